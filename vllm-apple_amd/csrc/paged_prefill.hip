// Chunked-prefill paged attention on MFMA (gfx950).
//
// Reference semantics: paged_attention_v2_prefill
// (vllm_apple/metal/kernels/paged_attention_v2.metal:375-478): query row t
// (sequence token_to_seq[t], position positions[t]) attends to cache positions
// [0, positions[t]] through that sequence's block table.  The cached prefix and
// the causal mask inside the chunk both follow from the positions, so the
// kernel needs no query_start_loc and accepts any token order.
//
// Work decomposition
//   block = 4 waves = (token subtile, query head) pairs of one kv head: 4 heads
//           x 32 tokens for GQA groups >= 4, 2 x 64 for pairs, 1 x 128 for MHA.
//           All waves share every K/V tile staged in LDS.
//   grid  = (query tile, kv_head x head chunk).
//   For each distinct sequence among the tile's tokens (normally one) the
//   workgroup walks 64-key tiles of that sequence's cache:
//     S^T[64 keys x 32 queries] = K Q^T   (2 x D/16 mfma 32x32x16)
//     P = exp2(S*scale*log2e - m), causal/row mask as -inf (fp16: Q is
//       prescaled by scale*log2e and the accumulators start at -m, so the
//       MFMAs deliver the exponent directly)
//     O^T[D x 32 queries]      += V^T P^T (D/32 x 4 mfma 32x32x16)
//   The MFMA output layout of S^T (lane = query, 16 keys per lane) is the B
//   operand layout of the PV product, so the per-query softmax statistics sit
//   in the lanes that own the query's accumulators.
//
// Memory: K/V tiles move from HBM straight into LDS with the gfx950 direct
// loads (global_load_lds_dwordx4: lane i of a wave writes LDS bytes
// [16i, 16i+16) after the wave-uniform base in M0), double-buffered, so the
// next tile streams in during this tile's math with no registers, address
// arithmetic or LDS stores of its own.  The loads are inline asm the compiler
// does not track; an explicit wait and barrier per tile publish each tile.  Wave w
// fetches the tile's 16-key group w, which lies inside one cache block.
// Rows are unpadded; 16-byte chunks are XOR-swizzled by row so that both the
// K operand reads (ds_read_b128 down 32 rows) and the transposed V^T reads
// (ds_read_b64_tr_b16: within each 16-lane group, lanes 4r..4r+3 name 8-byte
// pieces of row r and lane i receives element i of rows 0..3) hit distinct
// banks.  V rows past the context or in a missing block are zero-filled, so
// masked keys (P = 0) contribute exactly zero.
//
// Head sizes: the kernel computes at D in {32, 64, 96, 128}; a head size hd
// below D (a multiple of 8) runs the next larger D with the chunks past hd
// zero-filled in LDS instead of loaded, Q's past hd zero, and only the first
// hd dims of a row written (the kPad instantiations).
#include "common.h"

namespace vaa {
namespace {

constexpr int kQT = 32;       // query tokens per wave (MFMA columns)
constexpr int kKT = 64;       // keys per tile: four 16-key groups, one per wave
constexpr int kWavesP = 4;    // waves per workgroup
constexpr int kXcds = 8;      // accelerator complex dies on MI355X
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold (log2 units)
constexpr int kThreadsP = kWavesP * kWave;
constexpr int kMaxPrefillSplits = 1024;  // grid z of the split-K prefill
static_assert(kKT == 16 * kWavesP, "one 16-key group per wave");

typedef short i16x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const f16* q;
  const f16* kc;
  const f16* vc;
  const int32_t* bt;
  const int32_t* tok_seq;
  const int32_t* pos;
  f16* out;
  float scale_log2;
  int hd;                     // head size (<= D; the kPad kernels mask dims hd .. D-1)
  int num_tokens, num_seqs, max_blocks, block_size, G;
  int bs_shift;               // log2(block_size) when it is a power of two, else -1
  // block_size is a multiple of 16, so each wave's 16-key group lies in one
  // block.  Otherwise (the kPad kernels only) each row finds its own block.
  int bs16;
  int heads_per_wg, subtiles, head_chunks;
  int tiles_y, padded_tiles;  // logical grid rows; workgroups in use (multiple of 8)
  // Split-K over the keys (grid z): split z covers key tiles
  // [z*split_tiles, (z+1)*split_tiles), the last one the rest.  A row whose
  // context spans more than one split leaves a partial (unnormalised O, max
  // in the log2 domain, sum) per split in row (token*H + head)*n_splits + z
  // of ws_acc / ws_ml, and prefill_merge_kernel writes its output; split 0
  // writes the other rows directly.  split_tiles = 0: no split.
  int split_tiles, n_splits, num_q_heads;
  float* ws_acc;
  float* ws_ml;
  int64_t num_blocks;
  // Byte strides in 32 bits (narrow = 1 when the block strides fit 32 bits and
  // a block's token offsets 31): the full-group fast path of the fetch.
  int narrow;
  uint32_t ksb2, vsb2, kst2, vst2;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int64_t q_st, q_sh, o_st, o_sh;
};

template <int D>
struct PCfg {
  static constexpr int CH = D / 8;             // 16-byte chunks per row
  static constexpr int NK = D / 16;            // QK mfma steps (K-dim 16)
  static constexpr int NDT = D / 32;           // PV output tiles of 32 dims
  static constexpr int TILE = kKT * D;         // halves per staged K or V tile
  static constexpr int NI = CH / 4;            // direct loads per wave per tile (K or V)
  static constexpr int ROWB = D * 2;           // bytes per LDS row
};

// Chunk swizzle: physical chunk = logical chunk ^ swz(row).  For 8 or 16
// chunks per row the XOR takes all 8 values over 8 consecutive rows (K reads
// conflict-free) and distinct pairs over 4 aligned rows (V^T reads
// conflict-free); for 4 or 12 chunks it stays inside aligned groups of 4.
template <int D>
__device__ __forceinline__ int swz(int row) {
  if constexpr (D == 64 || D == 128) return ((row & 3) << 1) | ((row >> 2) & 1);
  else return (row >> 1) & 3;
}

// K tiles at D = 128: the chunk XOR takes all 16 values over 16 consecutive
// rows, so a ds_read_b128 of one logical chunk down 16 rows hits 16 distinct
// chunk slots (measured 201 against 121 B/clk per CU with the 8-value XOR).
// V keeps swz, which the transposed reads need.
template <int D>
__device__ __forceinline__ int swzk(int row) {
  if constexpr (D == 128) return row & 15;
  else return swz<D>(row);
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
  return v;
}

// max / sum of x over lanes l and l ^ 32.  v_permlane32_swap exchanges the
// upper half of its first operand with the lower half of its second, so with
// x in both, one result holds x's lower half twice and the other its upper
// half twice: a VALU exchange with no LDS round trip.  The sum adds the same
// two values in both halves, so both hold the identical result.
__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::x4 lds_tr4(const f16* p) {
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(typename Elem<T>::x4, r);
}

// s_waitcnt vmcnt(0) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4 left at its maximum, lgkmcnt 11:8): every direct load and LDS
// access of this wave has landed.
__device__ __forceinline__ void wait_all() { __builtin_amdgcn_s_waitcnt(0x0070); }
// A wave-uniform 32-bit read through the scalar unit (s_load_dword, via the
// constant address space: the block table is not written during the
// kernel).  lgkmcnt counts it, so waiting for it does not wait for the vector
// loads in flight, which complete in order.
__device__ __forceinline__ int32_t scalar_load_i32(const int32_t* p) {
  return *((const __attribute__((address_space(4))) int32_t*)(reinterpret_cast<uintptr_t>(p)));
}

// Workgroup barrier for LDS traffic only: s_waitcnt lgkmcnt(0) (vmcnt and
// expcnt at their maxima), so outstanding global loads stay in flight.
__device__ __forceinline__ void lds_bar() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}


// One 16-byte direct load per lane into LDS at lds + 16 * lane, issued as
// inline asm so that the compiler does not track it: a tracked LDS DMA makes
// it wait for every outstanding LDS read (lgkmcnt(0)) before any operand use,
// which defeats the read-ahead.  The explicit wait_all() + barrier at each
// tile boundary orders the DMA against the reads.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(lds)
               : "memory", "m0");
}
// The same from a wave-uniform base address (an SGPR pair) plus each lane's
// 32-bit byte offset: no per-lane 64-bit address arithmetic.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}

// The block-table entries of 64 consecutive blocks sit in one VGPR (one per
// lane) and are read with readlane, so the tile loop issues no scalar loads.
struct BlockWindow {
  int base;  // first block index held
  int vals;  // lane i: physical block of block base + i, or -1
};

__device__ __forceinline__ void window_load(const PrefillArgs& a, const int32_t* bts, int base,
                                            BlockWindow& w) {
  const int e = base + static_cast<int>(threadIdx.x % kWave);
  w.base = base;
  w.vals = e < a.max_blocks ? bts[e] : -1;
}

// Physical block of block index bi (wave-uniform), or -1 when the entry is
// missing or out of range.
__device__ __forceinline__ int64_t window_block(const PrefillArgs& a, const int32_t* bts,
                                                int bi, BlockWindow& w) {
  if (bi >= w.base + kWave) window_load(a, bts, bi, w);
  const int64_t phys = __builtin_amdgcn_readlane(w.vals, bi - w.base);
  return (phys >= 0 && phys < a.num_blocks) ? phys : -1;
}

// Loop-invariant per-lane addressing.
template <int D>
struct Lanes {
  uint32_t koff[PCfg<D>::NI];  // byte offset of this lane's chunk inside its K group
  uint32_t voff[PCfg<D>::NI];
  int row[PCfg<D>::NI];        // row inside the 16-key group for each direct load
  int kaddr[PCfg<D>::NK];      // LDS byte address of the K operand for step s
  int vaddr[PCfg<D>::NDT];     // LDS byte address of the V^T operand for dim tile dt
  uint32_t kval, vval;         // bit q: direct load q's K / V chunk lies below hd
};

template <int D>
__device__ __forceinline__ void lanes_init(const PrefillArgs& a, int wave, int lane,
                                           Lanes<D>& L) {
  using C = PCfg<D>;
#pragma unroll
  for (int q = 0; q < C::NI; ++q) {
    const int P = 64 * (wave * C::NI + q) + lane;  // chunk slot in the tile
    const int R = P / C::CH;                         // tile row (16*wave .. +15)
    const int lck = (P % C::CH) ^ swzk<D>(R);        // logical chunks stored there
    const int lcv = (P % C::CH) ^ swz<D>(R);
    L.row[q] = R & 15;
    L.koff[q] = static_cast<uint32_t>((R & 15) * a.k_st * 2 + lck * 16);
    L.voff[q] = static_cast<uint32_t>((R & 15) * a.v_st * 2 + lcv * 16);
  }
  L.kval = 0;
  L.vval = 0;
#pragma unroll
  for (int q = 0; q < C::NI; ++q) {
    const int P = 64 * (wave * C::NI + q) + lane;
    const int R = P / C::CH;
    L.kval |= (((P % C::CH) ^ swzk<D>(R)) * 8 < a.hd ? 1u : 0u) << q;
    L.vval |= (((P % C::CH) ^ swz<D>(R)) * 8 < a.hd ? 1u : 0u) << q;
  }
  const int qj = lane & 31, hb = lane >> 5;
  const int sk = swzk<D>(qj);
#pragma unroll
  for (int s2 = 0; s2 < C::NK; ++s2)
    L.kaddr[s2] = qj * C::ROWB + ((hb * (C::CH / 2) + s2) ^ sk) * 16;
  const int g16 = lane >> 4, i16 = lane & 15;
  const int r = 4 * hb + (i16 >> 2), j4 = i16 & 3;
  const int sv = swz<D>(r);
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
    L.vaddr[dt] = r * C::ROWB + ((4 * dt + 2 * (g16 & 1) + (j4 >> 1)) ^ sv) * 16 + (j4 & 1) * 8;
}

// First key position of the sequence's context [0, kv_len) that lies in an
// invalid block-table entry, or INT32_MAX.  A row whose context [0, lim]
// reaches it is never written (paged_attention_v2.metal:428); checking this
// once per sequence keeps the abort rule out of the tile loop.  The caller
// guarantees ceil(kv_len / block_size) <= max_blocks.
__device__ __forceinline__ int first_bad_key(const PrefillArgs& a, const int32_t* bts,
                                             int kv_len, int lane) {
  const int nb = (kv_len + a.block_size - 1) / a.block_size;
  int bad = INT32_MAX;
  for (int i = lane; i < nb; i += kWave) {
    const int64_t e = bts[i];
    if (e < 0 || e >= a.num_blocks) bad = min(bad, i);
  }
  bad = wave_min_i(bad);
  return bad == INT32_MAX ? INT32_MAX : bad * a.block_size;
}

// Splits a row at position pos spans: its context [0, pos] covers
// ceil((pos + 1) / kKT) key tiles; the last split takes any excess.
__device__ __forceinline__ int row_splits(const PrefillArgs& a, int pos) {
  const int tiles = (pos + kKT) / kKT;
  return min(a.n_splits, (tiles + a.split_tiles - 1) / a.split_tiles);
}

// Streams one 64-key tile into (kd, vd): wave w copies 16-key group w with
// direct loads, or zeros for rows past the context and for a missing block.
// kbase / vbase point at this kv head's slice of block 0.
template <int D, bool kPad>
__device__ __forceinline__ void tile_fetch(const PrefillArgs& a, const int32_t* bts,
                                           const char* kbase, const char* vbase, int key0,
                                           int kv_len, int wave, int lane, const Lanes<D>& L,
                                           BlockWindow& w, f16* kd, f16* vd,
                                           int phys_hint = -2) {
  using C = PCfg<D>;
  const int k0 = key0 + 16 * wave;
  if constexpr (!kPad) {
    // Full 16-key group in a valid block (every group but a sequence's
    // last): one window read, a 32-bit offset product per half and eight
    // direct loads from a wave-uniform base.  phys_hint (>= -1): the
    // group's block-table entry, read by the caller.
    if (a.narrow && k0 + 16 <= kv_len) {
      const int bi = a.bs_shift >= 0 ? (k0 >> a.bs_shift) : k0 / a.block_size;
      int phys;
      if (phys_hint >= -1) {
        phys = phys_hint;
      } else {
        if (bi >= w.base + kWave) window_load(a, bts, bi, w);
        phys = __builtin_amdgcn_readlane(w.vals, bi - w.base);
      }
      if (phys >= 0 && phys < a.num_blocks) {
        const uint32_t row0 = static_cast<uint32_t>(k0 - bi * a.block_size);
        const char* kb = kbase + static_cast<uint64_t>(static_cast<uint32_t>(phys)) * a.ksb2 +
                         row0 * a.kst2;
        const char* vb = vbase + static_cast<uint64_t>(static_cast<uint32_t>(phys)) * a.vsb2 +
                         row0 * a.vst2;
        const uint32_t kl = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
            reinterpret_cast<uintptr_t>(kd) + 1024 * (wave * C::NI)));
        const uint32_t vl = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
            reinterpret_cast<uintptr_t>(vd) + 1024 * (wave * C::NI)));
#pragma unroll
        for (int q = 0; q < C::NI; ++q) {
          dma16s(kb, L.koff[q], kl + 1024 * q);
          dma16s(vb, L.voff[q], vl + 1024 * q);
        }
        return;
      }
    }
  }
  int nvalid = 0, row0 = 0;
  int64_t mine = -1;
  if (k0 < kv_len) {
    const int bi = a.bs_shift >= 0 ? (k0 >> a.bs_shift) : k0 / a.block_size;
    mine = window_block(a, bts, bi, w);
    row0 = k0 - bi * a.block_size;
    if (mine >= 0) nvalid = min(16, kv_len - k0);
  }
  char* kdst = reinterpret_cast<char*>(kd) + 1024 * (wave * C::NI);
  char* vdst = reinterpret_cast<char*>(vd) + 1024 * (wave * C::NI);
  const uint32_t kl0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(kdst)));
  const uint32_t vl0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(vdst)));
  if constexpr (kPad) {
    if (!a.bs16) {
      // block_size not a multiple of 16: the group's rows may lie in several
      // blocks; each finds its own in the window (which is moved so that it
      // covers the group's last row).  Rows past the context or in a missing
      // block are zeros.
      if (k0 < kv_len) {
        const int last = min(k0 + 15, kv_len - 1) / a.block_size;
        if (last >= w.base + kWave) window_load(a, bts, k0 / a.block_size, w);
      }
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int q = 0; q < C::NI; ++q) {
        const int tok = k0 + L.row[q];
        const int bq = min(tok, kv_len - 1) / a.block_size;
        const int64_t ph = __shfl(w.vals, max(0, min(kWave - 1, bq - w.base)), kWave);
        const bool ok = tok < kv_len && ph >= 0 && ph < a.num_blocks;
        const int64_t rin = tok - static_cast<int64_t>(bq) * a.block_size;
        const char* kr = kbase + 2 * (ph * a.k_sb + rin * a.k_st) +
                         (L.koff[q] - static_cast<uint32_t>(L.row[q] * a.k_st * 2));
        const char* vr = vbase + 2 * (ph * a.v_sb + rin * a.v_st) +
                         (L.voff[q] - static_cast<uint32_t>(L.row[q] * a.v_st * 2));
        if (ok && ((L.kval >> q) & 1u)) dma16(kr, kl0 + 1024 * q);
        else *reinterpret_cast<u32x4*>(kdst + 1024 * q + 16 * lane) = z;
        if (ok && ((L.vval >> q) & 1u)) dma16(vr, vl0 + 1024 * q);
        else *reinterpret_cast<u32x4*>(vdst + 1024 * q + 16 * lane) = z;
      }
      return;
    }
  }
  if (nvalid > 0) {
    const char* kb = kbase + 2 * (mine * a.k_sb + static_cast<int64_t>(row0) * a.k_st);
    const char* vb = vbase + 2 * (mine * a.v_sb + static_cast<int64_t>(row0) * a.v_st);
    const u32x4 z = {0u, 0u, 0u, 0u};
    if (nvalid == 16) {  // every tile but a sequence's last
#pragma unroll
      for (int q = 0; q < C::NI; ++q) {
        if constexpr (kPad) {
          // Chunks past hd: zeros instead of the next row's elements.
          if ((L.kval >> q) & 1u) dma16(kb + L.koff[q], kl0 + 1024 * q);
          else *reinterpret_cast<u32x4*>(kdst + 1024 * q + 16 * lane) = z;
          if ((L.vval >> q) & 1u) dma16(vb + L.voff[q], vl0 + 1024 * q);
          else *reinterpret_cast<u32x4*>(vdst + 1024 * q + 16 * lane) = z;
        } else {
          dma16s(kb, L.koff[q], kl0 + 1024 * q);
          dma16s(vb, L.voff[q], vl0 + 1024 * q);
        }
      }
      return;
    }
#pragma unroll
    for (int q = 0; q < C::NI; ++q) {
      if (L.row[q] < nvalid) {
        if (!kPad || ((L.kval >> q) & 1u)) dma16(kb + L.koff[q], kl0 + 1024 * q);
        else *reinterpret_cast<u32x4*>(kdst + 1024 * q + 16 * lane) = z;
        if (!kPad || ((L.vval >> q) & 1u)) dma16(vb + L.voff[q], vl0 + 1024 * q);
        else *reinterpret_cast<u32x4*>(vdst + 1024 * q + 16 * lane) = z;
      } else {
        *reinterpret_cast<u32x4*>(kdst + 1024 * q + 16 * lane) = z;
        *reinterpret_cast<u32x4*>(vdst + 1024 * q + 16 * lane) = z;
      }
    }
  } else {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < C::NI; ++q) {
      *reinterpret_cast<u32x4*>(kdst + 1024 * q + 16 * lane) = z;
      *reinterpret_cast<u32x4*>(vdst + 1024 * q + 16 * lane) = z;
    }
  }
}

// One 64-key tile for this wave's 32 query rows: S^T = K Q^T as two
// independent 32-key MFMA row blocks, online softmax over both, then
// O^T += V^T P^T over four 16-key groups.  The LDS operand reads run ahead
// of their MFMAs (kKAhead K reads, kVAhead V^T pairs; the first V^T pairs
// are issued before the softmax, whose VALU work then hides their latency),
// and scheduling barriers keep the compiler from hoisting every read (which
// would not fit the register budget of two waves per SIMD).  With the direct
// loads untracked (dma16) the compiler waits for each read with a partial
// lgkmcnt, so a few reads ahead suffice.  fp16 at D = 128 reads three K
// operands ahead: its accumulator-initialisation tile (minit) takes the
// registers of the fourth (256 VGPRs, no spills); the rest keep four.
template <int D, typename T>
constexpr int kKAhead = (D == 128 && !Elem<T>::kSplitP) ? 3 : 4;
constexpr int kVAhead = 4;

template <int D, typename T>
__device__ __forceinline__ void tile_math(const PrefillArgs& a, const f16* kt, const f16* vt,
                                          int key0, int lim, int hb, const Lanes<D>& L,
                                          const u32x4 (&qb)[PCfg<D>::NK], float& m_run,
                                          float& l_part, f32x16 (&acc)[PCfg<D>::NDT],
                                          f32x16& minit) {
  using C = PCfg<D>;
  using X4 = typename Elem<T>::x4;
  using X8 = typename Elem<T>::x8;
  constexpr int NKR = 2 * C::NK;   // K operand reads (b128)
  constexpr int NPV = C::NDT * 4;  // PV MFMAs, one V^T pair each
  const char* kbytes = reinterpret_cast<const char*>(kt);
  const char* vbytes = reinterpret_cast<const char*>(vt);
  // S^T block j: A lane = K[32j + l%32][hb*D/2 + 8s .. +7]; read i covers
  // step i/2 of block i%2.
  u32x4 kA[NKR];
  auto kread = [&](int i) {
    kA[i] = *reinterpret_cast<const u32x4*>(kbytes + L.kaddr[i >> 1] + 32 * (i & 1) * C::ROWB);
  };
#pragma unroll
  for (int i = 0; i < kKAhead<D, T> && i < NKR; ++i) kread(i);
  __builtin_amdgcn_sched_barrier(0);
  // fp16: Q is prescaled by scale*log2(e) and both accumulator chains start
  // at -m_sub (minit), so S^T comes out of the MFMAs as s - m_sub in the
  // log2 domain and p = 2^(that) is one v_exp_f32.
  f32x16 sacc[2];
  if constexpr (!Elem<T>::kSplitP) {
    sacc[0] = minit;
    sacc[1] = minit;
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[j][r] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < NKR; ++i) {
    if (i + kKAhead<D, T> < NKR) kread(i + kKAhead<D, T>);
    sacc[i & 1] = Elem<T>::mfma32x32x16(__builtin_bit_cast(X8, kA[i]),
                                        __builtin_bit_cast(X8, qb[i >> 1]), sacc[i & 1]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // V^T for MFMA i (key group i / NDT, dim tile i % NDT) from the
  // transposing LDS read.
  X4 vlo[NPV], vhi[NPV];
  auto vread = [&](int i) {
    const int g = i / C::NDT, dt = i % C::NDT;
    const f16* vp = reinterpret_cast<const f16*>(vbytes + L.vaddr[dt] + 16 * g * C::ROWB);
    vlo[i] = lds_tr4<T>(vp);
    vhi[i] = lds_tr4<T>(vp + 8 * D);
  };
#pragma unroll
  for (int i = 0; i < kVAhead && i < NPV; ++i) vread(i);
  __builtin_amdgcn_sched_barrier(0);
  // Lane holds keys 32j + 8(r/4) + 4hb + r%4 for query qj.  The mask is only
  // evaluated when some row of the wave cannot see the whole tile.
  const int rel = lim - key0;
  if (__builtin_amdgcn_ballot_w64(rel < kKT - 1) != 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kl = 32 * j + 8 * (r >> 2) + 4 * hb + (r & 3);
        if (kl > rel) sacc[j][r] = -INFINITY;
      }
  }
  // Two chains of three-operand maxima (v_max3_f32) over the lane's 32 keys.
  float mx0 = fmaxf(sacc[0][0], sacc[0][1]), mx1 = fmaxf(sacc[1][0], sacc[1][1]);
#pragma unroll
  for (int r = 2; r < 16; r += 2) {
    mx0 = fmaxf(fmaxf(mx0, sacc[0][r]), sacc[0][r + 1]);
    mx1 = fmaxf(fmaxf(mx1, sacc[1][r]), sacc[1][r + 1]);
  }
  // pb[g]: B operand for 16-key group g (keys 16g + 8(i/4) + 4hb + i%4);
  // with Elem<T>::kSplitP (bf16) p = pb + pl, two PV products.
  X8 pb[4], pl[4];
  if constexpr (!Elem<T>::kSplitP) {
    // rel = this tile's row max relative to m_sub.  Lazy rescale: keep the
    // reference max unless a score exceeds it by more than 2^8 (p stays
    // <= 256, exact in fp16); the wave-uniform branch is taken on a row's
    // first tile and on rare outliers only.  Only lanes whose max grows
    // rescale (a fully masked lane keeps m_run = -inf).
    const float rel = half_max(fmaxf(mx0, mx1));
    const bool fresh = m_run == -INFINITY;
    if (__builtin_amdgcn_ballot_w64(rel > (fresh ? -INFINITY : kRescaleLog2)) != 0) {
      float shift = 0.f;
      if (rel > (fresh ? -INFINITY : 0.f)) {
        const float m_new = rel + (fresh ? 0.f : m_run);
        const float alpha = fast_exp2(m_run - m_new);  // 0 when m_run = -inf
        l_part *= alpha;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) acc[dt] *= alpha;
        m_run = m_new;
        shift = rel;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[j][r] -= shift;
      const float mi = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
      for (int r = 0; r < 16; ++r) minit[r] = mi;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        pb[2 * j + (r >> 3)][r & 7] = Elem<T>::from_f(fast_exp2(sacc[j][r]));
    // The row sum takes the probabilities as the PV product sees them (the
    // rounded fp16 values), two per v_dot2c_f32_f16 against (1, 1).
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 one = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
    float l0 = 0.f, l1 = 0.f;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      l0 = __builtin_amdgcn_fdot2(h2{pb[gq][0], pb[gq][1]}, one, l0, false);
      l1 = __builtin_amdgcn_fdot2(h2{pb[gq][2], pb[gq][3]}, one, l1, false);
      l0 = __builtin_amdgcn_fdot2(h2{pb[gq][4], pb[gq][5]}, one, l0, false);
      l1 = __builtin_amdgcn_fdot2(h2{pb[gq][6], pb[gq][7]}, one, l1, false);
    }
    l_part += l0 + l1;
  } else {
    const float mx = half_max(fmaxf(mx0, mx1)) * a.scale_log2;
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleLog2) != 0 && mx > m_run) {
      const float alpha = fast_exp2(m_run - mx);  // 0 when m_run = -inf
      l_part *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) acc[dt] *= alpha;
      m_run = mx;
    }
    const float m_sub = (m_run == -INFINITY) ? 0.f : m_run;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(sacc[j][r], a.scale_log2, -m_sub));
        pb[2 * j + (r >> 3)][r & 7] = Elem<T>::from_f(p);
        pl[2 * j + (r >> 3)][r & 7] =
            Elem<T>::from_f(p - Elem<T>::to_f(pb[2 * j + (r >> 3)][r & 7]));
        l_part += p;
      }
  }
  __builtin_amdgcn_sched_barrier(0);
  // O^T += V^T P^T.
#pragma unroll
  for (int i = 0; i < NPV; ++i) {
    if (i + kVAhead < NPV) vread(i + kVAhead);
    const int g = i / C::NDT, dt = i % C::NDT;
    const X8 va = {vlo[i][0], vlo[i][1], vlo[i][2], vlo[i][3],
                   vhi[i][0], vhi[i][1], vhi[i][2], vhi[i][3]};
    acc[dt] = Elem<T>::mfma32x32x16(va, pb[g], acc[dt]);
    if constexpr (Elem<T>::kSplitP) acc[dt] = Elem<T>::mfma32x32x16(va, pl[g], acc[dt]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int D, typename T, bool kPad>
__global__ void __launch_bounds__(kThreadsP) __attribute__((amdgpu_waves_per_eu(2, 2)))
paged_prefill_kernel(PrefillArgs a) {
  using C = PCfg<D>;
  // Two K and two V tile buffers; the direct loads into one are ordered
  // against the reads of the other by the per-tile wait and barrier.
  __shared__ __align__(16) f16 k0s[C::TILE];
  __shared__ __align__(16) f16 k1s[C::TILE];
  __shared__ __align__(16) f16 v0s[C::TILE];
  __shared__ __align__(16) f16 v1s[C::TILE];
  __shared__ int red[2][kWavesP];

  // XCD-aware placement: the hardware hands consecutive workgroup ids to the
  // 8 XCDs in turn, so id i runs on XCD i % 8.  Give each XCD a contiguous
  // range of (kv head, query tile) work so the query tiles that reuse one
  // sequence's K/V tiles share that XCD's L2.  The second half of an XCD's
  // range is walked backwards: its workgroups take the CUs' second slots in
  // dispatch order, so a CU pairs an early query tile of a chunk (short
  // causal context) with a late one (long context) and the CUs finish
  // together (C3: 6 % faster than pairing equal tiles).
  const int gx = gridDim.x;
  const int id = blockIdx.x + gx * blockIdx.y;
  if (id >= a.padded_tiles) return;  // grid rounding beyond the padded count
  const int per_xcd = a.padded_tiles / kXcds;
  int kx = id / kXcds;
  if (kx >= per_xcd / 2) kx = per_xcd - 1 - (kx - per_xcd / 2);
  const int logical = (id % kXcds) * per_xcd + kx;
  if (logical >= gx * a.tiles_y) return;
  const int tile_x = logical % gx, tile_y = logical / gx;
  const int split = blockIdx.z;
  const int kvh = tile_y / a.head_chunks;
  const int hchunk = tile_y % a.head_chunks;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int hw = wave % a.heads_per_wg, sub = wave / a.heads_per_wg;
  const int ghead = hchunk * a.heads_per_wg + hw;             // head index in the group
  const bool math = sub < a.subtiles && ghead < a.G;         // this wave computes
  const int head = kvh * a.G + (ghead < a.G ? ghead : 0);
  const int qj = lane & 31, hb = lane >> 5;

  // Per-lane query token (lanes l and l+32 share token qj).
  const int tok = tile_x * (kQT * a.subtiles) + (sub < a.subtiles ? sub : 0) * kQT + qj;
  int tseq = -1, tpos = -1;
  if (sub < a.subtiles && tok < a.num_tokens) {
    tseq = a.tok_seq[tok];
    tpos = a.pos[tok];
  }
  // Q^T as B operand: lane holds Q[token qj][hb*D/2 + 8s .. +7], s < NK.
  // Issued right after the token's sequence and position, before the rows
  // are validated (a row past num_tokens reads the last token's row; an
  // invalid row's scores are all masked), so the load is in flight during
  // the sequence discovery; prescaled before the first tile's math.
  u32x4 qb[C::NK];
  {
    const int qtok = min(tok, a.num_tokens - 1);
    const f16* qp = a.q + static_cast<int64_t>(qtok) * a.q_st + head * a.q_sh + hb * (D / 2);
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      if constexpr (kPad)
        qb[s] = (hb * (D / 2) + 8 * s < a.hd) ? ld16(qp + 8 * s) : u32x4{0u, 0u, 0u, 0u};
      else
        qb[s] = ld16(qp + 8 * s);
    }
  }
  bool q_ready = false;
  bool row_ok = tseq >= 0 && tseq < a.num_seqs && tpos >= 0;
  if (row_ok) {
    const int64_t nb = (static_cast<int64_t>(tpos) + a.block_size) / a.block_size;
    if (nb > a.max_blocks) row_ok = false;  // context longer than the table
  }
  bool done = !row_ok;
  bool aborted = false;

  f32x16 minit;
#pragma unroll
  for (int r = 0; r < 16; ++r) minit[r] = 0.f;

  float m_run = -INFINITY, l_part = 0.f;
  f32x16 acc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  Lanes<D> L;
  lanes_init<D>(a, wave, lane, L);
  const char* kbase = reinterpret_cast<const char*>(a.kc + kvh * a.k_sh);
  const char* vbase = reinterpret_cast<const char*>(a.vc + kvh * a.v_sh);

  while (true) {
    // Next sequence among the workgroup's unfinished tokens, and its context.
    int s = wave_min_i(done ? INT32_MAX : tseq);
    if (lane == 0) red[0][wave] = s;
    lds_bar();
    s = red[0][0];
#pragma unroll
    for (int w = 1; w < kWavesP; ++w) s = min(s, red[0][w]);
    if (s == INT32_MAX) break;
    const bool active = !done && tseq == s;
    int kv_len = wave_max_i(active ? tpos + 1 : 0);
    if (lane == 0) red[1][wave] = kv_len;
    lds_bar();
    kv_len = red[1][0];
#pragma unroll
    for (int w = 1; w < kWavesP; ++w) kv_len = max(kv_len, red[1][w]);
    const int n_kt = (kv_len + kKT - 1) / kKT;
    const int32_t* bts = a.bt + static_cast<int64_t>(s) * a.max_blocks;
    const int lim = active ? tpos : -1;  // last key position this row may see
    // This workgroup's key tiles of the sequence: all of them, or its split.
    int t_lo = 0, t_hi = n_kt;
    if (a.split_tiles > 0) {
      t_lo = split * a.split_tiles;
      if (split != a.n_splits - 1) t_hi = min(n_kt, t_lo + a.split_tiles);
    }

    // Double buffer: the next tile's direct loads are issued before this
    // tile's math; one wait + barrier per tile publishes it.
    if (t_lo < t_hi) {
      // The first tile's block-table entry with a scalar load (its own
      // counter: the fetch does not wait behind the Q loads in flight); the
      // window for the later tiles is loaded by the next fetch.
      int phys0 = -2;
      if constexpr (!kPad) {
        const int k0 = t_lo * kKT + 16 * wave;
        const int bi = a.bs_shift >= 0 ? (k0 >> a.bs_shift) : k0 / a.block_size;
        if (a.narrow && k0 + 16 <= kv_len && bi < a.max_blocks)
          phys0 = scalar_load_i32(bts + bi);
      }
      BlockWindow win;
      if (phys0 >= -1) {
        // Loaded by the first fetch that needs it.
        win.base = -(1 << 30);
        win.vals = -1;
      } else {
        window_load(a, bts, a.bs_shift >= 0 ? (t_lo * kKT) >> a.bs_shift
                                            : (t_lo * kKT) / a.block_size, win);
      }
      tile_fetch<D, kPad>(a, bts, kbase, vbase, t_lo * kKT, kv_len, wave, lane, L, win, k0s, v0s,
                          phys0);
      // The abort check's table reads overlap the first tile's loads.
      if (lim >= first_bad_key(a, bts, kv_len, lane)) aborted = true;
      wait_all();
      __builtin_amdgcn_s_barrier();
      if constexpr (!Elem<T>::kSplitP) {
        if (!q_ready) {
          // fp16: Q prescaled by scale*log2(e), rounded once to fp16.
#pragma unroll
          for (int s2 = 0; s2 < C::NK; ++s2) {
            f16x8 h = __builtin_bit_cast(f16x8, qb[s2]);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              h[e] = static_cast<f16>(static_cast<float>(h[e]) * a.scale_log2);
            qb[s2] = __builtin_bit_cast(u32x4, h);
          }
          q_ready = true;
        }
      }
      for (int kt = t_lo; kt < t_hi; kt += 2) {
        if (kt + 1 < t_hi)
          tile_fetch<D, kPad>(a, bts, kbase, vbase, (kt + 1) * kKT, kv_len, wave, lane, L, win, k1s,
                        v1s);
        if (math) tile_math<D, T>(a, k0s, v0s, kt * kKT, lim, hb, L, qb, m_run, l_part, acc, minit);
        wait_all();
        __builtin_amdgcn_s_barrier();
        if (kt + 1 >= t_hi) break;
        if (kt + 2 < t_hi)
          tile_fetch<D, kPad>(a, bts, kbase, vbase, (kt + 2) * kKT, kv_len, wave, lane, L, win, k0s,
                        v0s);
        if (math)
          tile_math<D, T>(a, k1s, v1s, (kt + 1) * kKT, lim, hb, L, qb, m_run, l_part, acc, minit);
        wait_all();
        __builtin_amdgcn_s_barrier();
      }
    }
    if (t_lo >= t_hi && lim >= first_bad_key(a, bts, kv_len, lane)) aborted = true;
    done = done || active;
  }

  if (!math) return;
  const float l_tot = half_sum(l_part);
  if (!row_ok) return;
  if (a.split_tiles > 0) {
    const int rs = row_splits(a, tpos);
    if (rs > 1) {
      // Partial of this split (fully masked: max -inf, sum 0); an aborted
      // row is marked by a negative sum, which the merge leaves unwritten.
      if (split >= rs) return;
      const int64_t row =
          (static_cast<int64_t>(tok) * a.num_q_heads + head) * a.n_splits + split;
      float* dst = a.ws_acc + row * D;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 v = {acc[dt][4 * rg], acc[dt][4 * rg + 1], acc[dt][4 * rg + 2],
                           acc[dt][4 * rg + 3]};
          *reinterpret_cast<f32x4*>(dst + 32 * dt + 8 * rg + 4 * hb) = v;
        }
      }
      if (hb == 0) {
        a.ws_ml[row * 2 + 0] = m_run;
        a.ws_ml[row * 2 + 1] = aborted ? -1.f : l_tot;
      }
      return;
    }
    if (split != 0) return;  // the row's keys all lie in split 0
  }
  if (aborted) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  f16* op = a.out + static_cast<int64_t>(tok) * a.o_st + head * a.o_sh;
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      typename Elem<T>::x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = Elem<T>::from_f(acc[dt][4 * rg + i] * inv);
      const int d = 32 * dt + 8 * rg + 4 * hb;
      if (!kPad || d < a.hd) *reinterpret_cast<typename Elem<T>::x4*>(op + d) = o;
    }
  }
}

// Log-sum-exp merge of the split rows' partials: out = sum_z 2^(m_z - M) acc_z /
// sum_z 2^(m_z - M) l_z with M the largest m_z of a piece that saw keys.  One
// 256-thread workgroup per token; a thread takes four dimensions of one head
// for each of kMergeItems heads at a time, and walks the pieces once with a
// running maximum (each piece rescales the sums when it raises it), so the
// loads of every piece and item are independent and in flight together (a
// first pass for the maximum put a dependent round trip before the partial
// loads).  Rows the reference leaves unwritten stay untouched: the same
// validity rules as the attention kernel, and the abort mark of split 0.
constexpr int kMergeThreads = 256;
constexpr int kMergeItems = 4;

template <int D, typename T>
__global__ void __launch_bounds__(kMergeThreads) prefill_merge_kernel(PrefillArgs a) {
  const int tok = blockIdx.x;
  const int seq = a.tok_seq[tok], pos = a.pos[tok];
  if (seq < 0 || seq >= a.num_seqs || pos < 0) return;
  if ((static_cast<int64_t>(pos) + a.block_size) / a.block_size > a.max_blocks) return;
  const int rs = row_splits(a, pos);
  if (rs <= 1) return;
  constexpr int G4 = D / 4;
  const int H = a.num_q_heads;
  for (int it0 = threadIdx.x; it0 < H * G4; it0 += kMergeThreads * kMergeItems) {
    int64_t row0[kMergeItems];
    float M[kMergeItems], den[kMergeItems];
    f32x4 num[kMergeItems];
    bool aborted[kMergeItems];
#pragma unroll
    for (int i = 0; i < kMergeItems; ++i) {
      const int it = min(it0 + i * kMergeThreads, H * G4 - 1);
      row0[i] = (static_cast<int64_t>(tok) * H + it / G4) * a.n_splits;
      M[i] = -INFINITY;
      den[i] = 0.f;
      num[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      aborted[i] = false;
    }
    for (int z = 0; z < rs; ++z) {
#pragma unroll
      for (int i = 0; i < kMergeItems; ++i) {
        const int it = min(it0 + i * kMergeThreads, H * G4 - 1);
        const int64_t row = row0[i] + z;
        const float mz = a.ws_ml[row * 2], lz = a.ws_ml[row * 2 + 1];
        const f32x4 az = *reinterpret_cast<const f32x4*>(a.ws_acc + row * D + (it % G4) * 4);
        if (z == 0 && lz < 0.f) aborted[i] = true;
        if (!(lz > 0.f)) continue;  // a piece that saw no keys (max -inf)
        const float Mn = fmaxf(M[i], mz);
        const float so = fast_exp2(M[i] - Mn);  // 0 while M = -inf
        const float sn = fast_exp2(mz - Mn);
        num[i] = num[i] * so + az * sn;
        den[i] = den[i] * so + lz * sn;
        M[i] = Mn;
      }
    }
#pragma unroll
    for (int i = 0; i < kMergeItems; ++i) {
      const int it = it0 + i * kMergeThreads;
      if (it >= H * G4 || aborted[i]) continue;
      const int head = it / G4, d = (it % G4) * 4;
      if (d >= a.hd) continue;  // padded dims (hd is a multiple of 8)
      T* o = reinterpret_cast<T*>(a.out) + static_cast<int64_t>(tok) * a.o_st + head * a.o_sh + d;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = Elem<T>::from_f(den[i] > 0.f ? num[i][e] / den[i] : 0.f);
    }
  }
}

template <int D, typename T, bool kPad>
int launch_prefill(const PrefillArgs& a, int num_kv_heads, hipStream_t stream) {
  const int per_wg = kQT * a.subtiles;
  const int gx = (a.num_tokens + per_wg - 1) / per_wg, gy = num_kv_heads * a.head_chunks;
  // Pad the grid to a multiple of the XCD count so every logical tile has a
  // slot under the XCD remap (surplus workgroups exit at once).
  const int total = gx * gy, padded = (total + kXcds - 1) / kXcds * kXcds;
  PrefillArgs b = a;
  b.tiles_y = gy;
  b.padded_tiles = padded;
  dim3 grid(gx, (padded + gx - 1) / gx, a.split_tiles > 0 ? a.n_splits : 1);
  hipLaunchKernelGGL((paged_prefill_kernel<D, T, kPad>), grid, dim3(kThreadsP), 0, stream, b);
  const int st = check_launch("paged_prefill_kernel");
  if (st || a.split_tiles <= 0) return st;
  hipLaunchKernelGGL((prefill_merge_kernel<D, T>), dim3(a.num_tokens), dim3(kMergeThreads), 0,
                     stream, b);
  return check_launch("prefill_merge_kernel");
}

}  // namespace
}  // namespace vaa

using namespace vaa;

namespace vaa {
namespace {

// Split-K plan for max_seq_len: key tiles per split and the number of splits.
int prefill_split_plan(const char* what, const vaa_attn_params* p, int split_keys,
                       int* split_tiles, int* n_splits) {
  if (split_keys <= 0 || split_keys % kKT != 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: split_keys=%d must be a positive multiple of %d",
                what, split_keys, kKT);
  int64_t max_len = p->max_seq_len;
  const int64_t cap = static_cast<int64_t>(p->max_blocks_per_seq) * p->block_size;
  if (max_len > cap) max_len = cap;
  if (max_len < 1) max_len = 1;
  const int64_t tiles = (max_len + kKT - 1) / kKT, per = split_keys / kKT;
  const int64_t ns = (tiles + per - 1) / per;
  if (ns > kMaxPrefillSplits)
    return fail(VAA_ERR_UNSUPPORTED, "%s: split_keys=%d cuts max_seq_len=%lld into %lld > %d splits",
                what, split_keys, (long long)max_len, (long long)ns, kMaxPrefillSplits);
  *split_tiles = static_cast<int>(per);
  *n_splits = static_cast<int>(ns);
  return VAA_OK;
}

size_t prefill_ws_bytes(const vaa_attn_params* p, int num_tokens, int n_splits) {
  if (n_splits <= 1 || num_tokens <= 0) return 0;
  return static_cast<size_t>(num_tokens) * p->num_query_heads * n_splits *
         (static_cast<size_t>(padded_head(p->head_size)) + 2) * sizeof(float);
}

int prefill_impl(const char* what, const vaa_attn_params* p, const uint16_t* query,
                 const uint16_t* key_cache, const uint16_t* value_cache,
                 const int32_t* block_table, const int32_t* token_to_seq,
                 const int32_t* positions, uint16_t* output, int num_tokens, int split_keys,
                 void* workspace, size_t workspace_bytes, void* stream) {
  if (!p) return fail(VAA_ERR_INVALID_ARG, "%s: null params", what);
  if (!head_size_ok(p->head_size))
    return fail(VAA_ERR_UNSUPPORTED, "%s: head_size=%d (a multiple of 8 up to 128)", what,
                p->head_size);
  if (p->block_size <= 0 || p->num_kv_heads <= 0 || p->num_query_heads <= 0 ||
      p->num_query_heads % p->num_kv_heads != 0 ||
      p->queries_per_kv != p->num_query_heads / p->num_kv_heads ||
      p->max_blocks_per_seq <= 0 || p->num_blocks <= 0 || p->num_seqs < 0 ||
      num_tokens < 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: bad shape params", what);
  if (!valid_dtype(p->dtype))
    return fail(VAA_ERR_UNSUPPORTED, "%s: dtype=%d", what, p->dtype);
  if (p->num_query_heads > 65535)
    return fail(VAA_ERR_UNSUPPORTED, "%s: num_query_heads=%d", what, p->num_query_heads);
  int split_tiles = 0, n_splits = 1;
  if (split_keys != 0) {
    const int st = prefill_split_plan(what, p, split_keys, &split_tiles, &n_splits);
    if (st) return st;
    if (n_splits <= 1) split_tiles = 0;  // one split: the plain kernel
  }
  if (num_tokens == 0) return VAA_OK;
  if (!query || !key_cache || !value_cache || !block_table || !token_to_seq ||
      !positions || !output)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  const int64_t strides[] = {p->k_stride_block, p->k_stride_head, p->k_stride_token,
                             p->v_stride_block, p->v_stride_head, p->v_stride_token,
                             p->q_stride_token, p->q_stride_head, p->o_stride_token,
                             p->o_stride_head};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0)
      return fail(VAA_ERR_INVALID_ARG, "%s: strides must be multiples of 8 elements", what);
  if (!aligned16(query) || !aligned16(key_cache) || !aligned16(value_cache) ||
      !aligned16(output))
    return fail(VAA_ERR_INVALID_ARG, "%s: tensors must be 16-byte aligned", what);
  PrefillArgs a;
  a.split_tiles = split_tiles;
  a.n_splits = n_splits;
  a.num_q_heads = p->num_query_heads;
  a.ws_acc = nullptr;
  a.ws_ml = nullptr;
  if (split_tiles > 0) {
    const size_t need = prefill_ws_bytes(p, num_tokens, n_splits);
    if (!workspace || workspace_bytes < need)
      return fail(VAA_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu needed", what,
                  workspace_bytes, need);
    if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
      return fail(VAA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", what);
    const size_t rows = static_cast<size_t>(num_tokens) * p->num_query_heads * n_splits;
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + rows * padded_head(p->head_size);
  }
  a.q = reinterpret_cast<const f16*>(query);
  a.kc = reinterpret_cast<const f16*>(key_cache);
  a.vc = reinterpret_cast<const f16*>(value_cache);
  a.bt = block_table;
  a.tok_seq = token_to_seq;
  a.pos = positions;
  a.out = reinterpret_cast<f16*>(output);
  a.scale_log2 = p->scale * kLog2e;
  a.hd = p->head_size;
  a.num_tokens = num_tokens;
  a.num_seqs = p->num_seqs;
  a.max_blocks = p->max_blocks_per_seq;
  a.block_size = p->block_size;
  a.bs_shift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if (p->block_size == (1 << sh)) a.bs_shift = sh;
  a.bs16 = p->block_size % 16 == 0 ? 1 : 0;
  a.G = p->queries_per_kv;
  // Waves = (token subtile, head) pairs: 4 heads x 32 tokens when the group
  // has >= 3 heads, 2 x 64 for pairs, 1 x 128 for MHA.
  if (a.G >= 3) {
    a.heads_per_wg = a.G >= 4 ? 4 : 3;
    a.subtiles = 1;
  } else {
    a.heads_per_wg = a.G;
    a.subtiles = kWavesP / a.G;
  }
  a.head_chunks = (a.G + a.heads_per_wg - 1) / a.heads_per_wg;
  a.num_blocks = p->num_blocks;
  {
    const int64_t bs = p->block_size;
    const bool fits = p->k_stride_block * 2 < (int64_t(1) << 32) &&
                      p->v_stride_block * 2 < (int64_t(1) << 32) &&
                      p->k_stride_token * 2 * bs < (int64_t(1) << 31) &&
                      p->v_stride_token * 2 * bs < (int64_t(1) << 31);
    a.narrow = fits ? 1 : 0;
    a.ksb2 = fits ? static_cast<uint32_t>(p->k_stride_block * 2) : 0u;
    a.vsb2 = fits ? static_cast<uint32_t>(p->v_stride_block * 2) : 0u;
    a.kst2 = fits ? static_cast<uint32_t>(p->k_stride_token * 2) : 0u;
    a.vst2 = fits ? static_cast<uint32_t>(p->v_stride_token * 2) : 0u;
  }
  a.k_sb = p->k_stride_block; a.k_sh = p->k_stride_head; a.k_st = p->k_stride_token;
  a.v_sb = p->v_stride_block; a.v_sh = p->v_stride_head; a.v_st = p->v_stride_token;
  a.q_st = p->q_stride_token; a.q_sh = p->q_stride_head;
  a.o_st = p->o_stride_token; a.o_sh = p->o_stride_head;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = p->dtype == VAA_DTYPE_BF16;
  // Head sizes below the computed size, and block sizes that are not a
  // multiple of 16, run the kPad kernels.
  const bool pad = padded_head(p->head_size) != p->head_size || p->block_size % 16 != 0;
#define VAA_PREFILL_CASE(DP)                                                 \
  case DP:                                                                   \
    if (pad)                                                                 \
      return bf ? launch_prefill<DP, bf16, true>(a, p->num_kv_heads, s)      \
                : launch_prefill<DP, f16, true>(a, p->num_kv_heads, s);      \
    return bf ? launch_prefill<DP, bf16, false>(a, p->num_kv_heads, s)       \
              : launch_prefill<DP, f16, false>(a, p->num_kv_heads, s);
  switch (padded_head(p->head_size)) {
    VAA_PREFILL_CASE(32)
    VAA_PREFILL_CASE(64)
    VAA_PREFILL_CASE(96)
    VAA_PREFILL_CASE(128)
  }
#undef VAA_PREFILL_CASE
  return fail(VAA_ERR_UNSUPPORTED, "head_size=%d", p->head_size);
}

}  // namespace
}  // namespace vaa

extern "C" int vaa_paged_attention_prefill(const vaa_attn_params* p,
                                           const uint16_t* query,
                                           const uint16_t* key_cache,
                                           const uint16_t* value_cache,
                                           const int32_t* block_table,
                                           const int32_t* token_to_seq,
                                           const int32_t* positions,
                                           uint16_t* output, int num_tokens,
                                           void* stream) {
  return prefill_impl("vaa_paged_attention_prefill", p, query, key_cache, value_cache,
                      block_table, token_to_seq, positions, output, num_tokens, 0, nullptr, 0,
                      stream);
}

extern "C" size_t vaa_paged_attention_prefill_workspace_size(const vaa_attn_params* p,
                                                             int num_tokens, int split_keys) {
  if (!p || p->max_blocks_per_seq <= 0 || p->block_size <= 0 || p->num_query_heads <= 0)
    return 0;
  int split_tiles = 0, n_splits = 1;
  if (prefill_split_plan("vaa_paged_attention_prefill_workspace_size", p, split_keys,
                         &split_tiles, &n_splits) != VAA_OK)
    return 0;
  return prefill_ws_bytes(p, num_tokens, n_splits);
}

extern "C" int vaa_paged_attention_prefill_split(const vaa_attn_params* p,
                                                 const uint16_t* query,
                                                 const uint16_t* key_cache,
                                                 const uint16_t* value_cache,
                                                 const int32_t* block_table,
                                                 const int32_t* token_to_seq,
                                                 const int32_t* positions, uint16_t* output,
                                                 int num_tokens, int split_keys,
                                                 void* workspace, size_t workspace_bytes,
                                                 void* stream) {
  if (split_keys == 0)
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_paged_attention_prefill_split: split_keys must be a positive multiple of %d",
                kKT);
  return prefill_impl("vaa_paged_attention_prefill_split", p, query, key_cache, value_cache,
                      block_table, token_to_seq, positions, output, num_tokens, split_keys,
                      workspace, workspace_bytes, stream);
}
