// Paged decode attention for gfx950 (CDNA4), GQA, split-K with a log-sum-exp
// merge, optional fused write of the new token's K/V.
//
// Reference semantics: paged_attention_fused.metal:107-328 and
// paged_attention_v2.metal:49-261 (online softmax in fp32 over the first
// seq_len cache positions of the sequence, kv head = q head / queries_per_kv,
// zero row for seq_len <= 0).
//
// Work decomposition
//   grid     = (partition, kv_head x head chunk, seq); one workgroup serves
//              every query head of the GQA group (up to 16, the MFMA columns),
//              so each K/V byte is read from HBM once.  Larger groups (MQA
//              with many heads) are cut into ceil(G/16) chunks of at most 16
//              heads, one workgroup each.
//   block    = 8 waves; each wave streams a contiguous run of 16-token tiles
//              with its own (max, sum, acc) and the waves are combined in LDS
//              at the end.  Fixed partitions of at most 1024 tokens use
//              4-wave workgroups, two per CU: one's start-up overlaps the
//              other's streaming.  The shared balanced split
//              (VAA_PARTITION_BALANCED_SHARED), for a decode that runs beside
//              another kernel, uses 4-wave workgroups too, four per CU's
//              worth of the split: a concurrent kernel's workgroups hold some
//              CUs, and the shorter pieces let the dispatcher give the free
//              CUs more of them.
//   split-K  = only when the (seq, kv_head) pairs cannot fill the GPU or the
//              lengths are unequal; partials (max, sum, acc) go to a workspace
//              and a second kernel merges them (log-sum-exp).  The merge is a
//              separate launch on purpose: a cross-workgroup handoff inside
//              one launch needs agent-scope release/acquire (an L2 writeback
//              and invalidate per workgroup on every XCD), which measured 3x
//              slower than the kernel boundary.
//
// Head sizes: the kernels compute at D in {32, 64, 96, 128}; a head size hd
// below D (any multiple of 8, e.g. 80 or 112, as the reference's generic
// kernels take any head size up to 128: paged_attention_fused.metal:208-233)
// runs the next larger D with the tail dims zero: Q and K chunks past hd load
// as zeros (so they add nothing to Q.K), V chunks past hd are not loaded, and
// only the first hd dims of a row are written.  Those kernels are the kPad
// instantiations; the four native sizes compile without the masks.
//
// Per 16-token tile a wave does
//   S^T[16 tok x 16 heads] = K[16 x D] * Q^T[D x 16]   (D/32 x mfma 16x16x32)
//   P = exp2(S*scale*log2e - m)                         (fp32, heads on lanes)
//   O^T[D x 16 heads]     += V^T[D x 16] * P^T[16 x 16] (D/16 x mfma 16x16x16)
// Heads >= queries_per_kv are zero columns.  S^T (not S) is computed so the
// MFMA output layout (lane = head, 4 tokens per lane) is exactly the B operand
// layout of the PV product and the per-head softmax statistics live in the
// same lanes as the head's accumulators: no shuffles besides the 2-step
// cross-lane max.
//
// Memory: each lane loads 16-byte pieces of one K row straight into the MFMA
// A-operand registers.  The contraction index is permuted identically in K
// and Q: MFMA step s, lane group g holds dims 32s + 8g .. +7, so the four
// lane groups of one token read 64 contiguous bytes per load instruction.  V
// is loaded with fully coalesced 16-byte loads, stored to a per-wave LDS tile
// (XOR-swizzled 16-byte chunks) and read back transposed with the gfx950
// ds_read_b64_tr_b16 (one read per MFMA operand).  The K/V stream is
// read once per call, so its loads carry the nontemporal hint (MI355X
// headline: 72 -> 79 % of HBM peak on one box; the hint on the earlier K lane
// map, 16-byte pieces 64 bytes apart, had cost 8 points); the balanced
// split hints V only (issue_tile).  Loads run one tile ahead of the math in
// two buffers (the 4-wave fixed-partition kernel: two tiles ahead in three
// rotating buffers), and the wave's block-table entries sit in a VGPR (one
// per lane) read with readlane, so the steady-state loop issues no scalar
// memory loads.
#include "common.h"

#include <atomic>

namespace vaa {
namespace {

typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;   // waves per workgroup
constexpr int kShortPartTiles = 64;  // fixed partitions up to 1024 tokens run 4-wave workgroups
// Balanced split: 4-wave workgroups, two per CU's worth of the split alone
// (C2u 0.115 -> 0.105 ms and C4 0.575 -> 0.547 ms against one 8-wave workgroup
// per CU, one box), four per CU's worth for VAA_PARTITION_BALANCED_SHARED
// beside a concurrent kernel (C5 step beside the prefill: 3, 4, 6, 8 ->
// 0.577, 0.571, 0.579, 0.587 ms; two: 0.597).  Three workgroups per CU's
// worth at three waves per SIMD: C2u the same, C4 and the C5 step slower.
//
// Loads run one tile ahead in the balanced and the 8-wave kernels (against
// two ahead, one box: C2u 0.1031-0.1035 -> 0.1011-0.1014 ms, headline
// 0.1631-0.1632 -> 0.1622-0.1623 ms, C1 7.1 -> 6.5 us) and two ahead in the
// 4-wave fixed-partition kernel (C4 at 512-token partitions: one ahead 0.685
// against 0.638 ms).
constexpr int kBalWaves = kWaves / 2;
constexpr int kBalPerCu = 2;
constexpr int kSharedPerCu = 4;
constexpr int kTile = 16;   // tokens per MFMA tile

// Tensors are raw 16-bit storage; the kernels' element type T (fp16 or bf16)
// gives the values their meaning.
struct DecodeArgs {
  const f16* q;
  f16* kc;
  f16* vc;
  const int32_t* bt;
  const int32_t* seq_lens;
  f16* out;
  const f16* new_k;
  const f16* new_v;
  // Split-K partials, one row per (piece, query head): unnormalised acc [D]
  // and (max in the log2 domain, sum).  Fixed partitions use rows
  // (seq*H + qhead)*max_parts + part; the balanced split uses
  // (y*(max_parts + num_seqs) + c + seq)*Gc + h, with y = kv head x head
  // chunk, max_parts = workgroups per y, and keeps its geometry in ws_hdr
  // (per, starts[0..num_seqs]).
  float* ws_acc;
  float* ws_ml;
  int* ws_hdr;
  float scale_log2;
  int hd;  // head size (<= D; the kPad kernels mask dims hd .. D-1)
  int num_seqs, max_blocks, block_size, num_kv_heads, num_q_heads, G;
  // block_size is a multiple of 16, so every 16-token tile lies in one block.
  // Otherwise (the kPad kernels only) each row of a tile finds its own block.
  int bs16;
  int Gc, chunks;  // query heads per chunk (<= 16) and chunks per kv head
  int part_tiles, max_parts;
  int lds_main;  // bytes of LDS before the balanced split's prefix sums
  int64_t num_blocks;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int64_t q_st, q_sh, o_st, o_sh, n_st, n_sh;
};

template <int D>
struct Cfg {
  static constexpr int NS = D / 32;               // QK mfma count (K-dim 32)
  static constexpr int NDT = D / 16;              // PV mfma count (16 dims each)
  static constexpr int CH = D / 8;                // 16-byte chunks per row
  static constexpr int VLD = kTile * CH / kWave;  // V loads per lane per tile
  static constexpr bool SWZ = (CH == 8 || CH == 16);
};

template <int D>
__device__ __forceinline__ int swz(int row) {
  if constexpr (Cfg<D>::SWZ) return ((row >> 2) & 3) << 1;
  return 0;
}

template <int D>
struct Tile {
  u32x4 k[Cfg<D>::NS];
  u32x4 v[Cfg<D>::VLD];
};

// Per-lane constants of the tile loads and LDS traffic.
template <int D>
struct LaneMap {
  uint32_t koff;               // element offset of this lane's K piece in a tile (step 0)
  uint32_t voff[Cfg<D>::VLD];  // element offset of V chunk i in a tile
  int vrow[Cfg<D>::VLD];       // tile row of V chunk i
  uint32_t wlds[Cfg<D>::VLD];  // LDS element offset where V chunk i is stored
  uint32_t trbase;             // V^T transposing read: this lane's 8-byte piece at chunk 0
  int trsw;                    // chunk swizzle of its row
  uint32_t kval, vval;         // kPad: bit s / i set when K step s / V chunk i is below hd
};

// Block-table window: lane i of `vals` holds the entry of block blk0 + i, so a
// chunk of up to 64 tiles (block_size 16) reads its physical blocks with
// readlane and the pipelined loop issues no scalar or table loads.
__device__ __forceinline__ int load_window(const DecodeArgs& a, int seq, int blk0, int lane) {
  const int e = blk0 + lane;
  return e < a.max_blocks ? a.bt[static_cast<int64_t>(seq) * a.max_blocks + e] : -1;
}

__device__ __forceinline__ int64_t window_block(const DecodeArgs& a, int vals, int blk0,
                                                int j) {
  return __builtin_amdgcn_readlane(vals, (j * kTile) / a.block_size - blk0);
}

// V rows always load with the nontemporal hint; K rows too when kStream.
// kStream is on for the fixed partitions (headline 78.4-78.7 % with V alone
// hinted, 78.8-79.1 % with both, one box) and off for the balanced split:
// beside a concurrent prefill the hint on K cost the C5 attention step 3 %
// (0.638-0.642 against 0.610-0.612 ms), and on the split alone C2u (0.1051
// against 0.1009 ms, one box).
template <int D, bool kStream = true, bool kPad = false>
__device__ __forceinline__ void issue_tile(const DecodeArgs& a, int64_t kbase,
                                          int64_t vbase, const LaneMap<D>& m,
                                          int64_t phys, int j, Tile<D>& t) {
  const int row0 = (j * kTile) % a.block_size;
  if (phys < 0 || phys >= a.num_blocks) phys = 0;  // masked by the caller
  const f16* kb = a.kc + kbase + phys * a.k_sb + row0 * a.k_st;
  const f16* vb = a.vc + vbase + phys * a.v_sb + row0 * a.v_st;
  const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int s = 0; s < Cfg<D>::NS; ++s) {
    if (kPad && !((m.kval >> s) & 1u)) {
      t.k[s] = z;
      continue;
    }
    t.k[s] = kStream ? ld16_stream(kb + m.koff + 32 * s) : ld16(kb + m.koff + 32 * s);
  }
#pragma unroll
  for (int i = 0; i < Cfg<D>::VLD; ++i)
    t.v[i] = (!kPad || ((m.vval >> i) & 1u)) ? ld16_stream(vb + m.voff[i]) : z;
}

// A tile whose rows may lie in different blocks (block_size not a multiple
// of 16): each row finds its physical block in the window (lane i of vals:
// block blk0 + i) with a cross-lane read.  Returns the rows that lie in valid
// blocks (bit r: row r); the others load row 0 of block 0 and are masked.
template <int D, bool kStream, bool kPad>
__device__ __forceinline__ uint32_t issue_tile_rows(const DecodeArgs& a, int64_t kbase,
                                                    int64_t vbase, const LaneMap<D>& m,
                                                    int vals, int blk0, int j, int lane,
                                                    Tile<D>& t) {
  using C = Cfg<D>;
  const int c16 = lane & 15, g = lane >> 4;
  auto row_at = [&](int row, int64_t& phys, int& rin) {
    const int tok = j * kTile + row;
    const int bi = tok / a.block_size;
    phys = __shfl(vals, bi - blk0, kWave);
    rin = tok - bi * a.block_size;
    const bool ok = phys >= 0 && phys < a.num_blocks;
    if (!ok) {
      phys = 0;
      rin = 0;
    }
    return ok;
  };
  const u32x4 z = {0u, 0u, 0u, 0u};
  int64_t pk;
  int rk;
  const bool kok = row_at(c16, pk, rk);
  const f16* kp = a.kc + kbase + pk * a.k_sb + rk * a.k_st + 8 * g;
#pragma unroll
  for (int s = 0; s < C::NS; ++s) {
    if (kPad && !((m.kval >> s) & 1u)) {
      t.k[s] = z;
      continue;
    }
    t.k[s] = kStream ? ld16_stream(kp + 32 * s) : ld16(kp + 32 * s);
  }
#pragma unroll
  for (int i = 0; i < C::VLD; ++i) {
    if (kPad && !((m.vval >> i) & 1u)) {
      t.v[i] = z;
      continue;
    }
    int64_t pv;
    int rv;
    row_at(m.vrow[i], pv, rv);
    const int ch = (i * kWave + lane) % C::CH;
    t.v[i] = ld16_stream(a.vc + vbase + pv * a.v_sb + rv * a.v_st + ch * 8);
  }
  return static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(kok && g == 0)) & 0xFFFFu;
}

// One tile of math.  vmask bit r: row r of the tile is a real token of a
// valid block (all 16 for every tile but the sequence's last one; none for
// an invalid block).
template <int D, typename T>
__device__ __forceinline__ void tile_math(const LaneMap<D>& m, const Tile<D>& t,
                                          const u32x4* qb, T* vt, uint32_t vmask, int g,
                                          float scale_log2, float& m_run, float& l_part,
                                          f32x4* acc) {
  using C = Cfg<D>;
  // V tile -> LDS; rows past the sequence end are zeroed so stale cache
  // contents (even NaN) can never reach the accumulators.
#pragma unroll
  for (int i = 0; i < C::VLD; ++i) {
    const u32x4 v = ((vmask >> m.vrow[i]) & 1u) ? t.v[i] : u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(vt + m.wlds[i]) = v;
  }
  // S^T = K Q^T.
  f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < C::NS; ++s) {
    s4 = Elem<T>::mfma16x16x32(__builtin_bit_cast(typename Elem<T>::x8, t.k[s]),
                               __builtin_bit_cast(typename Elem<T>::x8, qb[s]), s4);
  }
  // Online softmax in the log2 domain; lane = head, tokens 4g..4g+3.
  float x[4];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[r] = ((vmask >> (4 * g + r)) & 1u) ? s4[r] * scale_log2 : -INFINITY;
    mx = fmaxf(mx, x[r]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
  const float m_new = fmaxf(m_run, mx);
  if (m_new != m_run) {  // the running max moved: rescale (rare after warm-up)
    const float alpha = fast_exp2(m_run - m_new);  // 0 when m_run = -inf
    l_part *= alpha;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) acc[dt] *= alpha;
    m_run = m_new;
  }
  const float m_sub = (m_run == -INFINITY) ? 0.f : m_run;
  // The sum takes the probabilities as the PV product sees them: the rounded
  // fp16 value, or the bf16 pair hi + lo (Elem<T>::kSplitP).
  typename Elem<T>::x4 ph, pl;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float p = fast_exp2(x[r] - m_sub);
    ph[r] = Elem<T>::from_f(p);
    if constexpr (Elem<T>::kSplitP) {
      pl[r] = Elem<T>::from_f(p - Elem<T>::to_f(ph[r]));
      l_part += Elem<T>::to_f(ph[r]) + Elem<T>::to_f(pl[r]);
    } else {
      l_part += Elem<T>::to_f(ph[r]);
    }
  }
  // O^T += V^T P^T; lane receives V[4g+r][16dt + c16], r = 0..3, from one
  // transposing LDS read (four 16-bit reads before: headline 81.0-81.2 ->
  // 81.7-81.8 % of HBM peak, C2 uniform +1 point).
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) {
    const typename Elem<T>::x4 va = __builtin_bit_cast(
        typename Elem<T>::x4,
        __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vt + m.trbase + (((2 * dt) ^ m.trsw) << 3))));
    acc[dt] = Elem<T>::mfma16x16x16(va, ph, acc[dt]);
    if constexpr (Elem<T>::kSplitP) acc[dt] = Elem<T>::mfma16x16x16(va, pl, acc[dt]);
  }
}

// The peeled last tile of a sequence when block_size is not a multiple of
// 16: rows tok0 .. tok0 + nrows - 1 each read from their own block (pre, when
// has_pre: the table entries of blocks 0-63, lane i holding entry i); the row
// of the new token (new_row) comes from new_k/new_v and, when write_new, is
// written to its slot in the cache.  Returns the rows that are real tokens of
// valid blocks.
template <int D, bool kPad>
__device__ __forceinline__ uint32_t load_peeled_rows(const DecodeArgs& a, const LaneMap<D>& m,
                                                     int seq, int kvh, int64_t kbase,
                                                     int64_t vbase, int tok0, int nrows,
                                                     int new_row, bool write_new, bool has_pre,
                                                     int pre, int lane, Tile<D>& t) {
  using C = Cfg<D>;
  const int c16 = lane & 15, g = lane >> 4;
  auto row_at = [&](int row, int64_t& phys, int& rin) {
    const int tok = tok0 + row, bi = tok / a.block_size;
    if (has_pre && bi < kWave)
      phys = __shfl(pre, bi, kWave);  // -1 past max_blocks, as the table read
    else
      phys = bi < a.max_blocks ? a.bt[static_cast<int64_t>(seq) * a.max_blocks + bi] : -1;
    rin = tok - bi * a.block_size;
    const bool ok = phys >= 0 && phys < a.num_blocks;
    if (!ok) {
      phys = 0;
      rin = 0;
    }
    return ok;
  };
  int64_t pk;
  int rk;
  const bool kok = row_at(c16, pk, rk);
  f16* krow = a.kc + kbase + pk * a.k_sb + rk * a.k_st + 8 * g;
  const bool kmine = c16 == new_row && kok;
  const f16* kp = kmine ? a.new_k + seq * a.n_st + kvh * a.n_sh + 8 * g : krow;
#pragma unroll
  for (int s = 0; s < C::NS; ++s) {
    const bool in = !kPad || ((m.kval >> s) & 1u);
    t.k[s] = in ? ld16(kp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
    if (in && kmine && write_new) st16(krow + 32 * s, t.k[s]);
  }
#pragma unroll
  for (int i = 0; i < C::VLD; ++i) {
    if (kPad && !((m.vval >> i) & 1u)) {
      t.v[i] = u32x4{0u, 0u, 0u, 0u};
      continue;
    }
    int64_t pv;
    int rv;
    const bool vok = row_at(m.vrow[i], pv, rv);
    const int ch = (i * kWave + lane) % C::CH;
    f16* vrow = a.vc + vbase + pv * a.v_sb + rv * a.v_st + ch * 8;
    const bool vmine = m.vrow[i] == new_row && vok;
    const f16* vp = vmine ? a.new_v + seq * a.n_st + kvh * a.n_sh + ch * 8 : vrow;
    t.v[i] = ld16(vp);
    if (vmine && write_new) st16(vrow, t.v[i]);
  }
  return static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(kok && c16 < nrows && g == 0)) &
         0xFFFFu;
}

// Where the result of one (sequence, kv head, tile range) goes.
struct RangeOut {
  bool whole;         // the range is the whole sequence: normalised fp16 rows of out
  int64_t prow0;      // else: workspace row of the group's first query head
  int64_t prow_step;  // workspace row stride between the group's query heads
};

// The NW waves of the workgroup attend query heads qh0 .. qh0+nh-1 (nh <= 16,
// all of kv head kvh's group or a chunk of it) of
// sequence seq over the 16-token tiles [t0, t1) of its first L (clamped)
// positions: each wave streams a contiguous run of tiles, then the waves
// combine through LDS.  smem is reused on return only after the trailing
// barrier, so a workgroup may call this repeatedly.
//
// pre, when has_pre: the block-table window of blocks 0-63 of seq (lane i:
// entry i, as load_window gives it), loaded by the caller before the
// sequence's length arrived; a wave whose tiles all lie in those blocks
// (contexts up to 64 blocks) reads its physical blocks from it, one
// dependent global round trip fewer.
template <int D, typename T, int NW = kWaves, bool kStream = true, bool kPad = false,
          int kAhead = 1>
__device__ __forceinline__ void decode_range(const DecodeArgs& a, unsigned char* smem, int seq,
                                             int kvh, int qh0, int nh, int L, bool fused,
                                             bool write_new, int t0, int t1, const RangeOut& ro,
                                             bool trailing_barrier, bool has_pre = false,
                                             int pre = -1) {
  using C = Cfg<D>;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int c16 = lane & 15, g = lane >> 4;
  const int G = nh;
  const int n_tiles = (L + kTile - 1) / kTile;
  const int per = (t1 - t0 + NW - 1) / NW;
  const int jb = t0 + wave * per;
  const int je = min(jb + per, t1);

  // The sequence's last tile is peeled when it is partial or holds the new
  // token (fused KV write); every other tile is full and runs the pipeline.
  const int special = (fused || (L % kTile) != 0) ? n_tiles - 1 : n_tiles;
  const int jm = min(je, special);

  LaneMap<D> m;
  m.koff = c16 * static_cast<uint32_t>(a.k_st) + 8 * g;
#pragma unroll
  for (int i = 0; i < C::VLD; ++i) {
    const int f = i * kWave + lane;
    const int row = f / C::CH, ch = f % C::CH;
    m.vrow[i] = row;
    m.voff[i] = row * static_cast<uint32_t>(a.v_st) + ch * 8;
    m.wlds[i] = row * D + ((ch ^ swz<D>(row)) * 8);
  }
  m.kval = 0;
  m.vval = 0;
  if constexpr (kPad) {
#pragma unroll
    for (int s = 0; s < C::NS; ++s) m.kval |= (32 * s + 8 * g < a.hd ? 1u : 0u) << s;
#pragma unroll
    for (int i = 0; i < C::VLD; ++i)
      m.vval |= (((i * kWave + lane) % C::CH) * 8 < a.hd ? 1u : 0u) << i;
  }
  {
    // ds_read_b64_tr_b16: in each 16-lane group g, lane 4r + j names the
    // 8-byte piece j (dims 4j .. 4j + 3 of a 16-dim step) of token row
    // 4g + r, and lane i receives dim i of rows 4g .. 4g + 3.
    const int row = 4 * g + (c16 >> 2), j = c16 & 3;
    m.trsw = swz<D>(row);
    m.trbase = row * D + (j >> 1) * 8 + (j & 1) * 4;
  }
  const int64_t kbase = kvh * a.k_sh, vbase = kvh * a.v_sh;

  // Q^T as the B operand: lane holds Q[head c16][32s + 8g .. +7] for step s.
  u32x4 qb[C::NS];
  {
    const bool hv = c16 < G;
    const f16* qp = a.q + seq * a.q_st + (qh0 + (hv ? c16 : 0)) * a.q_sh + 8 * g;
#pragma unroll
    for (int s = 0; s < C::NS; ++s)
      qb[s] = (hv && (!kPad || ((m.kval >> s) & 1u))) ? ld16(qp + 32 * s)
                                                      : u32x4{0u, 0u, 0u, 0u};
  }

  T* vt = reinterpret_cast<T*>(smem) + wave * (kTile * D);
  float m_run = -INFINITY, l_part = 0.f;
  f32x4 acc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Each chunk covers the tiles of 64 consecutive blocks (one VGPR of
  // block-table entries).  With block_size not a multiple of 16 (kPad
  // kernels only) a chunk ends at the last tile that lies wholly before the
  // window's end.
  const bool in_pre = has_pre && jm * kTile <= kWave * a.block_size;
  for (int cb = jb; cb < jm;) {
    const int blk0 = in_pre ? 0 : (cb * kTile) / a.block_size;
    const int ce = min(jm, ((blk0 + kWave) * a.block_size) / kTile);
    const int vals = in_pre ? pre : load_window(a, seq, blk0, lane);
    // Issues tile jj into r; returns its rows of valid blocks.
    auto issue = [&](int jj, Tile<D>& r) -> uint32_t {
      if (kPad && !a.bs16)
        return issue_tile_rows<D, kStream, kPad>(a, kbase, vbase, m, vals, blk0, jj, lane, r);
      const int64_t p = window_block(a, vals, blk0, jj);
      issue_tile<D, kStream, kPad>(a, kbase, vbase, m, p, jj, r);
      return (p < 0 || p >= a.num_blocks) ? 0u : 0xFFFFu;
    };
    // Prefetch indices past the chunk are clamped to its last tile (an L2
    // hit), which keeps the loop free of branches around loads.
    const int jl = ce - 1;
    if constexpr (kAhead == 1) {
      // Two tile buffers; loads run one tile ahead.
      Tile<D> r0, r1;
      uint32_t v0 = issue(cb, r0), v1;
      int j = cb;
      for (; j + 2 <= ce; j += 2) {
        v1 = issue(j + 1, r1);
        tile_math<D, T>(m, r0, qb, vt, v0, g, a.scale_log2, m_run, l_part, acc);
        v0 = issue(min(j + 2, jl), r0);
        tile_math<D, T>(m, r1, qb, vt, v1, g, a.scale_log2, m_run, l_part, acc);
      }
      if (j < ce) tile_math<D, T>(m, r0, qb, vt, v0, g, a.scale_log2, m_run, l_part, acc);
      cb = ce;
      continue;
    }
    // Three rotating tile buffers; loads run two tiles ahead.
    Tile<D> r0, r1, r2;
    uint32_t v0 = issue(cb, r0);
    uint32_t v1 = issue(min(cb + 1, jl), r1);
    uint32_t v2;
    int j = cb;
    for (; j + 3 <= ce; j += 3) {
      v2 = issue(min(j + 2, jl), r2);
      tile_math<D, T>(m, r0, qb, vt, v0, g, a.scale_log2, m_run, l_part, acc);
      v0 = issue(min(j + 3, jl), r0);
      tile_math<D, T>(m, r1, qb, vt, v1, g, a.scale_log2, m_run, l_part, acc);
      v1 = issue(min(j + 4, jl), r1);
      tile_math<D, T>(m, r2, qb, vt, v2, g, a.scale_log2, m_run, l_part, acc);
    }
    // Remainder (0..2 tiles): r0 holds tile j, r1 tile j+1.
    if (j < ce) {
      tile_math<D, T>(m, r0, qb, vt, v0, g, a.scale_log2, m_run, l_part, acc);
      if (j + 1 < ce)
        tile_math<D, T>(m, r1, qb, vt, v1, g, a.scale_log2, m_run, l_part, acc);
    }
    cb = ce;
  }

  // Peeled last tile: partial and/or carrying the new token, which is read
  // from new_k/new_v and, when write_new, written to the cache here (the
  // fused KV write; of the head chunks of one kv head only the first
  // writes, the others read the same token from new_k/new_v).
  if (special >= jb && special < je) {
    const int j = special;
    const int tok0 = j * kTile;
    const int new_row = fused ? (L - 1) - tok0 : -1;
    Tile<D> t;
    uint32_t vm;
    if (kPad && !a.bs16) {
      vm = load_peeled_rows<D, kPad>(a, m, seq, kvh, kbase, vbase, tok0, min(kTile, L - tok0),
                                     new_row, write_new, has_pre, pre, lane, t);
    } else {
      const int bi = tok0 / a.block_size;
      int64_t phys;
      if (has_pre && bi < kWave)
        phys = __builtin_amdgcn_readlane(pre, bi);  // -1 past max_blocks, as the table read
      else
        phys = bi < a.max_blocks ? a.bt[static_cast<int64_t>(seq) * a.max_blocks + bi] : -1;
      const bool bvalid = phys >= 0 && phys < a.num_blocks;
      vm = bvalid ? (1u << min(kTile, L - tok0)) - 1u : 0u;
      if (!bvalid) phys = 0;
      const int row0 = tok0 % a.block_size;
      f16* kb = a.kc + kbase + phys * a.k_sb + row0 * a.k_st;
      f16* vb = a.vc + vbase + phys * a.v_sb + row0 * a.v_st;
      {
        const bool mine = (c16 == new_row) && bvalid;
        const f16* kp = mine ? a.new_k + seq * a.n_st + kvh * a.n_sh + 8 * g
                             : kb + m.koff;
#pragma unroll
        for (int s = 0; s < C::NS; ++s) {
          const bool in = !kPad || ((m.kval >> s) & 1u);
          t.k[s] = in ? ld16(kp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
          if (in && mine && write_new) st16(kb + m.koff + 32 * s, t.k[s]);
        }
      }
#pragma unroll
      for (int i = 0; i < C::VLD; ++i) {
        if (kPad && !((m.vval >> i) & 1u)) {
          t.v[i] = u32x4{0u, 0u, 0u, 0u};
          continue;
        }
        const bool mine = (m.vrow[i] == new_row) && bvalid;
        const int ch = (i * kWave + lane) % C::CH;
        const f16* vp = mine ? a.new_v + seq * a.n_st + kvh * a.n_sh + ch * 8 : vb + m.voff[i];
        t.v[i] = ld16(vp);
        if (mine && write_new) st16(vb + m.voff[i], t.v[i]);
      }
    }
    tile_math<D, T>(m, t, qb, vt, vm, g, a.scale_log2, m_run, l_part, acc);
  }

  // Sum over the four token groups of this head.
  l_part += __shfl_xor(l_part, 16, kWave);
  l_part += __shfl_xor(l_part, 32, kWave);

  // Cross-wave combine through LDS: wm/wl [wave][16], wa [wave][G][D].
  __syncthreads();
  float* wm = reinterpret_cast<float*>(smem);
  float* wl = wm + NW * 16;
  float* wa = wl + NW * 16;
  if (c16 < G) {
    if (g == 0) {
      wm[wave * 16 + c16] = m_run;
      wl[wave * 16 + c16] = l_part;
    }
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * dt + 4 * g + r;
        wa[(wave * G + c16) * D + d] = acc[dt][r];
      }
    }
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w * 16 + h]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = wm[w * 16 + h];
        if (mw == -INFINITY) continue;
        const float sc = fast_exp2(mw - M);
        num += sc * wa[(w * G + h) * D + d];
        den += sc * wl[w * 16 + h];
      }
    }
    if (ro.whole) {
      const int qh = qh0 + h;
      if (!kPad || d < a.hd)
        reinterpret_cast<T*>(a.out)[seq * a.o_st + qh * a.o_sh + d] =
            Elem<T>::from_f(den > 0.f ? num / den : 0.f);
    } else {
      const int64_t row = ro.prow0 + h * ro.prow_step;
      a.ws_acc[row * D + d] = num;
      if (d == 0) {
        a.ws_ml[row * 2 + 0] = M;
        a.ws_ml[row * 2 + 1] = den;
      }
    }
  }
  if (trailing_barrier) __syncthreads();
}

// Zero output rows of a sequence with seq_len <= 0 (the reference leaves them
// unwritten in a pre-zeroed buffer).
__device__ __forceinline__ void zero_rows(const DecodeArgs& a, int seq, int h0, int nh, int D) {
  for (int idx = threadIdx.x; idx < nh * D; idx += blockDim.x) {
    const int h = h0 + idx / D;
    a.out[seq * a.o_st + h * a.o_sh + idx % D] = f2h(0.f);
  }
}

__device__ __forceinline__ int clamped_len(const DecodeArgs& a, int seq) {
  const int L = a.seq_lens[seq];
  const int cap = a.max_blocks * a.block_size;
  return L > cap ? cap : L;
}

// Fixed partitions: grid (kv_head x head chunk, partition, seq), the kv head
// fastest: consecutive workgroups read the same cache blocks' heads, which lie
// side by side in HBM ([block][kv head][token][dim]), at about the same time
// (C4 with 512-token partitions: 62 -> 68 % of HBM peak against partition
// fastest).  NW waves per workgroup: 8 for long partitions; 4 for short
// ones, so that two workgroups share a CU and one's start-up (Q load, first
// tiles) overlaps the other's tail.
template <int D, typename T, int NW, bool kPad>
__global__ void __launch_bounds__(NW* kWave) __attribute__((amdgpu_waves_per_eu(2)))
paged_decode_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int part = blockIdx.y, seq = blockIdx.z;
  const int kvh = blockIdx.x / a.chunks, hc = blockIdx.x % a.chunks;
  const int qh0 = kvh * a.G + hc * a.Gc, nh = min(a.Gc, a.G - hc * a.Gc);
  // The first partition's window, issued before the length is known
  // (independent loads, one round trip); later partitions start past it.
  const int pre = part == 0 ? load_window(a, seq, 0, static_cast<int>(threadIdx.x % kWave)) : -1;
  const int Lorig = a.seq_lens[seq];
  const int L = clamped_len(a, seq);
  if (L <= 0) {
    if (part == 0) zero_rows(a, seq, qh0, nh, a.hd);
    return;
  }
  const int part_tok = a.part_tiles * kTile;
  const int n_tiles = (L + kTile - 1) / kTile;
  const int n_parts = min((L + part_tok - 1) / part_tok, a.max_parts);
  if (part >= n_parts) return;
  const int t0 = part * a.part_tiles;
  const int t1 = (part == a.max_parts - 1) ? n_tiles : min(t0 + a.part_tiles, n_tiles);
  RangeOut ro;
  ro.whole = (n_parts == 1);
  ro.prow0 = (static_cast<int64_t>(seq) * a.num_q_heads + qh0) * a.max_parts + part;
  ro.prow_step = a.max_parts;
  decode_range<D, T, NW, true, kPad, NW == 4 ? 2 : 1>(
      a, smem, seq, kvh, qh0, nh, L, a.new_k != nullptr && Lorig == L, hc == 0, t0, t1, ro,
      false, part == 0, pre);
}

// Balanced split: the tiles of all sequences (for one kv head) are laid end
// to end and workgroup c of the kv head takes tiles [c*per, (c+1)*per), with
// per = max(ceil(total / gridDim.x), kBalMinTiles).  Every workgroup derives
// the same prefix sums of tiles per sequence from seq_lens, so the split
// follows the actual lengths without a host round trip.  A sequence inside
// one workgroup's range is finished there; the pieces of a sequence that
// crosses ranges go to workspace rows (y*(gridDim.x + num_seqs) + c + seq)*Gc
// + h, y = blockIdx.y (kv head x head chunk) -- distinct for distinct (c, seq)
// because the ranges and the sequences are both in increasing order -- and
// the merge kernel combines them.
constexpr int kBalMinTiles = 4 * kWaves;

__device__ __forceinline__ int tiles_of(const DecodeArgs& a, int seq) {
  const int L = clamped_len(a, seq);
  return L > 0 ? (L + kTile - 1) / kTile : 0;
}

// starts[s] = sum of tiles_of(s') for s' < s, s = 0..num_seqs (LDS).
__device__ __forceinline__ void tile_prefix(const DecodeArgs& a, int* starts, int* wsum) {
  const int B = a.num_seqs, nt = blockDim.x;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int per = (B + nt - 1) / nt;
  const int s0 = min(B, static_cast<int>(threadIdx.x) * per), s1 = min(B, s0 + per);
  int sum = 0;
  for (int s = s0; s < s1; ++s) sum += tiles_of(a, s);
  int x = sum;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) wsum[wave] = x;
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; ++w) off += wsum[w];
  int run = off + x - sum;
  for (int s = s0; s < s1; ++s) {
    starts[s] = run;
    run += tiles_of(a, s);
  }
  if (threadIdx.x == nt - 1) starts[B] = off + x;
  __syncthreads();
}

template <int D, typename T, int NW, bool kPad>
__global__ void __launch_bounds__(NW* kWave) __attribute__((amdgpu_waves_per_eu(2)))
paged_decode_balanced_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int c = blockIdx.x, y = blockIdx.y, nc = gridDim.x;
  const int kvh = y / a.chunks, hc = y % a.chunks;
  const int qh0 = kvh * a.G + hc * a.Gc, nh = min(a.Gc, a.G - hc * a.Gc);
  const int B = a.num_seqs;
  int* starts = reinterpret_cast<int*>(smem + a.lds_main);
  tile_prefix(a, starts, starts + B + 1);
  const int total = starts[B];
  const int per = max((total + nc - 1) / nc, kBalMinTiles);
  if (c == 0 && y == 0) {
    // Split geometry for the merge kernel.
    if (threadIdx.x == 0) a.ws_hdr[0] = per;
    for (int s = threadIdx.x; s <= B; s += blockDim.x) a.ws_hdr[1 + s] = starts[s];
  }
  const int r0 = c * per, r1 = min(total, r0 + per);
  if (r0 >= r1) return;
  // First sequence with tiles at or after r0.
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (starts[mid + 1] <= r0) lo = mid + 1;
    else hi = mid;
  }
  int seq = lo;
  for (int pos = r0; pos < r1; ++seq) {
    const int s0 = starts[seq], s1 = starts[seq + 1];
    if (s1 <= pos) continue;  // empty sequence
    const int t0 = pos - s0, t1 = min(r1, s1) - s0;
    RangeOut ro;
    ro.whole = (t0 == 0 && t1 == s1 - s0);
    ro.prow0 = (static_cast<int64_t>(y) * (nc + B) + c + seq) * a.Gc;
    ro.prow_step = 1;
    const int L = clamped_len(a, seq);
    decode_range<D, T, NW, false, kPad>(a, smem, seq, kvh, qh0, nh, L,
                           a.new_k != nullptr && a.seq_lens[seq] == L, hc == 0, t0, t1, ro,
                           true);
    pos = s0 + t1;
  }
}

// Merge for the balanced split: sequence seq spans workgroups
// starts[seq]/per .. (starts[seq+1]-1)/per of its kv head; when that is one
// workgroup the decode kernel wrote the row already.  Rows of empty
// sequences are zeroed here.
// Log-sum-exp merge of split partials (m_p, l_p, acc_p) in one pass:
//   out = sum_p 2^(m_p - M) acc_p / sum_p 2^(m_p - M) l_p,  M = max_p m_p,
// kept as a running maximum with the sums rescaled when it grows, so each
// piece's three loads are independent of the others and issue together.
// Pieces with l_p = 0 (nothing visible) are skipped.
struct MergeAcc {
  float M = -INFINITY, num = 0.f, den = 0.f;
  __device__ __forceinline__ void add(float mp, float lp, float ap) {
    if (!(lp > 0.f)) return;
    const float Mn = fmaxf(M, mp);
    const float so = fast_exp2(M - Mn);  // 0 while M = -inf
    const float sn = fast_exp2(mp - Mn);
    num = num * so + ap * sn;
    den = den * so + lp * sn;
    M = Mn;
  }
  __device__ __forceinline__ float value() const { return den > 0.f ? num / den : 0.f; }
};

// A thread merges four dimensions: the scale factors of a partition are
// computed once for its four partial sums, and each partial row is read
// with 16-byte loads (C4 with 512-token partitions: the step 0.645 -> 0.640
// ms, 69.5 -> 70.0 % of HBM peak).
struct MergeAcc4 {
  float M = -INFINITY, den = 0.f;
  f32x4 num = {0.f, 0.f, 0.f, 0.f};
  __device__ __forceinline__ void add(float mp, float lp, const f32x4& ap) {
    if (!(lp > 0.f)) return;
    const float Mn = fmaxf(M, mp);
    const float so = fast_exp2(M - Mn);  // 0 while M = -inf
    const float sn = fast_exp2(mp - Mn);
    num = num * so + ap * sn;
    den = den * so + lp * sn;
    M = Mn;
  }
};

// Balanced-split merge: a thread takes four dimensions of one query head,
// kBalMergeRows heads of a sequence per workgroup.
constexpr int kBalMergeRows = 4;

template <int D, typename T>
__global__ void __launch_bounds__(D / 4 * kBalMergeRows)
paged_decode_merge_balanced_kernel(DecodeArgs a) {
  constexpr int D4 = D / 4;
  const int qh = blockIdx.x * kBalMergeRows + threadIdx.x / D4, seq = blockIdx.y;
  const int d4 = threadIdx.x % D4;
  if (qh >= a.num_q_heads) return;
  const int B = a.num_seqs, nc = a.max_parts;
  if (4 * d4 >= a.hd) return;  // padded dims (hd is a multiple of 8)
  T* o = reinterpret_cast<T*>(a.out) + seq * a.o_st + qh * a.o_sh + 4 * d4;
  const int L = clamped_len(a, seq);
  if (L <= 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = Elem<T>::from_f(0.f);
    return;
  }
  const int per = a.ws_hdr[0];
  const int c0 = a.ws_hdr[1 + seq] / per, c1 = (a.ws_hdr[2 + seq] - 1) / per;
  if (c0 == c1) return;
  const int hg = qh % a.G, y = (qh / a.G) * a.chunks + hg / a.Gc, h = hg % a.Gc;
  const int64_t base = static_cast<int64_t>(y) * (nc + B) + seq;
  MergeAcc4 m;
#pragma unroll 4
  for (int c = c0; c <= c1; ++c) {
    const int64_t row = (base + c) * a.Gc + h;
    m.add(a.ws_ml[row * 2], a.ws_ml[row * 2 + 1],
          *reinterpret_cast<const f32x4*>(a.ws_acc + row * D + 4 * d4));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = Elem<T>::from_f(m.den > 0.f ? m.num[i] / m.den : 0.f);
}

// Second pass for split sequences:
//   out = sum_p 2^(m_p - M) acc_p / sum_p 2^(m_p - M) l_p,  M = max_p m_p.
// kMergeSplit thread groups of D/4 threads each merge every kMergeSplit-th
// partition (shorter dependent load chains for the long-context split); the
// group states are then merged the same way through LDS.
constexpr int kMergeSplit = 8;

template <int D, typename T>
__global__ void __launch_bounds__(D / 4 * kMergeSplit)
paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int D4 = D / 4;
  __shared__ float sml[kMergeSplit][2];
  __shared__ f32x4 snum[kMergeSplit][D4];
  const int qh = blockIdx.x, seq = blockIdx.y;
  const int d4 = threadIdx.x % D4, grp = threadIdx.x / D4;
  int L = a.seq_lens[seq];
  const int cap = a.max_blocks * a.block_size;
  if (L > cap) L = cap;
  if (L <= 0) return;  // zero row written by the decode kernel
  const int part_tok = a.part_tiles * kTile;
  const int n_parts = min((L + part_tok - 1) / part_tok, a.max_parts);
  if (n_parts <= 1) return;  // written directly by the decode kernel
  const int64_t row0 = (static_cast<int64_t>(seq) * a.num_q_heads + qh) * a.max_parts;
  MergeAcc4 m;
#pragma unroll 4
  for (int p = grp; p < n_parts; p += kMergeSplit)
    m.add(a.ws_ml[(row0 + p) * 2], a.ws_ml[(row0 + p) * 2 + 1],
          *reinterpret_cast<const f32x4*>(a.ws_acc + (row0 + p) * D + 4 * d4));
  if (d4 == 0) {
    sml[grp][0] = m.M;
    sml[grp][1] = m.den;
  }
  snum[grp][d4] = m.num;
  __syncthreads();
  if (grp != 0 || 4 * d4 >= a.hd) return;
  MergeAcc4 t;
#pragma unroll
  for (int g = 0; g < kMergeSplit; ++g) t.add(sml[g][0], sml[g][1], snum[g][d4]);
  T* o = reinterpret_cast<T*>(a.out) + seq * a.o_st + qh * a.o_sh + 4 * d4;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = Elem<T>::from_f(t.den > 0.f ? t.num[i] / t.den : 0.f);
}

// Merge of caller-supplied attention states (vaa_merge_attn_states): row
// (s, h) combines partial outputs o_p (normalised, fp32) with their
// log-sum-exps lse_p (natural log of the partition's softmax denominator),
//   out = sum_p e^(lse_p - LSE) o_p,  LSE = log sum_p e^(lse_p),
// through MergeAcc in the log2 domain (m_p = lse_p log2 e, l_p = 1).
// Partitions with lse_p = -inf (or NaN) hold no keys and are skipped; a row
// with none is zero, and its merged lse -inf.
struct StatesArgs {
  const float* part_out;   // [S, H, P, D]
  const float* part_lse;   // [S, H, P]
  const int32_t* num_parts;  // [S] or null (all P)
  f16* out;
  float* out_lse;          // [S, H] or null
  int H, P, D;
  int64_t o_st, o_sh;
};

template <typename T>
__global__ void __launch_bounds__(128) merge_states_kernel(StatesArgs a) {
  const int h = blockIdx.x, s = blockIdx.y;
  int n = a.P;
  if (a.num_parts) n = min(max(a.num_parts[s], 0), a.P);
  const int64_t row0 = (static_cast<int64_t>(s) * a.H + h) * a.P;
  for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
    MergeAcc m;
    for (int p = 0; p < n; ++p) {
      const float lse = a.part_lse[row0 + p];
      const bool has = lse > -INFINITY;  // false for -inf and NaN
      m.add(has ? lse * kLog2e : 0.f, has ? 1.f : 0.f, a.part_out[(row0 + p) * a.D + d]);
    }
    reinterpret_cast<T*>(a.out)[s * a.o_st + h * a.o_sh + d] = Elem<T>::from_f(m.value());
    if (a.out_lse && d == 0)
      a.out_lse[static_cast<int64_t>(s) * a.H + h] =
          m.den > 0.f ? (m.M + __builtin_log2f(m.den)) * (1.f / kLog2e) : -INFINITY;
  }
}

// Compute units of the current device, queried once per device.  Each
// entry is written with the same value by whichever thread gets there first
// (a relaxed atomic: concurrent first calls only repeat the query).
constexpr int kMaxDevices = 64;
std::atomic<int> g_num_cus[kMaxDevices];

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  if (dev >= 0 && dev < kMaxDevices) {
    const int n = g_num_cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int n = 0;
  if (dev < 0 ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0)
    n = 256;
  if (dev >= 0 && dev < kMaxDevices) g_num_cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

constexpr int kBalMaxSeqs = 8192;  // prefix sums of tiles per sequence live in LDS
constexpr int kMaxGroupCols = 16;  // query heads per workgroup: the MFMA's 16 columns

// A GQA group of G query heads is served in ceil(G/16) chunks of
// ceil(G/chunks) heads (the last one may hold fewer), one workgroup each.
inline int head_chunks(int G) { return (G + kMaxGroupCols - 1) / kMaxGroupCols; }
inline int heads_per_chunk(int G) {
  const int c = head_chunks(G);
  return (G + c - 1) / c;
}

// How a call splits its sequences.
struct Split {
  bool balanced;     // balanced split over the actual lengths
  bool shared;       // balanced, kSharedPerCu (else kBalPerCu) workgroups per CU's worth
  int part;          // fixed: tokens per partition (balanced: -1)
  int max_parts;     // fixed: partitions per sequence; balanced: workgroups per kv head
                     // and head chunk
  size_t ws_bytes;   // workspace needed (0: none)
  size_t hdr_bytes;  // balanced: bytes before the partial rows
};

// Fixed partitions with partition_size > 0; with 0 the size comes from
// max_seq_len alone (all sequences assumed at the maximum): split only as far
// as needed for the workgroups to cover every CU once, in multiples of
// 16 * kWaves tokens.  VAA_PARTITION_BALANCED: 4-wave workgroups, two per
// CU's worth, each taking an equal share of the tiles of all sequences (split
// on the device from seq_lens); VAA_PARTITION_BALANCED_SHARED: the same with
// four per CU's worth.
int plan_split(const vaa_attn_params* p, Split* sp) {
  const int64_t cap = static_cast<int64_t>(p->max_blocks_per_seq) * p->block_size;
  int64_t max_len = p->max_seq_len;
  if (max_len > cap) max_len = cap;
  if (max_len < 1) max_len = 1;
  const int quantum = kTile * kWaves;
  int64_t part = p->partition_size;
  const size_t row_bytes = (static_cast<size_t>(padded_head(p->head_size)) + 2) * sizeof(float);
  if (part == VAA_PARTITION_BALANCED || part == VAA_PARTITION_BALANCED_SHARED) {
    if (p->num_seqs > kBalMaxSeqs)
      return fail(VAA_ERR_UNSUPPORTED, "balanced split: num_seqs=%d > %d", p->num_seqs,
                  kBalMaxSeqs);
    const bool shared = part == VAA_PARTITION_BALANCED_SHARED;
    const int per_cu = shared ? kSharedPerCu : kBalPerCu;
    const int ys = p->num_kv_heads * head_chunks(p->queries_per_kv);
    const int wgs = (per_cu * num_cus() + ys - 1) / ys;
    sp->balanced = true;
    sp->shared = shared;
    sp->part = static_cast<int>(part);
    sp->max_parts = wgs < 1 ? 1 : wgs;
    sp->hdr_bytes = ((static_cast<size_t>(p->num_seqs) + 2) * sizeof(int) + 255) / 256 * 256;
    const size_t rows = static_cast<size_t>(ys) * (sp->max_parts + p->num_seqs) *
                        heads_per_chunk(p->queries_per_kv);
    sp->ws_bytes = sp->hdr_bytes + rows * row_bytes;
    return VAA_OK;
  }
  if (part > 0) {
    if (part % quantum != 0)
      return fail(VAA_ERR_INVALID_ARG,
                  "partition_size=%lld must be a positive multiple of %d",
                  (long long)part, quantum);
  } else if (part == 0) {
    const int64_t pairs = static_cast<int64_t>(p->num_seqs) * p->num_kv_heads *
                          head_chunks(p->queries_per_kv);
    int64_t splits = pairs > 0 ? (num_cus() + pairs - 1) / pairs : 1;
    if (splits < 1) splits = 1;
    part = (max_len + splits - 1) / splits;
    part = (part + quantum - 1) / quantum * quantum;
  } else {
    return fail(VAA_ERR_INVALID_ARG, "partition_size=%lld (use > 0, 0, %d or %d)",
                (long long)part, VAA_PARTITION_BALANCED, VAA_PARTITION_BALANCED_SHARED);
  }
  if (part > (int64_t{1} << 30)) part = int64_t{1} << 30;
  // Partitions index the grid's y dimension.
  if ((max_len + part - 1) / part > 65535)
    return fail(VAA_ERR_UNSUPPORTED,
                "partition_size=%lld splits max_seq_len=%lld into more than 65535 partitions",
                (long long)part, (long long)max_len);
  sp->balanced = false;
  sp->shared = false;
  sp->part = static_cast<int>(part);
  sp->max_parts = static_cast<int>((max_len + part - 1) / part);
  sp->hdr_bytes = 0;
  sp->ws_bytes = sp->max_parts <= 1 ? 0
                                    : static_cast<size_t>(p->num_seqs) * p->num_query_heads *
                                          sp->max_parts * row_bytes;
  return VAA_OK;
}

int check_params(const vaa_attn_params* p, const char* what) {
  if (!p) return fail(VAA_ERR_INVALID_ARG, "%s: null params", what);
  if (!head_size_ok(p->head_size))
    return fail(VAA_ERR_UNSUPPORTED, "%s: head_size=%d (a multiple of 8 up to 128)", what,
                p->head_size);
  if (p->block_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: block_size=%d must be positive", what, p->block_size);
  if (p->num_kv_heads <= 0 || p->num_query_heads <= 0 ||
      p->num_query_heads % p->num_kv_heads != 0 ||
      p->queries_per_kv != p->num_query_heads / p->num_kv_heads)
    return fail(VAA_ERR_INVALID_ARG, "%s: heads %d/%d, queries_per_kv=%d", what,
                p->num_query_heads, p->num_kv_heads, p->queries_per_kv);
  if (!valid_dtype(p->dtype))
    return fail(VAA_ERR_UNSUPPORTED, "%s: dtype=%d (VAA_DTYPE_F16 or VAA_DTYPE_BF16)", what,
                p->dtype);
  if (p->num_seqs < 0 || p->max_blocks_per_seq <= 0 || p->num_blocks <= 0)
    return fail(VAA_ERR_INVALID_ARG,
                "%s: num_seqs=%d max_blocks_per_seq=%d num_blocks=%lld", what,
                p->num_seqs, p->max_blocks_per_seq, (long long)p->num_blocks);
  const int64_t strides[] = {p->k_stride_block, p->k_stride_head, p->k_stride_token,
                             p->v_stride_block, p->v_stride_head, p->v_stride_token,
                             p->q_stride_token, p->q_stride_head, p->o_stride_token,
                             p->o_stride_head};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0)
      return fail(VAA_ERR_INVALID_ARG,
                  "%s: strides must be non-negative multiples of 8 elements", what);
  // In-tile lane offsets are 32-bit.
  if (p->k_stride_token * kTile >= (int64_t{1} << 31) ||
      p->v_stride_token * kTile >= (int64_t{1} << 31))
    return fail(VAA_ERR_INVALID_ARG, "%s: token stride too large", what);
  return VAA_OK;
}

template <int D, typename T, bool kPad>
int launch_decode(const DecodeArgs& a0, bool balanced, bool shared, hipStream_t stream) {
  DecodeArgs a = a0;
  const size_t lds_tiles = static_cast<size_t>(kWaves) * kTile * D * sizeof(f16);
  const size_t lds_comb =
      (2 * kWaves * 16 + static_cast<size_t>(kWaves) * a.Gc * D) * sizeof(float);
  const size_t lds = lds_tiles > lds_comb ? lds_tiles : lds_comb;
  if (balanced) {
    const size_t lds_bal =
        std::max(static_cast<size_t>(kBalWaves) * kTile * D * sizeof(f16),
                 (2 * kBalWaves * 16 + static_cast<size_t>(kBalWaves) * a.Gc * D) * sizeof(float));
    a.lds_main = static_cast<int>((lds_bal + 15) / 16 * 16);
    const size_t lds_b =
        a.lds_main + (static_cast<size_t>(a.num_seqs) + 1 + kBalWaves) * sizeof(int);
    hipLaunchKernelGGL((paged_decode_balanced_kernel<D, T, kBalWaves, kPad>),
                       dim3(a.max_parts, a.num_kv_heads * a.chunks), dim3(kBalWaves * kWave),
                       lds_b, stream, a);
    int st = check_launch("paged_decode_balanced_kernel");
    if (st) return st;
    hipLaunchKernelGGL((paged_decode_merge_balanced_kernel<D, T>),
                       dim3((a.num_q_heads + kBalMergeRows - 1) / kBalMergeRows, a.num_seqs),
                       dim3(D / 4 * kBalMergeRows), 0, stream, a);
    return check_launch("paged_decode_merge_balanced_kernel");
  }
  dim3 grid(a.num_kv_heads * a.chunks, a.max_parts, a.num_seqs);
  if (a.max_parts > 1 && a.part_tiles <= kShortPartTiles) {
    constexpr int kNw = kWaves / 2;
    const size_t lds4 = std::max(static_cast<size_t>(kNw) * kTile * D * sizeof(f16),
                                 (2 * kNw * 16 + static_cast<size_t>(kNw) * a.Gc * D) *
                                     sizeof(float));
    hipLaunchKernelGGL((paged_decode_kernel<D, T, kNw, kPad>), grid, dim3(kNw * kWave), lds4,
                       stream, a);
  } else {
    hipLaunchKernelGGL((paged_decode_kernel<D, T, kWaves, kPad>), grid, dim3(kWaves * kWave),
                       lds, stream, a);
  }
  int st = check_launch("paged_decode_kernel");
  if (st || a.max_parts <= 1) return st;
  hipLaunchKernelGGL((paged_decode_merge_kernel<D, T>), dim3(a.num_q_heads, a.num_seqs),
                     dim3(D / 4 * kMergeSplit), 0, stream, a);
  return check_launch("paged_decode_merge_kernel");
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" size_t vaa_paged_attention_decode_workspace_size(const vaa_attn_params* p,
                                                            int32_t* partition_size_out) {
  if (!p || p->num_seqs <= 0 || p->block_size <= 0 || p->max_blocks_per_seq <= 0 ||
      p->num_kv_heads <= 0 || p->queries_per_kv <= 0)
    return 0;
  Split sp;
  if (plan_split(p, &sp) != VAA_OK) return 0;
  if (partition_size_out) *partition_size_out = sp.part;
  return sp.ws_bytes;
}

namespace vaa {
namespace {

// The body of vaa_paged_attention_decode, given the workspace; `what` names
// the entry point in error messages.
int decode_impl(const char* what, const vaa_attn_params* p, const uint16_t* query,
                uint16_t* key_cache, uint16_t* value_cache, const int32_t* block_table,
                const int32_t* seq_lens, uint16_t* output, const uint16_t* new_keys,
                const uint16_t* new_values, void* workspace, size_t workspace_bytes,
                void* stream) {
  int st = check_params(p, what);
  if (st) return st;
  if (p->num_seqs == 0) return VAA_OK;
  if (!query || !key_cache || !value_cache || !block_table || !seq_lens || !output)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if ((new_keys == nullptr) != (new_values == nullptr))
    return fail(VAA_ERR_INVALID_ARG,
                "%s: new_keys and new_values go together", what);
  if (new_keys && (p->new_kv_stride_token % 8 || p->new_kv_stride_head % 8 ||
                   !aligned16(new_keys) || !aligned16(new_values)))
    return fail(VAA_ERR_INVALID_ARG,
                "%s: new K/V must be 16-byte aligned rows", what);
  if (!aligned16(query) || !aligned16(key_cache) || !aligned16(value_cache))
    return fail(VAA_ERR_INVALID_ARG,
                "%s: query and caches must be 16-byte aligned", what);
  Split sp;
  st = plan_split(p, &sp);
  if (st) return st;

  DecodeArgs a;
  a.q = reinterpret_cast<const f16*>(query);
  a.kc = reinterpret_cast<f16*>(key_cache);
  a.vc = reinterpret_cast<f16*>(value_cache);
  a.bt = block_table;
  a.seq_lens = seq_lens;
  a.out = reinterpret_cast<f16*>(output);
  a.new_k = reinterpret_cast<const f16*>(new_keys);
  a.new_v = reinterpret_cast<const f16*>(new_values);
  a.ws_acc = nullptr;
  a.ws_ml = nullptr;
  a.ws_hdr = nullptr;
  if (sp.ws_bytes > 0) {
    if (!workspace || workspace_bytes < sp.ws_bytes)
      return fail(VAA_ERR_WORKSPACE,
                  "%s: workspace %zu bytes < %zu needed", what, workspace_bytes,
                  sp.ws_bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
      return fail(VAA_ERR_INVALID_ARG,
                  "%s: workspace must be 16-byte aligned", what);
    const int dp = padded_head(p->head_size);
    const size_t rows = (sp.ws_bytes - sp.hdr_bytes) / ((dp + 2) * sizeof(float));
    unsigned char* base = static_cast<unsigned char*>(workspace);
    a.ws_hdr = reinterpret_cast<int*>(base);
    a.ws_acc = reinterpret_cast<float*>(base + sp.hdr_bytes);
    a.ws_ml = a.ws_acc + rows * dp;
  }
  a.scale_log2 = p->scale * kLog2e;
  a.hd = p->head_size;
  a.num_seqs = p->num_seqs;
  a.max_blocks = p->max_blocks_per_seq;
  a.block_size = p->block_size;
  a.bs16 = p->block_size % kTile == 0 ? 1 : 0;
  a.num_kv_heads = p->num_kv_heads;
  a.num_q_heads = p->num_query_heads;
  a.G = p->queries_per_kv;
  a.chunks = head_chunks(a.G);
  a.Gc = heads_per_chunk(a.G);
  a.part_tiles = sp.balanced ? 0 : sp.part / kTile;
  a.max_parts = sp.max_parts;
  a.lds_main = 0;
  a.num_blocks = p->num_blocks;
  a.k_sb = p->k_stride_block; a.k_sh = p->k_stride_head; a.k_st = p->k_stride_token;
  a.v_sb = p->v_stride_block; a.v_sh = p->v_stride_head; a.v_st = p->v_stride_token;
  a.q_st = p->q_stride_token; a.q_sh = p->q_stride_head;
  a.o_st = p->o_stride_token; a.o_sh = p->o_stride_head;
  a.n_st = p->new_kv_stride_token; a.n_sh = p->new_kv_stride_head;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = p->dtype == VAA_DTYPE_BF16;
  // Head sizes below the computed size, and block sizes that are not a
  // multiple of 16, run the kPad kernels (masked dims, rows that find their
  // own blocks).
  const bool pad = padded_head(p->head_size) != p->head_size || p->block_size % kTile != 0;
#define VAA_DECODE_CASE(DP)                                                              \
  case DP:                                                                               \
    if (pad)                                                                             \
      return bf ? launch_decode<DP, bf16, true>(a, sp.balanced, sp.shared, s)            \
                : launch_decode<DP, f16, true>(a, sp.balanced, sp.shared, s);            \
    return bf ? launch_decode<DP, bf16, false>(a, sp.balanced, sp.shared, s)             \
              : launch_decode<DP, f16, false>(a, sp.balanced, sp.shared, s);
  switch (padded_head(p->head_size)) {
    VAA_DECODE_CASE(32)
    VAA_DECODE_CASE(64)
    VAA_DECODE_CASE(96)
    VAA_DECODE_CASE(128)
  }
#undef VAA_DECODE_CASE
  return fail(VAA_ERR_UNSUPPORTED, "head_size=%d", p->head_size);
}

}  // namespace
}  // namespace vaa

extern "C" int vaa_paged_attention_decode(const vaa_attn_params* p, const uint16_t* query,
                                          uint16_t* key_cache, uint16_t* value_cache,
                                          const int32_t* block_table, const int32_t* seq_lens,
                                          uint16_t* output, const uint16_t* new_keys,
                                          const uint16_t* new_values, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  return decode_impl("vaa_paged_attention_decode", p, query, key_cache, value_cache, block_table,
                     seq_lens, output, new_keys, new_values, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free decode.  The split-K partials live in a fixed device array
// instead of a caller workspace.  Each GPU the library runs on holds its own
// copy of the array (kScratchBytes) until the process ends.  In host code
// `scratch` names a host-side stand-in, not device memory: the kernels get
// the device address from hipGetSymbolAddress, taken once per device on the
// entry point's first call there with that device current.  The kernels
// write every row and header word they read in the same call (the partials
// of each split sequence, the balanced split's geometry), so nothing needs
// clearing between calls.  Calls that overlap on one GPU share the array and
// race.
constexpr size_t kScratchBytes = size_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace vaa {
namespace {

std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of this device's copy of `scratch`, or null with the error
// set.
void* scratch_ptr(const char* what) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(VAA_ERR_HIP, "%s: no current HIP device (or device id >= %d)", what, kMaxDevices);
    return nullptr;
  }
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr) return ptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    fail(VAA_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed: %s", what, hipGetErrorString(e));
    return nullptr;
  }
  g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  return ptr;
}

}  // namespace
}  // namespace vaa

extern "C" size_t vaa_paged_attention_decode_noalloc_max_workspace(void) {
  return kScratchBytes;
}

extern "C" int vaa_paged_attention_decode_noalloc(const vaa_attn_params* p,
                                                  const uint16_t* query, uint16_t* key_cache,
                                                  uint16_t* value_cache,
                                                  const int32_t* block_table,
                                                  const int32_t* seq_lens, uint16_t* output,
                                                  const uint16_t* new_keys,
                                                  const uint16_t* new_values, void* stream) {
  const char* what = "vaa_paged_attention_decode_noalloc";
  int st = check_params(p, what);
  if (st) return st;
  if (p->num_seqs == 0) return VAA_OK;
  Split sp;
  st = plan_split(p, &sp);
  if (st) return st;
  if (sp.ws_bytes > kScratchBytes)
    return fail(VAA_ERR_WORKSPACE,
                "%s: this split needs %zu bytes of partials, above the fixed %zu-byte device "
                "array (use VAA_PARTITION_BALANCED, larger partitions, or "
                "vaa_paged_attention_decode with a workspace)",
                what, sp.ws_bytes, kScratchBytes);
  void* ws = nullptr;
  if (sp.ws_bytes > 0) {
    ws = scratch_ptr(what);
    if (!ws) return VAA_ERR_HIP;
  }
  return decode_impl(what, p, query, key_cache, value_cache, block_table, seq_lens, output,
                     new_keys, new_values, ws, sp.ws_bytes > 0 ? kScratchBytes : 0, stream);
}

extern "C" int vaa_merge_attn_states(const float* partial_out, const float* partial_lse,
                                     const int32_t* num_parts, int num_seqs, int num_heads,
                                     int max_parts, int head_size, uint16_t* output,
                                     int64_t o_stride_token, int64_t o_stride_head,
                                     float* output_lse, int dtype, void* stream) {
  if (num_seqs < 0 || num_heads <= 0 || max_parts <= 0 || head_size <= 0)
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_merge_attn_states: num_seqs=%d num_heads=%d max_parts=%d head_size=%d",
                num_seqs, num_heads, max_parts, head_size);
  if (!valid_dtype(dtype))
    return fail(VAA_ERR_UNSUPPORTED, "vaa_merge_attn_states: dtype=%d", dtype);
  if (num_seqs == 0) return VAA_OK;
  if (!partial_out || !partial_lse || !output)
    return fail(VAA_ERR_INVALID_ARG, "vaa_merge_attn_states: null pointer");
  if (o_stride_token < 0 || o_stride_head < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_merge_attn_states: bad output strides");
  // Grid (num_heads, num_seqs): y is limited to 65535.
  if (num_seqs > 65535)
    return fail(VAA_ERR_UNSUPPORTED, "vaa_merge_attn_states: num_seqs=%d > 65535", num_seqs);
  StatesArgs a;
  a.part_out = partial_out;
  a.part_lse = partial_lse;
  a.num_parts = num_parts;
  a.out = reinterpret_cast<f16*>(output);
  a.out_lse = output_lse;
  a.H = num_heads;
  a.P = max_parts;
  a.D = head_size;
  a.o_st = o_stride_token;
  a.o_sh = o_stride_head;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == VAA_DTYPE_BF16)
    hipLaunchKernelGGL((merge_states_kernel<bf16>), dim3(num_heads, num_seqs), dim3(128), 0, st,
                       a);
  else
    hipLaunchKernelGGL((merge_states_kernel<f16>), dim3(num_heads, num_seqs), dim3(128), 0, st, a);
  return check_launch("merge_states_kernel");
}
