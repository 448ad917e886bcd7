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
//   workgroup walks 32-key tiles of that sequence's cache:
//     S^T[32 keys x 32 queries] = K Q^T   (D/16 x mfma 32x32x16)
//     P = exp2(S*scale*log2e - m), causal/row mask as -inf
//     O^T[D x 32 queries]      += V^T P^T (D/16 x mfma 32x32x16)
//   The MFMA output layout of S^T (lane = query, 16 keys per lane) is the B
//   operand layout of the PV product, so the per-query softmax statistics sit
//   in the lanes that own the query's accumulators.
// Memory: K/V tiles are double-buffered in LDS (padded rows of D+8 halves) and
// filled from registers that were loaded from HBM during the previous tile's
// math, so one barrier per tile separates load and use.  V^T operands come
// from LDS with the gfx950 transpose read (ds_read_b64_tr_b16): within each
// 16-lane group, lanes 4r..4r+3 name 8-byte pieces of row r and lane i
// receives element i of rows 0..3, which is exactly a 4-key column of V.
#include "common.h"

namespace vaa {
namespace {

constexpr int kQT = 32;       // query tokens per wave (MFMA columns)
constexpr int kKT = 32;       // keys per tile
constexpr int kWavesP = 4;    // waves per workgroup
constexpr int kXcds = 8;      // accelerator complex dies on MI355X
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold (log2 units)
constexpr int kThreadsP = kWavesP * kWave;

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
  int num_tokens, num_seqs, max_blocks, block_size, G;
  int heads_per_wg, subtiles, head_chunks;
  int tiles_y, padded_tiles;  // logical grid rows; workgroups in use (multiple of 8)
  int64_t num_blocks;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int64_t q_st, q_sh, o_st, o_sh;
};

template <int D>
struct PCfg {
  static constexpr int LD = D + 8;                      // padded LDS row (halves)
  static constexpr int CH = D / 8;                      // 16-byte chunks per row
  static constexpr int NK = D / 16;                     // QK mfma count (K-dim 16)
  static constexpr int NDT = D / 32;                    // PV output tiles of 32 dims
  static constexpr int TILE = kKT * LD;                 // halves per staged tile
  static constexpr int MAXC = (kKT * CH + kThreadsP - 1) / kThreadsP;  // chunks/thread
};

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

__device__ __forceinline__ f16x4 lds_tr4(const f16* p) {
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(f16x4, r);
}

// Registers holding this thread's share of one K/V tile on its way to LDS.
template <int D>
struct Stage {
  u32x4 k[PCfg<D>::MAXC];
  u32x4 v[PCfg<D>::MAXC];
};

// The block-table entries of 64 consecutive blocks sit in one VGPR (one per
// lane) and are read with readlane, so the tile loop issues no scalar loads
// whose latency would sit in front of the K/V loads.
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

// Each 16-row half of a 32-key tile lies inside one cache block (block_size
// is a multiple of 16), so its base address is uniform and every thread adds
// a constant in-tile offset.  Rows past kv_len and rows of an invalid block
// are zero-filled.  A row whose context [0, lim] reaches an invalid block
// aborts (is never written), as paged_attention_v2.metal:428 does.
template <int D>
__device__ __forceinline__ void stage_load(const PrefillArgs& a, const int32_t* bts, int kvh,
                                           int key0, int kv_len, int lim, BlockWindow& w,
                                           bool& aborted, Stage<D>& st) {
  using C = PCfg<D>;
  const f16* kb[2];
  const f16* vb[2];
  bool ok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k0 = key0 + 16 * h;
    const int bi = k0 / a.block_size;
    int64_t phys = -1;
    if (k0 < kv_len) {
      phys = window_block(a, bts, bi, w);
      if (phys < 0 && k0 <= lim) aborted = true;
    }
    ok[h] = phys >= 0;
    if (!ok[h]) phys = 0;
    const int row0 = k0 - bi * a.block_size;
    kb[h] = a.kc + phys * a.k_sb + kvh * a.k_sh + row0 * a.k_st;
    vb[h] = a.vc + phys * a.v_sb + kvh * a.v_sh + row0 * a.v_st;
  }
#pragma unroll
  for (int i = 0; i < C::MAXC; ++i) {
    const int f = threadIdx.x + i * kThreadsP;
    st.k[i] = u32x4{0u, 0u, 0u, 0u};
    st.v[i] = u32x4{0u, 0u, 0u, 0u};
    if (f < kKT * C::CH) {
      const int kr = f / C::CH, ch = f % C::CH;
      const int h = kr >> 4, r = kr & 15;
      if (ok[h] && key0 + kr < kv_len) {
        st.k[i] = ld16(kb[h] + r * a.k_st + ch * 8);
        st.v[i] = ld16(vb[h] + r * a.v_st + ch * 8);
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void stage_store(f16* ks, f16* vs, const Stage<D>& st) {
  using C = PCfg<D>;
#pragma unroll
  for (int i = 0; i < C::MAXC; ++i) {
    const int f = threadIdx.x + i * kThreadsP;
    if (f < kKT * C::CH) {
      const int kr = f / C::CH, ch = f % C::CH;
      *reinterpret_cast<u32x4*>(ks + kr * C::LD + ch * 8) = st.k[i];
      *reinterpret_cast<u32x4*>(vs + kr * C::LD + ch * 8) = st.v[i];
    }
  }
}

// One 32-key tile for this wave's 32 query rows: S^T = K Q^T, online
// softmax, O^T += V^T P^T.
template <int D>
__device__ __forceinline__ void tile_math(const PrefillArgs& a, const f16* kb, const f16* vb,
                                          int key0, int lim, int k_rd, int v_rd, int hb,
                                          const u32x4 (&qb)[PCfg<D>::NK], float& m_run,
                                          float& l_part, f32x16 (&acc)[PCfg<D>::NDT]) {
  using C = PCfg<D>;
  // S^T = K Q^T : A lane = K[key l%32][hb*D/2 + 8s .. +7].
  f32x16 sacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
  for (int s2 = 0; s2 < C::NK; ++s2) {
    const u32x4 kA = *reinterpret_cast<const u32x4*>(kb + k_rd + 8 * s2);
    sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, kA),
                                                  __builtin_bit_cast(f16x8, qb[s2]), sacc, 0,
                                                  0, 0);
  }
  // Lane holds keys 8(r/4) + 4hb + r%4 for query qj.  The mask is only
  // evaluated when some row of the wave cannot see the whole tile.
  const int rel = lim - key0;
  float mx = -INFINITY;
  if (__builtin_amdgcn_ballot_w64(rel < kKT - 1) != 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kl = 8 * (r >> 2) + 4 * hb + (r & 3);
      if (kl > rel) sacc[r] = -INFINITY;
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave)) * a.scale_log2;
  // Lazy rescale: keep the reference max unless a score exceeds it by more
  // than 2^8 (p stays <= 256, exact in fp16); the wave-uniform branch is
  // taken on a row's first tile and on rare outliers only.  Only lanes whose
  // max grows rescale (a fully masked lane keeps m_run = -inf and must not
  // form -inf - -inf).
  if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleLog2) != 0 && mx > m_run) {
    const float alpha = fast_exp2(m_run - mx);  // 0 when m_run = -inf
    l_part *= alpha;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) acc[dt] *= alpha;
    m_run = mx;
  }
  const float m_sub = (m_run == -INFINITY) ? 0.f : m_run;
  f16x8 pb[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float p = fast_exp2(fmaf(sacc[r], a.scale_log2, -m_sub));
    pb[r >> 3][r & 7] = f2h(p);
    l_part += p;
  }
  // O^T += V^T P^T; MFMA c covers keys 16c + 4hb + (i%4) + 8(i/4), i < 8.
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const f16* vp = vb + v_rd + (16 * c) * C::LD + 32 * dt;
      const f16x4 lo = lds_tr4(vp);
      const f16x4 hi = lds_tr4(vp + 8 * C::LD);
      const f16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[c], acc[dt], 0, 0, 0);
    }
  }
}

template <int D>
__global__ void __launch_bounds__(kThreadsP) __attribute__((amdgpu_waves_per_eu(2, 2)))
paged_prefill_kernel(PrefillArgs a) {
  using C = PCfg<D>;
  __shared__ __align__(16) f16 ks[2][C::TILE];
  __shared__ __align__(16) f16 vs[2][C::TILE];
  __shared__ int red[2][kWavesP];

  // XCD-aware placement: the hardware hands consecutive workgroup ids to the
  // 8 XCDs in turn, so id i runs on XCD i % 8.  Give each XCD a contiguous
  // range of (kv head, query tile) work so the query tiles that reuse one
  // sequence's K/V tiles share that XCD's L2.
  const int gx = gridDim.x;
  const int id = blockIdx.x + gx * blockIdx.y;
  if (id >= a.padded_tiles) return;  // grid rounding beyond the padded count
  const int per_xcd = a.padded_tiles / kXcds;
  const int logical = (id % kXcds) * per_xcd + id / kXcds;
  if (logical >= gx * a.tiles_y) return;
  const int tile_x = logical % gx, tile_y = logical / gx;
  const int kvh = tile_y / a.head_chunks;
  const int hchunk = tile_y % a.head_chunks;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int hw = wave % a.heads_per_wg, sub = wave / a.heads_per_wg;
  const int ghead = hchunk * a.heads_per_wg + hw;             // head index in the group
  const bool math = sub < a.subtiles && ghead < a.G;         // this wave computes
  const int head = kvh * a.G + (ghead < a.G ? ghead : 0);
  const int qj = lane & 31, hb = lane >> 5;
  const int g16 = lane >> 4, i16 = lane & 15;

  // Per-lane query token (lanes l and l+32 share token qj).
  const int tok = tile_x * (kQT * a.subtiles) + (sub < a.subtiles ? sub : 0) * kQT + qj;
  int tseq = -1, tpos = -1;
  if (sub < a.subtiles && tok < a.num_tokens) {
    tseq = a.tok_seq[tok];
    tpos = a.pos[tok];
  }
  bool row_ok = tseq >= 0 && tseq < a.num_seqs && tpos >= 0;
  if (row_ok) {
    const int64_t nb = (static_cast<int64_t>(tpos) + a.block_size) / a.block_size;
    if (nb > a.max_blocks) row_ok = false;  // context longer than the table
  }
  bool done = !row_ok;
  bool aborted = false;

  // Q^T as B operand: lane holds Q[token qj][hb*D/2 + 8s .. +7], s < NK.
  u32x4 qb[C::NK];
  {
    const bool ld = row_ok && math;
    const f16* qp = a.q + static_cast<int64_t>(ld ? tok : 0) * a.q_st + head * a.q_sh +
                    hb * (D / 2);
#pragma unroll
    for (int s = 0; s < C::NK; ++s) qb[s] = ld ? ld16(qp + 8 * s) : u32x4{0u, 0u, 0u, 0u};
  }

  float m_run = -INFINITY, l_part = 0.f;
  f32x16 acc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  // LDS element offsets of this lane's operand reads (constant over tiles).
  const int k_rd = qj * C::LD + hb * (D / 2);
  const int v_rd = (4 * hb + (i16 >> 2)) * C::LD + 16 * (g16 & 1) + 4 * (i16 & 3);

  while (true) {
    // Next sequence among the workgroup's unfinished tokens, and its context.
    int s = wave_min_i(done ? INT32_MAX : tseq);
    if (lane == 0) red[0][wave] = s;
    __syncthreads();
    s = red[0][0];
#pragma unroll
    for (int w = 1; w < kWavesP; ++w) s = min(s, red[0][w]);
    if (s == INT32_MAX) break;
    const bool active = !done && tseq == s;
    int kv_len = wave_max_i(active ? tpos + 1 : 0);
    if (lane == 0) red[1][wave] = kv_len;
    __syncthreads();
    kv_len = red[1][0];
#pragma unroll
    for (int w = 1; w < kWavesP; ++w) kv_len = max(kv_len, red[1][w]);
    const int n_kt = (kv_len + kKT - 1) / kKT;
    const int32_t* bts = a.bt + static_cast<int64_t>(s) * a.max_blocks;
    const int lim = active ? tpos : -1;  // last key position this row may see

    // Two register stages rotate so K/V loads run two tiles ahead of the
    // math; LDS holds the tile being computed and the next one.
    BlockWindow win;
    window_load(a, bts, 0, win);
    Stage<D> sa, sb;
    stage_load<D>(a, bts, kvh, 0, kv_len, lim, win, aborted, sa);
    if (n_kt > 1) stage_load<D>(a, bts, kvh, kKT, kv_len, lim, win, aborted, sb);
    stage_store<D>(ks[0], vs[0], sa);
    __syncthreads();
    for (int kt = 0; kt < n_kt; kt += 2) {
      if (kt + 2 < n_kt) stage_load<D>(a, bts, kvh, (kt + 2) * kKT, kv_len, lim, win, aborted, sa);
      if (math) tile_math<D>(a, ks[0], vs[0], kt * kKT, lim, k_rd, v_rd, hb, qb, m_run, l_part, acc);
      if (kt + 1 < n_kt) stage_store<D>(ks[1], vs[1], sb);
      __syncthreads();
      if (kt + 1 >= n_kt) break;
      if (kt + 3 < n_kt) stage_load<D>(a, bts, kvh, (kt + 3) * kKT, kv_len, lim, win, aborted, sb);
      if (math)
        tile_math<D>(a, ks[1], vs[1], (kt + 1) * kKT, lim, k_rd, v_rd, hb, qb, m_run, l_part, acc);
      if (kt + 2 < n_kt) stage_store<D>(ks[0], vs[0], sa);
      __syncthreads();
    }
    done = done || active;
  }

  if (!math) return;
  const float l_tot = l_part + __shfl_xor(l_part, 32, kWave);
  if (!row_ok || aborted) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  f16* op = a.out + static_cast<int64_t>(tok) * a.o_st + head * a.o_sh;
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = f2h(acc[dt][4 * rg + i] * inv);
      const int d = 32 * dt + 8 * rg + 4 * hb;
      *reinterpret_cast<f16x4*>(op + d) = o;
    }
  }
}

template <int D>
int launch_prefill(const PrefillArgs& a, int num_kv_heads, hipStream_t stream) {
  const int per_wg = kQT * a.subtiles;
  const int gx = (a.num_tokens + per_wg - 1) / per_wg, gy = num_kv_heads * a.head_chunks;
  // Pad the grid to a multiple of the XCD count so every logical tile has a
  // slot under the XCD remap (surplus workgroups exit at once).
  const int total = gx * gy, padded = (total + kXcds - 1) / kXcds * kXcds;
  PrefillArgs b = a;
  b.tiles_y = gy;
  b.padded_tiles = padded;
  dim3 grid(gx, (padded + gx - 1) / gx);
  hipLaunchKernelGGL(paged_prefill_kernel<D>, grid, dim3(kThreadsP), 0, stream, b);
  return check_launch("paged_prefill_kernel");
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_paged_attention_prefill(const vaa_attn_params* p,
                                           const uint16_t* query,
                                           const uint16_t* key_cache,
                                           const uint16_t* value_cache,
                                           const int32_t* block_table,
                                           const int32_t* token_to_seq,
                                           const int32_t* positions,
                                           uint16_t* output, int num_tokens,
                                           void* stream) {
  if (!p) return fail(VAA_ERR_INVALID_ARG, "vaa_paged_attention_prefill: null params");
  if (p->head_size != 32 && p->head_size != 64 && p->head_size != 96 &&
      p->head_size != 128)
    return fail(VAA_ERR_UNSUPPORTED,
                "vaa_paged_attention_prefill: head_size=%d not in {32,64,96,128}",
                p->head_size);
  if (p->block_size <= 0 || p->num_kv_heads <= 0 || p->num_query_heads <= 0 ||
      p->num_query_heads % p->num_kv_heads != 0 ||
      p->queries_per_kv != p->num_query_heads / p->num_kv_heads ||
      p->max_blocks_per_seq <= 0 || p->num_blocks <= 0 || p->num_seqs < 0 ||
      num_tokens < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_paged_attention_prefill: bad shape params");
  if (num_tokens == 0) return VAA_OK;
  if (!query || !key_cache || !value_cache || !block_table || !token_to_seq ||
      !positions || !output)
    return fail(VAA_ERR_INVALID_ARG, "vaa_paged_attention_prefill: null pointer");
  const int64_t strides[] = {p->k_stride_block, p->k_stride_head, p->k_stride_token,
                             p->v_stride_block, p->v_stride_head, p->v_stride_token,
                             p->q_stride_token, p->q_stride_head, p->o_stride_token,
                             p->o_stride_head};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0)
      return fail(VAA_ERR_INVALID_ARG,
                  "vaa_paged_attention_prefill: strides must be multiples of 8 elements");
  if (!aligned16(query) || !aligned16(key_cache) || !aligned16(value_cache) ||
      !aligned16(output))
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_paged_attention_prefill: tensors must be 16-byte aligned");
  PrefillArgs a;
  a.q = reinterpret_cast<const f16*>(query);
  a.kc = reinterpret_cast<const f16*>(key_cache);
  a.vc = reinterpret_cast<const f16*>(value_cache);
  a.bt = block_table;
  a.tok_seq = token_to_seq;
  a.pos = positions;
  a.out = reinterpret_cast<f16*>(output);
  a.scale_log2 = p->scale * kLog2e;
  a.num_tokens = num_tokens;
  a.num_seqs = p->num_seqs;
  a.max_blocks = p->max_blocks_per_seq;
  a.block_size = p->block_size;
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
  a.k_sb = p->k_stride_block; a.k_sh = p->k_stride_head; a.k_st = p->k_stride_token;
  a.v_sb = p->v_stride_block; a.v_sh = p->v_stride_head; a.v_st = p->v_stride_token;
  a.q_st = p->q_stride_token; a.q_sh = p->q_stride_head;
  a.o_st = p->o_stride_token; a.o_sh = p->o_stride_head;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (p->head_size) {
    case 32: return launch_prefill<32>(a, p->num_kv_heads, s);
    case 64: return launch_prefill<64>(a, p->num_kv_heads, s);
    case 96: return launch_prefill<96>(a, p->num_kv_heads, s);
    case 128: return launch_prefill<128>(a, p->num_kv_heads, s);
  }
  return fail(VAA_ERR_UNSUPPORTED, "head_size=%d", p->head_size);
}
