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
//   grid  = (32-token query tile, kv_head x head-chunk); a workgroup has one
//           wave per query head (up to 4 heads of the GQA group), and the
//           waves share every K/V tile staged in LDS.
//   For each distinct sequence among the tile's tokens (normally one), the
//   workgroup walks 32-key tiles of that sequence's cache:
//     S^T[32 keys x 32 queries] = K Q^T   (D/16 x mfma 32x32x16)
//     P = exp2(S*scale*log2e - m), causal/row mask as -inf
//     O^T[D x 32 queries]      += V^T P^T (D/16 x mfma 32x32x16)
//   The MFMA output layout of S^T (lane = query, 16 keys per lane) is the B
//   operand layout of the PV product, so the per-query softmax statistics sit
//   in the lanes that own the query's accumulators.
#include "common.h"

namespace vaa {
namespace {

constexpr int kQT = 32;        // query tokens per workgroup
constexpr int kKT = 32;        // keys per tile
constexpr int kMaxWaves = 4;   // query heads per workgroup

struct PrefillArgs {
  const f16* q;
  const f16* kc;
  const f16* vc;
  const int32_t* bt;
  const int32_t* tok_seq;
  const int32_t* pos;
  f16* out;
  float scale_log2;
  int num_tokens, num_seqs, max_blocks, block_size, G, head_chunks;
  int64_t num_blocks;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int64_t q_st, q_sh, o_st, o_sh;
};

template <int D>
struct PCfg {
  static constexpr int LD = D + 8;        // padded LDS row (halves)
  static constexpr int CH = D / 8;        // 16-byte chunks per row
  static constexpr int NK = D / 16;       // QK mfma count (K-dim 16)
  static constexpr int NDT = D / 32;      // PV output tiles of 32 dims
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

template <int D>
__global__ void __launch_bounds__(kMaxWaves* kWave)
paged_prefill_kernel(PrefillArgs a) {
  using C = PCfg<D>;
  __shared__ __align__(16) f16 ks[kKT * C::LD];
  __shared__ __align__(16) f16 vs[kKT * C::LD];
  __shared__ int s_bad;  // bit b set: 16-key sub-block b of the tile is invalid

  const int tile0 = blockIdx.x * kQT;
  const int kvh = blockIdx.y / a.head_chunks;
  const int hchunk = blockIdx.y % a.head_chunks;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int nthreads = blockDim.x;
  const int head = kvh * a.G + hchunk * kMaxWaves + wave;  // query head
  const int qj = lane & 31, hb = lane >> 5;

  // Per-lane query token (lanes l and l+32 share token qj).
  const int tok = tile0 + qj;
  int tseq = -1, tpos = -1;
  if (tok < a.num_tokens) {
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
    const bool ld = row_ok && head < kvh * a.G + a.G;
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

  while (true) {
    const int cand = done ? INT32_MAX : tseq;
    const int s = wave_min_i(cand);
    if (s == INT32_MAX) break;  // identical in every wave: same tokens
    const bool active = !done && tseq == s;
    const int kv_len = wave_max_i(active ? tpos + 1 : 0);
    const int n_kt = (kv_len + kKT - 1) / kKT;
    const int32_t* bts = a.bt + static_cast<int64_t>(s) * a.max_blocks;

    for (int kt = 0; kt < n_kt; ++kt) {
      const int key0 = kt * kKT;
      __syncthreads();  // previous tile fully consumed
      if (threadIdx.x == 0) s_bad = 0;
      __syncthreads();
      // Stage K and V rows [key0, key0+32) of sequence s into LDS.
      for (int f = threadIdx.x; f < kKT * C::CH; f += nthreads) {
        const int kr = f / C::CH, ch = f % C::CH;
        const int kpos = key0 + kr;
        const int bi = kpos / a.block_size;
        int64_t phys = bi < a.max_blocks ? bts[bi] : -1;
        const bool bvalid = phys >= 0 && phys < a.num_blocks;
        u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
        if (bvalid && kpos < kv_len) {
          const int row = kpos - bi * a.block_size;
          kv = ld16(a.kc + phys * a.k_sb + kvh * a.k_sh + row * a.k_st + ch * 8);
          vv = ld16(a.vc + phys * a.v_sb + kvh * a.v_sh + row * a.v_st + ch * 8);
        }
        if (!bvalid && kpos < kv_len && ch == 0) atomicOr(&s_bad, 1 << (kr / 16));
        *reinterpret_cast<u32x4*>(ks + kr * C::LD + ch * 8) = kv;
        *reinterpret_cast<u32x4*>(vs + kr * C::LD + ch * 8) = vv;
      }
      __syncthreads();
      // A row aborts (is never written) when a block inside its context is
      // invalid, as paged_attention_v2.metal:428 does.
      const int bad = s_bad;
      if (active && bad) {
        for (int b = 0; b < 2; ++b)
          if ((bad >> b) & 1)
            if (key0 + 16 * b <= tpos) aborted = true;
      }
      if (head >= kvh * a.G + a.G) continue;  // idle wave (G not a multiple of 4)

      // S^T = K Q^T : A lane = K[key l%32][hb*D/2 + 8s .. +7].
      f32x16 st;
#pragma unroll
      for (int r = 0; r < 16; ++r) st[r] = 0.f;
      const f16* krow = ks + qj * C::LD + hb * (D / 2);
#pragma unroll
      for (int s2 = 0; s2 < C::NK; ++s2) {
        const u32x4 kA = *reinterpret_cast<const u32x4*>(krow + 8 * s2);
        st = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, kA),
                                                    __builtin_bit_cast(f16x8, qb[s2]),
                                                    st, 0, 0, 0);
      }
      // Lane holds keys 8(r/4) + 4hb + r%4 for query qj.
      float x[16];
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kp = key0 + 8 * (r >> 2) + 4 * hb + (r & 3);
        const bool ok = active && kp <= tpos;
        x[r] = ok ? st[r] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_new == m_run) ? 1.f : fast_exp2(m_run - m_new);
      const float m_sub = (m_new == -INFINITY) ? 0.f : m_new;
      f16x8 pb[2];
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const f16 p = f2h(fast_exp2(x[r] - m_sub));
        pb[r >> 3][r & 7] = p;
        psum += h2f(p);
      }
      l_part = l_part * alpha + psum;
      m_run = m_new;
      if (alpha != 1.f) {
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) acc[dt] *= alpha;
      }
      // O^T += V^T P^T. MFMA c covers keys 16c + 4hb + (i%4) + 8(i/4), i < 8.
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        const int d = 32 * dt + qj;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          f16x8 va;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int key = 16 * c + 4 * hb + (i & 3) + 8 * (i >> 2);
            va[i] = vs[key * C::LD + d];
          }
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[c], acc[dt], 0, 0, 0);
        }
      }
    }
    done = done || active;
  }

  if (head >= kvh * a.G + a.G) return;
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
  const int waves = a.G < kMaxWaves ? a.G : kMaxWaves;
  dim3 grid((a.num_tokens + kQT - 1) / kQT, num_kv_heads * a.head_chunks);
  hipLaunchKernelGGL(paged_prefill_kernel<D>, grid, dim3(waves * kWave), 0, stream, a);
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
  a.head_chunks = (a.G + kMaxWaves - 1) / kMaxWaves;
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
