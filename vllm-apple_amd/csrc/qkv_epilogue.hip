// Fused QKV epilogue: bias add, NeoX rotary embedding on Q and K, and the KV
// write through slot_mapping, in one pass over the projection's Q/K/V views.
//
// The reference runs these as separate kernels over the planar QKV buffer
// [Q_all][K_all][V_all] (vllm_apple/engine/runner.py:919-1016):
//   bias_add_inplace_kernel on Q, K and V      engine/ops/qkv.py:391-416,
//                                              engine/ops/elementwise.py:252-259
//   rope_neox_kernel on Q and K                engine/ops/elementwise.py:185-239
//   kv_write_prefill (K and V -> cache)        engine/ops/kv_write.py:118-156
// each reading and writing Q/K/V through HBM again.  Here every 16-byte chunk
// is read once: biased (rounded to the 16-bit type, as the reference's
// in-place half add leaves it), rotated in fp32 with the same helper as the
// RoPE kernel, written back in place (Q, K; V only when a bias changed it),
// and K/V also go to their cache slot.  The result equals running the three
// kernels in turn.
//
// Work: a row of workgroups per token (the token's position and slot are read
// once); a thread takes one item of that token.  The Q and K items come first:
// a pair of 16-byte chunks (elements i..i+7 and i+rot/2..) of a head's
// rotated part, or one chunk of its unrotated tail [rot, D); then the V items,
// one chunk each, so no thread is idle.
#include "common.h"

#include <algorithm>

namespace vaa {
namespace {

struct EpiArgs {
  f16* q;
  f16* k;
  f16* v;
  const f16* bias;  // [H*D | KV*D | KV*D] or null
  const float* cosc;
  const float* sinc;
  const int32_t* pos;
  const void* slots;
  int slot_i64;
  f16* kc;
  f16* vc;
  int T, H, KV, D, rot, max_pos, bs;
  int64_t num_blocks;
  int64_t q_st, kv_st;  // token strides of q and of k / v (heads packed at stride D)
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
};

template <typename T>
__device__ __forceinline__ void unpack(u32x4 r, float* f) {
  const typename Elem<T>::x8 h = __builtin_bit_cast(typename Elem<T>::x8, r);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = Elem<T>::to_f(h[i]);
}

template <typename T>
__device__ __forceinline__ void load8(const f16* p, float* f) {
  unpack<T>(ld16(p), f);
}

template <typename T>
__device__ __forceinline__ u32x4 pack(const float* f) {
  typename Elem<T>::x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = Elem<T>::from_f(f[i]);
  return __builtin_bit_cast(u32x4, h);
}

// x + bias, rounded to T and widened again: the value the reference's in-place
// half add leaves in the buffer (for 16-bit operands the fp32 sum rounds to
// the same result as a direct half-precision add).
template <typename T>
__device__ __forceinline__ void add_bias(const f16* b, float* f) {
  float bf[8];
  load8<T>(b, bf);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = Elem<T>::to_f(Elem<T>::from_f(f[i] + bf[i]));
}

template <typename T>
__global__ void __launch_bounds__(1024) qkv_epilogue_kernel(EpiArgs a) {
  const int D = a.D, cpr = D / 8, half = a.rot / 2;
  const int rot_items = a.rot / 16;
  const int qk_items = rot_items + (D - a.rot) / 8;
  const int nqk = (a.H + a.KV) * qk_items;  // Q and K items of one token
  const int n_items = nqk + a.KV * cpr;     // plus the V chunks
  const int64_t cap = a.num_blocks * a.bs;
  for (int t = blockIdx.y; t < a.T; t += gridDim.y) {
    // Per-token values (wave-uniform).
    const int p = a.pos[t];
    const int64_t s = a.slot_i64 ? static_cast<const int64_t*>(a.slots)[t]
                                 : static_cast<const int32_t*>(a.slots)[t];
    const bool slot_ok = s >= 0 && s < cap;
    const int64_t blk = slot_ok ? s / a.bs : 0, off = slot_ok ? s % a.bs : 0;
    for (int it = blockIdx.x * blockDim.x + threadIdx.x; it < n_items;
         it += gridDim.x * blockDim.x) {
      int kind, j, item;  // kind 0 = query, 1 = key, 2 = value head
      if (it < nqk) {
        const int hh = it / qk_items;
        item = it - hh * qk_items;
        kind = hh < a.H ? 0 : 1;
        j = kind == 0 ? hh : hh - a.H;
      } else {
        const int r = it - nqk;
        j = r / cpr;
        item = r - j * cpr;
        kind = 2;
      }
      f16* x = kind == 0 ? a.q + t * a.q_st + static_cast<int64_t>(j) * D
                         : (kind == 1 ? a.k : a.v) + t * a.kv_st + static_cast<int64_t>(j) * D;
      const f16* b = nullptr;
      if (a.bias) {
        b = a.bias + (kind == 0 ? 0 : a.H * D + (kind - 1) * a.KV * D) + static_cast<int64_t>(j) * D;
      }
      // Cache row of this token for K/V heads (nullptr: padding or out of range).
      f16* crow = nullptr;
      if (kind > 0 && slot_ok) {
        crow = kind == 1 ? a.kc + blk * a.k_sb + j * a.k_sh + off * a.k_st
                         : a.vc + blk * a.v_sb + j * a.v_sh + off * a.v_st;
      }
    if (kind < 2 && item < rot_items) {
      const int i0 = 8 * item;
      float x0[8], x1[8], y0[8], y1[8];
      load8<T>(x + i0, x0);
      load8<T>(x + half + i0, x1);
      if (b) {
        add_bias<T>(b + i0, x0);
        add_bias<T>(b + half + i0, x1);
      }
      if (p >= 0 && p < a.max_pos) {
        float c[8], s[8];
        const float* cp = a.cosc + static_cast<int64_t>(p) * half + i0;
        const float* sp = a.sinc + static_cast<int64_t>(p) * half + i0;
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(cp);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(cp + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(sp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c[e] = c0[e];
          c[e + 4] = c1[e];
          s[e] = s0[e];
          s[e + 4] = s1[e];
        }
        rope_rotate8(x0, x1, c, s, y0, y1);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          y0[e] = x0[e];
          y1[e] = x1[e];
        }
      }
      const u32x4 w0 = pack<T>(y0), w1 = pack<T>(y1);
      st16(x + i0, w0);
      st16(x + half + i0, w1);
      if (crow) {
        st16(crow + i0, w0);
        st16(crow + half + i0, w1);
      }
    } else {
      // Unrotated chunk: the tail [rot, D) of a Q/K head, or any V chunk.
      const int c = kind < 2 ? a.rot / 8 + (item - rot_items) : item;
      u32x4 w = ld16(x + 8 * c);
      if (b) {
        float f[8];
        unpack<T>(w, f);
        add_bias<T>(b + 8 * c, f);
        w = pack<T>(f);
        st16(x + 8 * c, w);
      }
      if (crow) st16(crow + 8 * c, w);
    }
    }
  }
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_qkv_epilogue(const vaa_attn_params* p, uint16_t* query, uint16_t* key,
                                uint16_t* value, const uint16_t* bias, const float* cos_cache,
                                const float* sin_cache, int rotary_dim, int max_position,
                                const int32_t* positions, const void* slot_mapping,
                                int slot_index_type, uint16_t* key_cache,
                                uint16_t* value_cache, int num_tokens, void* stream) {
  const char* what = "vaa_qkv_epilogue";
  if (!p) return fail(VAA_ERR_INVALID_ARG, "%s: null params", what);
  if (!valid_dtype(p->dtype)) return fail(VAA_ERR_UNSUPPORTED, "%s: dtype=%d", what, p->dtype);
  if (num_tokens < 0) return fail(VAA_ERR_INVALID_ARG, "%s: num_tokens=%d", what, num_tokens);
  if (num_tokens == 0) return VAA_OK;
  const int D = p->head_size;
  if (D <= 0 || D % 16 != 0 || p->num_kv_heads <= 0 || p->num_query_heads <= 0 ||
      p->block_size <= 0 || p->num_blocks <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: head_size=%d heads=%d/%d block_size=%d", what, D,
                p->num_query_heads, p->num_kv_heads, p->block_size);
  if (rotary_dim <= 0 || rotary_dim > D || rotary_dim % 16 != 0)
    return fail(VAA_ERR_UNSUPPORTED, "%s: rotary_dim=%d (a multiple of 16, <= head_size)", what,
                rotary_dim);
  if (max_position < 0) return fail(VAA_ERR_INVALID_ARG, "%s: max_position=%d", what, max_position);
  if (!query || !key || !value || !cos_cache || !sin_cache || !positions || !slot_mapping ||
      !key_cache || !value_cache)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (slot_index_type != VAA_INDEX_I32 && slot_index_type != VAA_INDEX_I64)
    return fail(VAA_ERR_INVALID_ARG, "%s: slot_index_type=%d", what, slot_index_type);
  const int64_t strides[] = {p->q_stride_token, p->new_kv_stride_token, p->k_stride_block,
                             p->k_stride_head, p->k_stride_token, p->v_stride_block,
                             p->v_stride_head, p->v_stride_token};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0)
      return fail(VAA_ERR_INVALID_ARG, "%s: strides must be non-negative multiples of 8", what);
  if (p->q_stride_head != D || p->new_kv_stride_head != D)
    return fail(VAA_ERR_INVALID_ARG, "%s: heads must be packed at stride head_size", what);
  if (!aligned16(query) || !aligned16(key) || !aligned16(value) || !aligned16(key_cache) ||
      !aligned16(value_cache) || (bias && !aligned16(bias)) || !aligned16(cos_cache) ||
      !aligned16(sin_cache))
    return fail(VAA_ERR_INVALID_ARG, "%s: tensors must be 16-byte aligned", what);
  EpiArgs a;
  a.q = reinterpret_cast<f16*>(query);
  a.k = reinterpret_cast<f16*>(key);
  a.v = reinterpret_cast<f16*>(value);
  a.bias = reinterpret_cast<const f16*>(bias);
  a.cosc = cos_cache;
  a.sinc = sin_cache;
  a.pos = positions;
  a.slots = slot_mapping;
  a.slot_i64 = slot_index_type == VAA_INDEX_I64;
  a.kc = reinterpret_cast<f16*>(key_cache);
  a.vc = reinterpret_cast<f16*>(value_cache);
  a.T = num_tokens;
  a.H = p->num_query_heads;
  a.KV = p->num_kv_heads;
  a.D = D;
  a.rot = rotary_dim;
  a.max_pos = max_position;
  a.bs = p->block_size;
  a.num_blocks = p->num_blocks;
  a.q_st = p->q_stride_token;
  a.kv_st = p->new_kv_stride_token;
  a.k_sb = p->k_stride_block; a.k_sh = p->k_stride_head; a.k_st = p->k_stride_token;
  a.v_sb = p->v_stride_block; a.v_sh = p->v_stride_head; a.v_st = p->v_stride_token;
  // One row of workgroups per token: x covers the token's items, y the tokens.
  const int qk_items = rotary_dim / 16 + (D - rotary_dim) / 8;
  const int n_items = (a.H + a.KV) * qk_items + a.KV * (D / 8);
  // Workgroup sized to the token's items (whole waves, at most 1024 threads).
  const int wg = std::min(1024, (n_items + kWave - 1) / kWave * kWave);
  const dim3 grid((n_items + wg - 1) / wg, num_tokens < 65535 ? num_tokens : 65535);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (p->dtype == VAA_DTYPE_BF16)
    hipLaunchKernelGGL(qkv_epilogue_kernel<bf16>, grid, dim3(wg), 0, s, a);
  else
    hipLaunchKernelGGL(qkv_epilogue_kernel<f16>, grid, dim3(wg), 0, s, a);
  return check_launch("qkv_epilogue_kernel");
}
