// Bandwidth-bound layer ops next to attention: RMSNorm (+ post-norm residual),
// NeoX rotary embedding (in place on Q and K) and SwiGLU (silu(gate) * up).
// 16-bit in / 16-bit out (fp16, the reference's type, or bf16) with fp32
// arithmetic; 16-byte vector accesses when the views allow it, 2-byte
// fallbacks otherwise.  Rows read once carry the nontemporal hint (C5 on
// MI355X: RMSNorm 11.9 -> 10.9 us, RoPE 10.8 -> 10.1 us); the norm weights,
// read by every row, do not.
#include "common.h"

namespace vaa {
namespace {

template <typename T>
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
  const typename Elem<T>::x8 h = __builtin_bit_cast(typename Elem<T>::x8, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = Elem<T>::to_f(h[i]);
}
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* f) {
  typename Elem<T>::x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = Elem<T>::from_f(f[i]);
  return __builtin_bit_cast(u32x4, h);
}

// ---------------------------------------------------------------- RMSNorm --
// rmsnorm.py:78-173: out = half(float(x) * rsqrt(sum(x^2)/H + eps) * float(w)),
// plus float(residual) after the norm when a residual is given.
// One wave per row; NC 16-byte chunks per lane stay in registers so x is read
// from HBM once (NC == 0: rows too long for registers, second pass re-reads).
//
// kAdd: the residual add that precedes the norm in the reference's layer
// (runner.py:1107-1130: residual_add, copy to the residual buffer, norm in
// place) in one pass: h = half(x + r) is written back to r, and the norm of h
// goes to out (which may alias x).  The norm's arithmetic is the plain
// kernel's on h, so the result equals the three steps bit for bit.
constexpr int kNormRowsPerBlock = 4;

template <int NC, bool kAdd, typename T>
__global__ void __launch_bounds__(kNormRowsPerBlock* kWave)
rmsnorm_vec_kernel(const T* in, T* out, const T* w, T* res, int rows,
                   int H, int64_t in_st, int64_t out_st, int64_t res_st,
                   float eps) {
  const int row = blockIdx.x * kNormRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const int chunks = H / 8;
  const T* x = in + row * in_st;
  T* r = res ? res + row * res_st : nullptr;
  // The row's values: x, or (kAdd) h = half(x + r), written back to r.
  auto load = [&](int c) {
    const u32x4 v = ld16_stream(x + 8 * c);
    if constexpr (!kAdd) {
      return v;
    } else {
      float f[8], rf[8];
      unpack8<T>(v, f);
      unpack8<T>(ld16_stream(r + 8 * c), rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] += rf[e];
      const u32x4 h = pack8<T>(f);
      st16(r + 8 * c, h);
      return h;
    }
  };
  float ss = 0.f;
  u32x4 xv[NC > 0 ? NC : 1];
  if constexpr (NC > 0) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + i * kWave;
      xv[i] = c < chunks ? load(c) : u32x4{0u, 0u, 0u, 0u};
      float f[8];
      unpack8<T>(xv[i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  } else {
    for (int c = lane; c < chunks; c += kWave) {
      float f[8];
      unpack8<T>(load(c), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / static_cast<float>(H) + eps);
  T* o = out + row * out_st;
  auto emit = [&](int c, u32x4 v) {
    float f[8], wf[8];
    unpack8<T>(v, f);
    unpack8<T>(ld16(w + 8 * c), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (f[e] * rs) * wf[e];
    if (!kAdd && r) {
      float rf[8];
      unpack8<T>(ld16(r + 8 * c), rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] += rf[e];
    }
    st16(o + 8 * c, pack8<T>(f));
  };
  if constexpr (NC > 0) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + i * kWave;
      if (c < chunks) emit(c, xv[i]);
    }
  } else {
    // Second pass: h was written to r by this lane (kAdd), x otherwise.
    for (int c = lane; c < chunks; c += kWave) emit(c, ld16((kAdd ? r : x) + 8 * c));
  }
}

template <bool kAdd, typename T>
__global__ void __launch_bounds__(kNormRowsPerBlock* kWave)
rmsnorm_scalar_kernel(const T* in, T* out, const T* w, T* res,
                      int rows, int H, int64_t in_st, int64_t out_st,
                      int64_t res_st, float eps) {
  const int row = blockIdx.x * kNormRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const T* x = in + row * in_st;
  T* r = res ? res + row * res_st : nullptr;
  float ss = 0.f;
  for (int i = lane; i < H; i += kWave) {
    float v = Elem<T>::to_f(x[i]);
    if constexpr (kAdd) {
      const T h = Elem<T>::from_f(v + Elem<T>::to_f(r[i]));
      r[i] = h;
      v = Elem<T>::to_f(h);
    }
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / static_cast<float>(H) + eps);
  T* o = out + row * out_st;
  const T* src = kAdd ? r : x;
  for (int i = lane; i < H; i += kWave) {
    float v = (Elem<T>::to_f(src[i]) * rs) * Elem<T>::to_f(w[i]);
    if (!kAdd && r) v += Elem<T>::to_f(r[i]);
    o[i] = Elem<T>::from_f(v);
  }
}

// ------------------------------------------------------------------- RoPE --
// elementwise.py:185-239: for pair i < rot/2 of every q and k head,
//   (x_i, x_{i+rot/2}) <- (x_i c - x_{i+rot/2} s, x_i s + x_{i+rot/2} c)
// with c, s = cos/sin_cache[positions[t], i] (fp32), in place.
template <typename E>
struct RopeArgs {
  E* q;
  E* k;
  const float* cosc;
  const float* sinc;
  const int32_t* pos;
  int T, H, KV, D, rot, max_pos;
  int64_t q_st, k_st;
};

// One thread rotates 8 consecutive pairs of one head.
template <typename T>
__global__ void __launch_bounds__(256) rope_neox_vec_kernel(RopeArgs<T> a) {
  const int half = a.rot / 2;
  const int groups = half / 8;
  const int heads = a.H + (a.k ? a.KV : 0);
  const int64_t total = static_cast<int64_t>(a.T) * heads * groups;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int gi = static_cast<int>(idx % groups);
    const int64_t th = idx / groups;
    const int hh = static_cast<int>(th % heads);
    const int t = static_cast<int>(th / heads);
    const int p = a.pos[t];
    if (p < 0 || p >= a.max_pos) continue;
    T* x = hh < a.H ? a.q + t * a.q_st + static_cast<int64_t>(hh) * a.D
                      : a.k + t * a.k_st + static_cast<int64_t>(hh - a.H) * a.D;
    const int i0 = 8 * gi;
    const float* cp = a.cosc + static_cast<int64_t>(p) * half + i0;
    const float* sp = a.sinc + static_cast<int64_t>(p) * half + i0;
    float c[8], s[8], x0[8], x1[8];
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
    unpack8<T>(ld16_stream(x + i0), x0);
    unpack8<T>(ld16_stream(x + i0 + half), x1);
    float y0[8], y1[8];
    rope_rotate8(x0, x1, c, s, y0, y1);
    st16(x + i0, pack8<T>(y0));
    st16(x + i0 + half, pack8<T>(y1));
  }
}

template <typename T>
__global__ void __launch_bounds__(256) rope_neox_scalar_kernel(RopeArgs<T> a) {
  const int half = a.rot / 2;
  const int heads = a.H + (a.k ? a.KV : 0);
  const int64_t total = static_cast<int64_t>(a.T) * heads * half;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int i = static_cast<int>(idx % half);
    const int64_t th = idx / half;
    const int hh = static_cast<int>(th % heads);
    const int t = static_cast<int>(th / heads);
    const int p = a.pos[t];
    if (p < 0 || p >= a.max_pos) continue;
    T* x = hh < a.H ? a.q + t * a.q_st + static_cast<int64_t>(hh) * a.D
                      : a.k + t * a.k_st + static_cast<int64_t>(hh - a.H) * a.D;
    const float c = a.cosc[static_cast<int64_t>(p) * half + i];
    const float s = a.sinc[static_cast<int64_t>(p) * half + i];
    const float x0 = Elem<T>::to_f(x[i]), x1 = Elem<T>::to_f(x[i + half]);
    x[i] = Elem<T>::from_f(x0 * c - x1 * s);
    x[i + half] = Elem<T>::from_f(x0 * s + x1 * c);
  }
}

// ----------------------------------------------------------------- SwiGLU --
// elementwise.py:114-124: out = half(g / (1 + exp(-g)) * u) in fp32.
template <typename T>
__global__ void __launch_bounds__(256)
silu_mul_vec_kernel(const T* gate, const T* up, T* out, int64_t rows,
                    int64_t cols, int64_t g_st, int64_t u_st, int64_t o_st) {
  const int64_t cpr = cols / 8;
  const int64_t total = rows * cpr;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cpr, c = (idx % cpr) * 8;
    float g[8], u[8], y[8];
    unpack8<T>(ld16_stream(gate + r * g_st + c), g);
    unpack8<T>(ld16_stream(up + r * u_st + c), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = silu_mul1(g[e], u[e]);
    st16(out + r * o_st + c, pack8<T>(y));
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
silu_mul_scalar_kernel(const T* gate, const T* up, T* out, int64_t rows,
                       int64_t cols, int64_t g_st, int64_t u_st, int64_t o_st) {
  const int64_t total = rows * cols;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cols, c = idx % cols;
    out[r * o_st + c] = Elem<T>::from_f(
        silu_mul1(Elem<T>::to_f(gate[r * g_st + c]), Elem<T>::to_f(up[r * u_st + c])));
  }
}

int64_t grid_for(int64_t work, int64_t per_block, int64_t cap) {
  int64_t b = (work + per_block - 1) / per_block;
  if (b < 1) b = 1;
  return b > cap ? cap : b;
}

}  // namespace
}  // namespace vaa

using namespace vaa;

namespace vaa {
namespace {

template <bool kAdd, typename T>
int launch_rmsnorm(const char* what, const void* in_, void* out_, const void* w_, void* r_, int T_,
                   int H, int64_t in_st, int64_t out_st, int64_t r_st, float eps, hipStream_t s) {
  const T* in = static_cast<const T*>(in_);
  T* out = static_cast<T*>(out_);
  const T* w = static_cast<const T*>(w_);
  T* r = static_cast<T*>(r_);
  const dim3 grid((T_ + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
  const dim3 block(kNormRowsPerBlock * kWave);
  const bool vec = H % 8 == 0 && aligned16(in) && aligned16(out) && aligned16(w) &&
                   (!r || aligned16(r)) && in_st % 8 == 0 && out_st % 8 == 0 &&
                   (!r || r_st % 8 == 0);
  if (!vec) {
    hipLaunchKernelGGL((rmsnorm_scalar_kernel<kAdd, T>), grid, block, 0, s, in, out, w, r, T_,
                       H, in_st, out_st, r_st, eps);
    return check_launch(what);
  }
  const int per_lane = (H / 8 + kWave - 1) / kWave;
#define VAA_NORM(NC)                                                                \
  hipLaunchKernelGGL((rmsnorm_vec_kernel<NC, kAdd, T>), grid, block, 0, s, in, out, w, r, \
                     T_, H, in_st, out_st, r_st, eps)
  if (per_lane <= 1) VAA_NORM(1);
  else if (per_lane <= 2) VAA_NORM(2);
  else if (per_lane <= 4) VAA_NORM(4);
  else if (per_lane <= 8) VAA_NORM(8);
  else if (per_lane <= 10) VAA_NORM(10);
  else if (per_lane <= 16) VAA_NORM(16);
  else VAA_NORM(0);
#undef VAA_NORM
  return check_launch(what);
}

template <typename T>
int launch_rope(const RopeArgs<T>& a, bool vec, int64_t heads, hipStream_t s) {
  const int half = a.rot / 2;
  if (vec) {
    const int64_t work = static_cast<int64_t>(a.T) * heads * (half / 8);
    hipLaunchKernelGGL((rope_neox_vec_kernel<T>), dim3(grid_for(work, 256, 1 << 20)),
                       dim3(256), 0, s, a);
    return check_launch("rope_neox_vec_kernel");
  }
  const int64_t work = static_cast<int64_t>(a.T) * heads * half;
  hipLaunchKernelGGL((rope_neox_scalar_kernel<T>), dim3(grid_for(work, 256, 1 << 20)),
                     dim3(256), 0, s, a);
  return check_launch("rope_neox_scalar_kernel");
}

template <typename T>
int launch_silu(const void* g_, const void* u_, void* o_, int64_t rows, int64_t cols,
                int64_t g_st, int64_t u_st, int64_t o_st, hipStream_t s) {
  const T* g = static_cast<const T*>(g_);
  const T* u = static_cast<const T*>(u_);
  T* o = static_cast<T*>(o_);
  const bool vec = cols % 8 == 0 && aligned16(g) && aligned16(u) && aligned16(o) &&
                   (rows == 1 || (g_st % 8 == 0 && u_st % 8 == 0 && o_st % 8 == 0));
  if (vec) {
    const int64_t work = rows * (cols / 8);
    hipLaunchKernelGGL((silu_mul_vec_kernel<T>), dim3(grid_for(work, 256, 1 << 16)), dim3(256),
                       0, s, g, u, o, rows, cols, g_st, u_st, o_st);
    return check_launch("silu_mul_vec_kernel");
  }
  hipLaunchKernelGGL((silu_mul_scalar_kernel<T>), dim3(grid_for(rows * cols, 256, 1 << 16)),
                     dim3(256), 0, s, g, u, o, rows, cols, g_st, u_st, o_st);
  return check_launch("silu_mul_scalar_kernel");
}

}  // namespace
}  // namespace vaa

extern "C" int vaa_rmsnorm(const uint16_t* input, uint16_t* output,
                           const uint16_t* weight, const uint16_t* residual,
                           int num_tokens, int hidden_size, int64_t input_stride,
                           int64_t output_stride, int64_t residual_stride,
                           float eps, int dtype, void* stream) {
  if (num_tokens < 0 || hidden_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_rmsnorm: num_tokens=%d hidden_size=%d",
                num_tokens, hidden_size);
  if (!valid_dtype(dtype)) return fail(VAA_ERR_UNSUPPORTED, "vaa_rmsnorm: dtype=%d", dtype);
  if (num_tokens == 0) return VAA_OK;
  if (!input || !output || !weight)
    return fail(VAA_ERR_INVALID_ARG, "vaa_rmsnorm: null pointer");
  if (input_stride < hidden_size || output_stride < hidden_size ||
      (residual && residual_stride < hidden_size))
    return fail(VAA_ERR_INVALID_ARG, "vaa_rmsnorm: row stride < hidden_size");
  // The residual is only read here.
  void* r = const_cast<uint16_t*>(residual);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == VAA_DTYPE_BF16
             ? launch_rmsnorm<false, bf16>("rmsnorm_kernel", input, output, weight, r, num_tokens,
                                           hidden_size, input_stride, output_stride,
                                           residual_stride, eps, s)
             : launch_rmsnorm<false, f16>("rmsnorm_kernel", input, output, weight, r, num_tokens,
                                          hidden_size, input_stride, output_stride,
                                          residual_stride, eps, s);
}

extern "C" int vaa_add_rmsnorm(const uint16_t* input, uint16_t* residual, const uint16_t* weight,
                               uint16_t* output, int num_tokens, int hidden_size,
                               int64_t input_stride, int64_t residual_stride,
                               int64_t output_stride, float eps, int dtype, void* stream) {
  const char* what = "vaa_add_rmsnorm";
  if (num_tokens < 0 || hidden_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: num_tokens=%d hidden_size=%d", what, num_tokens,
                hidden_size);
  if (!valid_dtype(dtype)) return fail(VAA_ERR_UNSUPPORTED, "%s: dtype=%d", what, dtype);
  if (num_tokens == 0) return VAA_OK;
  if (!input || !residual || !weight || !output)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (input_stride < hidden_size || output_stride < hidden_size ||
      residual_stride < hidden_size)
    return fail(VAA_ERR_INVALID_ARG, "%s: row stride < hidden_size", what);
  if (static_cast<const void*>(output) == static_cast<const void*>(residual))
    return fail(VAA_ERR_INVALID_ARG, "%s: output must not alias residual", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == VAA_DTYPE_BF16
             ? launch_rmsnorm<true, bf16>("add_rmsnorm_kernel", input, output, weight, residual,
                                          num_tokens, hidden_size, input_stride, output_stride,
                                          residual_stride, eps, s)
             : launch_rmsnorm<true, f16>("add_rmsnorm_kernel", input, output, weight, residual,
                                         num_tokens, hidden_size, input_stride, output_stride,
                                         residual_stride, eps, s);
}

extern "C" int vaa_rope_neox(uint16_t* query, uint16_t* key,
                             const float* cos_cache, const float* sin_cache,
                             const int32_t* positions, int num_tokens,
                             int num_heads, int num_kv_heads, int head_size,
                             int rotary_dim, int64_t q_stride_token,
                             int64_t k_stride_token, int max_position,
                             int dtype, void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || rotary_dim <= 0 ||
      rotary_dim > head_size || rotary_dim % 2 != 0 || max_position <= 0 ||
      (key && num_kv_heads <= 0))
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_rope_neox: heads=%d/%d head_size=%d rotary_dim=%d max_position=%d",
                num_heads, num_kv_heads, head_size, rotary_dim, max_position);
  if (!valid_dtype(dtype)) return fail(VAA_ERR_UNSUPPORTED, "vaa_rope_neox: dtype=%d", dtype);
  if (num_tokens == 0) return VAA_OK;
  if (!query || !cos_cache || !sin_cache || !positions)
    return fail(VAA_ERR_INVALID_ARG, "vaa_rope_neox: null pointer");
  if (q_stride_token < static_cast<int64_t>(num_heads) * head_size ||
      (key && k_stride_token < static_cast<int64_t>(num_kv_heads) * head_size))
    return fail(VAA_ERR_INVALID_ARG, "vaa_rope_neox: token stride too small");
  const int half = rotary_dim / 2;
  const bool vec = half % 8 == 0 && head_size % 8 == 0 && aligned16(query) &&
                   (!key || aligned16(key)) && aligned16(cos_cache) &&
                   aligned16(sin_cache) && q_stride_token % 8 == 0 &&
                   (!key || k_stride_token % 8 == 0);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t heads = num_heads + (key ? num_kv_heads : 0);
  if (dtype == VAA_DTYPE_BF16) {
    RopeArgs<bf16> a{reinterpret_cast<bf16*>(query), reinterpret_cast<bf16*>(key), cos_cache,
                     sin_cache, positions, num_tokens, num_heads, num_kv_heads, head_size,
                     rotary_dim, max_position, q_stride_token, k_stride_token};
    return launch_rope(a, vec, heads, s);
  }
  RopeArgs<f16> a{reinterpret_cast<f16*>(query), reinterpret_cast<f16*>(key), cos_cache,
                  sin_cache, positions, num_tokens, num_heads, num_kv_heads, head_size,
                  rotary_dim, max_position, q_stride_token, k_stride_token};
  return launch_rope(a, vec, heads, s);
}

extern "C" int vaa_silu_mul_2d(const uint16_t* gate, const uint16_t* up,
                               uint16_t* output, int64_t rows, int64_t cols,
                               int64_t gate_stride, int64_t up_stride,
                               int64_t output_stride, int dtype, void* stream) {
  if (rows < 0 || cols < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_silu_mul: rows=%lld cols=%lld",
                (long long)rows, (long long)cols);
  if (!valid_dtype(dtype)) return fail(VAA_ERR_UNSUPPORTED, "vaa_silu_mul: dtype=%d", dtype);
  if (rows == 0 || cols == 0) return VAA_OK;
  if (!gate || !up || !output)
    return fail(VAA_ERR_INVALID_ARG, "vaa_silu_mul: null pointer");
  if (rows > 1 && (gate_stride < cols || up_stride < cols || output_stride < cols))
    return fail(VAA_ERR_INVALID_ARG, "vaa_silu_mul: row stride < cols");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == VAA_DTYPE_BF16
             ? launch_silu<bf16>(gate, up, output, rows, cols, gate_stride, up_stride,
                                 output_stride, s)
             : launch_silu<f16>(gate, up, output, rows, cols, gate_stride, up_stride,
                                output_stride, s);
}

extern "C" int vaa_silu_mul(const uint16_t* gate, const uint16_t* up,
                            uint16_t* output, int64_t num_elements, int dtype, void* stream) {
  return vaa_silu_mul_2d(gate, up, output, 1, num_elements, num_elements,
                         num_elements, num_elements, dtype, stream);
}
