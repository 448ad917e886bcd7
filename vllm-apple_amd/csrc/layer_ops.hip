// Bandwidth-bound layer ops next to attention: RMSNorm (+ post-norm residual),
// NeoX rotary embedding (in place on Q and K) and SwiGLU (silu(gate) * up).
// All fp16 in / fp16 out with fp32 arithmetic; 16-byte vector accesses when
// the views allow it, 2-byte fallbacks otherwise.
#include "common.h"

namespace vaa {
namespace {

__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
  const f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = h2f(h[i]);
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = f2h(f[i]);
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

template <int NC, bool kAdd>
__global__ void __launch_bounds__(kNormRowsPerBlock* kWave)
rmsnorm_vec_kernel(const f16* in, f16* out, const f16* w, f16* res, int T,
                   int H, int64_t in_st, int64_t out_st, int64_t res_st,
                   float eps) {
  const int row = blockIdx.x * kNormRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= T) return;
  const int chunks = H / 8;
  const f16* x = in + row * in_st;
  f16* r = res ? res + row * res_st : nullptr;
  // The row's values: x, or (kAdd) h = half(x + r), written back to r.
  auto load = [&](int c) {
    const u32x4 v = ld16(x + 8 * c);
    if constexpr (!kAdd) {
      return v;
    } else {
      float f[8], rf[8];
      unpack8(v, f);
      unpack8(ld16(r + 8 * c), rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] += rf[e];
      const u32x4 h = pack8(f);
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
      unpack8(xv[i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  } else {
    for (int c = lane; c < chunks; c += kWave) {
      float f[8];
      unpack8(load(c), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / static_cast<float>(H) + eps);
  f16* o = out + row * out_st;
  auto emit = [&](int c, u32x4 v) {
    float f[8], wf[8];
    unpack8(v, f);
    unpack8(ld16(w + 8 * c), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (f[e] * rs) * wf[e];
    if (!kAdd && r) {
      float rf[8];
      unpack8(ld16(r + 8 * c), rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] += rf[e];
    }
    st16(o + 8 * c, pack8(f));
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

template <bool kAdd>
__global__ void __launch_bounds__(kNormRowsPerBlock* kWave)
rmsnorm_scalar_kernel(const f16* in, f16* out, const f16* w, f16* res,
                      int T, int H, int64_t in_st, int64_t out_st,
                      int64_t res_st, float eps) {
  const int row = blockIdx.x * kNormRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= T) return;
  const f16* x = in + row * in_st;
  f16* r = res ? res + row * res_st : nullptr;
  float ss = 0.f;
  for (int i = lane; i < H; i += kWave) {
    float v = h2f(x[i]);
    if constexpr (kAdd) {
      const f16 h = f2h(v + h2f(r[i]));
      r[i] = h;
      v = h2f(h);
    }
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / static_cast<float>(H) + eps);
  f16* o = out + row * out_st;
  const f16* src = kAdd ? r : x;
  for (int i = lane; i < H; i += kWave) {
    float v = (h2f(src[i]) * rs) * h2f(w[i]);
    if (!kAdd && r) v += h2f(r[i]);
    o[i] = f2h(v);
  }
}

// ------------------------------------------------------------------- RoPE --
// elementwise.py:185-239: for pair i < rot/2 of every q and k head,
//   (x_i, x_{i+rot/2}) <- (x_i c - x_{i+rot/2} s, x_i s + x_{i+rot/2} c)
// with c, s = cos/sin_cache[positions[t], i] (fp32), in place.
struct RopeArgs {
  f16* q;
  f16* k;
  const float* cosc;
  const float* sinc;
  const int32_t* pos;
  int T, H, KV, D, rot, max_pos;
  int64_t q_st, k_st;
};

// One thread rotates 8 consecutive pairs of one head.
__global__ void __launch_bounds__(256) rope_neox_vec_kernel(RopeArgs a) {
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
    f16* x = hh < a.H ? a.q + t * a.q_st + static_cast<int64_t>(hh) * a.D
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
    unpack8(ld16(x + i0), x0);
    unpack8(ld16(x + i0 + half), x1);
    float y0[8], y1[8];
    rope_rotate8(x0, x1, c, s, y0, y1);
    st16(x + i0, pack8(y0));
    st16(x + i0 + half, pack8(y1));
  }
}

__global__ void __launch_bounds__(256) rope_neox_scalar_kernel(RopeArgs a) {
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
    f16* x = hh < a.H ? a.q + t * a.q_st + static_cast<int64_t>(hh) * a.D
                      : a.k + t * a.k_st + static_cast<int64_t>(hh - a.H) * a.D;
    const float c = a.cosc[static_cast<int64_t>(p) * half + i];
    const float s = a.sinc[static_cast<int64_t>(p) * half + i];
    const float x0 = h2f(x[i]), x1 = h2f(x[i + half]);
    x[i] = f2h(x0 * c - x1 * s);
    x[i + half] = f2h(x0 * s + x1 * c);
  }
}

// ----------------------------------------------------------------- SwiGLU --
// elementwise.py:114-124: out = half(g / (1 + exp(-g)) * u) in fp32.
__device__ __forceinline__ float silu_mul1(float g, float u) {
  const float e = fast_exp2(-g * kLog2e);
  return (g * __builtin_amdgcn_rcpf(1.f + e)) * u;
}

__global__ void __launch_bounds__(256)
silu_mul_vec_kernel(const f16* gate, const f16* up, f16* out, int64_t rows,
                    int64_t cols, int64_t g_st, int64_t u_st, int64_t o_st) {
  const int64_t cpr = cols / 8;
  const int64_t total = rows * cpr;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cpr, c = (idx % cpr) * 8;
    float g[8], u[8], y[8];
    unpack8(ld16(gate + r * g_st + c), g);
    unpack8(ld16(up + r * u_st + c), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = silu_mul1(g[e], u[e]);
    st16(out + r * o_st + c, pack8(y));
  }
}

__global__ void __launch_bounds__(256)
silu_mul_scalar_kernel(const f16* gate, const f16* up, f16* out, int64_t rows,
                       int64_t cols, int64_t g_st, int64_t u_st, int64_t o_st) {
  const int64_t total = rows * cols;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cols, c = idx % cols;
    out[r * o_st + c] = f2h(silu_mul1(h2f(gate[r * g_st + c]), h2f(up[r * u_st + c])));
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

template <bool kAdd>
int launch_rmsnorm(const char* what, const f16* in, f16* out, const f16* w, f16* r, int T, int H,
                   int64_t in_st, int64_t out_st, int64_t r_st, float eps, hipStream_t s) {
  const dim3 grid((T + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
  const dim3 block(kNormRowsPerBlock * kWave);
  const bool vec = H % 8 == 0 && aligned16(in) && aligned16(out) && aligned16(w) &&
                   (!r || aligned16(r)) && in_st % 8 == 0 && out_st % 8 == 0 &&
                   (!r || r_st % 8 == 0);
  if (!vec) {
    hipLaunchKernelGGL(rmsnorm_scalar_kernel<kAdd>, grid, block, 0, s, in, out, w, r, T, H,
                       in_st, out_st, r_st, eps);
    return check_launch(what);
  }
  const int per_lane = (H / 8 + kWave - 1) / kWave;
#define VAA_NORM(NC)                                                                       \
  hipLaunchKernelGGL((rmsnorm_vec_kernel<NC, kAdd>), grid, block, 0, s, in, out, w, r, T, H, \
                     in_st, out_st, r_st, eps)
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

}  // namespace
}  // namespace vaa

extern "C" int vaa_rmsnorm(const uint16_t* input, uint16_t* output,
                           const uint16_t* weight, const uint16_t* residual,
                           int num_tokens, int hidden_size, int64_t input_stride,
                           int64_t output_stride, int64_t residual_stride,
                           float eps, void* stream) {
  if (num_tokens < 0 || hidden_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_rmsnorm: num_tokens=%d hidden_size=%d",
                num_tokens, hidden_size);
  if (num_tokens == 0) return VAA_OK;
  if (!input || !output || !weight)
    return fail(VAA_ERR_INVALID_ARG, "vaa_rmsnorm: null pointer");
  if (input_stride < hidden_size || output_stride < hidden_size ||
      (residual && residual_stride < hidden_size))
    return fail(VAA_ERR_INVALID_ARG, "vaa_rmsnorm: row stride < hidden_size");
  // The residual is only read here.
  return launch_rmsnorm<false>(
      "rmsnorm_kernel", reinterpret_cast<const f16*>(input), reinterpret_cast<f16*>(output),
      reinterpret_cast<const f16*>(weight),
      const_cast<f16*>(reinterpret_cast<const f16*>(residual)), num_tokens, hidden_size,
      input_stride, output_stride, residual_stride, eps, static_cast<hipStream_t>(stream));
}

extern "C" int vaa_add_rmsnorm(const uint16_t* input, uint16_t* residual, const uint16_t* weight,
                               uint16_t* output, int num_tokens, int hidden_size,
                               int64_t input_stride, int64_t residual_stride,
                               int64_t output_stride, float eps, void* stream) {
  const char* what = "vaa_add_rmsnorm";
  if (num_tokens < 0 || hidden_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: num_tokens=%d hidden_size=%d", what, num_tokens,
                hidden_size);
  if (num_tokens == 0) return VAA_OK;
  if (!input || !residual || !weight || !output)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (input_stride < hidden_size || output_stride < hidden_size ||
      residual_stride < hidden_size)
    return fail(VAA_ERR_INVALID_ARG, "%s: row stride < hidden_size", what);
  if (static_cast<const void*>(output) == static_cast<const void*>(residual))
    return fail(VAA_ERR_INVALID_ARG, "%s: output must not alias residual", what);
  return launch_rmsnorm<true>(
      "add_rmsnorm_kernel", reinterpret_cast<const f16*>(input), reinterpret_cast<f16*>(output),
      reinterpret_cast<const f16*>(weight), reinterpret_cast<f16*>(residual), num_tokens,
      hidden_size, input_stride, output_stride, residual_stride, eps,
      static_cast<hipStream_t>(stream));
}

extern "C" int vaa_rope_neox(uint16_t* query, uint16_t* key,
                             const float* cos_cache, const float* sin_cache,
                             const int32_t* positions, int num_tokens,
                             int num_heads, int num_kv_heads, int head_size,
                             int rotary_dim, int64_t q_stride_token,
                             int64_t k_stride_token, int max_position,
                             void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || rotary_dim <= 0 ||
      rotary_dim > head_size || rotary_dim % 2 != 0 || max_position <= 0 ||
      (key && num_kv_heads <= 0))
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_rope_neox: heads=%d/%d head_size=%d rotary_dim=%d max_position=%d",
                num_heads, num_kv_heads, head_size, rotary_dim, max_position);
  if (num_tokens == 0) return VAA_OK;
  if (!query || !cos_cache || !sin_cache || !positions)
    return fail(VAA_ERR_INVALID_ARG, "vaa_rope_neox: null pointer");
  if (q_stride_token < static_cast<int64_t>(num_heads) * head_size ||
      (key && k_stride_token < static_cast<int64_t>(num_kv_heads) * head_size))
    return fail(VAA_ERR_INVALID_ARG, "vaa_rope_neox: token stride too small");
  RopeArgs a{reinterpret_cast<f16*>(query), reinterpret_cast<f16*>(key), cos_cache,
             sin_cache, positions, num_tokens, num_heads, num_kv_heads, head_size,
             rotary_dim, max_position, q_stride_token, k_stride_token};
  const int half = rotary_dim / 2;
  const bool vec = half % 8 == 0 && head_size % 8 == 0 && aligned16(query) &&
                   (!key || aligned16(key)) && aligned16(cos_cache) &&
                   aligned16(sin_cache) && q_stride_token % 8 == 0 &&
                   (!key || k_stride_token % 8 == 0);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t heads = num_heads + (key ? num_kv_heads : 0);
  if (vec) {
    const int64_t work = static_cast<int64_t>(num_tokens) * heads * (half / 8);
    hipLaunchKernelGGL(rope_neox_vec_kernel, dim3(grid_for(work, 256, 1 << 20)),
                       dim3(256), 0, s, a);
    return check_launch("rope_neox_vec_kernel");
  }
  const int64_t work = static_cast<int64_t>(num_tokens) * heads * half;
  hipLaunchKernelGGL(rope_neox_scalar_kernel, dim3(grid_for(work, 256, 1 << 20)),
                     dim3(256), 0, s, a);
  return check_launch("rope_neox_scalar_kernel");
}

extern "C" int vaa_silu_mul_2d(const uint16_t* gate, const uint16_t* up,
                               uint16_t* output, int64_t rows, int64_t cols,
                               int64_t gate_stride, int64_t up_stride,
                               int64_t output_stride, void* stream) {
  if (rows < 0 || cols < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_silu_mul: rows=%lld cols=%lld",
                (long long)rows, (long long)cols);
  if (rows == 0 || cols == 0) return VAA_OK;
  if (!gate || !up || !output)
    return fail(VAA_ERR_INVALID_ARG, "vaa_silu_mul: null pointer");
  if (rows > 1 && (gate_stride < cols || up_stride < cols || output_stride < cols))
    return fail(VAA_ERR_INVALID_ARG, "vaa_silu_mul: row stride < cols");
  const f16* g = reinterpret_cast<const f16*>(gate);
  const f16* u = reinterpret_cast<const f16*>(up);
  f16* o = reinterpret_cast<f16*>(output);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = cols % 8 == 0 && aligned16(g) && aligned16(u) && aligned16(o) &&
                   (rows == 1 || (gate_stride % 8 == 0 && up_stride % 8 == 0 &&
                                  output_stride % 8 == 0));
  if (vec) {
    const int64_t work = rows * (cols / 8);
    hipLaunchKernelGGL(silu_mul_vec_kernel, dim3(grid_for(work, 256, 1 << 16)),
                       dim3(256), 0, s, g, u, o, rows, cols, gate_stride, up_stride,
                       output_stride);
    return check_launch("silu_mul_vec_kernel");
  }
  hipLaunchKernelGGL(silu_mul_scalar_kernel, dim3(grid_for(rows * cols, 256, 1 << 16)),
                     dim3(256), 0, s, g, u, o, rows, cols, gate_stride, up_stride,
                     output_stride);
  return check_launch("silu_mul_scalar_kernel");
}

extern "C" int vaa_silu_mul(const uint16_t* gate, const uint16_t* up,
                            uint16_t* output, int64_t num_elements, void* stream) {
  return vaa_silu_mul_2d(gate, up, output, 1, num_elements, num_elements,
                         num_elements, num_elements, stream);
}
