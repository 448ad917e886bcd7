// Gated-MLP up projection with the SwiGLU epilogue, on the matrix cores:
//
//   out[t, i] = round16(silu(g) * u),  g = x[t, :] . w_gate[i, :],  u = x[t, :] . w_up[i, :]
//
// with g and u accumulated in fp32 and never rounded to 16 bits.  The
// reference runs this as two GEMMs into [T, I] gate and up buffers followed by
// a silu_mul pass over both (vllm_apple/engine/ops/mlp.py:247-330 with
// elementwise.py:114-124); here the epilogue reads g and u from the
// accumulators, so neither intermediate is written or read back.
//
// Tiling (one 4-wave workgroup per CU, all 160 KB of LDS):
//   workgroup = 256 tokens x 128 output columns: a 256 x 256 product of the
//               token rows of x against 256 weight rows (128 gate, then the
//               128 up rows of the same columns);
//   wave w    = tokens 128*(w/2) .. +128 x columns 64*(w%2) .. +64, a 4 x 4
//               grid of 32x32 MFMA tiles (two gate and two up row blocks by
//               four token blocks), so the gate and up values of one output
//               sit in the same lane, in the same accumulator position;
//   k-step    = 64 hidden elements.  The product is computed transposed,
//               W x^T, with v_mfma_f32_32x32x16: the A operand is 8 weights of
//               one row and the B operand 8 activations of one token, both
//               read from LDS with ds_read_b128.  Lanes 0-31 take the first
//               half of the step's 64 elements and lanes 32-63 the second
//               (the contraction index is a sum, so any assignment that the
//               two operands share is exact).
//
// Memory: both operands are rows contiguous in the hidden dimension.  They
// move from HBM to LDS with direct loads (buffer_load_dwordx4 ... lds: lane i
// of a wave writes LDS bytes [16i, 16i + 16) after the wave-uniform base in
// M0).  The loads are inline asm, so the compiler does not track them (it
// would otherwise wait for every one of them before any LDS read); the
// kernel orders each LDS read behind its own counted vmcnt wait and barrier.
// Weight tiles go through a ring of three 32 KB stages and activation tiles
// through two, all of LDS: during step k the wave issues the activation
// loads of step k + 1 and then the weight loads of step k + 2, one load
// after every second MFMA of the step's first half, so the weight stream,
// which comes from HBM, has two steps to land and the activations, which
// come from L2 and the Infinity Cache, one.  The 16-byte chunks of each 128-byte LDS row are XOR-swizzled by row & 7,
// so the eight consecutive rows that an operand read spans per 128 bytes hit
// distinct banks.  Token rows past num_tokens read the last token's row
// (always in bounds) and their outputs are not stored.
//
// Workgroup order: the 8 XCDs each take a contiguous range of (column tile,
// token tile) pairs, token tile fastest, so all the token tiles that share a
// weight tile run at the same time on one XCD and read it through its L2.
#include "common.h"

namespace vaa {
namespace {

constexpr int kGT = 256;                         // tokens per workgroup
constexpr int kGI = 128;                         // output columns per workgroup
constexpr int kGK = 64;                          // hidden elements per k-step
constexpr int kGWaves = 4;
constexpr int kGThreads = kGWaves * kWave;
constexpr int kGRowB = kGK * 2;                  // bytes per LDS row
constexpr int kGTileB = 256 * kGRowB;            // one operand tile: 256 rows, 32 KB
constexpr int kGLoads = kGTileB / (kGThreads * 16);  // direct loads per wave per operand
constexpr int kGXcds = 8;
static_assert(kGLoads == 8, "eight 1 KB direct loads per wave and operand");

// Word 3 of a raw buffer resource on gfx9-family parts: 32-bit data format,
// no swizzle, offsets checked against the byte range in word 2.
constexpr int kBufDword3 = 0x00020000;

typedef int i32x4v __attribute__((ext_vector_type(4)));

// Raw buffer resource for [base, base + bytes), in scalar registers.
__device__ __forceinline__ i32x4v buffer_rsrc(const char* base, int bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4v r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((b >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = kBufDword3;
  return r;
}
// One direct load of 16 bytes per lane into LDS: lane i writes bytes
// [m0 + 16i, m0 + 16i + 16).  M0 is written here and used by nothing else
// in this kernel.
__device__ __forceinline__ void dma16(const i32x4v& rs, int voff, int soff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds"
               :
               : "v"(voff), "s"(m0), "s"(rs), "s"(soff)
               : "memory", "m0");
}

struct GluArgs {
  const char* x;
  const char* wg;
  const char* wu;
  char* out;
  int64_t xs, ws, os;  // row strides, bytes
  int num_tokens, ksteps, t_tiles, tiles;
};

// s_waitcnt vmcnt(8) lgkmcnt(0), at the top of step k: every vector memory
// load of this wave but the newest 8 has landed.  Loads complete in issue
// order and the newest 8 are the weights of step k + 1 (issued last in step
// k - 1), so the activations of step k (issued before them) and the weights
// of step k (issued in step k - 2) are in LDS, as far as this wave's loads
// go; the barrier that follows covers the other waves'.
__device__ __forceinline__ void glu_wait_tiles() { __builtin_amdgcn_s_waitcnt(0x0078); }

template <typename T>
__global__ void __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
gate_up_silu_kernel(GluArgs a) {
  __shared__ __align__(16) char smem[5 * kGTileB];  // W stages 0-2, x stages 0-1
  char* const w0 = smem;
  char* const w1 = smem + kGTileB;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)));

  const int per_xcd = static_cast<int>(gridDim.x) / kGXcds;
  const int logical = (static_cast<int>(blockIdx.x) % kGXcds) * per_xcd +
                      static_cast<int>(blockIdx.x) / kGXcds;
  if (logical >= a.tiles) return;
  const int t0 = (logical % a.t_tiles) * kGT;
  const int i0 = (logical / a.t_tiles) * kGI;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;

  // Direct-load sources, as buffer loads: a wave-uniform resource and k
  // offset, and a per-lane 32-bit offset.  Slot P of a tile is LDS row P / 8,
  // physical chunk P % 8, which holds logical chunk (P % 8) ^ (row & 7).
  // Weight rows 0-127 (waves 0 and 1) are the gate rows i0.., rows 128-255
  // (waves 2 and 3) the up rows of the same columns, so each wave reads one
  // weight matrix; its load q is 8 rows further on.  Every access stays
  // inside its resource's range (rows of x are clamped to num_tokens - 1).
  const char* wbase = (wave < 2 ? a.wg : a.wu) + static_cast<int64_t>(i0) * a.ws;
  const i32x4v wrs = buffer_rsrc(wbase, static_cast<int>(kGI * a.ws));
  const i32x4v xrs = buffer_rsrc(a.x, static_cast<int>(a.num_tokens * a.xs));
  const int rw = 8 * (wave & 1) * kGLoads + (lane >> 3);  // weight row of load 0, mod 128
  const int lc = (lane & 7) ^ (rw & 7);                    // a wave's rows agree mod 8
  const int woff = rw * static_cast<int>(a.ws) + lc * 16;
  const int wstep = 8 * static_cast<int>(a.ws);
  int xoff[kGLoads];
#pragma unroll
  for (int q = 0; q < kGLoads; ++q) {
    const int R = 8 * (wave * kGLoads + q) + (lane >> 3);
    xoff[q] = min(t0 + R, a.num_tokens - 1) * static_cast<int>(a.xs) + lc * 16;
  }
  const int dst0 = 1024 * wave * kGLoads;

  // Operand reads: row l % 32 of a 32-row block, logical chunk 4 (l / 32) + s.
  const int l32 = lane & 31, hb = lane >> 5;
  int rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) rd[s] = l32 * kGRowB + (((4 * hb + s) ^ (l32 & 7)) << 4);
  const int wi = wave & 1, wt = wave >> 1;
  // Weight row blocks: gate 64wi, 64wi + 32; up 128 + 64wi, 128 + 64wi + 32.
  const int wrow[4] = {64 * wi, 64 * wi + 32, kGI + 64 * wi, kGI + 64 * wi + 32};
  const int xrow0 = 128 * wt;

  f32x16 acc[4][4];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[f][c][r] = 0.f;

  // Direct load L of a step: 0-7 the activation tile of k-step kx into the
  // LDS address xst, 8-15 the weight tile of k-step kw into wst.
  auto load1 = [&](int L, int kbx, int kbw, uint32_t xst, uint32_t wst) {
    if (L < kGLoads)
      dma16(xrs, xoff[L], kbx, xst + dst0 + 1024 * L);
    else
      dma16(wrs, woff, kbw + (L - kGLoads) * wstep, wst + dst0 + 1024 * (L - kGLoads));
  };
  auto frags = [&](const char* wt_, const char* xt_, int s, u32x4 (&A)[4], u32x4 (&B)[4]) {
#pragma unroll
    for (int f = 0; f < 4; ++f)
      A[f] = *reinterpret_cast<const u32x4*>(wt_ + wrow[f] * kGRowB + rd[s]);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      B[c] = *reinterpret_cast<const u32x4*>(xt_ + (xrow0 + 32 * c) * kGRowB + rd[s]);
  };
  auto mfmas = [&](const u32x4 (&A)[4], const u32x4 (&B)[4], bool ld, int L0, int kbx, int kbw,
                   uint32_t xst, uint32_t wst) {
#pragma unroll
    for (int idx = 0; idx < 16; ++idx) {
      const int f = idx >> 2, c = idx & 3;
      acc[f][c] = Elem<T>::mfma32x32x16(__builtin_bit_cast(typename Elem<T>::x8, A[f]),
                                        __builtin_bit_cast(typename Elem<T>::x8, B[c]),
                                        acc[f][c]);
      if (ld && (idx & 1)) load1(L0 + (idx >> 1), kbx, kbw, xst, wst);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const int n = a.ksteps;
  // Step ks: weights in W stage ks % 3, activations in x stage ks % 2; it
  // loads the activations of step ks + 1 and then the weights of ks + 2.
  auto step = [&](int ks) {
    glu_wait_tiles();
    __syncthreads();
    const char* cw = smem + (ks % 3) * kGTileB;
    const char* cx = smem + (3 + (ks & 1)) * kGTileB;
    const uint32_t xst = lds0 + (3 + ((ks + 1) & 1)) * kGTileB;
    const uint32_t wst = lds0 + ((ks + 2) % 3) * kGTileB;
    const int kbx = min(ks + 1, n - 1) * kGRowB;
    const int kbw = min(ks + 2, n - 1) * kGRowB;
    u32x4 A0[4], B0[4], A1[4], B1[4];
    frags(cw, cx, 0, A0, B0);
    frags(cw, cx, 1, A1, B1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(A0, B0, true, 0, kbx, kbw, xst, wst);
    frags(cw, cx, 2, A0, B0);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(A1, B1, true, 8, kbx, kbw, xst, wst);
    frags(cw, cx, 3, A1, B1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(A0, B0, false, 0, 0, 0, 0, 0);
    mfmas(A1, B1, false, 0, 0, 0, 0, 0);
  };
  // Prologue: weights of steps 0 and 1, activations of step 0, issued so
  // that at the top of every step the newest 8 loads are the only ones that
  // may still be in flight (the weights of the next step).
#pragma unroll
  for (int q = 0; q < kGLoads; ++q) dma16(wrs, woff, q * wstep, lds0 + dst0 + 1024 * q);
#pragma unroll
  for (int q = 0; q < kGLoads; ++q)
    dma16(xrs, xoff[q], 0, lds0 + 3 * kGTileB + dst0 + 1024 * q);
#pragma unroll
  for (int q = 0; q < kGLoads; ++q)
    dma16(wrs, woff, min(1, n - 1) * kGRowB + q * wstep, lds0 + kGTileB + dst0 + 1024 * q);
  for (int ks = 0; ks < n; ++ks) step(ks);
  // Every load has landed before the workgroup ends and its LDS is released.
  __builtin_amdgcn_s_waitcnt(0x0070);

  // Epilogue, staged through LDS so that the output leaves in whole rows.
  // The lane holds token xrow0 + 32c + l32 and, for row block f, columns
  // 8 (r / 4) + 4 hb + r % 4 of that block: four runs of four consecutive
  // columns.  silu(g) u is formed in registers and written as 8-byte pieces
  // into a [256 tokens][128 columns] tile (token rows 0-127 in w0, 128-255
  // in w1, 256 bytes each, 16-byte chunks XOR-swizzled by row & 15 so the 32
  // token rows of one write hit distinct banks); then each row goes out as
  // sixteen 16-byte stores.
  __syncthreads();  // every wave is done with the operand tiles
  char* stage = wt == 0 ? w0 : w1;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int row = 32 * c + l32;  // within this wave's 128 token rows
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int col = 64 * wi + 32 * j + 8 * g4 + 4 * hb;
        T v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = Elem<T>::from_f(silu_mul1(acc[j][c][4 * g4 + e], acc[2 + j][c][4 * g4 + e]));
        const int chunk = (col >> 3) ^ (row & 15);
        *reinterpret_cast<u32x2*>(stage + row * 256 + chunk * 16 + (col & 7) * 2) =
            __builtin_bit_cast(u32x2, v);
      }
  }
  __syncthreads();
  const int tid = threadIdx.x;
  const int ch = tid & 15;
#pragma unroll 4
  for (int r0 = 0; r0 < kGT; r0 += kGThreads / 16) {
    const int row = r0 + (tid >> 4);
    const int tok = t0 + row;
    if (tok < a.num_tokens) {
      const char* src = (row < 128 ? w0 : w1) + (row & 127) * 256 + ((ch ^ (row & 15)) << 4);
      *reinterpret_cast<u32x4*>(a.out + static_cast<int64_t>(tok) * a.os + 2 * (i0 + 8 * ch)) =
          *reinterpret_cast<const u32x4*>(src);
    }
  }
}

template <typename T>
int launch_gate_up_silu(const GluArgs& a0, hipStream_t stream) {
  GluArgs a = a0;
  const int grid = (a.tiles + kGXcds - 1) / kGXcds * kGXcds;
  hipLaunchKernelGGL((gate_up_silu_kernel<T>), dim3(grid), dim3(kGThreads), 0, stream, a);
  return check_launch("gate_up_silu_kernel");
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_gate_up_silu(const uint16_t* x, int64_t x_stride, const uint16_t* w_gate,
                                const uint16_t* w_up, int64_t w_stride, uint16_t* output,
                                int64_t output_stride, int num_tokens, int hidden_size,
                                int intermediate_size, int dtype, void* stream) {
  const char* what = "vaa_gate_up_silu";
  if (!valid_dtype(dtype)) return fail(VAA_ERR_UNSUPPORTED, "%s: dtype=%d", what, dtype);
  if (num_tokens < 0 || hidden_size <= 0 || intermediate_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: num_tokens=%d hidden_size=%d intermediate_size=%d",
                what, num_tokens, hidden_size, intermediate_size);
  if (hidden_size % kGK != 0 || intermediate_size % kGI != 0)
    return fail(VAA_ERR_UNSUPPORTED,
                "%s: hidden_size=%d must be a multiple of %d and intermediate_size=%d of %d",
                what, hidden_size, kGK, intermediate_size, kGI);
  if (num_tokens == 0) return VAA_OK;
  if (!x || !w_gate || !w_up || !output) return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (x_stride < hidden_size || w_stride < hidden_size || output_stride < intermediate_size ||
      x_stride % 8 != 0 || w_stride % 8 != 0 || output_stride % 8 != 0)
    return fail(VAA_ERR_INVALID_ARG,
                "%s: strides x=%lld w=%lld out=%lld (x, w: multiples of 8 >= hidden_size; out: "
                "a multiple of 8 >= intermediate_size)",
                what, (long long)x_stride, (long long)w_stride, (long long)output_stride);
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(output))
    return fail(VAA_ERR_INVALID_ARG, "%s: x, weights and output must be 16-byte aligned", what);
  GluArgs a;
  a.x = reinterpret_cast<const char*>(x);
  a.wg = reinterpret_cast<const char*>(w_gate);
  a.wu = reinterpret_cast<const char*>(w_up);
  a.out = reinterpret_cast<char*>(output);
  a.xs = 2 * x_stride;
  a.ws = 2 * w_stride;
  a.os = 2 * output_stride;
  a.num_tokens = num_tokens;
  a.ksteps = hidden_size / kGK;
  a.t_tiles = (num_tokens + kGT - 1) / kGT;
  const int64_t tiles = static_cast<int64_t>(a.t_tiles) * (intermediate_size / kGI);
  // Load offsets and buffer ranges are 31-bit: activation rows from x,
  // weight rows from the workgroup's first row.
  if (tiles > (1 << 30) || static_cast<int64_t>(num_tokens) * a.xs >= (int64_t(1) << 31) ||
      static_cast<int64_t>(kGI) * a.ws >= (int64_t(1) << 31))
    return fail(VAA_ERR_UNSUPPORTED, "%s: problem too large", what);
  a.tiles = static_cast<int>(tiles);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == VAA_DTYPE_F16 ? launch_gate_up_silu<f16>(a, s) : launch_gate_up_silu<bf16>(a, s);
}
