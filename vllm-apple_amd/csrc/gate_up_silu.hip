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
#ifndef VAA_GLU_SMALL_TOKENS
#define VAA_GLU_SMALL_TOKENS 128
#endif
constexpr int kSmallTokens = VAA_GLU_SMALL_TOKENS;  // the few-token kernel up to this many tokens
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
// The same with the nontemporal hint, for weight tiles that one call reads
// once: with few token tiles (T <= 1024 here, and the small-token kernel) the
// hint speeds the weight stream up (C5 MLP shape: 16 tokens 0.117 -> 0.105
// ms, 6.4 TB/s of weights; 256 tokens 0.181 -> 0.170 ms).  With more token
// tiles the tiles that share a weight tile read it again through L2, and the
// hint stopped helping (2104 tokens: 1.254 against 1.248 ms).
__device__ __forceinline__ void dma16_stream(const i32x4v& rs, int voff, int soff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, %3 offen nt lds"
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

template <typename T, bool kStreamW>
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
    else if constexpr (kStreamW)
      dma16_stream(wrs, woff, kbw + (L - kGLoads) * wstep, wst + dst0 + 1024 * (L - kGLoads));
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

// ---------------------------------------------------------------------------
// Few tokens (decode-sized batches, T <= 128): the weights are the stream
// (671 MB at hidden 5120 x 2 x intermediate 32768) and the product is small,
// so the 256-token tile above spends most of its MFMAs on padding and runs
// one workgroup per CU.  Here a workgroup owns 64 output columns (64 gate and
// the 64 up rows of the same columns) and all tokens (TB blocks of 32): its
// weight tile is 16 KB per 64-element k-step, so two workgroups share a CU
// and 512 of them cover intermediate 32768.  Tiles move with the same direct
// loads, swizzled 128-byte LDS rows and counted waits as above; weights go
// through a ring of three stages (two steps of lookahead), activations
// through two.  Wave w computes column half c = w & 1 (gate block c and up
// block 2 + c, 32 rows each).  With an even number of token blocks the
// other wave bit picks half of them (every k sub-step, epilogue straight from
// the registers); with one or three, it picks a k half of every step (two of
// the four 16-element sub-steps) for every token block, the k halves are
// summed through LDS and waves 0 and 1 apply the SiLU epilogue.
// Token rows past num_tokens read the last token's row; their outputs are
// not stored.
constexpr int kSCols = 64;                    // output columns per workgroup
constexpr int kSWTile = 2 * kSCols * kGRowB;  // weight tile per k-step: 128 rows, 16 KB
constexpr int kSWStages = 3;

// s_waitcnt vmcnt(4) lgkmcnt(0): all of this wave's loads but the newest 4
// (its weight loads of the next step) have landed.
__device__ __forceinline__ void glu_small_wait() { __builtin_amdgcn_s_waitcnt(0x0074); }

template <typename T, int TB>
__global__ void __launch_bounds__(kGThreads) gate_up_silu_small_kernel(GluArgs a) {
  extern __shared__ __align__(16) char smem[];  // W stages, then x stages
  constexpr int kXTile = TB * 32 * kGRowB;
  constexpr bool kTokSplit = TB % 2 == 0;   // waves split the token blocks, else the k sub-steps
  constexpr int NB = kTokSplit ? TB / 2 : TB;  // token blocks per wave
  constexpr int NS = kTokSplit ? 4 : 2;        // 16-element sub-steps per wave and step
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)));
  const int i0 = blockIdx.x * kSCols;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;

  // Loads: weight rows 0-63 are the gate rows i0.., 64-127 the up rows;
  // wave w loads rows 32w .. 32w + 31 (four 1 KB loads of 8 rows) and the
  // activation loads w, w + 4, ... of the TB * 4 in a tile.
  const char* wbase = (wave < 2 ? a.wg : a.wu) + static_cast<int64_t>(i0) * a.ws;
  const i32x4v wrs = buffer_rsrc(wbase, static_cast<int>(kSCols * a.ws));
  const i32x4v xrs = buffer_rsrc(a.x, static_cast<int>(a.num_tokens * a.xs));
  const int rw = 32 * (wave & 1) + (lane >> 3);  // weight row of load 0 within its matrix
  const int lc = (lane & 7) ^ (rw & 7);
  const int woff = rw * static_cast<int>(a.ws) + lc * 16;
  const int wstep = 8 * static_cast<int>(a.ws);
  int xoff[TB];
#pragma unroll
  for (int j = 0; j < TB; ++j) {
    const int R = 8 * (wave + 4 * j) + (lane >> 3);
    xoff[j] = min(R, a.num_tokens - 1) * static_cast<int>(a.xs) + lc * 16;
  }
  const uint32_t wdst = 1024 * 4 * wave;

  const int l32 = lane & 31, hb = lane >> 5;
  const int c = wave & 1, kh = wave >> 1;
  const int b0 = kTokSplit ? kh * NB : 0;  // first token block of this wave
  int rd[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    rd[s] = l32 * kGRowB + (((4 * hb + (kTokSplit ? s : 2 * kh + s)) ^ (l32 & 7)) << 4);

  f32x16 g[NB], u[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) g[b][r] = u[b][r] = 0.f;

  const int n = a.ksteps;
  auto load_w = [&](int ks, uint32_t dst) {
    const int kb = min(ks, n - 1) * kGRowB;
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16_stream(wrs, woff, kb + q * wstep, dst + wdst + 1024 * q);
  };
  auto load_x = [&](int ks, uint32_t dst) {
    const int kb = min(ks, n - 1) * kGRowB;
#pragma unroll
    for (int j = 0; j < TB; ++j) dma16(xrs, xoff[j], kb, dst + 1024 * (wave + 4 * j));
  };
  const uint32_t xlds = lds0 + kSWStages * kSWTile;
  load_w(0, lds0);
  load_x(0, xlds);
  load_w(1, lds0 + kSWTile);
  for (int ks = 0; ks < n; ++ks) {
    glu_small_wait();
    __syncthreads();
    const char* cw = smem + (ks % kSWStages) * kSWTile;
    const char* cx = smem + kSWStages * kSWTile + (ks & 1) * kXTile;
    load_x(ks + 1, xlds + ((ks + 1) & 1) * kXTile);
    load_w(ks + 2, lds0 + ((ks + 2) % kSWStages) * kSWTile);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4 ag = *reinterpret_cast<const u32x4*>(cw + (32 * c) * kGRowB + rd[s]);
      const u32x4 au = *reinterpret_cast<const u32x4*>(cw + (kSCols + 32 * c) * kGRowB + rd[s]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const u32x4 bx = *reinterpret_cast<const u32x4*>(cx + (32 * (b0 + b)) * kGRowB + rd[s]);
        g[b] = Elem<T>::mfma32x32x16(__builtin_bit_cast(typename Elem<T>::x8, ag),
                                     __builtin_bit_cast(typename Elem<T>::x8, bx), g[b]);
        u[b] = Elem<T>::mfma32x32x16(__builtin_bit_cast(typename Elem<T>::x8, au),
                                     __builtin_bit_cast(typename Elem<T>::x8, bx), u[b]);
      }
    }
  }
  // Every load has landed and every wave is done with the tiles before the
  // LDS is reused for the k-half sums.
  __builtin_amdgcn_s_waitcnt(0x0070);
  if constexpr (kTokSplit) {
    // Lane holds token 32(b0 + b) + l32 and, of column half c, columns
    // 8 (r / 4) + 4 hb + r % 4.
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int tok = 32 * (b0 + b) + l32;
      if (tok >= a.num_tokens) continue;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        T v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = Elem<T>::from_f(silu_mul1(g[b][4 * r4 + e], u[b][4 * r4 + e]));
        *reinterpret_cast<u32x2*>(a.out + static_cast<int64_t>(tok) * a.os +
                                  2 * (i0 + 32 * c + 8 * r4 + 4 * hb)) =
            __builtin_bit_cast(u32x2, v);
      }
    }
  } else {
    __syncthreads();
    constexpr int kVals = 2 * TB * 16;
    float* part = reinterpret_cast<float*>(smem) + c * kVals * kWave + lane;
    if (kh == 1) {
#pragma unroll
      for (int b = 0; b < TB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          part[(32 * b + r) * kWave] = g[b][r];
          part[(32 * b + 16 + r) * kWave] = u[b][r];
        }
    }
    __syncthreads();
    if (kh == 1) return;
    // Lane holds token 32b + l32 and, of column half c, columns
    // 8 (r / 4) + 4 hb + r % 4.
#pragma unroll
    for (int b = 0; b < TB; ++b) {
      const int tok = 32 * b + l32;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        T v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * r4 + e;
          v[e] = Elem<T>::from_f(silu_mul1(g[b][r] + part[(32 * b + r) * kWave],
                                           u[b][r] + part[(32 * b + 16 + r) * kWave]));
        }
        if (tok < a.num_tokens)
          *reinterpret_cast<u32x2*>(a.out + static_cast<int64_t>(tok) * a.os +
                                    2 * (i0 + 32 * c + 8 * r4 + 4 * hb)) =
              __builtin_bit_cast(u32x2, v);
      }
    }
  }
}

template <typename T, int TB>
int launch_small(const GluArgs& a, int inter, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(kSWStages) * kSWTile + 2 * TB * 32 * kGRowB;
  hipLaunchKernelGGL((gate_up_silu_small_kernel<T, TB>), dim3(inter / kSCols), dim3(kGThreads),
                     lds, stream, a);
  return check_launch("gate_up_silu_small_kernel");
}

template <typename T>
int launch_gate_up_silu_small(const GluArgs& a, int inter, hipStream_t stream) {
  switch ((a.num_tokens + 31) / 32) {
    case 1: return launch_small<T, 1>(a, inter, stream);
    case 2: return launch_small<T, 2>(a, inter, stream);
    case 3: return launch_small<T, 3>(a, inter, stream);
    default: return launch_small<T, 4>(a, inter, stream);
  }
}

template <typename T>
int launch_gate_up_silu(const GluArgs& a0, hipStream_t stream) {
  GluArgs a = a0;
  const int grid = (a.tiles + kGXcds - 1) / kGXcds * kGXcds;
  // Weight tiles read by at most four token tiles stream with the hint.
  if (a.t_tiles <= 4)
    hipLaunchKernelGGL((gate_up_silu_kernel<T, true>), dim3(grid), dim3(kGThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((gate_up_silu_kernel<T, false>), dim3(grid), dim3(kGThreads), 0, stream, a);
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
  if (num_tokens <= kSmallTokens)
    return dtype == VAA_DTYPE_F16 ? launch_gate_up_silu_small<f16>(a, intermediate_size, s)
                                  : launch_gate_up_silu_small<bf16>(a, intermediate_size, s);
  return dtype == VAA_DTYPE_F16 ? launch_gate_up_silu<f16>(a, s) : launch_gate_up_silu<bf16>(a, s);
}
