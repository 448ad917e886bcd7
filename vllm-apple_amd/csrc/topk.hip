// Top-k selection over logits rows: the k largest values of each row and
// their column indices, sorted by value (descending), ties by lower index.
//
// Reference: EngineTopK / topk_select (vllm_apple/engine/ops/topk.py:40-412),
// which cuts the logits read back to the host from vocab * 2 bytes to k * 6
// bytes per token.  There, one threadgroup per row keeps insertion-sorted
// per-thread lists and merges them in threadgroup memory.
//
// Here a row is cut into S chunks of at most kChunkMax columns, one workgroup
// per chunk, so a 32-row decode batch still fills the chip.  A workgroup loads
// its whole chunk into registers with every load in flight at once (one HBM
// round trip) and selects on order-preserving 16-bit keys: a lower bound L
// from k thread-group maxima (the top k are all >= L; on logits only ~1-5% of
// a chunk is), the items >= L listed in LDS, and each listed item's rank
// among them as its output position.  Flat or heavily tied rows, where too
// many items reach L, take a radix select of the k-th key first.
// A survivor's word is key << 32 | (0xffffffff - column), so "larger word" is
// "larger key, then lower column": ranking the words breaks ties by column,
// and 0 pads below every real entry (key 0 still has a non-zero low word).
// With S = 1 the ranks index the output; with S > 1 each chunk writes its
// survivors to the workspace sorted, and the merge kernel selects k of the S
// lists the same way.  Large batches at k <= 64 (thousands of chunks) select
// each chunk on one wave instead (topk_chunk_wave_kernel): the same bound,
// list and rank on ballots and cross-lane scans, with no workgroup barrier.
#include "common.h"

namespace vaa {
namespace {

constexpr int kTkThreads = 256;
constexpr int kMaxK = 256;
constexpr int kChunkMax = 8 * 8 * kTkThreads;   // 16384 columns: 8 register slices
constexpr int kChunkPref = 2 * 8 * kTkThreads;  // 4096 columns: 2 slices, high occupancy
constexpr int kMergeNj = 2;
constexpr int kMergeMax = kMergeNj * 8 * kTkThreads;  // 4096 merge candidates per row
constexpr int kChunkMin = 2048;                       // smallest chunk worth a workgroup
constexpr int kTargetGroups = 1024;                   // 4 workgroups per CU

// Order-preserving map of a 16-bit float (fp16 or bf16: sign, then magnitude
// bits) to an unsigned key: larger value -> larger key.
__host__ __device__ __forceinline__ uint32_t sort_key(uint32_t bits) {
  return (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
}
__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
  return (key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu);
}
__device__ __forceinline__ uint64_t pack(uint32_t key, uint32_t col) {
  return (static_cast<uint64_t>(key) << 32) | (0xffffffffu - col);
}

struct TopkArgs {
  const uint16_t* logits;
  int32_t* idx_out;
  uint16_t* val_out;
  uint64_t* ws;  // [T][S][k] survivors of each chunk (S > 1)
  int T, V, k, S, C;  // S chunks of C columns (C % 8 == 0 when vec)
  int vec;            // rows are 16-byte aligned: 16-byte loads, else 2-byte loads
  int64_t row_st, out_st;
};

constexpr int kCandMax = 1024;  // items >= K ranked directly

struct SelSmem {
  int hist[256];
  int res[2];
  int sc[kTkThreads / kWave];
  int n_cand;
  uint32_t lb;
  uint64_t cand[kCandMax];
};

// Block-wide exclusive scan of one int per thread (256 threads).
__device__ __forceinline__ int block_excl_scan(int v, int* sc, int& total) {
  const int tid = threadIdx.x, lane = tid % kWave, w = tid / kWave;
  int x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) sc[w] = x;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kTkThreads / kWave; ++i) {
    const int s = sc[i];
    if (i < w) off += s;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return off + x - v;
}

// Finds, from the top of a 256-bin histogram, the bin where the running count
// reaches `need` (the histogram holds at least `need`); res = {bin, count
// strictly above it}.
__device__ __forceinline__ void pick_bin(const int* hist, int need, int* res) {
  if (threadIdx.x < kWave) {
    // Lane l owns bins 255-4l .. 252-4l (descending order).
    const int lane = threadIdx.x;
    int c[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = hist[255 - 4 * lane - i];
      s += c[i];
    }
    int x = s;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    int above = x - s;  // count in the bins above this lane's group
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (above < need && above + c[i] >= need) {
        res[0] = 255 - 4 * lane - i;
        res[1] = above;
      }
      above += c[i];
    }
  }
  __syncthreads();
}

// Makes the packed keys opaque to the compiler at a phase boundary, so each
// phase unpacks them again (two VALU ops a key) instead of keeping all the
// unpacked keys of the previous phase alive.
template <int NJ>
__device__ __forceinline__ void reload(uint32_t (&kp)[NJ][4]) {
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(kp[j][q]));
}

// Top-k of the items a workgroup holds in registers.  Item (j, e) of thread t
// is number (j * 256 + t) * 8 + e in the item order.  kp[j][q] packs the keys
// of items (j, 2q) and (j, 2q+1) in its low and high halves; word(j, e) is the
// item's 64-bit word.  Items n_real and above are padding: key 0 (the lowest),
// kept out of every count and list, and after every real item in item order.
// Ties at the k-th key go to the lower column: by the words' low halves, or,
// on the ordered path, by item order, which must then agree with column order
// for equal keys.  out(r, word) receives the item of rank r = 0..k-1.
//
//   bound    group g = the threads t with t % k == g (k <= 256: none is
//            empty); L = min over groups of the group's largest key.  The k
//            group maxima are distinct items >= L, so the top k are all >= L.
//            A group made of padding has maximum 0, and L = 0 is still a bound.
//            On logits ~4k items of a chunk are >= L: only those reach the
//            LDS atomics of the two histogram passes.
//   pass 1   histogram of the high byte of keys >= L -> the bin holding the
//            k-th largest key K and the count above it;
//   pass 2   histogram of the low byte inside that bin -> K and the counts
//            above and equal to it (bins above K's hold keys > K >= L only,
//            so the counts are exact);
//   list     every item >= K (k plus the extra ties at K) goes to an LDS list,
//            at offsets from a block scan of per-thread counts;
//   rank     each listed word's rank among the listed words is its output
//            position when < k (words are distinct: distinct columns).  Its
//            LDS traffic grows with the square of the list, which is why the
//            list is cut at K rather than at L.
// When more than kCandMax items tie at K, an ordered compaction lists exactly
// k of them instead, ties taken in item order.
template <int NJ, class Word, class Out>
__device__ __forceinline__ void select_topk(uint32_t (&kp)[NJ][4], int n_real, int k,
                                            SelSmem& sm, Word word, Out out) {
  const int tid = threadIdx.x;
  auto key_of = [&](int j, int e) { return (kp[j][e / 2] >> (16 * (e & 1))) & 0xffffu; };
  auto real = [&](int j, int e) { return (j * kTkThreads + tid) * 8 + e < n_real; };
  // Lists every real item whose key is >= lo, while the list has room: each
  // thread counts its items, a block scan gives its offset.  The count lands
  // in sm.n_cand (it may exceed kCandMax); ends with a barrier.
  auto list_ge = [&](uint32_t lo) {
    reload(kp);
    int c = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j * kTkThreads * 8 >= n_real) break;  // block-uniform
#pragma unroll
      for (int e = 0; e < 8; ++e) c += (key_of(j, e) >= lo && real(j, e)) ? 1 : 0;
    }
    int total;
    int pos = block_excl_scan(c, sm.sc, total);
    if (c > 0) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j * kTkThreads * 8 >= n_real) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (key_of(j, e) >= lo && real(j, e)) {
            if (pos < kCandMax) sm.cand[pos] = word(j, e);
            ++pos;
          }
        }
      }
    }
    if (tid == 0) sm.n_cand = total;
    __syncthreads();
  };
  // Bound.
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (j * kTkThreads * 8 >= n_real) break;
#pragma unroll
    for (int q = 0; q < 4; ++q) m = max(m, max(kp[j][q] & 0xffffu, kp[j][q] >> 16));
  }
  sm.hist[tid] = 0;
  if (tid == 0) {
    sm.lb = 0xffffu;
    sm.n_cand = 0;
  }
  __syncthreads();
  atomicMax(&sm.hist[tid % k], static_cast<int>(m));
  __syncthreads();
  if (tid < k) atomicMin(&sm.lb, static_cast<uint32_t>(sm.hist[tid]));
  __syncthreads();
  const uint32_t L = sm.lb;
  int n_items;
  {
    // Pass 1: high byte of keys >= L.
    sm.hist[tid] = 0;
    reload(kp);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j * kTkThreads * 8 >= n_real) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t key = key_of(j, e);
        if (key >= L && real(j, e)) atomicAdd(&sm.hist[key >> 8], 1);
      }
    }
    __syncthreads();
    pick_bin(sm.hist, k, sm.res);
    const uint32_t hi = static_cast<uint32_t>(sm.res[0]);
    const int above_hi = sm.res[1];
    __syncthreads();
    // Pass 2: low byte inside bin `hi` (bins above `hi` hold keys > K >= L
    // only, so the counts above K are exact).
    sm.hist[tid] = 0;
    reload(kp);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j * kTkThreads * 8 >= n_real) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t key = key_of(j, e);
        if ((key >> 8) == hi && key >= L && real(j, e)) atomicAdd(&sm.hist[key & 0xffu], 1);
      }
    }
    __syncthreads();
    pick_bin(sm.hist, k - above_hi, sm.res);
    const uint32_t kth = (hi << 8) | static_cast<uint32_t>(sm.res[0]);
    const int above = above_hi + sm.res[1];         // keys > K
    const int n_ge = above + sm.hist[kth & 0xffu];  // keys >= K
    if (n_ge <= kCandMax) {
      list_ge(kth);
      n_items = n_ge;
    } else {
      // Ordered compaction of exactly k items.  An item's position is
      // (# keys > K before it) + min(# keys == K before it, need_eq).
      const int need_eq = k - above;
      int gt_run = 0, eq_run = 0;
      reload(kp);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j * kTkThreads * 8 >= n_real) break;
        int ngt = 0, neq = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t key = key_of(j, e);
          ngt += key > kth ? 1 : 0;
          neq += key == kth ? 1 : 0;
        }
        int tot;
        const int pre = block_excl_scan(ngt | (neq << 16), sm.sc, tot);  // counts < 65536
        int g = gt_run + (pre & 0xffff), q = eq_run + (pre >> 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t key = key_of(j, e);
          if (key > kth) {
            sm.cand[g + (q < need_eq ? q : need_eq)] = word(j, e);
            ++g;
          } else if (key == kth) {
            if (q < need_eq) sm.cand[g + q] = word(j, e);
            ++q;
          }
        }
        gt_run += tot & 0xffff;
        eq_run += tot >> 16;
      }
      n_items = k;
    }
    __syncthreads();
  }
  // Rank of each listed word.
  for (int i = tid; i < n_items; i += kTkThreads) {
    const uint64_t w = sm.cand[i];
    int r = 0;
#pragma unroll 16
    for (int t = 0; t < n_items; ++t) r += sm.cand[t] > w ? 1 : 0;
    if (r < k) out(r, w);
  }
  __syncthreads();
}

__device__ __forceinline__ void write_final(const TopkArgs& a, int row, int r, uint64_t w) {
  a.idx_out[row * a.out_st + r] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(w));
  a.val_out[row * a.out_st + r] = static_cast<uint16_t>(key_bits(static_cast<uint32_t>(w >> 32)));
}

// One workgroup per (row, chunk); NJ register slices hold NJ * 2048 columns.
template <int NJ>
__global__ void __launch_bounds__(kTkThreads) topk_chunk_kernel(TopkArgs a) {
  __shared__ SelSmem sm;
  const int tid = threadIdx.x;
  const int64_t n_work = static_cast<int64_t>(a.T) * a.S;
  for (int64_t w = blockIdx.x; w < n_work; w += gridDim.x) {
    const int row = static_cast<int>(w / a.S), s = static_cast<int>(w % a.S);
    const int c0 = s * a.C;
    const int c1 = min(a.V, c0 + a.C);
    const uint16_t* x = a.logits + row * a.row_st;
    // Columns past c1 are padding (key 0); they come last in item order.
    uint32_t kp[NJ][4];
    if (a.vec) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int col = c0 + (j * kTkThreads + tid) * 8;
        const u32x4 raw = col + 8 <= c1 ? ld16(x + col) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          kp[j][q] = col + 8 <= c1
                         ? sort_key(raw[q] & 0xffffu) | (sort_key(raw[q] >> 16) << 16)
                         : 0u;
      }
      // A chunk whose end is not a multiple of 8 (the row's last) has a tail.
      const int tail0 = c0 + ((c1 - c0) & ~7);
      if (tail0 < c1 && tid == ((tail0 - c0) / 8) % kTkThreads) {
        const int jt = ((tail0 - c0) / 8) / kTkThreads;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if (j != jt) continue;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (tail0 + e < c1) kp[j][e / 2] |= sort_key(x[tail0 + e]) << (16 * (e & 1));
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int col = c0 + (j * kTkThreads + tid) * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t k2 = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (col + 2 * q + h < c1) k2 |= sort_key(x[col + 2 * q + h]) << (16 * h);
          kp[j][q] = k2;
        }
      }
    }
    const int k_eff = min(a.k, c1 - c0);
    auto word = [&](int j, int e) {
      const uint32_t key = (kp[j][e / 2] >> (16 * (e & 1))) & 0xffffu;
      return pack(key, c0 + (j * kTkThreads + tid) * 8 + e);
    };
    // S == 1: the ranks index the output.  S > 1: a sorted list per chunk
    // (the merge's ordered path relies on it).
    uint64_t* list = a.ws + w * a.k;
    select_topk<NJ>(kp, c1 - c0, k_eff, sm, word, [&](int r, uint64_t wd) {
      if (a.S == 1)
        write_final(a, row, r, wd);
      else
        list[r] = wd;
    });
  }
}

// One wave per (row, chunk) for k <= 64 and chunks of at most 4096 columns:
// the selection runs on wave-wide primitives (ballots, cross-lane scans) and
// a per-wave LDS list, with no workgroup barrier or LDS histogram, so the
// four waves of a workgroup and the workgroups of a CU run independently.
//   load     lane l holds items (j * 64 + l) * 8 + e, j, e < 8: eight 16-byte
//            loads, all in flight at once;
//   bound    L = the k-th largest of the 64 lane maxima, found bit by bit with
//            ballots (the largest t that at least k lane maxima reach).  The
//            k lanes whose maxima are >= L hold k distinct items >= L, so the
//            top k are all >= L;
//   list     the real items >= L go to the wave's LDS list at offsets from a
//            wave scan of per-lane counts;
//   cut      a list of 65 to 128 words (the usual case on logits) is cut at
//            the exact k-th key among its words, bit by bit over the listed
//            keys, so that the rank below runs over about k words;
//   rank     each listed word's rank among the listed words is its output
//            position when < k.
// When more than kWaveCand items reach L (flat or heavily tied rows), the
// k-th key K is found the same bit-by-bit way over all items, and the list is
// cut at K, or, with too many ties at K, filled by an ordered compaction of
// exactly k items (ties taken in item order, which is column order).
constexpr int kTkWaves = kTkThreads / kWave;  // waves per workgroup
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
constexpr int kWaveChunk = 8 * 8 * kWave;     // 4096 columns per wave
constexpr int kWaveK = kWave;                 // the bound takes the k-th of 64 lane maxima
constexpr int kWaveCand = 512;                // list capacity per wave
// The wave kernel once there are at least this many chunks: below, a wave per
// chunk leaves the SIMDs too few waves to hide its serial phases (vocab
// 128256 in 32 chunks, k = 50, wave against workgroup kernel: 32 rows 21.1
// against 17.7 us; 64 rows 22.5 / 24.6; 128 rows 26.9 / 35.5; 256 rows 38.3 /
// 59.4; 512 rows 57.3 / 106.2).
constexpr int kWaveMinWork = 2048;

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Exclusive prefix sum over the lanes of a wave; total = the wave's sum.
__device__ __forceinline__ int wave_excl_scan(int v, int lane, int& total) {
  int x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  total = __shfl(x, kWave - 1, kWave);
  return x - v;
}

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// entries (a wave's LDS operations complete in order; the clobber keeps the
// compiler from moving accesses across).
__device__ __forceinline__ void wave_lds_fence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__global__ void __launch_bounds__(kTkThreads) topk_chunk_wave_kernel(TopkArgs a) {
  __shared__ uint64_t cand_all[kTkWaves][kWaveCand];
  const int lane = threadIdx.x % kWave;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  uint64_t* cand = cand_all[wv];
  const int64_t n_work = static_cast<int64_t>(a.T) * a.S;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kTkWaves + wv; w < n_work;
       w += static_cast<int64_t>(gridDim.x) * kTkWaves) {
    const int row = static_cast<int>(w / a.S), s = static_cast<int>(w % a.S);
    const int c0 = s * a.C;
    const int c1 = min(a.V, c0 + a.C);
    const int n_real = c1 - c0;
    const uint16_t* x = a.logits + row * a.row_st;
    // Items n_real and above are padding: key 0, kept out of every count.
    // Rows are 16-byte aligned (the launch checks a.vec).
    uint32_t kp[8][4];
    {
      // All eight loads are issued before any is used (one round trip); a
      // lane past the chunk's last full group of 8 reloads the chunk's first
      // group, which exists when n_real >= 8, and discards it.
      u32x4 raw[8];
      if (n_real >= 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int col = c0 + (j * kWave + lane) * 8;
          raw[j] = ld16(x + (col + 8 <= c1 ? col : c0));
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int col = c0 + (j * kWave + lane) * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          kp[j][q] = col + 8 <= c1
                         ? sort_key(raw[j][q] & 0xffffu) | (sort_key(raw[j][q] >> 16) << 16)
                         : 0u;
      }
      // A chunk whose end is not a multiple of 8 (the row's last) has a tail.
      const int tail0 = c0 + (n_real & ~7);
      if (tail0 < c1 && lane == ((tail0 - c0) / 8) % kWave) {
        const int jt = ((tail0 - c0) / 8) / kWave;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (j != jt) continue;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (tail0 + e < c1) kp[j][e / 2] |= sort_key(x[tail0 + e]) << (16 * (e & 1));
        }
      }
    }
    const int k = min(a.k, n_real);
    uint64_t* list = a.ws + w * a.k;
    auto key_of = [&](int j, int e) { return (kp[j][e / 2] >> (16 * (e & 1))) & 0xffffu; };
    // Bits e of slice j for the real items with key >= lo: item (j, e) is
    // real for e < n_real - (j * 64 + lane) * 8.
    auto sel_ge = [&](int j, uint32_t lo) {
      const int rj = n_real - (j * kWave + lane) * 8;
      const uint32_t real = rj >= 8 ? 0xffu : (rj <= 0 ? 0u : (1u << rj) - 1u);
      uint32_t bits = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) bits |= key_of(j, e) >= lo ? (1u << e) : 0u;
      return bits & real;
    };
    // This lane's real items with key >= lo.
    auto count_ge = [&](uint32_t lo) {
      reload(kp);
      int c = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) c += __builtin_popcount(sel_ge(j, lo));
      return c;
    };
    // Bound: the largest t that at least k lane maxima reach (the lane
    // maximum over packed pairs with v_pk_max_u16; padding keys are 0).
    uint32_t m;
    {
      u16x2 mm = __builtin_bit_cast(u16x2, kp[0][0]);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          mm = __builtin_elementwise_max(mm, __builtin_bit_cast(u16x2, kp[j][q]));
      m = max(static_cast<uint32_t>(mm[0]), static_cast<uint32_t>(mm[1]));
    }
    uint32_t L = 0;
#pragma unroll
    for (int b = 15; b >= 0; --b) {
      const uint32_t t = L | (1u << b);
      if (__popcll(__ballot(m >= t)) >= k) L = t;
    }
    // Items >= L: one compare per item, kept as 8 bits per slice.
    reload(kp);
    uint32_t selb[8];
    int c = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      selb[j] = sel_ge(j, L);
      c += __builtin_popcount(selb[j]);
    }
    int n_list;
    int pos = wave_excl_scan(c, lane, n_list);
    uint32_t K = L;
    bool ordered = false;
    if (n_list > kWaveCand) {
      // The k-th key over all real items, bit by bit, and the list cut there.
      K = 0;
#pragma unroll 1
      for (int b = 15; b >= 0; --b) {
        const uint32_t t = K | (1u << b);
        if (wave_sum_i(count_ge(t)) >= k) K = t;
      }
      reload(kp);
      c = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        selb[j] = sel_ge(j, K);
        c += __builtin_popcount(selb[j]);
      }
      pos = wave_excl_scan(c, lane, n_list);
      ordered = n_list > kWaveCand;
    }
    // Key of item (j, e) for a lane-varying e (a select over the slice's four
    // packed registers).
    auto key_at = [&](int j, int e) {
      const uint32_t v = (e >> 1) == 0 ? kp[j][0]
                       : (e >> 1) == 1 ? kp[j][1]
                       : (e >> 1) == 2 ? kp[j][2]
                                       : kp[j][3];
      return (v >> (16 * (e & 1))) & 0xffffu;
    };
    int n_items;
    if (!ordered) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t bits = selb[j];
        while (bits) {
          const int e = __builtin_ctz(bits);
          bits &= bits - 1;
          cand[pos++] = pack(key_at(j, e), c0 + (j * kWave + lane) * 8 + e);
        }
      }
      n_items = n_list;
    } else {
      // Ordered compaction of exactly k items: an item's position is
      // (# keys > K before it) + min(# keys == K before it, need_eq).
      const int above = wave_sum_i(count_ge(K + 1));
      const int need_eq = k - above;
      int gt_run = 0, eq_run = 0;
      reload(kp);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t ge = selb[j], gt = sel_ge(j, K + 1), eq = ge & ~gt;
        int tot;
        const int pre = wave_excl_scan(__builtin_popcount(gt) | (__builtin_popcount(eq) << 16),
                                       lane, tot);  // counts < 65536
        int g = gt_run + (pre & 0xffff), q = eq_run + (pre >> 16);
        uint32_t bits = ge;
        while (bits) {
          const int e = __builtin_ctz(bits);
          bits &= bits - 1;
          const uint64_t wd = pack(key_at(j, e), c0 + (j * kWave + lane) * 8 + e);
          if ((gt >> e) & 1u) {
            cand[g + (q < need_eq ? q : need_eq)] = wd;
            ++g;
          } else {
            if (q < need_eq) cand[g + q] = wd;
            ++q;
          }
        }
        gt_run += tot & 0xffff;
        eq_run += tot >> 16;
      }
      n_items = k;
    }
    wave_lds_fence();
    // A list longer than the wave (up to two words per lane, the usual case
    // on logits) is cut at the exact k-th key K among its words first (the
    // bit-by-bit search over the listed keys), so that the quadratic rank
    // below runs over about k words, one per lane.  Longer lists (flat rows)
    // are ranked whole.
    if (n_items > kWave && n_items <= 2 * kWave) {
      constexpr int kSl = 2;
      const int ns = (n_items + kWave - 1) / kWave;  // wave-uniform
      uint64_t wv8[kSl];
      int ck[kSl];
#pragma unroll
      for (int sl = 0; sl < kSl; ++sl) {
        const int i = sl * kWave + lane;
        wv8[sl] = (sl < ns && i < n_items) ? cand[i] : 0;
        ck[sl] = (sl < ns && i < n_items) ? static_cast<int>(wv8[sl] >> 32) : -1;
      }
      uint32_t Kc = 0;
#pragma unroll 1
      for (int b = 15; b >= 0; --b) {
        const int t = static_cast<int>(Kc | (1u << b));
        int cnt = 0;
#pragma unroll
        for (int sl = 0; sl < kSl; ++sl)
          if (sl < ns) cnt += __popcll(__ballot(ck[sl] >= t));
        if (cnt >= k) Kc = static_cast<uint32_t>(t);
      }
      int c2 = 0;
#pragma unroll
      for (int sl = 0; sl < kSl; ++sl) c2 += ck[sl] >= static_cast<int>(Kc) ? 1 : 0;
      int n2;
      int p2 = wave_excl_scan(c2, lane, n2);
      wave_lds_fence();  // every lane has read its words before the list is rewritten
#pragma unroll
      for (int sl = 0; sl < kSl; ++sl)
        if (ck[sl] >= static_cast<int>(Kc)) cand[p2++] = wv8[sl];
      n_items = n2;
      wave_lds_fence();
    }
    // Rank of each listed word; S == 1: the ranks index the output, else a
    // sorted list per chunk.
    for (int i = lane; i < n_items; i += kWave) {
      const uint64_t wd = cand[i];
      int r = 0;
#pragma unroll 8
      for (int t = 0; t < n_items; ++t) r += cand[t] > wd ? 1 : 0;
      if (r < k) {
        if (a.S == 1)
          write_final(a, row, r, wd);
        else
          list[r] = wd;
      }
    }
    wave_lds_fence();
  }
}

// One workgroup per row: k of the S sorted survivor lists.
__global__ void __launch_bounds__(kTkThreads) topk_merge_kernel(TopkArgs a) {
  __shared__ SelSmem sm;
  const int tid = threadIdx.x;
  const int n = a.S * a.k;
  for (int row = blockIdx.x; row < a.T; row += gridDim.x) {
    const uint64_t* in = a.ws + static_cast<int64_t>(row) * n;
    // Lists hold min(k, chunk length) survivors; only the last chunk can be
    // shorter than k, so the padding (word 0) comes last in item order.
    const int last_len = a.V - (a.S - 1) * a.C;
    const int n_real = n - a.k + min(a.k, last_len);
    uint64_t wd[kMergeNj][8];
    uint32_t kp[kMergeNj][4];
#pragma unroll
    for (int j = 0; j < kMergeNj; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = (j * kTkThreads + tid) * 8 + e;
        wd[j][e] = i < n_real ? in[i] : 0;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        kp[j][q] = static_cast<uint32_t>(wd[j][2 * q] >> 32) |
                   (static_cast<uint32_t>(wd[j][2 * q + 1] >> 32) << 16);
    }
    // Lists are sorted (key desc, column asc) and in column order, so item
    // order agrees with column order for equal keys.
    select_topk<kMergeNj>(kp, n_real, a.k, sm, [&](int j, int e) { return wd[j][e]; },
                          [&](int r, uint64_t w) { write_final(a, row, r, w); });
  }
}

// Chunking of a row: S chunks of C columns.  Chunks of at most kChunkPref
// columns where the merge can hold the survivors (at most kMergeMax / k
// chunks), never more than kChunkMax (the registers); more chunks while the
// grid is below kTargetGroups workgroups and chunks stay >= kChunkMin columns.
// Returns false when no chunking fits.
bool plan_chunks(int T, int V, int k, int* S_out, int* C_out) {
  const int s_min = (V + kChunkMax - 1) / kChunkMax;
  const int s_max_merge = kMergeMax / k;
  int S = max(s_min, min((V + kChunkPref - 1) / kChunkPref, s_max_merge));
  if (T > 0 && static_cast<int64_t>(T) * S < kTargetGroups) {
    const int want = (kTargetGroups + T - 1) / T;
    const int cap = (V + kChunkMin - 1) / kChunkMin;
    S = max(S, min(want, cap));
  }
  if (S > 1) S = min(S, s_max_merge);
  if (S < 1) S = 1;
  int C = (V + S - 1) / S;
  C = (C + 7) & ~7;
  if (C > kChunkMax) return false;
  S = (V + C - 1) / C;
  if (S > 1 && S > s_max_merge) return false;
  // Every chunk but the last holds >= k columns (C > 1024 >= k whenever S > 1),
  // which the merge's padding order relies on.
  if (S > 1 && C < k) return false;
  *S_out = S;
  *C_out = C;
  return true;
}

int check_topk(int num_tokens, int vocab_size, int k, const char* what) {
  if (num_tokens < 0 || vocab_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: num_tokens=%d vocab_size=%d", what, num_tokens,
                vocab_size);
  if (k < 1 || k > kMaxK || k > vocab_size)
    return fail(VAA_ERR_UNSUPPORTED, "%s: k=%d (1..%d, at most vocab_size)", what, k, kMaxK);
  int S, C;
  if (!plan_chunks(num_tokens, vocab_size, k, &S, &C))
    return fail(VAA_ERR_UNSUPPORTED, "%s: vocab_size=%d too large for k=%d (at most %d)", what,
                vocab_size, k, kChunkMax * (kMergeMax / k));
  return VAA_OK;
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_topk_workspace_size(int num_tokens, int vocab_size, int k,
                                       size_t* workspace_bytes) {
  const char* what = "vaa_topk_workspace_size";
  if (!workspace_bytes) return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  const int st = check_topk(num_tokens, vocab_size, k, what);
  if (st != VAA_OK) return st;
  int S, C;
  plan_chunks(num_tokens, vocab_size, k, &S, &C);
  *workspace_bytes = S > 1 ? static_cast<size_t>(num_tokens) * S * k * sizeof(uint64_t) : 0;
  return VAA_OK;
}

extern "C" int vaa_topk_logits(const uint16_t* logits, int num_tokens, int vocab_size,
                               int64_t row_stride, int k, int32_t* indices, uint16_t* values,
                               int64_t out_stride, void* workspace, size_t workspace_bytes,
                               void* stream) {
  const char* what = "vaa_topk_logits";
  int st = check_topk(num_tokens, vocab_size, k, what);
  if (st != VAA_OK) return st;
  if (num_tokens == 0) return VAA_OK;
  if (!logits || !indices || !values)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (row_stride < vocab_size || out_stride < k)
    return fail(VAA_ERR_INVALID_ARG, "%s: row_stride < vocab_size or out_stride < k", what);
  if ((reinterpret_cast<uintptr_t>(logits) & 1u) != 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: logits must be 2-byte aligned", what);
  TopkArgs a;
  plan_chunks(num_tokens, vocab_size, k, &a.S, &a.C);
  const size_t need = a.S > 1 ? static_cast<size_t>(num_tokens) * a.S * k * sizeof(uint64_t) : 0;
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(VAA_ERR_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) needed, got %zu",
                what, need, workspace ? workspace_bytes : static_cast<size_t>(0));
  a.logits = logits;
  a.idx_out = indices;
  a.val_out = values;
  a.ws = static_cast<uint64_t*>(workspace);
  a.T = num_tokens;
  a.V = vocab_size;
  a.k = k;
  a.vec = (row_stride % 8 == 0 && aligned16(logits)) ? 1 : 0;
  a.row_st = row_stride;
  a.out_st = out_stride;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_work = static_cast<int64_t>(num_tokens) * a.S;
  const int grid1 = static_cast<int>(n_work < (1 << 20) ? n_work : (1 << 20));
  if (a.vec && a.k <= kWaveK && a.C <= kWaveChunk && n_work >= kWaveMinWork) {
    const int64_t wgs = (n_work + kTkWaves - 1) / kTkWaves;
    hipLaunchKernelGGL(topk_chunk_wave_kernel, dim3(static_cast<int>(wgs < (1 << 20) ? wgs : (1 << 20))),
                       dim3(kTkThreads), 0, s, a);
  } else if (a.C <= 2 * 8 * kTkThreads)
    hipLaunchKernelGGL(topk_chunk_kernel<2>, dim3(grid1), dim3(kTkThreads), 0, s, a);
  else if (a.C <= 4 * 8 * kTkThreads)
    hipLaunchKernelGGL(topk_chunk_kernel<4>, dim3(grid1), dim3(kTkThreads), 0, s, a);
  else
    hipLaunchKernelGGL(topk_chunk_kernel<8>, dim3(grid1), dim3(kTkThreads), 0, s, a);
  st = check_launch("topk_chunk_kernel");
  if (st != VAA_OK || a.S == 1) return st;
  const int grid2 = num_tokens < (1 << 20) ? num_tokens : (1 << 20);
  hipLaunchKernelGGL(topk_merge_kernel, dim3(grid2), dim3(kTkThreads), 0, s, a);
  return check_launch("topk_merge_kernel");
}
