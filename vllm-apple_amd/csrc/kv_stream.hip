// Read-only stream of the K and V rows that a paged decode step reads, as a
// measured ceiling for the decode's HBM roofline.  No counterpart in the
// reference: the decode kernel's bandwidth is quoted against the 8 TB/s
// peak, and this kernel reads the same rows through the same block tables
// with the same loads (16 bytes per lane, nontemporal) and does nothing else
// with them but fold them into a checksum.
//
//   sink[s * num_kv_heads + h] = XOR of every 32-bit word of the K and V rows
//                                of positions [0, seq_lens[s]) of sequence s,
//                                kv head h
//
// Rows whose block-table entry is negative or past num_blocks, or lies past
// max_blocks_per_seq, are skipped; a sequence with seq_len <= 0 gives 0.
// One 8-wave workgroup per (sequence, kv head), as the decode runs one
// sequence per workgroup at the headline shape; wave w takes the 16-token
// tiles w, w + 8, ... and keeps the loads of the next tile in flight while it
// folds the current one.
#include "common.h"

namespace vaa {
namespace {

constexpr int kStreamWaves = 8;
constexpr int kStreamTile = 16;  // tokens per tile, inside one block

struct StreamArgs {
  const char* kc;
  const char* vc;
  const int32_t* bt;
  const int32_t* seq_lens;
  uint32_t* sink;
  int max_blocks, block_size, num_kv_heads;
  int64_t num_blocks;
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;  // byte strides
};

// NL 16-byte loads per lane and operand cover one tile of 16 rows x D.
template <int D>
struct STile {
  static constexpr int CH = D / 8;             // 16-byte chunks per row
  static constexpr int NL = kStreamTile * CH / kWave;
  u32x4 k[NL], v[NL];
};

template <int D>
__device__ __forceinline__ void stream_issue(const StreamArgs& a, const int32_t* bts, int len,
                                             const char* kh, const char* vh, int j, int lane,
                                             STile<D>& t) {
  constexpr int CH = STile<D>::CH;
  const u32x4 z = {0u, 0u, 0u, 0u};
  const int tok0 = j * kStreamTile;
  int64_t phys = -1;
  if (tok0 < len && tok0 / a.block_size < a.max_blocks) phys = bts[tok0 / a.block_size];
  const bool ok = phys >= 0 && phys < a.num_blocks;
  const int row0 = tok0 % a.block_size;
#pragma unroll
  for (int i = 0; i < STile<D>::NL; ++i) {
    const int c = lane + kWave * i;
    const int row = c / CH, col = c % CH;
    if (ok && tok0 + row < len) {
      t.k[i] = ld16_stream(kh + phys * a.k_sb + (row0 + row) * a.k_st + 16 * col);
      t.v[i] = ld16_stream(vh + phys * a.v_sb + (row0 + row) * a.v_st + 16 * col);
    } else {
      t.k[i] = z;
      t.v[i] = z;
    }
  }
}

template <int D>
__device__ __forceinline__ uint32_t stream_fold(const STile<D>& t) {
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < STile<D>::NL; ++i)
    x ^= t.k[i][0] ^ t.k[i][1] ^ t.k[i][2] ^ t.k[i][3] ^ t.v[i][0] ^ t.v[i][1] ^ t.v[i][2] ^
         t.v[i][3];
  return x;
}

template <int D>
__global__ void __launch_bounds__(kStreamWaves * kWave) kv_stream_kernel(StreamArgs a) {
  __shared__ uint32_t red[kStreamWaves];
  const int s = blockIdx.x, h = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int len = a.seq_lens[s];
  const int ntiles = len > 0 ? (len + kStreamTile - 1) / kStreamTile : 0;
  const int32_t* bts = a.bt + static_cast<int64_t>(s) * a.max_blocks;
  const char* kh = a.kc + h * a.k_sh;
  const char* vh = a.vc + h * a.v_sh;
  uint32_t x = 0;
  STile<D> t0, t1;
  int j = wave;
  stream_issue<D>(a, bts, len, kh, vh, j, lane, t0);
  for (; j < ntiles; j += 2 * kStreamWaves) {
    stream_issue<D>(a, bts, len, kh, vh, j + kStreamWaves, lane, t1);
    x ^= stream_fold<D>(t0);
    stream_issue<D>(a, bts, len, kh, vh, j + 2 * kStreamWaves, lane, t0);
    x ^= stream_fold<D>(t1);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, kWave);
  if (lane == 0) red[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < kStreamWaves; ++w) r ^= red[w];
    a.sink[static_cast<int64_t>(s) * a.num_kv_heads + h] = r;
  }
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_kv_stream_read(const vaa_attn_params* p, const uint16_t* key_cache,
                                  const uint16_t* value_cache, const int32_t* block_table,
                                  const int32_t* seq_lens, uint32_t* sink, void* stream) {
  const char* what = "vaa_kv_stream_read";
  if (!p) return fail(VAA_ERR_INVALID_ARG, "%s: null params", what);
  const int D = p->head_size;
  if (D != 32 && D != 64 && D != 96 && D != 128)
    return fail(VAA_ERR_UNSUPPORTED, "%s: head_size=%d (32, 64, 96 or 128)", what, D);
  if (p->num_seqs < 0 || p->num_kv_heads <= 0 || p->block_size <= 0 ||
      p->block_size % kStreamTile != 0 || p->max_blocks_per_seq <= 0 || p->num_blocks <= 0)
    return fail(VAA_ERR_INVALID_ARG,
                "%s: num_seqs=%d num_kv_heads=%d block_size=%d (a multiple of 16) "
                "max_blocks_per_seq=%d num_blocks=%lld",
                what, p->num_seqs, p->num_kv_heads, p->block_size, p->max_blocks_per_seq,
                (long long)p->num_blocks);
  if (p->num_seqs == 0) return VAA_OK;
  if (!key_cache || !value_cache || !block_table || !seq_lens || !sink)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (!aligned16(key_cache) || !aligned16(value_cache) || p->k_stride_token % 8 != 0 ||
      p->v_stride_token % 8 != 0 || p->k_stride_head % 8 != 0 || p->v_stride_head % 8 != 0 ||
      p->k_stride_block % 8 != 0 || p->v_stride_block % 8 != 0)
    return fail(VAA_ERR_INVALID_ARG,
                "%s: caches must be 16-byte aligned with strides in multiples of 8 elements",
                what);
  if (p->num_kv_heads > 65535)
    return fail(VAA_ERR_UNSUPPORTED, "%s: num_kv_heads=%d", what, p->num_kv_heads);
  StreamArgs a;
  a.kc = reinterpret_cast<const char*>(key_cache);
  a.vc = reinterpret_cast<const char*>(value_cache);
  a.bt = block_table;
  a.seq_lens = seq_lens;
  a.sink = sink;
  a.max_blocks = p->max_blocks_per_seq;
  a.block_size = p->block_size;
  a.num_kv_heads = p->num_kv_heads;
  a.num_blocks = p->num_blocks;
  a.k_sb = 2 * p->k_stride_block;
  a.k_sh = 2 * p->k_stride_head;
  a.k_st = 2 * p->k_stride_token;
  a.v_sb = 2 * p->v_stride_block;
  a.v_sh = 2 * p->v_stride_head;
  a.v_st = 2 * p->v_stride_token;
  const dim3 grid(p->num_seqs, p->num_kv_heads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (D) {
    case 32: hipLaunchKernelGGL(kv_stream_kernel<32>, grid, dim3(kStreamWaves * kWave), 0, s, a); break;
    case 64: hipLaunchKernelGGL(kv_stream_kernel<64>, grid, dim3(kStreamWaves * kWave), 0, s, a); break;
    case 96: hipLaunchKernelGGL(kv_stream_kernel<96>, grid, dim3(kStreamWaves * kWave), 0, s, a); break;
    default: hipLaunchKernelGGL(kv_stream_kernel<128>, grid, dim3(kStreamWaves * kWave), 0, s, a); break;
  }
  return check_launch(what);
}
