// Read-only stream of the K and V rows that a paged decode step reads, as a
// measured ceiling for the decode's HBM roofline.  No counterpart in the
// reference: the decode kernel's bandwidth is quoted against the 8 TB/s
// peak, and this kernel reads the same rows through the same block tables
// with the same loads (16 bytes per lane, nontemporal) and does nothing else
// with them but fold them into a checksum.
//
//   sink[(s * parts + q) * num_kv_heads + h] = XOR of every 32-bit word of
//       the K and V rows of positions [q * P, min((q + 1) * P, seq_lens[s]))
//       of sequence s, kv head h
//
// with P = partition_size (parts = ceil(max_seq_len / P)) as the decode's
// fixed split-K partitions cut a context, or P = infinity (parts = 1) when
// partition_size is 0.  Rows whose block-table entry is negative or past
// num_blocks, or lies past max_blocks_per_seq, are skipped; an empty piece
// gives 0.  One workgroup per (kv head, piece, sequence), kv head fastest, as
// the decode's grid: 8 waves, or 4 for pieces of up to 1024 tokens (the
// decode's short partitions); wave w takes the piece's 16-token tiles w,
// w + NW, ... and keeps the loads of the next tile in flight while it folds
// the current one.
#include "common.h"

namespace vaa {
namespace {

constexpr int kStreamTile = 16;  // tokens per tile, inside one block
constexpr int kShortPiece = 1024;  // pieces up to this many tokens run 4 waves

struct StreamArgs {
  const char* kc;
  const char* vc;
  const int32_t* bt;
  const int32_t* seq_lens;
  uint32_t* sink;
  int max_blocks, block_size, num_kv_heads;
  int piece_tiles, parts;  // 16-token tiles per piece, pieces per sequence
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

template <int D, int NW>
__global__ void __launch_bounds__(NW * kWave) kv_stream_kernel(StreamArgs a) {
  __shared__ uint32_t red[NW];
  const int h = blockIdx.x, q = blockIdx.y, s = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int len = a.seq_lens[s];
  const int ntiles = len > 0 ? (len + kStreamTile - 1) / kStreamTile : 0;
  const int t_lo = q * a.piece_tiles;
  const int t_hi = min(ntiles, t_lo + a.piece_tiles);
  const int32_t* bts = a.bt + static_cast<int64_t>(s) * a.max_blocks;
  const char* kh = a.kc + h * a.k_sh;
  const char* vh = a.vc + h * a.v_sh;
  uint32_t x = 0;
  if (t_lo < t_hi) {
    // Tiles past t_hi load nothing: stream_issue zeroes rows past the
    // piece's last key.
    const int lim = min(len, t_hi * kStreamTile);
    STile<D> t0, t1;
    int j = t_lo + wave;
    stream_issue<D>(a, bts, lim, kh, vh, j, lane, t0);
    for (; j < t_hi; j += 2 * NW) {
      stream_issue<D>(a, bts, lim, kh, vh, j + NW, lane, t1);
      x ^= stream_fold<D>(t0);
      stream_issue<D>(a, bts, lim, kh, vh, j + 2 * NW, lane, t0);
      x ^= stream_fold<D>(t1);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, kWave);
  if (lane == 0) red[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) r ^= red[w];
    a.sink[(static_cast<int64_t>(s) * a.parts + q) * a.num_kv_heads + h] = r;
  }
}

template <int D>
void launch_stream(const StreamArgs& a, dim3 grid, bool short_pieces, hipStream_t s) {
  if (short_pieces)
    hipLaunchKernelGGL((kv_stream_kernel<D, 4>), grid, dim3(4 * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((kv_stream_kernel<D, 8>), grid, dim3(8 * kWave), 0, s, a);
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
      p->block_size % kStreamTile != 0 || p->max_blocks_per_seq <= 0 || p->num_blocks <= 0 ||
      p->partition_size < 0 || p->partition_size % kStreamTile != 0 ||
      (p->partition_size > 0 && p->max_seq_len <= 0))
    return fail(VAA_ERR_INVALID_ARG,
                "%s: num_seqs=%d num_kv_heads=%d block_size=%d (a multiple of 16) "
                "max_blocks_per_seq=%d num_blocks=%lld partition_size=%d (0 or a multiple of "
                "16, with max_seq_len > 0) max_seq_len=%d",
                what, p->num_seqs, p->num_kv_heads, p->block_size, p->max_blocks_per_seq,
                (long long)p->num_blocks, p->partition_size, p->max_seq_len);
  if (p->num_seqs == 0) return VAA_OK;
  if (!key_cache || !value_cache || !block_table || !seq_lens || !sink)
    return fail(VAA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (!aligned16(key_cache) || !aligned16(value_cache) || p->k_stride_token % 8 != 0 ||
      p->v_stride_token % 8 != 0 || p->k_stride_head % 8 != 0 || p->v_stride_head % 8 != 0 ||
      p->k_stride_block % 8 != 0 || p->v_stride_block % 8 != 0)
    return fail(VAA_ERR_INVALID_ARG,
                "%s: caches must be 16-byte aligned with strides in multiples of 8 elements",
                what);
  const int P = p->partition_size;
  const int parts = P > 0 ? (p->max_seq_len + P - 1) / P : 1;
  if (p->num_seqs > 65535 || parts > 65535)
    return fail(VAA_ERR_UNSUPPORTED, "%s: num_seqs=%d pieces per sequence=%d (at most 65535)",
                what, p->num_seqs, parts);
  StreamArgs a;
  a.kc = reinterpret_cast<const char*>(key_cache);
  a.vc = reinterpret_cast<const char*>(value_cache);
  a.bt = block_table;
  a.seq_lens = seq_lens;
  a.sink = sink;
  a.max_blocks = p->max_blocks_per_seq;
  a.block_size = p->block_size;
  a.num_kv_heads = p->num_kv_heads;
  a.piece_tiles = P > 0 ? P / kStreamTile : (1 << 30) / kStreamTile;
  a.parts = parts;
  a.num_blocks = p->num_blocks;
  a.k_sb = 2 * p->k_stride_block;
  a.k_sh = 2 * p->k_stride_head;
  a.k_st = 2 * p->k_stride_token;
  a.v_sb = 2 * p->v_stride_block;
  a.v_sh = 2 * p->v_stride_head;
  a.v_st = 2 * p->v_stride_token;
  const dim3 grid(p->num_kv_heads, parts, p->num_seqs);
  const bool short_pieces = P > 0 && P <= kShortPiece;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (D) {
    case 32: launch_stream<32>(a, grid, short_pieces, s); break;
    case 64: launch_stream<64>(a, grid, short_pieces, s); break;
    case 96: launch_stream<96>(a, grid, short_pieces, s); break;
    default: launch_stream<128>(a, grid, short_pieces, s); break;
  }
  return check_launch(what);
}
