// Integer metadata for the prefill path, computed on the device so a step
// needs no host round trip: token -> sequence map, absolute positions and
// slot mapping.  Bit-exact integer arithmetic.
#include "common.h"

namespace vaa {
namespace {

// runner.py:526-546 (token_to_seq = repeat_interleave(arange(S), diff(qsl)))
// and apple_model_runner.py:1188-1200 (seq_lens are full lengths, so the
// chunk's first token sits at seq_len - query_len).
__global__ void __launch_bounds__(256)
token_index_kernel(const int32_t* qsl, const int32_t* seq_lens, int num_seqs,
                   int num_tokens, int32_t* tok_seq, int32_t* pos) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= num_tokens) return;
  int s = -1, p = -1;
  if (num_seqs > 0 && t >= qsl[0] && t < qsl[num_seqs]) {
    // Largest s with qsl[s] <= t: skips empty query ranges.
    int lo = 0, hi = num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (qsl[mid] <= t) lo = mid; else hi = mid - 1;
    }
    s = lo;
    const int qlen = qsl[s + 1] - qsl[s];
    p = seq_lens[s] - qlen + (t - qsl[s]);
  }
  tok_seq[t] = s;
  pos[t] = p;
}

// apple_model_runner.py:1202-1249: slot = block_ids[pos // bs] * bs + pos % bs,
// falling back to slot = pos when the block list is shorter than pos // bs.
__global__ void __launch_bounds__(256)
slot_mapping_kernel(const int32_t* bt, int max_blocks, int bs,
                    const int32_t* tok_seq, const int32_t* pos, int num_seqs,
                    int num_tokens, int64_t* slots) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= num_tokens) return;
  const int s = tok_seq[t], p = pos[t];
  int64_t out = -1;
  if (s >= 0 && s < num_seqs && p >= 0) {
    const int bi = p / bs;
    const int32_t b = bi < max_blocks ? bt[static_cast<int64_t>(s) * max_blocks + bi] : -1;
    out = b >= 0 ? static_cast<int64_t>(b) * bs + p % bs : static_cast<int64_t>(p);
  }
  slots[t] = out;
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_build_token_index(const int32_t* query_start_loc,
                                     const int32_t* seq_lens, int num_seqs,
                                     int num_tokens, int32_t* token_to_seq,
                                     int32_t* positions, void* stream) {
  if (num_seqs < 0 || num_tokens < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_build_token_index: num_seqs=%d num_tokens=%d",
                num_seqs, num_tokens);
  if (num_tokens == 0) return VAA_OK;
  if (!query_start_loc || !token_to_seq || !positions || (num_seqs > 0 && !seq_lens))
    return fail(VAA_ERR_INVALID_ARG, "vaa_build_token_index: null pointer");
  hipLaunchKernelGGL(token_index_kernel, dim3((num_tokens + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), query_start_loc, seq_lens,
                     num_seqs, num_tokens, token_to_seq, positions);
  return check_launch("token_index_kernel");
}

extern "C" int vaa_build_slot_mapping(const int32_t* block_table, int max_blocks_per_seq,
                                      int block_size, const int32_t* token_to_seq,
                                      const int32_t* positions, int num_seqs,
                                      int num_tokens, int64_t* slot_mapping,
                                      void* stream) {
  if (num_tokens < 0 || block_size <= 0 || max_blocks_per_seq < 0 || num_seqs < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_build_slot_mapping: bad sizes");
  if (num_tokens == 0) return VAA_OK;
  if (!token_to_seq || !positions || !slot_mapping ||
      (num_seqs > 0 && max_blocks_per_seq > 0 && !block_table))
    return fail(VAA_ERR_INVALID_ARG, "vaa_build_slot_mapping: null pointer");
  hipLaunchKernelGGL(slot_mapping_kernel, dim3((num_tokens + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), block_table, max_blocks_per_seq,
                     block_size, token_to_seq, positions, num_seqs, num_tokens,
                     slot_mapping);
  return check_launch("slot_mapping_kernel");
}
