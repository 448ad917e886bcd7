// Bit-exact K/V cache writes: slot_mapping scatter, decode-position write and
// the two entry points that replace the reference's CPU memcpy library.
//
// One thread moves one 16-byte chunk (8 fp16) of K and the same chunk of V;
// consecutive threads walk a head row, so a wave reads and writes whole
// 256-byte rows (D = 128) with 16-byte accesses.  The destination of each
// token comes from a small "resolver" (slot, decode position, or explicit
// block/offset) that returns false to skip the token.  The new K/V rows are
// read once, with the nontemporal hint (C3 chunk write 5.90 -> 5.67 us); the
// cache rows are stored normally, since attention reads them next.
#include "common.h"

namespace vaa {
namespace {

struct CacheDst {
  uint16_t* k;
  uint16_t* v;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
};

struct NewSrc {
  const uint16_t* k;
  const uint16_t* v;
  int64_t s_tok, s_head;
};

// slot_mapping (kv_write.py:130-146): block = slot / bs, offset = slot % bs.
template <typename IdxT>
struct SlotResolver {
  const IdxT* slots;
  int block_size;
  int64_t capacity;  // num_blocks * block_size
  __device__ bool operator()(int t, int64_t& block, int64_t& off) const {
    int64_t s = static_cast<int64_t>(slots[t]);
    if (s < 0 || s >= capacity) return false;
    block = s / block_size;
    off = s % block_size;
    return true;
  }
};

// Decode position (paged_attention_fused.metal:73-86, kv_write.py:86-99).
struct DecodeResolver {
  const int32_t* block_table;
  const int32_t* seq_lens;
  int max_blocks_per_seq;
  int block_size;
  int64_t num_blocks;
  __device__ bool operator()(int s, int64_t& block, int64_t& off) const {
    int L = seq_lens[s];
    if (L <= 0) return false;
    int pos = L - 1;
    int bi = pos / block_size;
    if (bi >= max_blocks_per_seq) return false;
    int phys = block_table[static_cast<int64_t>(s) * max_blocks_per_seq + bi];
    if (phys < 0 || phys >= num_blocks) return false;
    block = phys;
    off = pos % block_size;
    return true;
  }
};

// Explicit (block id, offset) arrays (kv_write.c:50-57).  The reference
// trusts both; here a token is skipped unless 0 <= block < num_blocks and
// 0 <= offset < off_limit, the offsets whose whole [KV, D] write stays inside
// the block's stride_block elements (offset_limit()), so a bad offset can
// neither spill into the neighbouring block nor past the last one.
struct BatchResolver {
  const int64_t* block_ids;
  const int64_t* offsets;
  int64_t num_blocks;
  int64_t off_limit;
  __device__ bool operator()(int t, int64_t& block, int64_t& off) const {
    int64_t b = block_ids[t], o = offsets[t];
    if (b < 0 || b >= num_blocks || o < 0 || o >= off_limit) return false;
    block = b;
    off = o;
    return true;
  }
};

// One token whose block and offset the host has already checked.
struct SingleResolver {
  int64_t block_id, offset;
  __device__ bool operator()(int, int64_t& block, int64_t& off) const {
    block = block_id;
    off = offset;
    return true;
  }
};

// Number of token offsets o >= 0 for which the write of one token,
// elements [o*st, o*st + (kv-1)*sh + d) of its block, ends within the
// block's sb elements: o*st + (kv-1)*sh + d <= sb.  0 when even offset 0
// does not fit; unbounded (INT64_MAX) for a zero token stride.
int64_t offset_limit(int64_t sb, int64_t sh, int64_t st, int kv, int d) {
  const int64_t room = sb - static_cast<int64_t>(kv - 1) * sh - d;
  if (room < 0) return 0;
  if (st <= 0) return INT64_MAX;
  return room / st + 1;
}

// VEC = 8: 16-byte chunks (all pointers/strides 8-element aligned);
// VEC = 1: 2-byte fallback for unaligned views.
template <int VEC, typename Resolver>
__global__ void __launch_bounds__(256)
kv_copy_kernel(CacheDst dst, NewSrc src, Resolver resolve, int num_tokens,
               int num_kv_heads, int head_size) {
  const int chunks = head_size / VEC;
  const int64_t total = static_cast<int64_t>(num_tokens) * num_kv_heads * chunks;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(idx % chunks);
    const int64_t th = idx / chunks;
    const int h = static_cast<int>(th % num_kv_heads);
    const int t = static_cast<int>(th / num_kv_heads);
    int64_t block, off;
    if (!resolve(t, block, off)) continue;
    const int64_t e = static_cast<int64_t>(c) * VEC;
    const int64_t so = t * src.s_tok + h * src.s_head + e;
    const int64_t dk = block * dst.k_sb + h * dst.k_sh + off * dst.k_st + e;
    const int64_t dv = block * dst.v_sb + h * dst.v_sh + off * dst.v_st + e;
    if constexpr (VEC == 8) {
      st16(dst.k + dk, ld16_stream(src.k + so));
      st16(dst.v + dv, ld16_stream(src.v + so));
    } else {
      dst.k[dk] = src.k[so];
      dst.v[dv] = src.v[so];
    }
  }
}

bool chunk_aligned(const CacheDst& d, const NewSrc& s, int head_size) {
  return head_size % 8 == 0 && aligned16(d.k) && aligned16(d.v) &&
         aligned16(s.k) && aligned16(s.v) && d.k_sb % 8 == 0 &&
         d.k_sh % 8 == 0 && d.k_st % 8 == 0 && d.v_sb % 8 == 0 &&
         d.v_sh % 8 == 0 && d.v_st % 8 == 0 && s.s_tok % 8 == 0 &&
         s.s_head % 8 == 0;
}

template <typename Resolver>
int launch_copy(const CacheDst& dst, const NewSrc& src, const Resolver& r,
                int num_tokens, int num_kv_heads, int head_size,
                hipStream_t stream, const char* what) {
  if (num_tokens <= 0) return VAA_OK;
  const bool vec = chunk_aligned(dst, src, head_size);
  const int64_t total = static_cast<int64_t>(num_tokens) * num_kv_heads *
                        (vec ? head_size / 8 : head_size);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (vec) {
    hipLaunchKernelGGL((kv_copy_kernel<8, Resolver>), dim3(blocks), dim3(256), 0,
                       stream, dst, src, r, num_tokens, num_kv_heads, head_size);
  } else {
    hipLaunchKernelGGL((kv_copy_kernel<1, Resolver>), dim3(blocks), dim3(256), 0,
                       stream, dst, src, r, num_tokens, num_kv_heads, head_size);
  }
  return check_launch(what);
}

int check_common(int num_kv_heads, int head_size, const void* k, const void* v,
                 const void* sk, const void* sv, const char* what, int num_tokens = 1) {
  if (num_tokens > 0 && (!k || !v || !sk || !sv))
    return fail(VAA_ERR_INVALID_ARG, "%s: null cache or source pointer", what);
  if (num_kv_heads <= 0 || head_size <= 0)
    return fail(VAA_ERR_INVALID_ARG, "%s: num_kv_heads=%d head_size=%d", what,
                num_kv_heads, head_size);
  return VAA_OK;
}

CacheDst dst_from(const vaa_attn_params* p, uint16_t* k, uint16_t* v) {
  return CacheDst{k, v, p->k_stride_block, p->k_stride_head, p->k_stride_token,
                  p->v_stride_block, p->v_stride_head, p->v_stride_token};
}

}  // namespace
}  // namespace vaa

using namespace vaa;

extern "C" int vaa_write_kv_batch(uint16_t* key_dst, uint16_t* value_dst,
                                  const uint16_t* key_src,
                                  const uint16_t* value_src,
                                  const int64_t* block_ids,
                                  const int64_t* token_offsets, int num_tokens,
                                  int num_kv_heads, int head_size,
                                  int64_t stride_block, int64_t stride_head,
                                  int64_t stride_token, int64_t num_blocks,
                                  void* stream) {
  int st = check_common(num_kv_heads, head_size, key_dst, value_dst, key_src,
                        value_src, "vaa_write_kv_batch", num_tokens);
  if (st) return st;
  if (num_tokens < 0 || (num_tokens > 0 && (!block_ids || !token_offsets)))
    return fail(VAA_ERR_INVALID_ARG, "vaa_write_kv_batch: bad token arrays");
  if (stride_block < 0 || stride_head < 0 || stride_token < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_write_kv_batch: negative stride");
  CacheDst d{key_dst, value_dst, stride_block, stride_head, stride_token,
             stride_block, stride_head, stride_token};
  NewSrc s{key_src, value_src, static_cast<int64_t>(num_kv_heads) * head_size,
           head_size};
  BatchResolver r{block_ids, token_offsets, num_blocks,
                  offset_limit(stride_block, stride_head, stride_token, num_kv_heads, head_size)};
  return launch_copy(d, s, r, num_tokens, num_kv_heads, head_size,
                     static_cast<hipStream_t>(stream), "vaa_write_kv_batch");
}

extern "C" int vaa_write_kv_single(uint16_t* key_dst, uint16_t* value_dst,
                                   const uint16_t* key_src,
                                   const uint16_t* value_src, int64_t block_id,
                                   int64_t token_offset, int num_kv_heads,
                                   int head_size, int64_t stride_block,
                                   int64_t stride_head, int64_t stride_token,
                                   int64_t num_blocks, void* stream) {
  int st = check_common(num_kv_heads, head_size, key_dst, value_dst, key_src,
                        value_src, "vaa_write_kv_single");
  if (st) return st;
  if (stride_block < 0 || stride_head < 0 || stride_token < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_write_kv_single: negative stride");
  // Both indices are host values: reject them here instead of skipping.
  if (block_id < 0 || block_id >= num_blocks)
    return fail(VAA_ERR_INVALID_ARG, "vaa_write_kv_single: block_id=%lld outside [0, %lld)",
                (long long)block_id, (long long)num_blocks);
  const int64_t lim =
      offset_limit(stride_block, stride_head, stride_token, num_kv_heads, head_size);
  if (token_offset < 0 || token_offset >= lim)
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_write_kv_single: token_offset=%lld outside the block (valid: 0..%lld)",
                (long long)token_offset, (long long)lim - 1);
  CacheDst d{key_dst, value_dst, stride_block, stride_head, stride_token,
             stride_block, stride_head, stride_token};
  NewSrc s{key_src, value_src, static_cast<int64_t>(num_kv_heads) * head_size,
           head_size};
  SingleResolver r{block_id, token_offset};
  return launch_copy(d, s, r, 1, num_kv_heads, head_size,
                     static_cast<hipStream_t>(stream), "vaa_write_kv_single");
}

extern "C" int vaa_kv_write_slots(const vaa_attn_params* p, uint16_t* key_cache,
                                  uint16_t* value_cache,
                                  const void* slot_mapping, int slot_index_type,
                                  const uint16_t* new_keys,
                                  const uint16_t* new_values, int num_tokens,
                                  void* stream) {
  if (!p) return fail(VAA_ERR_INVALID_ARG, "vaa_kv_write_slots: null params");
  if (!valid_dtype(p->dtype))  // a 16-bit copy either way
    return fail(VAA_ERR_UNSUPPORTED, "vaa_kv_write_slots: dtype=%d", p->dtype);
  int st = check_common(p->num_kv_heads, p->head_size, key_cache, value_cache,
                        new_keys, new_values, "vaa_kv_write_slots", num_tokens);
  if (st) return st;
  if (p->block_size <= 0 || p->num_blocks < 0)
    return fail(VAA_ERR_INVALID_ARG, "vaa_kv_write_slots: block_size=%d",
                p->block_size);
  if (num_tokens < 0 || (num_tokens > 0 && !slot_mapping))
    return fail(VAA_ERR_INVALID_ARG, "vaa_kv_write_slots: bad slot_mapping");
  CacheDst d = dst_from(p, key_cache, value_cache);
  NewSrc s{new_keys, new_values, p->new_kv_stride_token, p->new_kv_stride_head};
  const int64_t cap = p->num_blocks * p->block_size;
  hipStream_t strm = static_cast<hipStream_t>(stream);
  if (slot_index_type == VAA_INDEX_I64) {
    SlotResolver<int64_t> r{static_cast<const int64_t*>(slot_mapping),
                            p->block_size, cap};
    return launch_copy(d, s, r, num_tokens, p->num_kv_heads, p->head_size, strm,
                       "vaa_kv_write_slots");
  }
  if (slot_index_type == VAA_INDEX_I32) {
    SlotResolver<int32_t> r{static_cast<const int32_t*>(slot_mapping),
                            p->block_size, cap};
    return launch_copy(d, s, r, num_tokens, p->num_kv_heads, p->head_size, strm,
                       "vaa_kv_write_slots");
  }
  return fail(VAA_ERR_INVALID_ARG, "vaa_kv_write_slots: slot_index_type=%d",
              slot_index_type);
}

extern "C" int vaa_kv_write_decode(const vaa_attn_params* p, uint16_t* key_cache,
                                   uint16_t* value_cache,
                                   const int32_t* block_table,
                                   const int32_t* seq_lens,
                                   const uint16_t* new_keys,
                                   const uint16_t* new_values, void* stream) {
  if (!p) return fail(VAA_ERR_INVALID_ARG, "vaa_kv_write_decode: null params");
  if (!valid_dtype(p->dtype))
    return fail(VAA_ERR_UNSUPPORTED, "vaa_kv_write_decode: dtype=%d", p->dtype);
  int st = check_common(p->num_kv_heads, p->head_size, key_cache, value_cache,
                        new_keys, new_values, "vaa_kv_write_decode", p->num_seqs);
  if (st) return st;
  if (p->block_size <= 0 || p->max_blocks_per_seq <= 0 || p->num_seqs < 0)
    return fail(VAA_ERR_INVALID_ARG,
                "vaa_kv_write_decode: block_size=%d max_blocks_per_seq=%d",
                p->block_size, p->max_blocks_per_seq);
  if (p->num_seqs > 0 && (!block_table || !seq_lens))
    return fail(VAA_ERR_INVALID_ARG, "vaa_kv_write_decode: null block_table");
  CacheDst d = dst_from(p, key_cache, value_cache);
  NewSrc s{new_keys, new_values, p->new_kv_stride_token, p->new_kv_stride_head};
  DecodeResolver r{block_table, seq_lens, p->max_blocks_per_seq, p->block_size,
                   p->num_blocks};
  return launch_copy(d, s, r, p->num_seqs, p->num_kv_heads, p->head_size,
                     static_cast<hipStream_t>(stream), "vaa_kv_write_decode");
}
