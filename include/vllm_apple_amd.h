/*
 * vllm_apple_amd.h -- C ABI of the MI355X (gfx950) paged-attention hot path.
 *
 * Every entry point takes device pointers owned by the caller, explicit
 * element strides and a HIP stream (passed as void*), enqueues its kernels on
 * that stream and returns without synchronising.  The return value is a
 * status code (VAA_OK == 0, negative on error); vaa_last_error() returns a
 * thread-local message for the last failure on the calling thread.
 *
 * Data types: K/V cache, queries, outputs and activations are 16-bit floats
 * (uint16_t storage): IEEE fp16, the reference's type, or bfloat16, chosen by
 * vaa_attn_params.dtype for the attention entry points and by a dtype
 * argument (VAA_DTYPE_F16 / VAA_DTYPE_BF16) for the layer ops.  Block tables, sequence lengths, token->sequence maps
 * and positions are int32.  Slot mappings may be int32 (engine) or int64
 * (vLLM metadata), selected by an argument.
 *
 * Cache layouts are described by (stride_block, stride_head, stride_token)
 * in elements, so both layouts used by the reference are first-class:
 *   kernel/engine layout  K,V each [num_blocks, num_kv_heads, block_size, D]
 *       (vllm_apple/metal/kv_cache.py:213-219, engine/kv_cache.py:142-148)
 *   vLLM-facing layout    kv_cache[2, num_blocks, block_size, num_kv_heads, D]
 *       (vllm_apple/v1/attention/backends/metal_attn.py:171-185)
 * The innermost (head_size) dimension must be contiguous.
 *
 * Device-side guards: every kernel skips (never dereferences) a block id
 * outside [0, num_blocks), a slot outside [0, num_blocks*block_size) and a
 * token offset whose write would leave its block, so a bad index cannot
 * fault the GPU or write outside the block it names.  Range validation that
 * raises errors is done on the host by the Python layer, as the reference
 * does (vllm_apple/engine/kv_cache.py:300-420).
 */
#ifndef VLLM_APPLE_AMD_H_
#define VLLM_APPLE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VAA_ABI_VERSION 5

enum {
  VAA_OK = 0,
  VAA_ERR_INVALID_ARG = -1,  /* bad shape, stride, alignment or null pointer */
  VAA_ERR_UNSUPPORTED = -2,  /* head size / block size / group size not built */
  VAA_ERR_HIP = -3,          /* HIP runtime error (launch or device query)    */
  VAA_ERR_WORKSPACE = -4     /* split-K workspace missing or too small        */
};

/* Index element types for slot mappings. */
enum { VAA_INDEX_I32 = 0, VAA_INDEX_I64 = 1 };

/* 16-bit element types of caches, queries, new K/V and outputs. */
enum { VAA_DTYPE_F16 = 0, VAA_DTYPE_BF16 = 1 };

/*
 * vaa_attn_params.partition_size for decode:
 *   > 0  fixed split-K partitions of that many tokens (a multiple of 128);
 *   0    automatic, from max_seq_len alone;
 *   VAA_PARTITION_BALANCED  4-wave workgroups, two per CU's worth, each
 *        taking an equal share of the 16-token tiles of all sequences, split
 *        on the device from seq_lens (for unequal lengths; at most 8192
 *        sequences).
 *   VAA_PARTITION_BALANCED_SHARED  the same split with four workgroups per
 *        CU's worth, for a decode that runs concurrently with another kernel
 *        (a mixed step's prefill on a second stream): its smaller shares
 *        then fill the CUs the other kernel leaves.  A little slower than
 *        VAA_PARTITION_BALANCED when decode runs alone.
 */
#define VAA_PARTITION_BALANCED (-1)
#define VAA_PARTITION_BALANCED_SHARED (-2)

/*
 * Attention parameters.  Mirrors FusedAttentionParams / PagedAttentionParams
 * (vllm_apple/metal/kernels/paged_attention_fused.metal:24-49,
 *  vllm_apple/engine/ops/attention.py:51-157) with 64-bit strides, plus the
 * cache capacity (device-side guard) and the split-K partition size.
 */
typedef struct vaa_attn_params {
  float scale;                /* softmax scale, usually 1/sqrt(head_size)     */
  int32_t num_seqs;           /* rows of block_table / seq_lens               */
  int32_t max_seq_len;        /* upper bound of seq_lens (sizes the grid)     */
  int32_t max_blocks_per_seq; /* block_table row stride in elements           */
  int32_t head_size;          /* 32, 64, 96 or 128                            */
  int32_t block_size;         /* tokens per cache block, multiple of 16       */
  int32_t num_kv_heads;
  int32_t num_query_heads;
  int32_t queries_per_kv;     /* num_query_heads / num_kv_heads               */
  int32_t partition_size;     /* split-K tokens per partition; 0 = automatic,
                                 VAA_PARTITION_BALANCED(_SHARED) = split by
                                 lengths                                      */
  int64_t num_blocks;         /* cache capacity in blocks                     */
  int64_t k_stride_block, k_stride_head, k_stride_token;
  int64_t v_stride_block, v_stride_head, v_stride_token;
  int64_t q_stride_token, q_stride_head;
  int64_t o_stride_token, o_stride_head;
  int64_t new_kv_stride_token, new_kv_stride_head; /* new K and new V        */
  int32_t dtype;              /* VAA_DTYPE_F16 (0, the reference's type) or
                                 VAA_DTYPE_BF16: element type of the cache,
                                 queries, new K/V and outputs; fp32 math      */
} vaa_attn_params;

/* Thread-local message describing the last error on this thread. */
const char* vaa_last_error(void);
int vaa_abi_version(void);

/* ------------------------------------------------------------------------
 * KV cache writes (bit-exact copies)
 * ---------------------------------------------------------------------- */

/*
 * Replaces metal_write_kv_batch (vllm_apple/metal/native/kv_write.c:33-78),
 * bound by ctypes at vllm_apple/metal/bridge/metal_paged_attention_v2.py:574-607.
 * Same arguments, now device pointers, plus num_blocks (guard) and a stream.
 * Source K/V are contiguous [num_tokens, num_kv_heads, head_size]; for each
 * token t and head h the head_size elements go to
 * block_ids[t]*stride_block + h*stride_head + token_offsets[t]*stride_token.
 * The reference trusts both indices.  Here a token is skipped when its block
 * id is outside [0, num_blocks) or its offset o is negative or so large that
 * the token's write leaves the block:
 *   o*stride_token + (num_kv_heads-1)*stride_head + head_size > stride_block
 * (for both cache layouts that is o >= block_size).
 */
int vaa_write_kv_batch(uint16_t* key_dst, uint16_t* value_dst,
                       const uint16_t* key_src, const uint16_t* value_src,
                       const int64_t* block_ids, const int64_t* token_offsets,
                       int num_tokens, int num_kv_heads, int head_size,
                       int64_t stride_block, int64_t stride_head,
                       int64_t stride_token, int64_t num_blocks, void* stream);

/*
 * Replaces metal_write_kv_single (vllm_apple/metal/native/kv_write.c:84-107):
 * one token, block id and offset passed by value.  Since both are host
 * values, a block id or offset that vaa_write_kv_batch would skip is
 * rejected with VAA_ERR_INVALID_ARG and nothing is enqueued.
 */
int vaa_write_kv_single(uint16_t* key_dst, uint16_t* value_dst,
                        const uint16_t* key_src, const uint16_t* value_src,
                        int64_t block_id, int64_t token_offset,
                        int num_kv_heads, int head_size, int64_t stride_block,
                        int64_t stride_head, int64_t stride_token,
                        int64_t num_blocks, void* stream);

/*
 * Replaces the kv_write_prefill kernel (vllm_apple/engine/ops/kv_write.py:118-156,
 * host KVWriteOp.encode_prefill :336-402) and the torch scatter path
 * (vllm_apple/v1/attention/backends/base_attn.py:308-342): for token t with
 * s = slot_mapping[t] >= 0, K[s/bs, h, s%bs, :] = new_keys[t, h, :] and the
 * same for V.  Negative slots (padding) and slots >= num_blocks*block_size
 * are skipped.  Uses p->num_kv_heads, head_size, block_size, num_blocks,
 * k_/v_stride_*, new_kv_stride_*.
 */
int vaa_kv_write_slots(const vaa_attn_params* p, uint16_t* key_cache,
                       uint16_t* value_cache, const void* slot_mapping,
                       int slot_index_type, const uint16_t* new_keys,
                       const uint16_t* new_values, int num_tokens,
                       void* stream);

/*
 * Replaces kv_write_decode (vllm_apple/metal/kernels/paged_attention_fused.metal:55-101,
 * guarded variant vllm_apple/engine/ops/kv_write.py:66-114, host
 * KVWriteOp.encode_decode :261-334): the new token of sequence s is written
 * at position seq_lens[s]-1 through block_table.  seq_len <= 0, a block index
 * >= max_blocks_per_seq or an invalid physical block -> no write.
 */
int vaa_kv_write_decode(const vaa_attn_params* p, uint16_t* key_cache,
                        uint16_t* value_cache, const int32_t* block_table,
                        const int32_t* seq_lens, const uint16_t* new_keys,
                        const uint16_t* new_values, void* stream);

/* ------------------------------------------------------------------------
 * Paged attention
 * ---------------------------------------------------------------------- */

/*
 * Bytes of split-K workspace vaa_paged_attention_decode needs for these
 * parameters (0 when every sequence fits one partition).  The partition size
 * actually used is written to *partition_size_out when it is non-null.
 */
size_t vaa_paged_attention_decode_workspace_size(const vaa_attn_params* p,
                                                 int32_t* partition_size_out);

/*
 * Paged decode attention with GQA.  Replaces paged_attention_fused_h128 /
 * paged_attention_fused_generic (vllm_apple/metal/kernels/paged_attention_fused.metal:107-328),
 * paged_attention_v2_decode[_h128] (paged_attention_v2.metal:49-261) and the
 * host PagedAttentionOp.encode_decode_fused (vllm_apple/engine/ops/attention.py:369-537).
 *
 * For sequence s, query head h, kv head h / queries_per_kv:
 *   out[s,h,:] = sum_{j < L} softmax_j(scale * q[s,h,:] . K_j) V_j,  L = seq_lens[s]
 * with fp32 accumulation; seq_len <= 0 gives a zero row.  When new_keys and
 * new_values are non-null the token at position L-1 is taken from them and
 * written to the cache in the same launch (the fused KV write); when they are
 * null the cache must already hold it.  Long contexts are split into
 * partitions (p->partition_size, see VAA_PARTITION_BALANCED) whose partial
 * (max, sum, acc) go to the workspace and are merged (log-sum-exp) by a
 * second kernel on the same stream; the workspace must hold
 * vaa_paged_attention_decode_workspace_size(p) bytes, 16-byte aligned (it may
 * be null when that size is 0), and must not be shared by calls that can run
 * concurrently.
 */
int vaa_paged_attention_decode(const vaa_attn_params* p, const uint16_t* query,
                               uint16_t* key_cache, uint16_t* value_cache,
                               const int32_t* block_table,
                               const int32_t* seq_lens, uint16_t* output,
                               const uint16_t* new_keys,
                               const uint16_t* new_values, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * vaa_paged_attention_decode without a workspace argument: it allocates
 * nothing and takes no caller memory beyond its inputs and outputs.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * vaa_paged_attention_decode otherwise.  The split-K partials go to a fixed
 * device array of vaa_paged_attention_decode_noalloc_max_workspace() bytes
 * (32 MiB), one per GPU, held until the process ends; a split that needs
 * more (vaa_paged_attention_decode_workspace_size) is refused with
 * VAA_ERR_WORKSPACE before anything is enqueued.  The stream must belong to
 * the current device.  All calls on one GPU share its array: calls that can
 * overlap on one GPU (different streams, no ordering) race and must not be
 * made.
 */
size_t vaa_paged_attention_decode_noalloc_max_workspace(void);
int vaa_paged_attention_decode_noalloc(const vaa_attn_params* p, const uint16_t* query,
                                       uint16_t* key_cache, uint16_t* value_cache,
                                       const int32_t* block_table, const int32_t* seq_lens,
                                       uint16_t* output, const uint16_t* new_keys,
                                       const uint16_t* new_values, void* stream);

/*
 * Merge of attention states: the split-K second pass on its own, for partial
 * results the caller computed (partitions of one context decoded apart, a
 * context split across GPUs, a shared prefix and a per-request suffix).  No
 * counterpart in the reference, whose kernels never split a context; the
 * arithmetic is that of vaa_paged_attention_decode's merge pass.
 *   partial_out  fp32 [num_seqs, num_heads, max_parts, head_size], each
 *                partition's normalised output o_p (contiguous);
 *   partial_lse  fp32 [num_seqs, num_heads, max_parts], lse_p = log of the
 *                partition's softmax denominator, sum_j e^(scale q.k_j), in
 *                natural log; -inf for a partition without keys;
 *   num_parts    int32 [num_seqs]: partitions of each sequence (the first
 *                num_parts[s] of max_parts), or null for all max_parts.
 * out[s, h, :] = sum_p e^(lse_p - LSE) o_p with LSE = log sum_p e^(lse_p),
 * rounded to the 16-bit dtype at strides (o_stride_token, o_stride_head); a
 * row with no keys is zero.  output_lse (fp32 [num_seqs, num_heads], may be
 * null) receives LSE (-inf for no keys), so merges can be chained.
 */
int vaa_merge_attn_states(const float* partial_out, const float* partial_lse,
                          const int32_t* num_parts, int num_seqs, int num_heads,
                          int max_parts, int head_size, uint16_t* output,
                          int64_t o_stride_token, int64_t o_stride_head, float* output_lse,
                          int dtype, void* stream);

/*
 * Chunked-prefill paged attention (MFMA).  Replaces paged_attention_v2_prefill
 * (vllm_apple/metal/kernels/paged_attention_v2.metal:375-478, host
 * PagedAttentionOp.encode_prefill vllm_apple/engine/ops/attention.py:290-367).
 * Token t (query row t) of sequence token_to_seq[t] attends to cache
 * positions [0, positions[t]] through that sequence's block table, so the
 * cached prefix and the causal mask inside the chunk both follow from the
 * positions.  The chunk's own K/V must already be in the cache.  Rows with
 * an invalid sequence, a negative position, a context longer than the block
 * table or an invalid block inside the context are left unwritten, as in the
 * reference kernel.
 */
int vaa_paged_attention_prefill(const vaa_attn_params* p, const uint16_t* query,
                                const uint16_t* key_cache,
                                const uint16_t* value_cache,
                                const int32_t* block_table,
                                const int32_t* token_to_seq,
                                const int32_t* positions, uint16_t* output,
                                int num_tokens, void* stream);

/*
 * The same prefill with split-K over the keys, for batches whose contexts
 * are unequal (a long prefix next to short ones): key tiles are cut into
 * pieces of split_keys positions (a positive multiple of 64; the last piece
 * takes any excess past p->max_seq_len), one workgroup per (query tile, kv
 * head, piece), and rows whose context spans several pieces are combined by
 * a log-sum-exp merge -- the split/merge structure of
 * paged_attention_v2.metal's partitions (:49-261) applied to the prefill
 * kernel (:375-478).  Same results and unwritten-row rules as
 * vaa_paged_attention_prefill.  workspace: at least
 * vaa_paged_attention_prefill_workspace_size(p, num_tokens, split_keys) bytes,
 * 16-byte aligned (0 bytes when max_seq_len fits one piece).
 */
size_t vaa_paged_attention_prefill_workspace_size(const vaa_attn_params* p, int num_tokens,
                                                  int split_keys);
int vaa_paged_attention_prefill_split(const vaa_attn_params* p, const uint16_t* query,
                                      const uint16_t* key_cache, const uint16_t* value_cache,
                                      const int32_t* block_table, const int32_t* token_to_seq,
                                      const int32_t* positions, uint16_t* output,
                                      int num_tokens, int split_keys, void* workspace,
                                      size_t workspace_bytes, void* stream);

/*
 * token_to_seq and positions for a flattened batch, computed on the device
 * from query_start_loc [num_seqs+1] and full seq_lens [num_seqs]:
 *   token_to_seq = repeat_interleave(arange(num_seqs), diff(query_start_loc))
 *       (vllm_apple/engine/runner.py:526-546)
 *   positions[t] = seq_lens[s] - query_len[s] + (t - query_start_loc[s])
 *       (full seq_lens include the new tokens, apple_model_runner.py:1188-1200)
 * Tokens outside [query_start_loc[0], query_start_loc[num_seqs]) get -1.
 */
int vaa_build_token_index(const int32_t* query_start_loc,
                          const int32_t* seq_lens, int num_seqs,
                          int num_tokens, int32_t* token_to_seq,
                          int32_t* positions, void* stream);

/*
 * slot_mapping[t] = block_table[s, pos/bs]*bs + pos%bs for s = token_to_seq[t],
 * pos = positions[t]; when the block index is past the table width or the
 * entry is negative the slot is pos itself, as the reference runner does
 * (vllm_apple/v1/worker/apple_model_runner.py:1202-1249).  Invalid s or
 * negative pos -> -1.  Output is int64 (vLLM metadata type).
 */
int vaa_build_slot_mapping(const int32_t* block_table, int max_blocks_per_seq,
                           int block_size, const int32_t* token_to_seq,
                           const int32_t* positions, int num_seqs,
                           int num_tokens, int64_t* slot_mapping,
                           void* stream);

/* ------------------------------------------------------------------------
 * Layer ops next to attention.  `dtype` is VAA_DTYPE_F16 (the reference's
 * fp16) or VAA_DTYPE_BF16 for every 16-bit tensor of the call; arithmetic is
 * fp32, results round to nearest even.  Another value is VAA_ERR_UNSUPPORTED.
 * ---------------------------------------------------------------------- */

/*
 * RMSNorm.  Replaces rmsnorm_kernel / rmsnorm_residual_kernel
 * (vllm_apple/engine/ops/rmsnorm.py:78-173, host EngineRMSNorm.encode :226-321):
 *   out = half(float(x) * rsqrt(mean(float(x)^2) + eps) * float(w)) [+ residual]
 * The residual (may be null) is added after the norm, as the reference
 * kernel does.  Row strides are in elements.
 */
int vaa_rmsnorm(const uint16_t* input, uint16_t* output, const uint16_t* weight,
                const uint16_t* residual, int num_tokens, int hidden_size,
                int64_t input_stride, int64_t output_stride,
                int64_t residual_stride, float eps, int dtype, void* stream);

/*
 * Residual add + RMSNorm in one pass.  Replaces the reference layer's three
 * steps between the O projection and the MLP, and between the MLP and the
 * next layer's input norm (vllm_apple/engine/runner.py:871-887,1107-1130,
 * 1165-1171: encode_residual_add, encode_copy into the residual buffer,
 * EngineRMSNorm.encode in place):
 *   h = half(float(input) + float(residual));  residual <- h;
 *   output = half(float(h) * rsqrt(mean(float(h)^2) + eps) * float(w))
 * bit for bit as those steps.  output may alias input, not residual.
 */
int vaa_add_rmsnorm(const uint16_t* input, uint16_t* residual, const uint16_t* weight,
                    uint16_t* output, int num_tokens, int hidden_size, int64_t input_stride,
                    int64_t residual_stride, int64_t output_stride, float eps, int dtype,
                    void* stream);

/*
 * NeoX (split-half) rotary embedding, in place on query [T, num_heads, D] and
 * key [T, num_kv_heads, D] (token strides given, heads contiguous at stride
 * head_size).  Replaces rope_neox_kernel (vllm_apple/engine/ops/elementwise.py:185-239,
 * host EngineRoPE.encode :699-766).  cos_cache/sin_cache are fp32
 * [max_position, rotary_dim/2]; tokens whose position is outside
 * [0, max_position) are left unrotated.  key may be null.
 */
int vaa_rope_neox(uint16_t* query, uint16_t* key, const float* cos_cache,
                  const float* sin_cache, const int32_t* positions,
                  int num_tokens, int num_heads, int num_kv_heads,
                  int head_size, int rotary_dim, int64_t q_stride_token,
                  int64_t k_stride_token, int max_position, int dtype, void* stream);

/*
 * SwiGLU: out = round16(silu(float(g)) * float(u)).  Replaces silu_mul_kernel
 * (vllm_apple/engine/ops/elementwise.py:114-124, host encode_silu_mul
 * :496-532) over num_elements contiguous elements.
 */
int vaa_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* output,
                 int64_t num_elements, int dtype, void* stream);

/*
 * Row-strided SwiGLU over [rows, cols] (e.g. gate/up halves of vLLM's
 * [T, 2I] projection output).  Strides in elements.  No counterpart entry
 * point in the reference; same arithmetic as vaa_silu_mul.
 */
int vaa_silu_mul_2d(const uint16_t* gate, const uint16_t* up, uint16_t* output,
                    int64_t rows, int64_t cols, int64_t gate_stride,
                    int64_t up_stride, int64_t output_stride, int dtype, void* stream);

/*
 * Gated-MLP up projection with the SwiGLU epilogue, on the matrix cores:
 *   output[t, i] = round16(silu(g) * u),
 *   g = sum_h x[t, h] w_gate[i, h],   u = sum_h x[t, h] w_up[i, h],
 * with g and u accumulated in fp32 and not rounded before the epilogue
 * (silu and the product as vaa_silu_mul).  Replaces the reference's gated
 * path of EngineMLP (vllm_apple/engine/ops/mlp.py:247-330): gate_proj and
 * up_proj GEMMs into [T, I] intermediates (weights [I, H], transpose_B) and
 * encode_silu_mul over them (elementwise.py:114-124); the fused gate_up_proj
 * weight [2I, H] is passed as w_gate = w, w_up = w + I * w_stride.
 * x: [num_tokens, hidden_size] at row stride x_stride; weights at row stride
 * w_stride; output [num_tokens, intermediate_size] at row stride
 * output_stride (strides in elements).  hidden_size must be a multiple of
 * 64 and intermediate_size of 128 (VAA_ERR_UNSUPPORTED otherwise); x and
 * the weights and the output 16-byte aligned, with strides that are
 * multiples of 8.
 */
int vaa_gate_up_silu(const uint16_t* x, int64_t x_stride, const uint16_t* w_gate,
                     const uint16_t* w_up, int64_t w_stride, uint16_t* output,
                     int64_t output_stride, int num_tokens, int hidden_size,
                     int intermediate_size, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Fused QKV epilogue
 * ---------------------------------------------------------------------- */

/*
 * Bias add + NeoX rotary embedding + KV write in one pass over the QKV
 * projection's output.  No single counterpart in the reference; it fuses the
 * three kernels the reference runs in turn over its planar QKV buffer
 * (vllm_apple/engine/runner.py:919-1016): bias_add_inplace_kernel on Q, K and V
 * (engine/ops/qkv.py:391-416, elementwise.py:252-259), rope_neox_kernel on Q
 * and K (elementwise.py:185-239) and kv_write_prefill (kv_write.py:118-156).
 * For token t:
 *   q[t] <- rope(q[t] + bias_q)            in place
 *   k[t] <- rope(k[t] + bias_k)            in place, and to the cache slot
 *   v[t] <- v[t] + bias_v                  in place, and to the cache slot
 * where the biased values are rounded to the 16-bit type before the rotation
 * (the reference's half add), rope rotates the first rotary_dim elements by
 * cos/sin_cache[positions[t]] (fp32 [max_position, rotary_dim/2]; positions
 * outside the table are left unrotated) and the slot rule is
 * vaa_kv_write_slots's (slot_mapping[t] < 0 or past the cache: no write).
 * bias is [H*D | KV*D | KV*D] in the element type, or null.  query is
 * [T, H, D] with token stride p->q_stride_token, key and value [T, KV, D]
 * share p->new_kv_stride_token; heads are packed at stride D.  Uses
 * p->dtype, num_query_heads, num_kv_heads, head_size, block_size, num_blocks
 * and the k_/v_stride_* of the cache.  rotary_dim is a multiple of 16 and at
 * most head_size.
 */
int vaa_qkv_epilogue(const vaa_attn_params* p, uint16_t* query, uint16_t* key,
                     uint16_t* value, const uint16_t* bias, const float* cos_cache,
                     const float* sin_cache, int rotary_dim, int max_position,
                     const int32_t* positions, const void* slot_mapping,
                     int slot_index_type, uint16_t* key_cache, uint16_t* value_cache,
                     int num_tokens, void* stream);

/* ------------------------------------------------------------------------
 * Top-k logits selection
 * ---------------------------------------------------------------------- */

/*
 * The k largest values of each logits row and their column indices.
 * Replaces topk_select / topk_select_small_k (vllm_apple/engine/ops/topk.py:40-412,
 * host EngineTopK.encode :324-401), which cut the logits read back to the host
 * to k entries per token.  logits: [num_tokens, vocab_size] 16-bit floats (fp16
 * or bf16; the selection reads their bit patterns), 2-byte aligned, with
 * row_stride elements between rows (16-byte aligned rows are read 16 bytes at a
 * time).  Outputs indices int32 and values (the same 16-bit values)
 * [num_tokens, k] with out_stride between rows, sorted by value descending,
 * ties by lower column.  Values order as -NaN < -inf < ... < -0 < +0 < ... <
 * +inf < +NaN.  1 <= k <= 256 and k <= vocab_size (the reference caps k at 50,
 * or 8 on its small-k path); vocab_size <= 16384 * floor(4096 / k).
 *
 * A row is split over several workgroups when that fills the GPU better; the
 * chunks' survivors then go through `workspace`, whose size
 * vaa_topk_workspace_size returns (0: none needed, workspace may be null).  It
 * depends only on (num_tokens, vocab_size, k).  VAA_ERR_WORKSPACE when it is
 * missing, short or not 16-byte aligned.  Two launches at most, no allocation.
 */
int vaa_topk_workspace_size(int num_tokens, int vocab_size, int k, size_t* workspace_bytes);
int vaa_topk_logits(const uint16_t* logits, int num_tokens, int vocab_size,
                    int64_t row_stride, int k, int32_t* indices, uint16_t* values,
                    int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Measurement aid
 * ---------------------------------------------------------------------- */

/*
 * Read-only stream of the K and V rows a paged decode step reads, the
 * measured ceiling beside the decode's HBM roofline.  No counterpart in the
 * reference.  Reads, through block_table, the rows of positions
 * [0, seq_lens[s]) of every sequence s and kv head h with the decode's loads,
 * cut into pieces as the decode's fixed split-K partitions cut a context
 * (p->partition_size P, a multiple of 16, with parts = ceil(max_seq_len / P)
 * pieces per sequence; 0: one piece, parts = 1), one workgroup per piece, and
 * writes their checksum:
 *   sink[(s * parts + q) * num_kv_heads + h] = XOR of every 32-bit word of the
 *       K and V rows of positions [q P, min((q + 1) P, seq_lens[s]))
 * (rows whose table entry is negative, >= num_blocks or past
 * max_blocks_per_seq are skipped; an empty piece gives 0).  Uses the cache
 * fields of p (num_seqs, max_seq_len, max_blocks_per_seq, head_size
 * 32/64/96/128, block_size a multiple of 16, num_kv_heads, num_blocks, k/v
 * strides, partition_size); sink holds num_seqs * parts * num_kv_heads uint32.
 */
int vaa_kv_stream_read(const vaa_attn_params* p, const uint16_t* key_cache,
                       const uint16_t* value_cache, const int32_t* block_table,
                       const int32_t* seq_lens, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_APPLE_AMD_H_ */
