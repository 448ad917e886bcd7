/*
 * ORACLE -- test infrastructure, not product code.
 *
 * Plain-C CPU restatement of the reference's integer/byte work on the paged
 * attention path: KV-cache writes and the slot / token index rules.  Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker.
 *
 * Pinned by: tests/test_oracle_kv.py (against the reference's own
 * vllm_apple/metal/native/kv_write.c compiled into oracle/_ref, against the
 * reference's known-answer test tests/metal/test_kv_cache_layout.py:68-131,
 * and against permutation invariants on exhaustive small tables).
 */
#include <stdint.h>
#include <string.h>

/* kv_write_prefill semantics (vllm_apple/engine/ops/kv_write.py:118-156):
 * slot < 0 skipped; block = slot / bs, offset = slot % bs.  Slots past the
 * capacity are skipped as well (the library's device guard). */
void oracle_kv_write_slots(uint16_t* kc, uint16_t* vc, const int64_t* slots,
                           const uint16_t* k, const uint16_t* v, int T, int KV,
                           int D, int bs, int64_t num_blocks, int64_t sb,
                           int64_t sh, int64_t st, int64_t src_st,
                           int64_t src_sh) {
  const int64_t cap = num_blocks * bs;
  for (int t = 0; t < T; ++t) {
    const int64_t s = slots[t];
    if (s < 0 || s >= cap) continue;
    const int64_t b = s / bs, o = s % bs;
    for (int h = 0; h < KV; ++h) {
      const int64_t dst = b * sb + h * sh + o * st;
      const int64_t src = t * src_st + h * src_sh;
      memcpy(kc + dst, k + src, (size_t)D * 2);
      memcpy(vc + dst, v + src, (size_t)D * 2);
    }
  }
}

/* metal_write_kv_batch (vllm_apple/metal/native/kv_write.c:33-78): token t,
 * head h goes to block_ids[t]*sb + h*sh + offsets[t]*st.  The reference
 * trusts both indices; the library's contract (and this restatement) skips a
 * token whose block id is outside [0, num_blocks) or whose offset o is
 * negative or makes the write end past the block: o*st + (KV-1)*sh + D > sb.
 * In-range tokens are the reference's memcpy loop exactly. */
void oracle_write_kv_batch(uint16_t* kc, uint16_t* vc, const uint16_t* k,
                           const uint16_t* v, const int64_t* block_ids,
                           const int64_t* offsets, int T, int KV, int D,
                           int64_t sb, int64_t sh, int64_t st,
                           int64_t num_blocks) {
  for (int t = 0; t < T; ++t) {
    const int64_t b = block_ids[t], o = offsets[t];
    if (b < 0 || b >= num_blocks || o < 0) continue;
    if (o * st + (int64_t)(KV - 1) * sh + D > sb) continue;
    for (int h = 0; h < KV; ++h) {
      const int64_t dst = b * sb + h * sh + o * st;
      const int64_t src = ((int64_t)t * KV + h) * D;
      memcpy(kc + dst, k + src, (size_t)D * 2);
      memcpy(vc + dst, v + src, (size_t)D * 2);
    }
  }
}

/* kv_write_decode (paged_attention_fused.metal:55-101 with the guards of
 * vllm_apple/engine/ops/kv_write.py:86-99): position seq_len-1. */
void oracle_kv_write_decode(uint16_t* kc, uint16_t* vc, const int32_t* bt,
                            int max_blocks, const int32_t* seq_lens, int S,
                            const uint16_t* k, const uint16_t* v, int KV, int D,
                            int bs, int64_t num_blocks, int64_t sb, int64_t sh,
                            int64_t st, int64_t src_st, int64_t src_sh) {
  for (int s = 0; s < S; ++s) {
    const int L = seq_lens[s];
    if (L <= 0) continue;
    const int pos = L - 1;
    const int bi = pos / bs;
    if (bi >= max_blocks) continue;
    const int32_t phys = bt[(int64_t)s * max_blocks + bi];
    if (phys < 0 || phys >= num_blocks) continue;
    const int o = pos % bs;
    for (int h = 0; h < KV; ++h) {
      const int64_t dst = (int64_t)phys * sb + h * sh + (int64_t)o * st;
      const int64_t src = (int64_t)s * src_st + h * src_sh;
      memcpy(kc + dst, k + src, (size_t)D * 2);
      memcpy(vc + dst, v + src, (size_t)D * 2);
    }
  }
}

/* token_to_seq = repeat_interleave(arange(S), diff(qsl)) (runner.py:526-546);
 * positions = seq_len - query_len + i (apple_model_runner.py:1188-1200). */
void oracle_token_index(const int32_t* qsl, const int32_t* seq_lens, int S,
                        int T, int32_t* tok, int32_t* pos) {
  for (int t = 0; t < T; ++t) {
    tok[t] = -1;
    pos[t] = -1;
  }
  for (int s = 0; s < S; ++s) {
    const int q0 = qsl[s], q1 = qsl[s + 1];
    for (int t = q0; t < q1; ++t) {
      if (t < 0 || t >= T) continue;
      tok[t] = s;
      pos[t] = seq_lens[s] - (q1 - q0) + (t - q0);
    }
  }
}

/* slot = block_ids[pos // bs] * bs + pos % bs, else pos when the block list is
 * too short (apple_model_runner.py:1202-1249). */
void oracle_slot_mapping(const int32_t* bt, int max_blocks, int bs,
                         const int32_t* tok, const int32_t* pos, int S, int T,
                         int64_t* slots) {
  for (int t = 0; t < T; ++t) {
    const int s = tok[t], p = pos[t];
    if (s < 0 || s >= S || p < 0) {
      slots[t] = -1;
      continue;
    }
    const int bi = p / bs;
    const int32_t b = bi < max_blocks ? bt[(int64_t)s * max_blocks + bi] : -1;
    slots[t] = b >= 0 ? (int64_t)b * bs + p % bs : (int64_t)p;
  }
}
