// Host-side producers of the per-step metadata: Transformer.preparePrefill / prepareDecode
// (engine/Transformer.java:319-456) restated over plain arrays, so the model runner hands the
// scheduled sequences to the library once per step and the library builds, and uploads, what
// every attention layer of the step reads.  No device work happens here except through
// nva_step_set.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#include "../../include/nva.h"

namespace {

// Builds into vectors; shared by the caller-array and the context entry points.
struct Built {
  std::vector<int32_t> cu_q, cu_k, slots, lens, ids, tables;
  std::vector<float> pos;
  int32_t max_q = 0, max_k = 0, stride = 0;
  bool has_tables = false;
  char err[160] = {0};
};

int max_blocks(const nva_seq *seqs, int n) {
  int w = 0;
  for (int i = 0; i < n; i++) w = std::max(w, seqs[i].num_blocks);
  return w;
}

// prepareBlockTables, Transformer.java:319-330: rectangular, width = longest table, -1 padded.
void block_tables(const nva_seq *seqs, int n, Built &b) {
  b.stride = max_blocks(seqs, n);
  b.tables.assign((size_t)n * b.stride, -1);
  for (int i = 0; i < n; i++)
    for (int j = 0; j < seqs[i].num_blocks; j++) b.tables[(size_t)i * b.stride + j] = seqs[i].block_table[j];
  b.has_tables = true;
}

nva_status build_prefill(const nva_seq *seqs, int n, int bs, Built &b) {
  if (n < 0 || bs <= 0 || (n > 0 && !seqs)) {
    snprintf(b.err, sizeof(b.err), "bad arguments (num_seqs=%d, block_size=%d)", n, bs);
    return NVA_E_ARG;
  }
  b.cu_q.assign(1, 0);
  b.cu_k.assign(1, 0);
  bool any_table = false;
  for (int si = 0; si < n; si++) {
    const nva_seq &s = seqs[si];
    const int start = s.num_cached_tokens;
    const int qlen = s.num_scheduled;
    const int end = start + qlen;
    if (start < 0 || qlen < 0 || s.num_blocks < 0 || (s.num_blocks > 0 && !s.block_table)) {
      snprintf(b.err, sizeof(b.err), "sequence %d: bad window or table", si);
      return NVA_E_ARG;
    }
    for (int i = start; i < end; i++) {
      b.pos.push_back((float)i);
      b.ids.push_back(s.seq_id);
    }
    b.cu_q.push_back(b.cu_q.back() + qlen);
    b.cu_k.push_back(b.cu_k.back() + end);
    b.max_q = std::max(b.max_q, qlen);
    b.max_k = std::max(b.max_k, end);
    if (s.num_blocks == 0) continue;  // no pages yet: nothing to map
    any_table = true;
    // The window's slots, page by page; the first page may start mid-page.
    const int sb = start / bs;
    const int eb = (end + bs - 1) / bs;
    if (eb > s.num_blocks) {
      snprintf(b.err, sizeof(b.err),
               "sequence %d: block table has %d blocks but tokens [%d, %d) need %d", si,
               s.num_blocks, start, end, eb);
      return NVA_E_ARG;
    }
    for (int i = sb; i < eb; i++) {
      const int64_t base = (int64_t)s.block_table[i] * bs;
      const int64_t s0 = base + (i == sb ? start % bs : 0);
      const int64_t s1 = i != eb - 1 ? base + bs : base + end - (int64_t)i * bs;
      for (int64_t sl = s0; sl < s1; sl++) b.slots.push_back((int32_t)sl);
    }
  }
  if (b.cu_k.back() > b.cu_q.back() && any_table) block_tables(seqs, n, b);
  return NVA_OK;
}

nva_status build_decode(const nva_seq *seqs, int n, int bs, Built &b) {
  if (n < 0 || bs <= 0 || (n > 0 && !seqs)) {
    snprintf(b.err, sizeof(b.err), "bad arguments (num_seqs=%d, block_size=%d)", n, bs);
    return NVA_E_ARG;
  }
  b.pos.resize(n);
  b.slots.resize(n);
  b.lens.resize(n);
  b.ids.resize(n);
  for (int i = 0; i < n; i++) {
    const nva_seq &s = seqs[i];
    if (s.num_blocks <= 0 || !s.block_table) {
      snprintf(b.err, sizeof(b.err), "sequence %d has an empty block table", i);
      return NVA_E_ARG;
    }
    if (s.num_tokens <= 0) {
      snprintf(b.err, sizeof(b.err), "sequence %d has no tokens", i);
      return NVA_E_ARG;
    }
    const int nblocks = (s.num_tokens + bs - 1) / bs;  // Sequence.numBlocks
    const int last_tokens = s.num_tokens - (nblocks - 1) * bs;
    b.pos[i] = (float)(s.num_tokens - 1);
    b.lens[i] = s.num_tokens;
    b.ids[i] = s.seq_id;
    b.slots[i] = (int32_t)((int64_t)s.block_table[s.num_blocks - 1] * bs + last_tokens - 1);
  }
  block_tables(seqs, n, b);
  return NVA_OK;
}

nva_status export_to(const Built &b, int n, bool prefill, nva_step_meta *out) {
  if (!out) return NVA_E_ARG;
  auto copy = [](int32_t *dst, const std::vector<int32_t> &v) {
    if (dst && !v.empty()) std::copy(v.begin(), v.end(), dst);
  };
  if (prefill) {
    copy(out->cu_q, b.cu_q);
    copy(out->cu_k, b.cu_k);
  }
  copy(out->context_lens, b.lens);
  copy(out->slot_mapping, b.slots);
  copy(out->seq_ids, b.ids);
  if (out->positions && !b.pos.empty()) std::copy(b.pos.begin(), b.pos.end(), out->positions);
  if (out->block_tables && b.has_tables) copy(out->block_tables, b.tables);
  out->max_seqlen_q = b.max_q;
  out->max_seqlen_k = b.max_k;
  out->num_slots = (int32_t)b.slots.size();
  out->num_tokens = (int32_t)b.pos.size();
  out->bt_stride = b.has_tables ? b.stride : 0;
  out->has_tables = b.has_tables ? 1 : 0;
  (void)n;
  return NVA_OK;
}

nva_status upload(nva_ctx *ctx, const Built &b, int n, bool prefill) {
  return nva_step_set(ctx, prefill ? 1 : 0, prefill ? b.cu_q.data() : nullptr,
                      prefill ? b.cu_k.data() : nullptr, n, b.max_q, b.max_k, b.slots.data(),
                      (int)b.slots.size(), prefill ? nullptr : b.lens.data(),
                      b.has_tables ? b.tables.data() : nullptr, b.has_tables ? b.stride : 0,
                      b.ids.data(), b.pos.data(), (int)b.pos.size());
}

}  // namespace

// Error text of a failed build on a context (defined with the context in api.cpp).
__attribute__((visibility("hidden"))) nva_status nva_internal_fail(nva_ctx *ctx, nva_status st,
                                                                 const char *msg);

extern "C" {

nva_status nva_build_prefill_metadata(const nva_seq *seqs, int num_seqs, int block_size,
                                      nva_step_meta *out) {
  Built b;
  nva_status st = build_prefill(seqs, num_seqs, block_size, b);
  if (st != NVA_OK) return st;
  return export_to(b, num_seqs, true, out);
}

nva_status nva_build_decode_metadata(const nva_seq *seqs, int num_seqs, int block_size,
                                     nva_step_meta *out) {
  Built b;
  nva_status st = build_decode(seqs, num_seqs, block_size, b);
  if (st != NVA_OK) return st;
  return export_to(b, num_seqs, false, out);
}

nva_status nva_step_prepare_prefill(nva_ctx *ctx, const nva_seq *seqs, int num_seqs,
                                    int block_size) {
  if (!ctx) return NVA_E_ARG;
  Built b;
  nva_status st = build_prefill(seqs, num_seqs, block_size, b);
  if (st != NVA_OK) return nva_internal_fail(ctx, st, b.err);
  return upload(ctx, b, num_seqs, true);
}

nva_status nva_step_prepare_decode(nva_ctx *ctx, const nva_seq *seqs, int num_seqs,
                                   int block_size) {
  if (!ctx) return NVA_E_ARG;
  Built b;
  nva_status st = build_decode(seqs, num_seqs, block_size, b);
  if (st != NVA_OK) return nva_internal_fail(ctx, st, b.err);
  return upload(ctx, b, num_seqs, false);
}

}  // extern "C"
