/*
 * nva.h -- C ABI of the MI355X (gfx950) paged-attention library for nano-vllm-java.
 *
 * The library replaces the bodies of the reference's attention boundary:
 *   RotaryEmbedding.forward(positions, q, k, ctx)   layers/Norms.java:275-346
 *   Attention.forward(q, k, v, ctx)                  layers/Attention.java:152-171
 * and owns the state those methods read:
 *   KvCacheArena (per-layer K/V pages)               engine/KvCacheArena.java:63-142
 *   Context.set (per-step varlen / paging metadata)  internal/Context.java:39-59
 * (reference paths are relative to nano-vllm-java/src/main/java/com/igormaznitsa/nanollvm/).
 *
 * Conventions
 *   - Every function returns an nva_status; 0 is success.  nva_last_error() returns the
 *     message of the last failure on a context (the text the Java exception would carry).
 *   - Tensor arguments (q, k, v, outputs) are DEVICE pointers to row-major fp32 arrays:
 *     q/out [tokens, num_heads, head_dim], k/v [tokens, num_kv_heads, head_dim].
 *     Step metadata (cu_seqlens, slots, tables, positions) are HOST pointers; they are copied
 *     to the device once per nva_step_set() and shared by every layer of that step.
 *   - A forward call with num_tokens == 0 (or rows == 0) does nothing and succeeds; its tensor
 *     pointers may then be NULL (the reference returns an empty tensor).
 *   - All work is enqueued on the context's HIP stream and is asynchronous unless stated.
 *   - A context is used by one host thread at a time (the reference's single generate thread,
 *     Attention.java:41-44); there is no internal locking.  Its calls share its device buffers
 *     (plans, split partials), so their work must run in order on the device: after
 *     nva_ctx_set_stream() to a stream not ordered with the previous one, synchronise before
 *     the next call.
 *   - There is no CPU fallback: nva_ctx_create() fails with NVA_E_HIP when no HIP device is
 *     usable.
 */
#ifndef NVA_H
#define NVA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t nva_status;

enum {
  NVA_OK = 0,
  NVA_E_ARG = 1,        /* bad argument (Java: IllegalArgumentException) */
  NVA_E_LAYER = 2,      /* layer index out of range, KvCacheArena.java:136-142 */
  NVA_E_ROPE_POS = 3,   /* RoPE position outside [0, maxPos), Norms.java:318-322 */
  NVA_E_SHARED_KV = 4,  /* shared-KV layer without slots or tables, Attention.java:189-191 */
  NVA_E_NO_ARENA = 5,   /* no KV arena bound (Java: NullPointerException), Attention.java:153 */
  NVA_E_NO_STEP = 6,    /* no step metadata set (Java: NullPointerException on Context) */
  NVA_E_HIP = 7,        /* HIP runtime error or no usable device */
  NVA_E_OOM = 8,        /* device or pinned allocation failed */
  NVA_E_UNSUPPORTED = 9 /* shape this build has no kernel for (e.g. head_dim % 4 != 0) */
};

typedef struct nva_ctx nva_ctx;
typedef struct nva_kv nva_kv;
typedef struct nva_rope nva_rope;

/* Constructor arguments of Attention(numHeads, headDim, scale, numKvHeads, slidingWindow,
 * kvLayerIndex, writeKv), Attention.java:108-125.  sliding_window <= 0 means full context. */
typedef struct nva_attn_desc {
  int32_t num_heads;
  int32_t head_dim;
  float scale;
  int32_t num_kv_heads;
  int32_t sliding_window;
  int32_t kv_layer_index;
  int32_t write_kv;
} nva_attn_desc;

/* RMSNorm(weight, eps, onePlusWeight) and RMSNorm.weightless(eps), layers/Norms.java:32-97.
 * weight is a DEVICE pointer to [width] fp32 (the model's resident norm weight), or NULL for
 * the weightless norm (identity gain).  one_plus_weight applies (1 + w) (Gemma 3). */
typedef struct nva_rms_norm {
  const float *weight;
  float eps;
  int32_t one_plus_weight;
} nva_rms_norm;

/* ------------------------------------------------------------------ context
 * Replaces the per-LLM engine objects that Transformer builds and closes
 * (engine/Transformer.java:113-143, 257-271). */
nva_status nva_ctx_create(int device, nva_ctx **out);
nva_status nva_ctx_destroy(nva_ctx *ctx);
/* Use an external HIP stream (hipStream_t) for all later work; NULL selects the device's
 * null stream (HIP's stream 0, torch's default stream).  Until this is called a context uses
 * its own stream, a blocking stream: work on it is ordered with work on the null stream
 * (hipMemcpy), so outputs may be copied out with hipMemcpy without nva_ctx_sync().  The
 * caller keeps an external stream alive while it is set; nva_ctx_stream() returns the
 * current one (save it first to restore it later). */
nva_status nva_ctx_set_stream(nva_ctx *ctx, void *hip_stream);
void *nva_ctx_stream(nva_ctx *ctx);
/* Blocks until all work enqueued on the context's stream has finished. */
nva_status nva_ctx_sync(nva_ctx *ctx);
const char *nva_last_error(nva_ctx *ctx);
const char *nva_status_string(nva_status status);
/* Per-kernel timing with HIP events on the context's stream (off by default).  Kernel names:
 * "rope_store", "store", "decode", "merge", "prefill", "gather", "linear", "rms_norm";
 * "attention" spans the attention kernels of one call (decode and prefill kernels that
 * overlap count once).  Host-side entries: "plan" (building a step's work plan on the host, once
 * per step and attention configuration, at its first layer) and "plan_upload" (copying it to
 * the device).  The name "device_bytes" instead returns in *launches the bytes of device memory
 * the context's grow-only work buffers hold (arenas and RoPE tables excluded). */
nva_status nva_ctx_set_timing(nva_ctx *ctx, int enable);
nva_status nva_ctx_kernel_stats(nva_ctx *ctx, const char *kernel, int64_t *launches,
                                double *total_ms);
nva_status nva_ctx_reset_stats(nva_ctx *ctx);

/* ------------------------------------------------------------------ KV arena
 * KvCacheArena(numBlocks, blockSize, numKvHeads, headDims[], allocateLayer[]),
 * KvCacheArena.java:63-90.  Each allocated layer owns zero-filled device buffers
 * K and V of shape [num_blocks, block_size, num_kv_heads, head_dims[layer]] fp32 (slot s is
 * block*block_size + offset, exactly the reference's layout).  allocate == NULL allocates every
 * layer; allocate[i] == 0 gives that layer no pages (the reference's numel-1 dummy). */
nva_status nva_kv_create(nva_ctx *ctx, int num_layers, int num_blocks, int block_size,
                         int num_kv_heads, const int32_t *head_dims, const uint8_t *allocate,
                         nva_kv **out);
/* KvCacheArena.close(), KvCacheArena.java:130-134: frees the device pages. */
nva_status nva_kv_destroy(nva_kv *kv);
/* The heap cap of Config.resolveNumKvcacheBlocks (llm/Config.java:93-125) with the device's free
 * HBM (hipMemGetInfo on the context's device, at the call) in place of
 * Runtime.getRuntime().maxMemory(): *blocks = max(32, floor(free * fraction / bytes_per_block)),
 * capped at INT32_MAX, where bytes_per_block = 2 * block_size * num_kv_heads * head_dims[l] * 4
 * summed over the layers that get pages (allocate == NULL: every layer; the reference skips
 * shared-KV layers the same way).  A query only: nothing is allocated.  The caller takes
 * min(estimated, *blocks) exactly as the reference does with its heap cap, then passes the
 * result to nva_kv_create.  fraction must be in (0, 1] (kvHeapFraction's range, Config.java:66-69);
 * *free_bytes (may be NULL) receives the free HBM the cap was computed from. */
nva_status nva_kv_blocks_that_fit(nva_ctx *ctx, int num_layers, int block_size, int num_kv_heads,
                                  const int32_t *head_dims, const uint8_t *allocate,
                                  float fraction, int *blocks, int64_t *free_bytes);
/* getKeyCache/getValueCache(layer), KvCacheArena.java:111-124: device pointers and the byte
 * size of each buffer (0 and NULL for an unallocated layer).  NVA_E_LAYER if out of range. */
nva_status nva_kv_layer(nva_kv *kv, int layer, void **key, void **value, int64_t *bytes);
/* Synchronous host<->device copies of a float range of one layer's K (which=0) or V
 * (which=1) buffer, for callers that inspect or pre-fill pages (Tensor.data() access). */
nva_status nva_kv_write(nva_kv *kv, int layer, int which, int64_t float_offset,
                        const float *host, int64_t count);
nva_status nva_kv_read(nva_kv *kv, int layer, int which, int64_t float_offset, float *host,
                       int64_t count);

/* ------------------------------------------------------------------ RoPE tables
 * RotaryEmbedding's [maxPos, headSize] cos|sin table, Norms.java:171-191.
 * nva_rope_create uploads the caller's own table (the Java table, so the bits are identical by
 * construction); nva_rope_create_theta builds it on the host with the reference's arithmetic
 * (invFreq = (float)(1/pow(base, 2i/d)); angle = (float)pos*invFreq as double; cos/sin cast to
 * float), Norms.java:183-204. */
nva_status nva_rope_create(nva_ctx *ctx, const float *cos_sin, int max_pos, int head_size,
                           nva_rope **out);
nva_status nva_rope_create_theta(nva_ctx *ctx, int head_size, int rotary_dim, int max_pos,
                                 float base, nva_rope **out);
nva_status nva_rope_destroy(nva_rope *rope);

/* ------------------------------------------------------------------ step metadata
 * Context.set(isPrefill, cuSeqlensQ, cuSeqlensK, maxSeqlenQ, maxSeqlenK, slotMapping,
 * contextLens, blockTables, seqIds), Context.java:39-59, plus the step's positions tensor
 * (Transformer.java:149-155).  Host arrays, copied to the device in one transfer:
 *   cu_q, cu_k       [num_seqs+1]  prefill only (NULL for decode)
 *   slot_mapping     [num_slots]   may be NULL (then the store is skipped, Attention.java:157)
 *   context_lens     [num_seqs]    decode only (NULL for prefill)
 *   block_tables     [num_seqs * bt_stride], -1 padded; NULL = no tables (dense prefill)
 *   seq_ids          [num_tokens]  optional, kept for the caller
 *   positions        [num_tokens]  fp32 positions, rounded like Math.round; may be NULL when
 *                                  RoPE is not used this step
 * For decode, num_seqs is the number of rows (one query token per sequence). */
nva_status nva_step_set(nva_ctx *ctx, int is_prefill, const int32_t *cu_q, const int32_t *cu_k,
                        int num_seqs, int max_seqlen_q, int max_seqlen_k,
                        const int32_t *slot_mapping, int num_slots,
                        const int32_t *context_lens, const int32_t *block_tables,
                        int bt_stride, const int32_t *seq_ids, const float *positions,
                        int num_tokens);
/* One scheduled sequence as the model runner sees it (engine/Sequence.java): host arrays.
 *   num_tokens         Sequence.numTokens(): every token of the sequence so far
 *   num_cached_tokens  prefill: tokens already in the pages (numCachedTokens)
 *   num_scheduled      prefill: tokens of this step's chunk (numScheduledTokens)
 *   block_table        the sequence's block ids (blockTable()), num_blocks entries */
typedef struct nva_seq {
  int32_t seq_id;
  int32_t num_tokens;
  int32_t num_cached_tokens;
  int32_t num_scheduled;
  const int32_t *block_table;
  int32_t num_blocks;
} nva_seq;

/* Step metadata as Context.set receives it, in caller-owned host arrays:
 *   cu_q, cu_k        [num_seqs + 1]   (prefill)
 *   slot_mapping      [tokens]         num_slots entries are written
 *   context_lens      [num_seqs]       (decode)
 *   seq_ids           [tokens]
 *   positions         [tokens]         fp32, as the step's positions tensor
 *   block_tables      [num_seqs * max(num_blocks)], -1 padded; bt_stride = max(num_blocks);
 *                     has_tables = 0 when the reference attaches none (prefill with no cached
 *                     prefix) */
typedef struct nva_step_meta {
  int32_t *cu_q, *cu_k;
  int32_t max_seqlen_q, max_seqlen_k;
  int32_t *slot_mapping;
  int32_t num_slots;
  int32_t *context_lens;
  int32_t *seq_ids;
  float *positions;
  int32_t num_tokens;
  int32_t *block_tables;
  int32_t bt_stride;
  int32_t has_tables;
} nva_step_meta;

/* Transformer.preparePrefill, engine/Transformer.java:342-418 (with prepareBlockTables,
 * :319-330): for each sequence the window [numCachedTokens, numCachedTokens + numScheduled)
 * gives positions, seq ids, cu_seqlens (Q: new tokens, K: full context through the window end)
 * and the slot of every new token in the sequence's pages (a sequence with an empty block table
 * adds no slots); block tables are attached only when cu_k.last > cu_q.last and some sequence
 * has a table.  Pure host code (no device, no context).  NVA_E_ARG where Java would throw
 * (a block table too short for the window). */
nva_status nva_build_prefill_metadata(const nva_seq *seqs, int num_seqs, int block_size,
                                      nva_step_meta *out);
/* Transformer.prepareDecode, engine/Transformer.java:427-456: one row per sequence with
 * position numTokens - 1, context length numTokens, and the slot
 * blockTable.last * blockSize + lastBlockNumTokens - 1 (Sequence.java:323-335); block tables
 * always attached.  NVA_E_ARG for an empty block table (Java: NoSuchElementException). */
nva_status nva_build_decode_metadata(const nva_seq *seqs, int num_seqs, int block_size,
                                     nva_step_meta *out);
/* The two producers above followed by nva_step_set: the per-step metadata of a scheduler step
 * built on the host and uploaded in one transfer. */
nva_status nva_step_prepare_prefill(nva_ctx *ctx, const nva_seq *seqs, int num_seqs,
                                    int block_size);
nva_status nva_step_prepare_decode(nva_ctx *ctx, const nva_seq *seqs, int num_seqs,
                                   int block_size);

/* Replaces the step's positions only (the positions tensor RotaryEmbedding.forward receives,
 * Norms.java:275, rounded with Math.round as at Norms.java:317).  Valid after nva_step_set. */
nva_status nva_step_positions(nva_ctx *ctx, const float *positions, int num_tokens);
/* Context.clear(), Context.java:61-74. */
nva_status nva_step_clear(nva_ctx *ctx);

/* ------------------------------------------------------------------ compute
 * RotaryEmbedding.forward(positions, q, k, ctx), Norms.java:275-346: q_out/k_out receive the
 * rotated q [tokens, hq, d] and k [tokens, hk, d].  Positions come from nva_step_set().
 * NVA_E_ROPE_POS if a rounded position is outside [0, max_pos) (no work is enqueued then). */
nva_status nva_rope_forward(nva_ctx *ctx, const nva_rope *rope, const float *q, const float *k,
                            int num_tokens, int hq, int hk, float *q_out, float *k_out);

/* Attention.forward(q, k, v, ctx), Attention.java:152-171: store k/v into the layer's pages
 * at the step's slots (when write_kv, the layer is allocated and num_slots == num_tokens;
 * negative slots skipped), then dense prefill, paged prefill (block tables present) or
 * decode, writing out [num_tokens, num_heads, head_dim].  Shared-KV layers (write_kv == 0)
 * read layer kv_layer_index without storing. */
nva_status nva_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc *desc,
                                 const float *q, const float *k, const float *v, int num_tokens,
                                 float *out);

/* nva_attention_forward without any allocation.  It has no counterpart in the reference: it is
 * for callers that cannot allocate device memory while they run attention (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * semantics and kernels as nva_attention_forward, and bit-identical results; the plan lists,
 * split partials and shared-KV gather rows go into a static device array of this library
 * (NVA_NOALLOC_SCRATCH_BYTES = 128 MiB, one per device, held until the process ends) instead of
 * the context's grow-only buffers, and the call makes no hipMalloc, hipFree or other allocating
 * call.  A step whose plan, partials and gathered rows need more than that fails with NVA_E_ARG
 * and a message giving the bytes needed.  Every call on a device shares that device's array and
 * it keeps the last call's contents: calls that overlap on one device (several host threads or
 * contexts, or streams not ordered with each other) race and must be serialised by the caller.
 * The step metadata still comes from nva_step_set(), whose buffers grow (allocate) when a step
 * is larger than every earlier one on the context. */
#define NVA_NOALLOC_SCRATCH_BYTES (128u << 20)
nva_status nva_attention_forward_noalloc(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc *desc,
                                         const float *q, const float *k, const float *v,
                                         int num_tokens, float *out);

/* The pair RotaryEmbedding.forward + Attention.forward as one call, the way the model layers
 * use them (models/internal/Qwen3ForCausalLM.java:207-222): one fused kernel rotates q and k
 * and stores rotated k and v into the pages, then the attention kernels run.  q_out/k_out
 * may be NULL (context-owned scratch is used).  Results are identical to calling the two
 * functions above in sequence. */
nva_status nva_rope_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                      const nva_attn_desc *desc, const float *q,
                                      const float *k, const float *v, int num_tokens,
                                      float *q_out, float *k_out, float *out);

/* RMSNorm.forward(x), layers/Norms.java:91-96 -> Ops.rmsNorm, tensor/Ops.java:444-500, over
 * x [rows, width] (device) into out [rows, width] (device; may equal x).  The sum of squares
 * follows ScalarFloatKernels.sumSquares (scalar/ScalarFloatKernels.java:55-70) bit for bit;
 * inv = (float)(1.0 / Math.sqrt(sum / width + eps)) in double. */
nva_status nva_rms_norm_forward(nva_ctx *ctx, const nva_rms_norm *norm, const float *x, int rows,
                                int width, float *out);

/* Linear.Row.forward (o_proj), models/internal/Qwen3ForCausalLM.java:221 -> Ops.linear,
 * tensor/Ops.java:84-124 -> MatmulRuntime.linear, tensor/MatmulRuntime.java:234-255:
 * y[rows, out] = x[rows, in] weight[out, in]^T (+ bias[out]).  x, weight, bias and y are
 * DEVICE pointers (x and weight 16-byte aligned, in % 4 == 0); bias may be NULL.  x is
 * typically the attention output [tokens, num_heads * head_dim] used in place (in < 4194304).
 * fp32 on MFMA; the sum order differs from the reference's gemv panels (fp32 rounding only).
 * Up to 16 rows run the library's weight-streaming GEMV, batches whose 32 x 32 output blocks fit
 * one per CU its 16 x 16- or 32 x 32-block kernels, and larger GEMMs its 128 x 64-tile kernel. */
nva_status nva_linear_forward(nva_ctx *ctx, const float *x, int rows, int in,
                              const float *weight, int out, const float *bias, float *y);

/* The per-head q/k (and Gemma 4 v) RMSNorm, RotaryEmbedding.forward and Attention.forward as
 * one call, the way the model layers chain them (Qwen3Attention.forward,
 * models/internal/Qwen3ForCausalLM.java:207-227 normHeads; Gemma3ForCausalLM.java:143-157;
 * Gemma4ForCausalLM.java:164-197 with its weightless v norm): one fused kernel normalises each
 * head row, rotates q and k, and stores rotated k and normalised v into the pages; then the
 * attention kernels run.  q_norm / k_norm / v_norm may each be NULL (no norm on that tensor).
 * q_out/k_out (may be NULL) receive the normalised, rotated q and k.  Results are identical to
 * nva_rms_norm_forward on each head row, then nva_rope_attention_forward. */
nva_status nva_norm_rope_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                           const nva_rms_norm *q_norm,
                                           const nva_rms_norm *k_norm,
                                           const nva_rms_norm *v_norm,
                                           const nva_attn_desc *desc, const float *q,
                                           const float *k, const float *v, int num_tokens,
                                           float *q_out, float *k_out, float *out);

/* The same, reading q, k and v from the packed qkv_proj output qkv [num_tokens,
 * (num_heads + 2 * num_kv_heads) * head_dim] -- per token the q heads, then the k heads, then
 * the v heads -- which the model layers split with Ops.splitLast before normHeads and RoPE
 * (models/internal/Qwen3ForCausalLM.java:210-214, Gemma3ForCausalLM.java:144-148,
 * LlamaForCausalLM.java:144-148).  The kernels read the packed rows in place, so no split copy is made.  Results are
 * identical to nva_norm_rope_attention_forward on the split tensors. */
nva_status nva_qkv_norm_rope_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                               const nva_rms_norm *q_norm,
                                               const nva_rms_norm *k_norm,
                                               const nva_rms_norm *v_norm,
                                               const nva_attn_desc *desc, const float *qkv,
                                               int num_tokens, float *q_out, float *k_out,
                                               float *out);

#ifdef __cplusplus
}
#endif

#endif /* NVA_H */
