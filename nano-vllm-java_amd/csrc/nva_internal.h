// Internal declarations shared by the C-ABI host code and the HIP kernels of libnva.so.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <stdint.h>

#include <algorithm>

namespace nva {

// One unit of the row kernel: one query row attending over the key range [kbeg, kend) of one
// sequence.  Decode rows, qLen == 1 prefill rows and the prefill fallback all use it.  A
// row whose key range is split produces partial (m, l, acc) results at index `part`; an
// unsplit row (part < 0) writes its output directly.
struct RowItem {
  int32_t qrow;   // row of q / out ([T, Hq, D])
  int32_t seq;    // block-table row (paged K/V)
  int32_t kbase;  // dense K/V: row of key 0 in k/v ([T, Hkv, D]); paged: unused
  int32_t kbeg;   // first key (absolute position in the sequence)
  int32_t kend;   // one past the last key
  int32_t part;   // partial-result slot, or -1
  // Paged items within at most two pages: block id of the first page + 1 (0: the kernel stages
  // the item's block ids from the table instead) and of the second page.
  int32_t blk_a, blk_b;
};

// Combines the partials of one split row (nparts >= 2) or zero-fills a row with no visible
// key (nparts == 0), as Attention.java:393-394 gives 0 when l == 0.  Partial maxima are in
// log2 units (scores are scaled by scale * log2(e) in every kernel).
struct MergeItem {
  int32_t qrow;
  int32_t first;
  int32_t nparts;
  int32_t pad;
};

// One segment of the MFMA prefill kernel: a tile of queries of one sequence, for one KV head
// (and a group of its query heads), over the keys [ks, ke).  A workgroup runs the segments of
// its slot one after another (a stream-K schedule: every slot gets the same number of key
// tiles, so a query tile whose keys straddle two slots becomes two segments whose partials are
// merged).
struct TileItem {
  int32_t seq;     // block-table row (paged) / sequence index
  int32_t qstart;  // row of the sequence's first query in q/out
  int32_t qlen;    // queries of the sequence
  int32_t q0;      // first query of this tile (index within the sequence)
  int32_t klen;    // keys of the sequence (kLen in the reference)
  int32_t kbase;   // dense K/V: row of key 0; paged: unused
  int32_t ks;      // first key of this workgroup's key chunk
  int32_t ke;      // one past the last key of the chunk
  int32_t part;    // partial-result base of a split tile, or -1 (whole key range: write out)
  int32_t nsplit;  // key chunks the tile is split into
  int32_t split;   // this chunk's index
  int32_t pad;
};

struct KvView {
  const float *k;        // paged: cache base; dense: k input base
  const float *v;
  const int32_t *table;  // block tables (paged) or nullptr (dense)
  int32_t bt_stride;
  int32_t block_size;
  int32_t bs_shift;      // log2(block_size) when a power of two, else -1
  int32_t paged;
};

struct RowLaunch {
  const float *q;
  float *out;
  KvView kv;
  const RowItem *items;
  int32_t num_items;
  int32_t hq, hkv, head_dim;
  float scale;
  float *part_m, *part_l, *part_acc;  // [P, Hq], [P, Hq], [P, Hq, D]
  int32_t mfma = 0;  // the planner chose the MFMA row kernel (row_mfma_supports, 5-16 heads)
  // XCD of the last workgroup of the kernel launched before this one on the stream (written by
  // that kernel), from which the launch picks the KV head of each workgroup; see xcd_hint in
  // RopeStoreLaunch.  rotate_heads: 2, 4 or 8 KV heads, d = 64 or 128, one workgroup per KV
  // head of an item.
  const int32_t *xcd_hint = nullptr;
  int32_t rotate_heads = 0;
};

struct MergeLaunch {
  float *out;
  const MergeItem *items;
  int32_t num_items;
  int32_t hq, head_dim;
  const float *part_m, *part_l, *part_acc;
};

struct TileLaunch {
  const float *q;
  float *out;
  KvView kv;
  const TileItem *items;     // segments, grouped by slot
  const int32_t *seg_off;    // [num_slots + 1]: slot s runs items [seg_off[s], seg_off[s+1])
  int32_t num_items;
  int32_t num_slots;         // workgroups along x (each runs its slot's segments in order)
  int32_t hq, hkv, head_dim;
  int32_t window;  // 0 = none
  float scale;
  float *part_m, *part_l, *part_acc;  // split tiles: [P, Hq], [P, Hq], [P, Hq, D]
};

// RMSNorm of every head row of one tensor (RMSNorm.forward over [T*H, d], Ops.java:444-500).
struct HeadNorm {
  const float *weight;  // [d], or null: weightless (identity gain)
  float eps;
  int32_t enabled;
  int32_t one_plus;     // apply (1 + w)
  int32_t pad;
};

struct RopeStoreLaunch {
  const float *q, *k, *v;     // inputs [T, hq, d], [T, hk, d], [T, hk, d]; k/v may be null
  float *q_out, *k_out;       // rotated outputs (k_out may be null)
  float *v_out;               // normalised v [T, hk, d] (only with a v norm; may be null)
  float *k_cache, *v_cache;   // store targets (null: no store)
  const int32_t *slots;       // [T] or null
  const int32_t *positions;   // [T] rounded, validated positions (null: no rotation)
  const float *cos_sin;       // [max_pos, d]
  int32_t tokens, hq, hk, head_dim;
  HeadNorm qn, kn, vn;        // per-head RMSNorm applied to q, k, v before rotation / store
  int32_t iters_per_wg;       // row kernel: row iterations per workgroup (set by the launcher)
  int32_t q_ld, k_ld, v_ld;   // floats per token of the q, k, v inputs (0: hq*d, hk*d, hk*d)
  // When non-null, the launch's last workgroup writes the id of the XCD it ran on here.  The
  // hardware hands consecutive workgroups to the 8 XCDs in turn, continuing across launches, so
  // the next launch's first workgroup lands on the XCD after it; the decode launch that follows
  // uses that to pair XCDs with KV heads (any value gives the same results).
  int32_t *xcd_hint;
};

// Standalone RMSNorm over rows of any width (RMSNorm.forward).
struct NormLaunch {
  const float *x;
  float *out;
  HeadNorm norm;
  int32_t rows, width;
};

// y[m, n] = x[m, k] w[n, k]^T (+ bias) with K split over `splits` slices of k_per_split.
struct LinearLaunch {
  const float *x, *w, *bias;
  float *y;
  float *part;  // [splits, m, n] partial sums when splits > 1
  int32_t m, n, k;
  int32_t splits, k_per_split;
};

struct GatherLaunch {
  const float *k_cache, *v_cache;
  float *k_out, *v_out;       // [T, hk, d]
  const int32_t *slots;
  int32_t tokens, row;        // row = hk * d floats
};

// Kernel launchers (each returns the hipGetLastError() of its launch).
hipError_t launch_rope_store(const RopeStoreLaunch &a, hipStream_t s, int num_cus);
hipError_t launch_rms_norm(const NormLaunch &a, hipStream_t s);
// LDS bytes the fused kernel needs for its head norms (0 when no norm is enabled).
size_t rope_store_norm_lds(const RopeStoreLaunch &a);
constexpr size_t kRopeNormMaxLds = 64 * 1024;
hipError_t launch_gather(const GatherLaunch &a, hipStream_t s);
hipError_t launch_zero(float *out, size_t n, hipStream_t s);
hipError_t launch_linear(const LinearLaunch &a, hipStream_t s);
// Weight-streaming GEMV for at most linear_gemv_max_rows() rows (no split, no partials).
hipError_t launch_gemv(const LinearLaunch &a, hipStream_t s);
// 32 x 32 blocks of y, one per workgroup, K split over the workgroup's linear_skinny_waves()
// waves; runs the reduce when splits > 1.
hipError_t launch_skinny(const LinearLaunch &a, hipStream_t s);

int linear_skinny_waves();
// 16 x 16 blocks, one per workgroup, K over its waves, no slices (a.splits must be 1).
hipError_t launch_skinny16(const LinearLaunch &a, hipStream_t s);
int linear_gemv_max_rows();
int linear_tile_rows();
int linear_tile_cols();
int linear_k_tile();
hipError_t launch_row_attention(const RowLaunch &a, int heads_per_wg, hipStream_t s);
hipError_t launch_merge(const MergeLaunch &a, int max_parts, hipStream_t s);
hipError_t launch_prefill_tiles(const TileLaunch &a, int heads_per_wg, hipStream_t s);

// Shapes the kernels are instantiated for.
bool row_kernel_supports(int head_dim, int heads_per_wg);
// Most query heads one row-kernel workgroup carries at this head dim (register budget).
int row_kernel_max_heads(int head_dim);
// The planner gives rows whose workgroups carry kRowMfmaMinHeads..kRowMfmaMaxHeads query heads
// of one KV head to the MFMA row kernel where it is built: d = 64 or 128, paged K/V with
// power-of-two pages of at least 16 tokens.  (From 5 heads per KV head it reads at 6.4-6.5 TB/s
// for any head count, where the row kernel falls to 5.3 TB/s at 8; at 3-4 heads the row kernel
// is as fast.)  Rows beside MFMA prefill tiles keep the row kernel when it covers the heads.
constexpr int kRowMfmaMinHeads = 5;
constexpr int kRowMfmaMaxHeads = 16;
bool row_mfma_supports(int head_dim, int paged, int block_size);
bool prefill_kernel_supports(int head_dim, int heads_per_wg);
// Prefill workgroups that can be resident on one CU at once (occupancy of the kernel), queried
// on the current device each call (callers cache it per device).
int prefill_blocks_per_cu(int head_dim, int heads_per_wg);

// Most pages one prefill key chunk may span (its block ids are staged in LDS).
constexpr int kPrefillTablePages = 128;
// Most pages one row-kernel work item may span (its block ids are staged in LDS).
constexpr int kRowTablePages = 64;
// Most partials per row that launch_merge folds with its row-wide kernel (one workgroup per
// query row, all heads) when a plan has many merge rows; rows with more take the per-(row,
// head) merge.
constexpr int kMergeRowsMaxParts = 8;

// Waves per prefill workgroup at this head dim (each wave owns 16 queries of one head; at
// d = 512 a pair of waves shares them, one half of the head dims each).
int prefill_waves(int head_dim);
// Most query heads one prefill workgroup carries at this head dim.
int prefill_max_heads(int head_dim);
// Query rows per prefill workgroup for a given heads-per-workgroup choice.
int prefill_tile_queries(int head_dim, int heads_per_wg);

}  // namespace nva
