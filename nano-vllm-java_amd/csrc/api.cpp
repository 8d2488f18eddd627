// C ABI of libnva.so: contexts, the device KV arena, per-step metadata upload, work planning
// and the Attention.forward / RotaryEmbedding.forward dispatch.  See include/nva.h.
//
// Host-side restatements (reference paths relative to
// nano-vllm-java/src/main/java/com/igormaznitsa/nanollvm/):
//   Attention.forward dispatch and store rule   layers/Attention.java:152-171
//   attendFromCache / gatherKvCache             layers/Attention.java:176-216
//   kLen and query offsets per branch           layers/Attention.java:245-299, 353-358
//   Math.round of positions and range check     layers/Norms.java:316-322
//   RoPE table arithmetic                       layers/Norms.java:183-204
//   KvCacheArena shapes and layer check         engine/KvCacheArena.java:63-142
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/nva.h"
#include "nva_internal.h"

using namespace nva;

// Device scratch of nva_attention_forward_noalloc: the plan lists, split partials and shared-KV
// gather rows of one call.  One copy per device, held from the library's load on that device
// until the process ends.  Host code never uses the name `scratch` as an address (on the host it
// is only a stand-in for the symbol): nva_ctx_create looks up each device's address once with
// hipGetSymbolAddress, and every later use goes through that address.  Nothing in it has to
// start at zero: every partial is written before the merge reads it, and the plan lists and
// gather rows are written by the call that reads them.
namespace {
constexpr size_t kScratchBytes = NVA_NOALLOC_SCRATCH_BYTES;
constexpr int kScratchDevices = 64;
}  // namespace
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// The scratch plan held by one device's array, so a call can skip copying the same plan again.
struct ScratchTag {
  uint64_t plan_id = 0;  // 0: no plan known to be held
  size_t offset = 0, bytes = 0;
};

// Per device: its address of `scratch` (looked up once, under the mutex, with that device
// current) and the tag of the plan it holds.
struct ScratchSlot {
  bool looked_up = false;
  hipError_t err = hipSuccess;
  char *ptr = nullptr;
  ScratchTag tag;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kScratchDevices];

// Called by nva_ctx_create with `device` current.
char *scratch_address(int device, hipError_t *err) {
  if (device < 0 || device >= kScratchDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot &slot = g_scratch[device];
  if (!slot.looked_up) {
    void *p = nullptr;
    slot.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    slot.ptr = slot.err == hipSuccess ? static_cast<char *>(p) : nullptr;
    slot.looked_up = true;
  }
  *err = slot.err;
  return slot.ptr;
}

ScratchTag &scratch_tag(int device) { return g_scratch[device].tag; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }


// Grow-only device buffer.
struct DevBuf {
  void *ptr = nullptr;
  size_t cap = 0;
  hipError_t reserve(size_t bytes) {
    if (bytes <= cap) return hipSuccess;
    if (ptr) {
      hipError_t e = hipFree(ptr);
      if (e != hipSuccess) return e;
      ptr = nullptr;
      cap = 0;
    }
    size_t want = std::max<size_t>(bytes, 4096);
    hipError_t e = hipMalloc(&ptr, want);
    if (e == hipSuccess) cap = want;
    return e;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
};

// Grow-only pinned host buffer whose last upload is tracked by an event, so it is only
// overwritten once the device has consumed it.
struct Staging {
  void *ptr = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
  hipError_t wait() {
    if (pending) {
      pending = false;
      return hipEventSynchronize(done);
    }
    return hipSuccess;
  }
  hipError_t reserve(size_t bytes) {
    hipError_t e = wait();
    if (e != hipSuccess) return e;
    if (!done) {
      e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
      if (e != hipSuccess) return e;
    }
    if (bytes <= cap) return hipSuccess;
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    cap = 0;
    size_t want = std::max<size_t>(bytes, 4096);
    e = hipHostMalloc(&ptr, want, hipHostMallocDefault);
    if (e == hipSuccess) cap = want;
    return e;
  }
  hipError_t upload(DevBuf &dst, size_t bytes, hipStream_t s) {
    hipError_t e = hipMemcpyAsync(dst.ptr, ptr, bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return e;
    e = hipEventRecord(done, s);
    if (e == hipSuccess) pending = true;
    return e;
  }
  void release() {
    if (pending) (void)hipEventSynchronize(done);
    pending = false;
    if (ptr) (void)hipHostFree(ptr);
    if (done) (void)hipEventDestroy(done);
    ptr = nullptr;
    done = nullptr;
    cap = 0;
  }
};

// A work plan: the flattened row / merge / tile lists for one attention configuration of the
// current step, built on the host and uploaded once, then reused by every layer with the same
// configuration.
struct PlanKey {
  int window, mfma, tile_q, wg_per_item, blocks_per_cu;
  int tile_groups;             // prefill grid height: KV heads x query-head groups
  int tokens;                  // rows of q / out in the forward call
  int paged;                   // keys through block tables (else dense k/v rows)
  int block_size, num_blocks;  // arena geometry the tables are checked against
  int head_dim, num_heads, num_kv_heads;  // size the work of a mixed plan's two kernels
  bool operator==(const PlanKey &o) const {
    return window == o.window && mfma == o.mfma && tile_q == o.tile_q &&
           head_dim == o.head_dim && num_heads == o.num_heads && num_kv_heads == o.num_kv_heads &&
           wg_per_item == o.wg_per_item && blocks_per_cu == o.blocks_per_cu &&
           tile_groups == o.tile_groups && tokens == o.tokens && paged == o.paged &&
           block_size == o.block_size && num_blocks == o.num_blocks;
  }
};

struct Plan {
  PlanKey key{};
  bool valid = false;
  int num_rows = 0, num_merge = 0, num_tiles = 0, num_parts = 0;
  int num_slots = 0;  // prefill stream-K slots (grid x)
  int max_parts = 0;  // most partials any merged row has
  bool covers_all = true;  // every output row is written by some kernel
  size_t off_rows = 0, off_merge = 0, off_tiles = 0, off_slots = 0;
  std::vector<char> host;  // the packed lists at the offsets above
  uint64_t id = 0;         // unique per build (identifies the plan held in a scratch array)
  bool on_device = false;  // host bytes uploaded to dev
  DevBuf dev;
  Staging stage;
};

// Workspace of the no-allocation entry point: the plan, the split partials and the shared-KV
// gather rows of one call live in fixed regions of a device's static scratch array instead of
// the context's grow-only buffers.  base is that device's address of the array (from
// hipGetSymbolAddress), used == bytes already taken (gather rows, at the front).
struct Scratch {
  char *base = nullptr;
  size_t used = 0;
};

struct PendingTiming {
  std::string name;
  hipEvent_t start, stop;
};

struct KernelStat {
  int64_t launches = 0;
  double ms = 0.0;
};

}  // namespace

struct nva_ctx {
  int device = 0;
  int num_cus = 256;
  hipStream_t own_stream = nullptr;
  hipStream_t side_stream = nullptr;  // decode rows of a mixed step run here, beside the tiles
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  hipStream_t stream = nullptr;
  std::string err;

  // Step metadata (host copies) and its device mirror.
  bool has_step = false;
  bool is_prefill = false;
  int num_seqs = 0;
  int num_tokens = 0;
  int max_q = 0, max_k = 0;
  int bt_stride = 0;
  int num_slots = 0;
  int64_t slot_max = -1;  // largest slot of the step (negative slots are skipped)
  bool has_cu = false, has_slots = false, has_ctx_lens = false, has_tables = false,
       has_pos = false;
  std::vector<int32_t> cu_q, cu_k, slots, ctx_lens, tables, seq_ids, pos;
  DevBuf d_step;
  Staging step_stage;
  size_t off_cu_q = 0, off_cu_k = 0, off_slots = 0, off_ctx = 0, off_tables = 0, off_pos = 0;

  std::vector<Plan *> plans;
  DevBuf d_part;     // split partials
  DevBuf d_q_rot;    // fused path scratch for rotated q
  DevBuf d_k_rot;    // fused path scratch for rotated k
  DevBuf d_v_norm;   // fused path scratch for normalised v (dense prefill with a v norm)
  DevBuf d_lin;      // split-K partial sums of the linear kernel
  DevBuf d_gather;   // shared-KV gather [2, T, Hkv, d]

  // One word the store / RoPE kernel writes the XCD of its last workgroup to, read by the decode
  // launch that follows (null if its allocation failed: no rotation).
  int32_t *xcd_hint = nullptr;

  // This device's address of the no-allocation scratch array (null if the lookup failed).
  char *scratch = nullptr;
  hipError_t scratch_err = hipSuccess;

  // Prefill occupancy (resident workgroups per CU) by (head dim, heads per workgroup), queried
  // once on this context's device.
  std::map<int, int> occupancy;

  bool timing = false;
  std::vector<PendingTiming> pending;
  std::vector<hipEvent_t> event_pool;
  std::map<std::string, KernelStat> stats;

  const int32_t *dev_i32(size_t off) const {
    return reinterpret_cast<const int32_t *>(static_cast<char *>(d_step.ptr) + off);
  }
};

struct nva_kv {
  nva_ctx *ctx = nullptr;
  int num_layers = 0, num_blocks = 0, block_size = 0, num_kv_heads = 0;
  std::vector<int32_t> head_dims;
  std::vector<float *> k, v;
  std::vector<int64_t> bytes;
};

struct nva_rope {
  nva_ctx *ctx = nullptr;
  int max_pos = 0, head_size = 0;
  float *table = nullptr;
};

namespace {

nva_status fail(nva_ctx *ctx, nva_status st, const char *fmt, ...) {
  if (ctx) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    ctx->err = buf;
  }
  return st;
}

nva_status hip_fail(nva_ctx *ctx, hipError_t e, const char *what) {
  return fail(ctx, e == hipErrorOutOfMemory ? NVA_E_OOM : NVA_E_HIP, "%s: %s", what,
              hipGetErrorString(e));
}

#define HIP_TRY(ctx, expr, what)                \
  do {                                          \
    hipError_t e_ = (expr);                     \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, what); \
  } while (0)

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Makes the context's device current for the scope of an entry point (its grow-only buffers
// are allocated, and its occupancy queried, on that device) and restores the caller's.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != device) (void)hipSetDevice(device);
  }
  explicit DeviceGuard(const nva_ctx *ctx) : DeviceGuard(ctx->device) {}
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

int ctx_prefill_blocks_per_cu(nva_ctx *ctx, int head_dim, int hpw) {
  const int key = head_dim * 16 + hpw;
  auto it = ctx->occupancy.find(key);
  if (it != ctx->occupancy.end()) return it->second;
  const int n = prefill_blocks_per_cu(head_dim, hpw);
  ctx->occupancy[key] = n;
  return n;
}

hipEvent_t take_event(nva_ctx *ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Brackets one kernel launch with timing events when timing is on.
struct Timed {
  nva_ctx *ctx;
  const char *name;
  hipStream_t stream;
  hipEvent_t start = nullptr;
  Timed(nva_ctx *c, const char *n, hipStream_t s = nullptr)
      : ctx(c), name(n), stream(s ? s : c->stream) {
    if (ctx->timing) {
      start = take_event(ctx);
      if (start) (void)hipEventRecord(start, stream);
    }
  }
  void done() {
    if (!start) return;
    hipEvent_t stop = take_event(ctx);
    if (!stop) return;
    (void)hipEventRecord(stop, stream);
    ctx->pending.push_back({name, start, stop});
    start = nullptr;
  }
};

void resolve_timings(nva_ctx *ctx) {
  for (auto &p : ctx->pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess &&
        hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      auto &s = ctx->stats[p.name];
      s.launches++;
      s.ms += ms;
    }
    ctx->event_pool.push_back(p.start);
    ctx->event_pool.push_back(p.stop);
  }
  ctx->pending.clear();
}

// Host time of one plan build (and its upload), kept as the "plan" entry of the kernel stats
// when timing is on: the per-step planning cost a scheduler step pays at its first layer.
struct HostTimed {
  nva_ctx *ctx;
  const char *name;
  std::chrono::steady_clock::time_point t0;
  bool on;
  HostTimed(nva_ctx *c, const char *n) : ctx(c), name(n), on(c->timing) {
    if (on) t0 = std::chrono::steady_clock::now();
  }
  ~HostTimed() {
    if (!on) return;
    const double ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    auto &s = ctx->stats[name];
    s.launches++;
    s.ms += ms;
  }
};

int pow2_shift(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int s = 0;
  while ((1 << s) < x) s++;
  return s;
}

int largest_pow2_divisor_upto(int rep, int cap) {
  int h = cap;
  while (h > 1 && rep % h) h >>= 1;
  return h;
}

// CUs for the tile grid of a mixed plan, one tile workgroup on each; the rows run on the other
// CUs and in the room left on the tile CUs.  The tile share f of the CUs minimises the longer of
// the two kernels: the tiles' time scales as 1/f, while the rows, being HBM-bound, keep
// 1 - f^1.8 of the whole chip's bandwidth.  That is below what the rows keep alone on the
// remaining CUs of a CU-masked stream (85% on half of the CUs, 68% on 3/8, 49% on 1/4), since
// beside tile workgroups they lose bandwidth too; for the Qwen3-4B-like mixed step it picks 160
// CUs, the best of a sweep over 128..208.  Solo rates: rows 6.5 TB/s, tiles 100 / 80 / 70
// TFLOP/s at head dim <= 128 / 256 / 512.
int64_t mixed_tile_cus(int num_cus, double row_bytes, double tile_flops, int head_dim) {
  const double tr = row_bytes / 6.5e12;
  const double tt =
      tile_flops / (head_dim <= 128 ? 100e12 : head_dim <= 256 ? 80e12 : 70e12);
  int best_s = 8;
  double best = 1e300;
  for (int s = 1; s < 16; s++) {
    const double f = s / 16.0;
    const double t = std::max(tr / (1.0 - std::pow(f, 1.8)), tt / f);
    if (t < best) {
      best = t;
      best_s = s;
    }
  }
  return (int64_t)num_cus * best_s / 16;
}

// One query row of the row kernel before splitting.
struct Row {
  int qrow, seq, kbase, kbeg, kend;
};

// Builds (or reuses) the host lists of the plan for this configuration of the current step;
// upload_plan() or the scratch path puts them on the device.
nva_status get_plan(nva_ctx *ctx, const PlanKey &key, Plan **out) {
  for (Plan *p : ctx->plans)
    if (p->valid && p->key == key) {
      *out = p;
      return NVA_OK;
    }
  HostTimed host_timer(ctx, "plan");
  Plan *plan = nullptr;
  for (Plan *p : ctx->plans)
    if (!p->valid) {
      plan = p;
      break;
    }
  if (!plan) {
    plan = new Plan();
    ctx->plans.push_back(plan);
  }

  const int W = key.window;
  const bool paged = key.paged != 0;
  std::vector<Row> rows;
  std::vector<TileItem> tiles;
  int covered = 0;
  // Every page a sequence reads must be a real block of the arena: the reference would throw
  // (ArrayIndexOutOfBounds) where a kernel would read out of bounds.
  auto check_pages = [&](int b, int klen) -> nva_status {
    if (klen <= 0) return NVA_OK;
    const int pages = (int)(((int64_t)klen + key.block_size - 1) / key.block_size);
    if (pages > ctx->bt_stride)
      return fail(ctx, NVA_E_ARG, "sequence %d needs %d pages but its block table has %d", b,
                  pages, ctx->bt_stride);
    const int32_t *t = ctx->tables.data() + (size_t)b * ctx->bt_stride;
    for (int j = 0; j < pages; j++)
      if (t[j] < 0 || t[j] >= key.num_blocks)
        return fail(ctx, NVA_E_ARG, "block table %d entry %d = %d is not a block in [0, %d)", b,
                    j, t[j], key.num_blocks);
    return NVA_OK;
  };
  if (!ctx->is_prefill) {
    // Decode, Attention.java:285-299: row b, kLen = contextLens[b], absQ = kLen - 1.
    const int n = key.tokens;
    rows.reserve(n);
    for (int b = 0; b < n; b++) {
      const int klen = ctx->ctx_lens[b];
      nva_status st = check_pages(b, klen);
      if (st != NVA_OK) return st;
      const int aq = klen - 1;
      const int kbeg = W > 0 ? std::max(0, aq - W + 1) : 0;
      rows.push_back({b, b, 0, kbeg, klen});
    }
    covered = n;
  } else {
    // Prefill, Attention.java:245-280: kLen = cuK[b+1]-cuK[b]; query qi at kLen-qLen+qi.
    if (ctx->num_seqs > 0 && ctx->cu_q[ctx->num_seqs] > key.tokens)
      return fail(ctx, NVA_E_ARG, "cuSeqlensQ ends at %d but q has %d rows",
                  ctx->cu_q[ctx->num_seqs], key.tokens);
    if (!paged && ctx->num_seqs > 0 && ctx->cu_k[ctx->num_seqs] > key.tokens)
      return fail(ctx, NVA_E_ARG, "cuSeqlensK ends at %d but k has %d rows",
                  ctx->cu_k[ctx->num_seqs], key.tokens);
    for (int b = 0; b < ctx->num_seqs; b++) {
      const int q0 = ctx->cu_q[b];
      const int qlen = ctx->cu_q[b + 1] - q0;
      const int klen = ctx->cu_k[b + 1] - ctx->cu_k[b];
      const int kbase = paged ? 0 : ctx->cu_k[b];
      if (qlen <= 0) continue;
      if (paged) {
        nva_status st = check_pages(b, klen);
        if (st != NVA_OK) return st;
      }
      covered += qlen;
      if (key.mfma && qlen >= 2 && klen >= qlen) {
        for (int t0 = 0; t0 < qlen; t0 += key.tile_q) {
          const int t1 = std::min(qlen, t0 + key.tile_q) - 1;
          const int aq0 = klen - qlen + t0, aq1 = klen - qlen + t1;
          TileItem ti;
          ti.seq = b;
          ti.qstart = q0;
          ti.qlen = qlen;
          ti.q0 = t0;
          ti.klen = klen;
          ti.kbase = kbase;
          ti.ks = W > 0 ? std::max(0, aq0 - W + 1) : 0;
          ti.ke = aq1 + 1;
          ti.part = -1;
          ti.nsplit = 1;
          ti.split = 0;
          ti.pad = 0;
          tiles.push_back(ti);
        }
      } else {
        for (int qi = 0; qi < qlen; qi++) {
          const int aq = klen - qlen + qi;
          const int kend = aq + 1;
          const int kbeg = W > 0 ? std::max(0, aq - W + 1) : 0;
          rows.push_back({q0 + qi, b, kbase, kbeg, kend});
        }
      }
    }
  }
  plan->covers_all = covered == key.tokens;

  // Stream-K schedule of the MFMA tiles.  The grid has exactly as many workgroups per head
  // group ("slots") as can be resident at once; the 32-key tiles of all query tiles are cut
  // into equal runs, one per slot, so every slot finishes at the same time.  A query tile whose
  // keys fall into several runs becomes several segments; they write partials (query-major,
  // segment-minor) that the merge kernel combines.  A segment also never spans more pages than
  // the kernel's LDS copy of the block table holds.
  std::vector<MergeItem> merges;
  std::vector<int32_t> seg_off;
  int parts = 0;
  int slots = 0;
  if (!tiles.empty()) {
    constexpr int KT = 32;
    int64_t total = 0;
    for (const TileItem &t : tiles) total += (t.ke - t.ks + KT - 1) / KT;
    // A mixed plan runs its rows on a second stream beside the tiles; the tile grid then has
    // one workgroup on each of a share of the CUs, and the rows take the rest.
    int64_t resident = (int64_t)ctx->num_cus * key.blocks_per_cu;
    if (!rows.empty()) {
      double row_bytes = 0.0, pairs = 0.0;
      for (const Row &r : rows) row_bytes += std::max(0, r.kend - r.kbeg);
      row_bytes *= 8.0 * key.num_kv_heads * key.head_dim;
      for (const TileItem &t : tiles) {
        const int n = std::min(key.tile_q, t.qlen - t.q0);
        for (int i = 0; i < n; i++) {
          const int aq = t.klen - t.qlen + t.q0 + i;
          pairs += W > 0 ? std::min(aq + 1, W) : aq + 1;
        }
      }
      const double flops = 4.0 * key.head_dim * key.num_heads * pairs;
      resident = std::max<int64_t>(key.tile_groups,
                                   mixed_tile_cus(ctx->num_cus, row_bytes, flops, key.head_dim));
    }
    slots = (int)std::max<int64_t>(1, std::min<int64_t>(total, resident / key.tile_groups));
    const int64_t page_cap =
        paged ? (int64_t)(kPrefillTablePages - 2) * key.block_size / KT * KT : INT32_MAX;
    // Two ways to cut the tiles into equal runs; the plan keeps the one that splits fewer
    // query rows (each split row writes and re-reads one partial per segment), unless that one
    // cuts a tile into more segments than the row-wide merge folds:
    //  (a) the query tiles in sequence order, laid end to end, cut at every slot boundary;
    //  (b) tiles longer than a run (cap = ceil(total / slots) key tiles) first, largest first,
    //      each filling whole empty slots and its remainder going to the fullest slot it fits;
    //      then the other tiles whole, largest first, each into the fullest slot it fits; what
    //      is left goes, piece by piece, to the emptiest slot.
    // Both give every slot the same number of key tiles (to one).  Measured splits (rows):
    // Qwen3-0.6B varlen prefill 512/1024/1536/2048 6784 (a) / 5696 (b), Gemma3 d = 256 global
    // 11648 / 8192, with a 512-key window 9472 / 8832.
    // Pieces of both cuts in flat arrays, grouped by tile in key order (the plan is rebuilt
    // every step, so it avoids a small allocation per tile).
    struct Piece {
      int tile, slot, k0, k1;
    };
    const int64_t cap_tiles = std::max<int64_t>(1, page_cap / KT);
    const int nt = (int)tiles.size();
    std::vector<int64_t> ntile(nt);
    for (int i = 0; i < nt; i++) ntile[i] = (tiles[i].ke - tiles[i].ks + KT - 1) / KT;
    // Rows written as partials, and the most segments of one tile.
    auto score = [&](const std::vector<Piece> &pc, int64_t *rows, int *most) {
      *rows = 0;
      *most = 1;
      for (size_t a = 0; a < pc.size();) {
        size_t b = a;
        while (b < pc.size() && pc[b].tile == pc[a].tile) b++;
        const int np = (int)(b - a);
        const TileItem &t = tiles[pc[a].tile];
        if (np > 1) *rows += (int64_t)np * std::min(key.tile_q, t.qlen - t.q0);
        *most = std::max(*most, np);
        a = b;
      }
    };
    std::vector<Piece> cut_a, cut_b;
    cut_a.reserve(nt + slots);
    {
      int64_t pos = 0;  // first key tile of the current query tile in the flattened order
      for (int i = 0; i < nt; i++) {
        const TileItem &t = tiles[i];
        const int64_t n = ntile[i];
        int64_t j = 0;
        while (j < n) {
          const int64_t g = pos + j;
          const int s_of = (int)std::min<int64_t>(slots - 1, g * slots / total);
          const int64_t s_end = ((int64_t)(s_of + 1) * total + slots - 1) / slots;  // exclusive
          int64_t take = std::min<int64_t>(n - j, s_end - g);
          take = std::max<int64_t>(1, std::min<int64_t>(take, cap_tiles));
          cut_a.push_back({i, s_of, t.ks + (int)(j * KT),
                           std::min<int>(t.ke, t.ks + (int)((j + take) * KT))});
          j += take;
        }
        pos += n;
      }
    }
    {
      const int64_t cap = (total + slots - 1) / slots;
      std::vector<int64_t> load(slots, 0), rem(nt, 0);
      struct Run {
        int tile, slot;
        int64_t n;
      };
      std::vector<Run> runs;
      runs.reserve(nt + 2 * slots);
      std::vector<int> order(nt);
      for (int i = 0; i < nt; i++) order[i] = i;
      std::stable_sort(order.begin(), order.end(),
                       [&](int x, int y) { return ntile[x] > ntile[y]; });
      auto fullest_fit = [&](int64_t n) {
        int best = -1;
        for (int b = 0; b < slots; b++)
          if (load[b] + n <= cap && (best < 0 || load[b] > load[best])) best = b;
        return best;
      };
      int empty = 0;  // slots below this index are not empty
      for (int i : order) {
        if (ntile[i] <= cap) continue;
        rem[i] = ntile[i];
        while (rem[i] >= cap) {
          while (empty < slots && load[empty] != 0) empty++;
          if (empty == slots) break;
          load[empty] = cap;
          runs.push_back({i, empty, cap});
          rem[i] -= cap;
        }
        if (rem[i] > 0) {
          const int b = fullest_fit(rem[i]);
          if (b >= 0) {
            load[b] += rem[i];
            runs.push_back({i, b, rem[i]});
            rem[i] = 0;
          }
        }
      }
      for (int i : order) {
        if (ntile[i] > cap) continue;
        const int b = fullest_fit(ntile[i]);
        if (b >= 0) {
          load[b] += ntile[i];
          runs.push_back({i, b, ntile[i]});
        } else {
          rem[i] = ntile[i];
        }
      }
      for (int i : order)
        while (rem[i] > 0) {
          int b = 0;
          for (int x = 1; x < slots; x++)
            if (load[x] < load[b]) b = x;
          const int64_t take = load[b] < cap ? std::min<int64_t>(rem[i], cap - load[b]) : rem[i];
          load[b] += take;
          runs.push_back({i, b, take});
          rem[i] -= take;
        }
      // Runs to key ranges, in key order; runs longer than the page cap split in their slot.
      std::stable_sort(runs.begin(), runs.end(),
                       [](const Run &x, const Run &y) { return x.tile < y.tile; });
      cut_b.reserve(runs.size());
      int64_t off = 0;
      for (size_t r = 0; r < runs.size(); r++) {
        if (r == 0 || runs[r].tile != runs[r - 1].tile) off = 0;
        const TileItem &t = tiles[runs[r].tile];
        int64_t c = runs[r].n;
        while (c > 0) {
          const int64_t take = std::min<int64_t>(c, cap_tiles);
          cut_b.push_back({runs[r].tile, runs[r].slot, t.ks + (int)(off * KT),
                           std::min<int>(t.ke, t.ks + (int)((off + take) * KT))});
          off += take;
          c -= take;
        }
      }
    }
    int64_t rows_a = 0, rows_b = 0;
    int most_a = 1, most_b = 1;
    score(cut_a, &rows_a, &most_a);
    score(cut_b, &rows_b, &most_b);
    const std::vector<Piece> &cut =
        rows_b < rows_a && most_b <= std::max(kMergeRowsMaxParts, most_a) ? cut_b : cut_a;
    // Segments grouped by slot (counting sort), each slot's in tile order.
    std::vector<int32_t> fill(slots + 1, 0);
    for (const Piece &pc : cut) fill[pc.slot + 1]++;
    for (int sl = 0; sl < slots; sl++) fill[sl + 1] += fill[sl];
    seg_off.assign(fill.begin(), fill.end());
    std::vector<TileItem> segs(cut.size());
    for (size_t a = 0; a < cut.size();) {
      size_t b = a;
      while (b < cut.size() && cut[b].tile == cut[a].tile) b++;
      const TileItem &t = tiles[cut[a].tile];
      const int np = (int)(b - a);
      const int rows = std::min(key.tile_q, t.qlen - t.q0);
      for (int pi = 0; pi < np; pi++) {
        TileItem c = t;
        c.ks = cut[a + pi].k0;
        c.ke = cut[a + pi].k1;
        c.part = np > 1 ? parts : -1;
        c.nsplit = np;
        c.split = pi;
        segs[fill[cut[a + pi].slot]++] = c;
      }
      if (np > 1) {
        for (int r = 0; r < rows; r++) merges.push_back({t.qstart + t.q0 + r, parts + r * np, np, 0});
        parts += rows * np;
      }
      a = b;
    }
    tiles.swap(segs);
  }

  // Chunk: the largest of 4096..64 keys that still gives the grid >= 8 workgroups per CU.  On
  // the 256-row, 1.8 M-key decode, 4096-key items run the kernel at 7.0 TB/s against 6.9 TB/s
  // at 1024 (fewer partials to write and merge) and 6.96 / 6.84 TB/s at 8192 / 16384 (a
  // longer tail).
  // When even 64-key items leave fewer than 8 workgroups per CU (a small step), the largest
  // multiple of 64 keys that still gives every CU a workgroup is taken instead: short items
  // cost more in fixed per-workgroup work and partials than they add in parallelism.  Measured
  // after a flush (decode kernel, HIP events): Gemma3 global decode (32 rows, 202 MB) 41.7 us
  // at 128 keys, 38.7 at 256, 38.3 at 384 (1.07 workgroups per CU; this rule's pick), 42.4 at
  // 512; Qwen3 decode of 8 rows 12.3 us at 64, 11.8 at 128 (the pick); the Gemma3 local layer
  // keeps 64.
  int64_t total = 0;
  for (const Row &r : rows) total += std::max(0, r.kend - r.kbeg);
  auto items_at = [&](int c) {
    int64_t items = 0;
    for (const Row &r : rows) {
      const int len = r.kend - r.kbeg;
      if (len > 0) items += (len + c - 1) / c;
    }
    return items * key.wg_per_item;
  };
  int chunk = 0;
  for (int c = 4096; c >= 64 && !chunk; c >>= 1)
    if (items_at(c) >= (int64_t)ctx->num_cus * 8) chunk = c;
  if (!chunk) {
    // items_at falls as the chunk grows: binary search over multiples of 64 in [64, 4096].
    int lo = 1, hi = 64;  // in units of 64 keys; lo satisfies the bound or is the fallback
    if (items_at(64) >= (int64_t)ctx->num_cus) {
      while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (items_at(64 * mid) >= (int64_t)ctx->num_cus) lo = mid;
        else hi = mid - 1;
      }
    }
    chunk = 64 * lo;
  }
  // A paged item of `chunk` keys spans at most (chunk - 1) / BS + 2 pages; the row kernel
  // stages at most kRowTablePages of them.
  if (key.paged) chunk = std::min(chunk, (kRowTablePages - 1) * key.block_size);

  std::vector<RowItem> items;
  items.reserve(rows.size() + total / chunk + 1);
  for (const Row &r : rows) {
    const int len = r.kend - r.kbeg;
    if (len <= 0) {
      merges.push_back({r.qrow, 0, 0, 0});
      continue;
    }
    const int rchunk = chunk;
    if (len <= rchunk) {
      items.push_back({r.qrow, r.seq, r.kbase, r.kbeg, r.kend, -1, 0, 0});
      continue;
    }
    const int n = (len + rchunk - 1) / rchunk;
    for (int j = 0; j < n; j++) {
      const int b0 = r.kbeg + j * rchunk;
      const int b1 = std::min(r.kend, b0 + rchunk);
      items.push_back({r.qrow, r.seq, r.kbase, b0, b1, parts + j, 0, 0});
    }
    merges.push_back({r.qrow, parts, n, 0});
    parts += n;
  }
  // Items within at most two pages carry the pages' block ids (RowItem::blk_a / blk_b).
  if (key.paged) {
    const int bs = key.block_size;
    for (RowItem &it : items) {
      if (it.kend <= it.kbeg) continue;
      const int p0 = it.kbeg / bs, p1 = (it.kend - 1) / bs;
      if (p1 - p0 > 1) continue;
      const int32_t *t = ctx->tables.data() + (size_t)it.seq * ctx->bt_stride;
      it.blk_a = t[p0] + 1;
      it.blk_b = p1 > p0 ? t[p1] : 0;
    }
  }
  // Longest items first: the workgroups dispatched last are the short row tails, so the chip
  // drains quickly at the end of the launch.  Items carry their own partial slot, so the
  // order does not change any result.
  std::stable_sort(items.begin(), items.end(), [](const RowItem &x, const RowItem &y) {
    return x.kend - x.kbeg > y.kend - y.kbeg;
  });
  // The kernels stage an item's (segment's) block ids in LDS; a plan that exceeded those
  // tables would be a planner bug, reported rather than launched.
  if (key.paged) {
    const int bs = key.block_size;
    for (const RowItem &it : items)
      if (it.kend > it.kbeg && (it.kend - 1) / bs - it.kbeg / bs + 1 > kRowTablePages)
        return fail(ctx, NVA_E_UNSUPPORTED, "row item spans more than %d pages", kRowTablePages);
    for (const TileItem &t : tiles)
      if (t.ke > t.ks && (t.ke - 1) / bs - t.ks / bs + 1 > kPrefillTablePages)
        return fail(ctx, NVA_E_UNSUPPORTED, "prefill segment spans more than %d pages",
                    kPrefillTablePages);
  }

  plan->key = key;
  plan->num_rows = (int)items.size();
  plan->num_merge = (int)merges.size();
  plan->num_tiles = (int)tiles.size();
  plan->num_parts = parts;
  plan->num_slots = slots;
  plan->max_parts = 0;
  for (const MergeItem &mi : merges) plan->max_parts = std::max(plan->max_parts, mi.nparts);
  plan->off_rows = 0;
  plan->off_merge = plan->off_rows + items.size() * sizeof(RowItem);
  plan->off_tiles = plan->off_merge + merges.size() * sizeof(MergeItem);
  plan->off_slots = plan->off_tiles + tiles.size() * sizeof(TileItem);
  plan->host.resize(plan->off_slots + seg_off.size() * sizeof(int32_t));
  char *h = plan->host.data();
  if (!items.empty()) memcpy(h + plan->off_rows, items.data(), items.size() * sizeof(RowItem));
  if (!merges.empty())
    memcpy(h + plan->off_merge, merges.data(), merges.size() * sizeof(MergeItem));
  if (!tiles.empty()) memcpy(h + plan->off_tiles, tiles.data(), tiles.size() * sizeof(TileItem));
  if (!seg_off.empty())
    memcpy(h + plan->off_slots, seg_off.data(), seg_off.size() * sizeof(int32_t));
  static std::atomic<uint64_t> next_id{1};
  plan->id = next_id.fetch_add(1);
  plan->on_device = false;
  plan->valid = true;
  *out = plan;
  return NVA_OK;
}

// The plan's lists in the context's device buffer (uploaded once per plan).
nva_status upload_plan(nva_ctx *ctx, Plan *plan) {
  const size_t bytes = plan->host.size();
  if (plan->on_device || bytes == 0) return NVA_OK;
  HostTimed host_timer(ctx, "plan_upload");
  HIP_TRY(ctx, plan->stage.reserve(bytes), "plan staging");
  HIP_TRY(ctx, plan->dev.reserve(bytes), "plan buffer");
  memcpy(plan->stage.ptr, plan->host.data(), bytes);
  HIP_TRY(ctx, plan->stage.upload(plan->dev, bytes, ctx->stream), "plan upload");
  plan->on_device = true;
  return NVA_OK;
}

KvView make_paged_view(nva_ctx *ctx, nva_kv *kv, int layer) {
  KvView v;
  v.k = kv->k[layer];
  v.v = kv->v[layer];
  v.table = ctx->has_tables ? ctx->dev_i32(ctx->off_tables) : nullptr;
  v.bt_stride = ctx->bt_stride;
  v.block_size = kv->block_size;
  v.bs_shift = pow2_shift(kv->block_size);
  v.paged = 1;
  return v;
}

KvView make_dense_view(const float *k, const float *v) {
  KvView view;
  view.k = k;
  view.v = v;
  view.table = nullptr;
  view.bt_stride = 0;
  view.block_size = 1;
  view.bs_shift = 0;
  view.paged = 0;
  return view;
}

// The plan of one attention call (the descriptor, the step, and whether keys are paged over
// an arena of num_blocks pages of block_size tokens or dense rows), plus the query heads per
// workgroup of the row and tile kernels.
nva_status attention_plan(nva_ctx *ctx, const nva_attn_desc &d, int paged, int block_size,
                          int num_blocks, int num_tokens, Plan **plan, int *hpw_row,
                          int *hpw_tile, bool *rows_mfma = nullptr) {
  const int rep = d.num_heads / d.num_kv_heads;
  // Query heads per row workgroup: the largest divisor of the GQA ratio the row kernel is built
  // for, so each K/V byte crosses HBM once per KV head (one head per workgroup at a ratio of 5
  // read it 5 times: 11.3 ms against 2.3 ms for the 256-row decode at 40 query heads).
  *hpw_row = 1;
  for (int h = std::min(rep, row_kernel_max_heads(d.head_dim)); h > 1; h--)
    if (rep % h == 0 && row_kernel_supports(d.head_dim, h)) {
      *hpw_row = h;
      break;
    }
  // Query heads per prefill workgroup: at most a quarter of its waves, so a workgroup covers at
  // least 64 queries of each head (measured: Gemma3 d = 256 prefill 13% faster with 2 heads
  // than with 4, Gemma 4 d = 512 3% faster with 1 than with 4, Qwen3-4B shape 4% faster with 2
  // than with 4).
  *hpw_tile = largest_pow2_divisor_upto(rep, prefill_max_heads(d.head_dim));
  const bool mfma = ctx->is_prefill && prefill_kernel_supports(d.head_dim, *hpw_tile);
  // The MFMA row kernel carries up to 16 heads of one KV head (it is used from 5).  Rows that
  // run beside MFMA prefill tiles (a mixed step) share the matrix pipes with them: there the row
  // kernel keeps 5 heads per KV head (40 query heads over 8 KV heads, Qwen3-4B-like mixed step:
  // attention 1.58-1.60 against 1.67-1.71 ms with MFMA rows), while 8 run as well or better on
  // MFMA (64 over 8: 2.14-2.25 against 2.25-2.28 ms), the row kernel's 8-head form being slow.
  bool mfma_rows = false;
  if (row_mfma_supports(d.head_dim, paged, block_size))
    for (int h = std::min(rep, kRowMfmaMaxHeads); h >= kRowMfmaMinHeads; h--)
      if (rep % h == 0) {
        if (!mfma || *hpw_row != h || h > kRowMfmaMinHeads) {
          *hpw_row = h;
          mfma_rows = true;
        }
        break;
      }
  if (rows_mfma) *rows_mfma = mfma_rows;
  if (!mfma_rows && !row_kernel_supports(d.head_dim, *hpw_row))
    return fail(ctx, NVA_E_UNSUPPORTED, "head_dim %d has no row kernel in this build",
                d.head_dim);
  PlanKey key;
  key.window = d.sliding_window > 0 ? d.sliding_window : 0;
  key.mfma = mfma ? 1 : 0;
  key.tile_q = mfma ? prefill_tile_queries(d.head_dim, *hpw_tile) : 0;
  key.wg_per_item = d.num_kv_heads * (rep / *hpw_row);
  key.blocks_per_cu = mfma ? ctx_prefill_blocks_per_cu(ctx, d.head_dim, *hpw_tile) : 0;
  key.tile_groups = mfma ? d.num_kv_heads * (rep / *hpw_tile) : 0;
  key.tokens = num_tokens;
  key.paged = paged;
  key.block_size = paged ? block_size : 0;
  key.num_blocks = paged ? num_blocks : 0;
  key.head_dim = d.head_dim;
  key.num_heads = d.num_heads;
  key.num_kv_heads = d.num_kv_heads;
  return get_plan(ctx, key, plan);
}

// Regions of the no-allocation array one call uses: [gather rows | plan lists | partials],
// each 256-byte aligned.
struct ScratchLayout {
  size_t plan_off = 0, part_off = 0, part_bytes = 0, end = 0;
};

ScratchLayout scratch_layout(size_t gather_bytes, const Plan &plan, const nva_attn_desc &d) {
  ScratchLayout l;
  const size_t parts = (size_t)plan.num_parts * d.num_heads;
  l.plan_off = align256(gather_bytes);
  l.part_off = align256(l.plan_off + plan.host.size());
  l.part_bytes = parts * (2 + (size_t)d.head_dim) * sizeof(float);
  l.end = l.part_off + l.part_bytes;
  return l;
}

// A kernel is about to write [begin, end) of this device's array: the plan recorded as held
// there no longer is, if the ranges meet.
void scratch_overwritten(int device, size_t begin, size_t end) {
  ScratchTag &tag = scratch_tag(device);
  if (tag.plan_id != 0 && begin < tag.offset + tag.bytes && tag.offset < end) tag = ScratchTag{};
}

bool stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Checks of a no-allocation call made before it launches anything (so a rejected call leaves
// the pages and the array untouched): the array must hold the call's gather rows, plan and
// partials, and under stream capture the plan must already be in it (a captured copy would
// only be recorded, not run, and the array would not hold what its tag says).
nva_status noalloc_prepare(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc &d, int num_tokens) {
  const bool dense = ctx->is_prefill && !ctx->has_tables;
  size_t gather = 0;
  if (dense && !d.write_kv) {
    gather = 2 * (size_t)num_tokens * d.num_kv_heads * d.head_dim * 4 + 16;
    if (gather > kScratchBytes)
      return fail(ctx, NVA_E_ARG,
                  "this call's gathered K/V rows need %zu bytes of device scratch; the "
                  "no-allocation entry point has %zu",
                  gather, kScratchBytes);
  }
  Plan *plan = nullptr;
  int hpw_row = 0, hpw_tile = 0;
  nva_status st = attention_plan(ctx, d, dense ? 0 : 1, dense ? 1 : kv->block_size,
                                 dense ? 0 : kv->num_blocks, num_tokens, &plan, &hpw_row,
                                 &hpw_tile);
  if (st != NVA_OK) return st;
  const ScratchLayout l = scratch_layout(gather, *plan, d);
  if (l.end > kScratchBytes)
    return fail(ctx, NVA_E_ARG,
                "this call needs %zu bytes of device scratch (plan %zu, partials %zu, gather "
                "%zu); the no-allocation entry point has %zu",
                l.end, plan->host.size(), l.part_bytes, gather, kScratchBytes);
  const ScratchTag &tag = scratch_tag(ctx->device);
  if (!plan->host.empty() && (tag.plan_id != plan->id || tag.offset != l.plan_off) &&
      stream_capturing(ctx->stream))
    return fail(ctx, NVA_E_ARG,
                "under stream capture the step's plan must already be in the device scratch "
                "array: make one call with this configuration outside capture first");
  return NVA_OK;
}

// The attention part of Attention.forward once the store (if any) is done.  With scr null the
// plan and partials use the context's buffers; otherwise the scratch array's regions.
nva_status run_attention(nva_ctx *ctx, const nva_attn_desc &d, const KvView &view,
                         int num_blocks, const float *q, int num_tokens, float *out,
                         Scratch *scr) {
  Plan *plan = nullptr;
  int hpw_row = 0, hpw_tile = 0;
  bool rows_mfma = false;
  nva_status st = attention_plan(ctx, d, view.paged, view.block_size, num_blocks, num_tokens,
                                 &plan, &hpw_row, &hpw_tile, &rows_mfma);
  if (st != NVA_OK) return st;
  const int window = d.sliding_window > 0 ? d.sliding_window : 0;

  const size_t parts = (size_t)plan->num_parts * d.num_heads;
  char *pbase = nullptr;
  float *pm = nullptr;
  if (!scr) {
    const size_t part_bytes = parts * (2 + (size_t)d.head_dim) * sizeof(float);
    st = upload_plan(ctx, plan);
    if (st != NVA_OK) return st;
    pbase = static_cast<char *>(plan->dev.ptr);
    if (parts > 0) HIP_TRY(ctx, ctx->d_part.reserve(part_bytes), "partial buffer");
    pm = static_cast<float *>(ctx->d_part.ptr);
  } else {
    // The sizes and the capture rule were checked before anything was launched
    // (noalloc_prepare); these are the same regions.
    const ScratchLayout l = scratch_layout(scr->used, *plan, d);
    pbase = scr->base + l.plan_off;
    pm = reinterpret_cast<float *>(scr->base + l.part_off);
    // Skip the copy when this device's array already holds this very plan at this offset.
    ScratchTag &tag = scratch_tag(ctx->device);
    if (!plan->host.empty() && (tag.plan_id != plan->id || tag.offset != l.plan_off)) {
      tag = ScratchTag{};
      HIP_TRY(ctx, hipMemcpyAsync(pbase, plan->host.data(), plan->host.size(),
                                  hipMemcpyHostToDevice, ctx->stream),
              "plan copy to scratch");
      tag.plan_id = plan->id;
      tag.offset = l.plan_off;
      tag.bytes = plan->host.size();
    }
    if (l.part_bytes > 0) scratch_overwritten(ctx->device, l.part_off, l.end);
  }

  // "attention" times the whole part below, kernels that overlap counted once.
  Timed span(ctx, "attention");
  if (!plan->covers_all) {
    // Rows outside every sequence stay zero, as Tensor.zeros in the reference.
    HIP_TRY(ctx, launch_zero(out, (size_t)num_tokens * d.num_heads * d.head_dim, ctx->stream),
            "zero output");
  }
  // A mixed step (MFMA tiles and rows in one plan) runs the HBM-bound rows on the side stream
  // while the MFMA-bound tiles run on the main stream; both write disjoint partials, and the
  // main stream waits for the side stream before the merge.  The tiles are issued first: the
  // plan sized their grid to a share of the CUs, which it only gets if the rows do not fill
  // the chip before it.
  const bool fork = plan->num_tiles > 0 && plan->num_rows > 0;
  if (fork) HIP_TRY(ctx, hipEventRecord(ctx->fork_ev, ctx->stream), "fork record");
  if (plan->num_tiles > 0) {
    TileLaunch t;
    t.q = q;
    t.out = out;
    t.kv = view;
    t.items = reinterpret_cast<const TileItem *>(pbase + plan->off_tiles);
    t.seg_off = reinterpret_cast<const int32_t *>(pbase + plan->off_slots);
    t.num_items = plan->num_tiles;
    t.num_slots = plan->num_slots;
    t.hq = d.num_heads;
    t.hkv = d.num_kv_heads;
    t.head_dim = d.head_dim;
    t.window = window;
    t.scale = d.scale;
    t.part_m = pm;
    t.part_l = pm + parts;
    t.part_acc = pm + 2 * parts;
    Timed tm(ctx, "prefill");
    HIP_TRY(ctx, launch_prefill_tiles(t, hpw_tile, ctx->stream), "prefill kernel launch");
    tm.done();
  }
  if (plan->num_rows > 0) {
    hipStream_t row_stream = ctx->stream;
    if (fork) {
      HIP_TRY(ctx, hipStreamWaitEvent(ctx->side_stream, ctx->fork_ev, 0), "fork wait");
      row_stream = ctx->side_stream;
    }
    RowLaunch r;
    r.q = q;
    r.out = out;
    r.kv = view;
    r.items = reinterpret_cast<const RowItem *>(pbase + plan->off_rows);
    r.num_items = plan->num_rows;
    r.hq = d.num_heads;
    r.hkv = d.num_kv_heads;
    r.head_dim = d.head_dim;
    r.scale = d.scale;
    r.part_m = pm;
    r.part_l = pm + parts;
    r.part_acc = pm + 2 * parts;
    r.mfma = rows_mfma ? 1 : 0;
    r.xcd_hint = ctx->xcd_hint;
    r.rotate_heads = (d.num_kv_heads == 8 || d.num_kv_heads == 4 || d.num_kv_heads == 2) &&
                     (d.head_dim == 128 || d.head_dim == 64) &&
                     hpw_row == d.num_heads / d.num_kv_heads;
    Timed tm(ctx, "decode", row_stream);
    HIP_TRY(ctx, launch_row_attention(r, hpw_row, row_stream), "decode kernel launch");
    tm.done();
  }
  if (fork) {
    HIP_TRY(ctx, hipEventRecord(ctx->join_ev, ctx->side_stream), "join record");
    HIP_TRY(ctx, hipStreamWaitEvent(ctx->stream, ctx->join_ev, 0), "join wait");
  }
  if (plan->num_merge > 0) {
    MergeLaunch mg;
    mg.out = out;
    mg.items = reinterpret_cast<const MergeItem *>(pbase + plan->off_merge);
    mg.num_items = plan->num_merge;
    mg.hq = d.num_heads;
    mg.head_dim = d.head_dim;
    mg.part_m = pm;
    mg.part_l = pm + parts;
    mg.part_acc = pm + 2 * parts;
    Timed tm(ctx, "merge");
    HIP_TRY(ctx, launch_merge(mg, plan->max_parts, ctx->stream), "merge kernel launch");
    tm.done();
  }
  span.done();
  return NVA_OK;
}

// Slots index the arena's num_blocks*block_size rows; the reference's arraycopy would throw
// for a slot past the end.
nva_status check_slots(nva_ctx *ctx, nva_kv *kv) {
  const int64_t rows = (int64_t)kv->num_blocks * kv->block_size;
  if (ctx->slot_max >= rows)
    return fail(ctx, NVA_E_ARG, "slot %lld outside the arena's %lld slots",
                (long long)ctx->slot_max, (long long)rows);
  return NVA_OK;
}

nva_status check_positions(nva_ctx *ctx, int num_tokens, int max_pos) {
  if (!ctx->has_pos) return fail(ctx, NVA_E_ARG, "the step has no positions");
  if (num_tokens > (int)ctx->pos.size())
    return fail(ctx, NVA_E_ARG, "%d tokens but the step has %d positions", num_tokens,
                (int)ctx->pos.size());
  for (int t = 0; t < num_tokens; t++) {
    const int p = ctx->pos[t];
    if (p < 0 || p >= max_pos)
      return fail(ctx, NVA_E_ROPE_POS, "RoPE position %d out of range [0, %d)", p, max_pos);
  }
  return NVA_OK;
}

nva_status check_desc(nva_ctx *ctx, const nva_attn_desc *d) {
  if (!d) return fail(ctx, NVA_E_ARG, "attention descriptor is null");
  if (d->num_heads <= 0 || d->num_kv_heads <= 0 || d->head_dim <= 0)
    return fail(ctx, NVA_E_ARG, "numHeads, numKvHeads and headDim must be > 0");
  if (d->num_heads % d->num_kv_heads)
    return fail(ctx, NVA_E_ARG, "numHeads %d is not a multiple of numKvHeads %d", d->num_heads,
                d->num_kv_heads);
  if (d->head_dim % 4) return fail(ctx, NVA_E_UNSUPPORTED, "headDim must be a multiple of 4");
  return NVA_OK;
}

// Shared prologue of nva_attention_forward / nva_rope_attention_forward.
nva_status check_forward(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc *desc, int num_tokens) {
  nva_status st = check_desc(ctx, desc);
  if (st != NVA_OK) return st;
  if (!kv) return fail(ctx, NVA_E_NO_ARENA, "KV cache arena not bound in Context");
  if (kv->ctx != ctx) return fail(ctx, NVA_E_ARG, "KV arena belongs to another context");
  if (desc->kv_layer_index < 0 || desc->kv_layer_index >= kv->num_layers)
    return fail(ctx, NVA_E_LAYER, "layerIndex out of range: %d (layers=%d)",
                desc->kv_layer_index, kv->num_layers);
  if (!ctx->has_step) return fail(ctx, NVA_E_NO_STEP, "no step metadata set on the context");
  if (num_tokens < 0) return fail(ctx, NVA_E_ARG, "num_tokens < 0");
  const int layer = desc->kv_layer_index;
  if (kv->k[layer] && (kv->head_dims[layer] != desc->head_dim ||
                       kv->num_kv_heads != desc->num_kv_heads))
    return fail(ctx, NVA_E_ARG, "layer %d pages are [.., %d, %d], attention wants [.., %d, %d]",
                layer, kv->num_kv_heads, kv->head_dims[layer], desc->num_kv_heads,
                desc->head_dim);
  if (!ctx->is_prefill) {
    if (!ctx->has_ctx_lens || !ctx->has_tables)
      return fail(ctx, NVA_E_ARG, "decode needs context lengths and block tables");
    if (num_tokens > ctx->num_seqs)
      return fail(ctx, NVA_E_ARG, "decode has %d rows but %d context lengths", num_tokens,
                  ctx->num_seqs);
  } else if (!ctx->has_cu) {
    return fail(ctx, NVA_E_ARG, "prefill needs cu_seqlens");
  }
  return NVA_OK;
}

// Which K/V the attention reads, Attention.java:161-170 and :176-195.  scr selects the
// no-allocation workspace (null: the context's buffers).
nva_status attention_after_store(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc &d,
                                 const float *q, const float *k, const float *v,
                                 int num_tokens, float *out, Scratch *scr = nullptr) {
  const int layer = d.kv_layer_index;
  const bool allocated = kv->k[layer] != nullptr;
  if (ctx->is_prefill && !ctx->has_tables) {
    if (d.write_kv) {
      if (!k || !v) return fail(ctx, NVA_E_ARG, "dense prefill needs k and v");
      return run_attention(ctx, d, make_dense_view(k, v), 0, q, num_tokens, out, scr);
    }
    // Shared-KV dense prefill: gather the producer's rows at the step's slots.
    if (!ctx->has_slots || ctx->num_slots != num_tokens)
      return fail(ctx, NVA_E_SHARED_KV,
                  "shared-KV attention needs slot mapping or block tables to read the "
                  "producer cache");
    if (!allocated) return fail(ctx, NVA_E_ARG, "producer layer %d has no pages", layer);
    nva_status sst = check_slots(ctx, kv);
    if (sst != NVA_OK) return sst;
    const size_t row = (size_t)d.num_kv_heads * d.head_dim;
    const size_t gather_bytes = 2 * (size_t)num_tokens * row * 4 + 16;
    float *gk = nullptr;
    if (!scr) {
      HIP_TRY(ctx, ctx->d_gather.reserve(gather_bytes), "gather buffer");
      gk = static_cast<float *>(ctx->d_gather.ptr);
    } else {
      // Size checked by noalloc_prepare.  The rows overwrite the front of the array.
      gk = reinterpret_cast<float *>(scr->base);
      scr->used = gather_bytes;
      scratch_overwritten(ctx->device, 0, gather_bytes);
    }
    float *gv = gk + (size_t)num_tokens * row;
    GatherLaunch g;
    g.k_cache = kv->k[layer];
    g.v_cache = kv->v[layer];
    g.k_out = gk;
    g.v_out = gv;
    g.slots = ctx->dev_i32(ctx->off_slots);
    g.tokens = num_tokens;
    g.row = (int)row;
    Timed tm(ctx, "gather");
    HIP_TRY(ctx, launch_gather(g, ctx->stream), "gather kernel launch");
    tm.done();
    return run_attention(ctx, d, make_dense_view(gk, gv), 0, q, num_tokens, out, scr);
  }
  if (!allocated) return fail(ctx, NVA_E_ARG, "layer %d has no pages to attend over", layer);
  if (!ctx->has_tables) return fail(ctx, NVA_E_ARG, "paged attention needs block tables");
  return run_attention(ctx, d, make_paged_view(ctx, kv, layer), kv->num_blocks, q,
                       num_tokens, out, scr);
}

// The kernels' view of an RMSNorm descriptor; NULL disables the norm.  Any eps is accepted, as
// in the reference (a negative var + eps gives NaN there too).
HeadNorm head_norm(const nva_rms_norm *n) {
  HeadNorm h{};
  if (n) {
    h.weight = n->weight;
    h.eps = n->eps;
    h.enabled = 1;
    h.one_plus = n->one_plus_weight ? 1 : 0;
  }
  return h;
}

// Math.round(float), Norms.java:317: floor(x + 1/2) evaluated exactly; NaN -> 0; saturating.
int32_t java_round(float x) {
  if (std::isnan(x)) return 0;
  const float f = std::floor(x);
  const float frac = x - f;
  const double r = (double)f + (frac >= 0.5f ? 1.0 : 0.0);
  if (r >= 2147483647.0) return 2147483647;
  if (r <= -2147483648.0) return (-2147483647 - 1);
  return (int32_t)r;
}

}  // namespace

// Records msg as the context's last error (the step producers in step.cpp report through it).
__attribute__((visibility("hidden"))) nva_status nva_internal_fail(nva_ctx *ctx, nva_status st,
                                                                 const char *msg) {
  return fail(ctx, st, "%s", msg);
}

extern "C" {

const char *nva_status_string(nva_status s) {
  switch (s) {
    case NVA_OK: return "ok";
    case NVA_E_ARG: return "invalid argument";
    case NVA_E_LAYER: return "layer index out of range";
    case NVA_E_ROPE_POS: return "RoPE position out of range";
    case NVA_E_SHARED_KV: return "shared-KV layer without slots or block tables";
    case NVA_E_NO_ARENA: return "no KV arena";
    case NVA_E_NO_STEP: return "no step metadata";
    case NVA_E_HIP: return "HIP error";
    case NVA_E_OOM: return "out of memory";
    case NVA_E_UNSUPPORTED: return "unsupported shape";
    default: return "unknown status";
  }
}

nva_status nva_ctx_create(int device, nva_ctx **out) {
  if (!out) return NVA_E_ARG;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return NVA_E_HIP;
  if (device < 0 || device >= n) return NVA_E_ARG;
  DeviceGuard dg(device);
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != device) return NVA_E_HIP;
  nva_ctx *ctx = new nva_ctx();
  ctx->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
    ctx->num_cus = prop.multiProcessorCount;
  // The context's own stream is a blocking stream, so it is ordered with work on the null
  // stream (hipMemcpy of inputs and outputs).  The side stream that runs decode rows beside
  // prefill tiles must overlap with whichever stream is current, so it is non-blocking and
  // joined through events.
  if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamDefault) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->side_stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->join_ev, hipEventDisableTiming) != hipSuccess) {
    if (ctx->join_ev) (void)hipEventDestroy(ctx->join_ev);
    if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
    if (ctx->side_stream) (void)hipStreamDestroy(ctx->side_stream);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return NVA_E_HIP;
  }
  ctx->stream = ctx->own_stream;
  if (hipMalloc(reinterpret_cast<void **>(&ctx->xcd_hint), 256) != hipSuccess ||
      hipMemset(ctx->xcd_hint, 0, 256) != hipSuccess) {
    if (ctx->xcd_hint) (void)hipFree(ctx->xcd_hint);
    ctx->xcd_hint = nullptr;
    (void)hipGetLastError();
  }
  ctx->scratch = scratch_address(device, &ctx->scratch_err);
  *out = ctx;
  return NVA_OK;
}

nva_status nva_ctx_destroy(nva_ctx *ctx) {
  if (!ctx) return NVA_OK;
  DeviceGuard dg(ctx);
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipStreamSynchronize(ctx->side_stream);
  resolve_timings(ctx);
  for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
  for (Plan *p : ctx->plans) {
    p->stage.release();
    p->dev.release();
    delete p;
  }
  ctx->step_stage.release();
  ctx->d_step.release();
  ctx->d_part.release();
  ctx->d_q_rot.release();
  ctx->d_k_rot.release();
  ctx->d_v_norm.release();
  ctx->d_lin.release();
  ctx->d_gather.release();
  if (ctx->xcd_hint) (void)hipFree(ctx->xcd_hint);
  (void)hipEventDestroy(ctx->fork_ev);
  (void)hipEventDestroy(ctx->join_ev);
  (void)hipStreamDestroy(ctx->side_stream);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
  return NVA_OK;
}

nva_status nva_ctx_set_stream(nva_ctx *ctx, void *hip_stream) {
  if (!ctx) return NVA_E_ARG;
  ctx->stream = static_cast<hipStream_t>(hip_stream);  // NULL: the device's null stream
  return NVA_OK;
}

void *nva_ctx_stream(nva_ctx *ctx) { return ctx ? ctx->stream : nullptr; }

nva_status nva_ctx_sync(nva_ctx *ctx) {
  if (!ctx) return NVA_E_ARG;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
  return NVA_OK;
}

const char *nva_last_error(nva_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

nva_status nva_ctx_set_timing(nva_ctx *ctx, int enable) {
  if (!ctx) return NVA_E_ARG;
  ctx->timing = enable != 0;
  return NVA_OK;
}

nva_status nva_ctx_kernel_stats(nva_ctx *ctx, const char *kernel, int64_t *launches,
                                double *total_ms) {
  if (!ctx || !kernel) return NVA_E_ARG;
  if (strcmp(kernel, "device_bytes") == 0) {
    // Device memory the context's grow-only buffers hold (not the arenas or RoPE tables).
    size_t b = ctx->d_step.cap + ctx->d_part.cap + ctx->d_q_rot.cap + ctx->d_k_rot.cap +
               ctx->d_v_norm.cap + ctx->d_lin.cap + ctx->d_gather.cap;
    for (const Plan *p : ctx->plans) b += p->dev.cap;
    if (launches) *launches = (int64_t)b;
    if (total_ms) *total_ms = 0.0;
    return NVA_OK;
  }
  resolve_timings(ctx);
  auto it = ctx->stats.find(kernel);
  if (launches) *launches = it == ctx->stats.end() ? 0 : it->second.launches;
  if (total_ms) *total_ms = it == ctx->stats.end() ? 0.0 : it->second.ms;
  return NVA_OK;
}

nva_status nva_ctx_reset_stats(nva_ctx *ctx) {
  if (!ctx) return NVA_E_ARG;
  resolve_timings(ctx);
  ctx->stats.clear();
  return NVA_OK;
}

// ------------------------------------------------------------------------------- KV arena

nva_status nva_kv_create(nva_ctx *ctx, int num_layers, int num_blocks, int block_size,
                         int num_kv_heads, const int32_t *head_dims, const uint8_t *allocate,
                         nva_kv **out) {
  if (!ctx || !out) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  *out = nullptr;
  if (num_layers <= 0) return fail(ctx, NVA_E_ARG, "numLayers must be > 0");
  if (num_blocks <= 0) return fail(ctx, NVA_E_ARG, "numBlocks must be > 0");
  if (block_size <= 0 || num_kv_heads <= 0 || !head_dims)
    return fail(ctx, NVA_E_ARG, "blockSize, numKvHeads must be > 0 and headDims non-null");
  nva_kv *kv = new nva_kv();
  kv->ctx = ctx;
  kv->num_layers = num_layers;
  kv->num_blocks = num_blocks;
  kv->block_size = block_size;
  kv->num_kv_heads = num_kv_heads;
  kv->head_dims.assign(head_dims, head_dims + num_layers);
  kv->k.assign(num_layers, nullptr);
  kv->v.assign(num_layers, nullptr);
  kv->bytes.assign(num_layers, 0);
  for (int i = 0; i < num_layers; i++) {
    if (allocate && !allocate[i]) continue;
    if (head_dims[i] <= 0) {
      nva_kv_destroy(kv);
      return fail(ctx, NVA_E_ARG, "headDims[%d] must be > 0", i);
    }
    const int64_t bytes =
        (int64_t)num_blocks * block_size * num_kv_heads * (int64_t)head_dims[i] * 4;
    void *pk = nullptr, *pv = nullptr;
    hipError_t e = hipMalloc(&pk, bytes);
    if (e == hipSuccess) e = hipMalloc(&pv, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(pk, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(pv, 0, bytes, ctx->stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // a failed allocation must not surface at a later launch check
      if (pk) (void)hipFree(pk);
      if (pv) (void)hipFree(pv);
      nva_kv_destroy(kv);
      return hip_fail(ctx, e, "KV arena allocation");
    }
    kv->k[i] = static_cast<float *>(pk);
    kv->v[i] = static_cast<float *>(pv);
    kv->bytes[i] = bytes;
  }
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "KV arena zero-fill");
  *out = kv;
  return NVA_OK;
}

nva_status nva_kv_blocks_that_fit(nva_ctx *ctx, int num_layers, int block_size, int num_kv_heads,
                                  const int32_t *head_dims, const uint8_t *allocate,
                                  float fraction, int *blocks, int64_t *free_bytes) {
  if (!ctx || !blocks) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (num_layers <= 0) return fail(ctx, NVA_E_ARG, "numLayers must be > 0");
  if (block_size <= 0 || num_kv_heads <= 0 || !head_dims)
    return fail(ctx, NVA_E_ARG, "blockSize, numKvHeads must be > 0 and headDims non-null");
  if (!(fraction > 0.0f && fraction <= 1.0f))
    return fail(ctx, NVA_E_ARG, "kvHeapFraction must be in (0, 1], got %g", (double)fraction);
  // Bytes of one page across the layers that get pages: K and V, Config.java:105-114.
  int64_t per_block = 0;
  for (int i = 0; i < num_layers; i++) {
    if (allocate && !allocate[i]) continue;
    if (head_dims[i] <= 0) return fail(ctx, NVA_E_ARG, "headDims[%d] must be > 0", i);
    per_block += 2 * (int64_t)block_size * num_kv_heads * head_dims[i] * 4;
  }
  if (per_block <= 0) return fail(ctx, NVA_E_ARG, "no layer gets pages");
  size_t free_b = 0, total_b = 0;
  HIP_TRY(ctx, hipMemGetInfo(&free_b, &total_b), "device memory query");
  // (long) (free * kvHeapFraction) / bytesPerBlock, at least 32 (Config.java:115-116).
  const int64_t budget = (int64_t)((double)free_b * (double)fraction);
  const int64_t cap = std::max<int64_t>(32, budget / per_block);
  *blocks = (int)std::min<int64_t>(cap, INT32_MAX);
  if (free_bytes) *free_bytes = (int64_t)free_b;
  return NVA_OK;
}

nva_status nva_kv_destroy(nva_kv *kv) {
  if (!kv) return NVA_OK;
  if (kv->ctx) (void)hipStreamSynchronize(kv->ctx->stream);
  for (size_t i = 0; i < kv->k.size(); i++) {
    if (kv->k[i]) (void)hipFree(kv->k[i]);
    if (kv->v[i]) (void)hipFree(kv->v[i]);
  }
  delete kv;
  return NVA_OK;
}

nva_status nva_kv_layer(nva_kv *kv, int layer, void **key, void **value, int64_t *bytes) {
  if (!kv) return NVA_E_ARG;
  if (layer < 0 || layer >= kv->num_layers)
    return fail(kv->ctx, NVA_E_LAYER, "layerIndex out of range: %d (layers=%d)", layer,
                kv->num_layers);
  if (key) *key = kv->k[layer];
  if (value) *value = kv->v[layer];
  if (bytes) *bytes = kv->bytes[layer];
  return NVA_OK;
}

static nva_status kv_copy(nva_kv *kv, int layer, int which, int64_t off, void *host,
                          int64_t count, bool to_device) {
  if (!kv || !host || count < 0 || off < 0 || (which != 0 && which != 1)) return NVA_E_ARG;
  nva_ctx *ctx = kv->ctx;
  DeviceGuard dg(ctx);
  if (layer < 0 || layer >= kv->num_layers)
    return fail(ctx, NVA_E_LAYER, "layerIndex out of range: %d (layers=%d)", layer,
                kv->num_layers);
  float *base = which == 0 ? kv->k[layer] : kv->v[layer];
  if (!base) return fail(ctx, NVA_E_ARG, "layer %d has no pages", layer);
  if ((off + count) * 4 > kv->bytes[layer])
    return fail(ctx, NVA_E_ARG, "range [%lld, %lld) outside the layer's %lld floats",
                (long long)off, (long long)(off + count), (long long)(kv->bytes[layer] / 4));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
  if (to_device)
    HIP_TRY(ctx, hipMemcpy(base + off, host, count * 4, hipMemcpyHostToDevice), "KV write");
  else
    HIP_TRY(ctx, hipMemcpy(host, base + off, count * 4, hipMemcpyDeviceToHost), "KV read");
  return NVA_OK;
}

nva_status nva_kv_write(nva_kv *kv, int layer, int which, int64_t float_offset,
                        const float *host, int64_t count) {
  return kv_copy(kv, layer, which, float_offset, const_cast<float *>(host), count, true);
}

nva_status nva_kv_read(nva_kv *kv, int layer, int which, int64_t float_offset, float *host,
                       int64_t count) {
  return kv_copy(kv, layer, which, float_offset, host, count, false);
}

// ------------------------------------------------------------------------------- RoPE tables

nva_status nva_rope_create(nva_ctx *ctx, const float *cos_sin, int max_pos, int head_size,
                           nva_rope **out) {
  if (!ctx || !out || !cos_sin) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  *out = nullptr;
  if (max_pos <= 0 || head_size <= 0 || head_size % 2)
    return fail(ctx, NVA_E_ARG, "RoPE table needs maxPos > 0 and an even headSize");
  const size_t bytes = (size_t)max_pos * head_size * 4;
  void *p = nullptr;
  HIP_TRY(ctx, hipMalloc(&p, bytes), "RoPE table allocation");
  hipError_t e = hipMemcpy(p, cos_sin, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(ctx, e, "RoPE table upload");
  }
  nva_rope *r = new nva_rope();
  r->ctx = ctx;
  r->max_pos = max_pos;
  r->head_size = head_size;
  r->table = static_cast<float *>(p);
  *out = r;
  return NVA_OK;
}

nva_status nva_rope_create_theta(nva_ctx *ctx, int head_size, int rotary_dim, int max_pos,
                                 float base, nva_rope **out) {
  if (!ctx || !out) return NVA_E_ARG;
  if (rotary_dim != head_size) return fail(ctx, NVA_E_ARG, "rotaryDim must equal headSize");
  if (max_pos <= 0 || head_size <= 0 || head_size % 2)
    return fail(ctx, NVA_E_ARG, "RoPE table needs maxPos > 0 and an even headSize");
  const int half = head_size / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; i++)
    inv[i] = (float)(1.0 / std::pow((double)base, (2.0 * i) / rotary_dim));
  std::vector<float> table((size_t)max_pos * head_size);
  for (int pos = 0; pos < max_pos; pos++)
    for (int i = 0; i < half; i++) {
      volatile float prod = (float)pos * inv[i];  // float product, as in Java
      const double freq = (double)prod;
      table[(size_t)pos * head_size + i] = (float)std::cos(freq);
      table[(size_t)pos * head_size + half + i] = (float)std::sin(freq);
    }
  return nva_rope_create(ctx, table.data(), max_pos, head_size, out);
}

nva_status nva_rope_destroy(nva_rope *rope) {
  if (!rope) return NVA_OK;
  if (rope->ctx) (void)hipStreamSynchronize(rope->ctx->stream);
  if (rope->table) (void)hipFree(rope->table);
  delete rope;
  return NVA_OK;
}

// ------------------------------------------------------------------------------- step

nva_status nva_step_set(nva_ctx *ctx, int is_prefill, const int32_t *cu_q, const int32_t *cu_k,
                        int num_seqs, int max_seqlen_q, int max_seqlen_k,
                        const int32_t *slot_mapping, int num_slots,
                        const int32_t *context_lens, const int32_t *block_tables,
                        int bt_stride, const int32_t *seq_ids, const float *positions,
                        int num_tokens) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (num_seqs < 0 || num_slots < 0 || num_tokens < 0 || bt_stride < 0)
    return fail(ctx, NVA_E_ARG, "negative count in step metadata");
  if (is_prefill && !cu_q) return fail(ctx, NVA_E_ARG, "prefill step needs cuSeqlensQ");
  if (is_prefill && !cu_k) return fail(ctx, NVA_E_ARG, "prefill step needs cuSeqlensK");
  if (block_tables && bt_stride <= 0 && num_seqs > 0)
    return fail(ctx, NVA_E_ARG, "block tables need bt_stride > 0");
  for (Plan *p : ctx->plans) p->valid = false;
  ctx->has_step = true;
  ctx->is_prefill = is_prefill != 0;
  ctx->num_seqs = num_seqs;
  ctx->num_tokens = num_tokens;
  ctx->max_q = max_seqlen_q;
  ctx->max_k = max_seqlen_k;
  ctx->bt_stride = block_tables ? bt_stride : 0;
  ctx->has_cu = cu_q && cu_k;
  ctx->has_slots = slot_mapping != nullptr;
  ctx->num_slots = slot_mapping ? num_slots : 0;
  ctx->has_ctx_lens = context_lens != nullptr;
  ctx->has_tables = block_tables != nullptr;
  ctx->has_pos = positions != nullptr;
  ctx->cu_q.assign(cu_q ? cu_q : nullptr, cu_q ? cu_q + num_seqs + 1 : nullptr);
  ctx->cu_k.assign(cu_k ? cu_k : nullptr, cu_k ? cu_k + num_seqs + 1 : nullptr);
  ctx->slots.assign(slot_mapping ? slot_mapping : nullptr,
                    slot_mapping ? slot_mapping + num_slots : nullptr);
  ctx->ctx_lens.assign(context_lens ? context_lens : nullptr,
                       context_lens ? context_lens + num_seqs : nullptr);
  ctx->tables.assign(block_tables ? block_tables : nullptr,
                     block_tables ? block_tables + (size_t)num_seqs * bt_stride : nullptr);
  ctx->seq_ids.assign(seq_ids ? seq_ids : nullptr, seq_ids ? seq_ids + num_tokens : nullptr);
  ctx->slot_max = -1;
  for (int32_t sl : ctx->slots) ctx->slot_max = std::max<int64_t>(ctx->slot_max, sl);
  ctx->pos.resize(positions ? num_tokens : 0);
  for (int t = 0; positions && t < num_tokens; t++) ctx->pos[t] = java_round(positions[t]);
  if (ctx->is_prefill) {
    for (int b = 0; b < num_seqs; b++)
      if (cu_q[b + 1] < cu_q[b] || cu_k[b + 1] < cu_k[b]) {
        ctx->has_step = false;
        return fail(ctx, NVA_E_ARG, "cu_seqlens must be non-decreasing");
      }
  }

  // One device blob: cu_q | cu_k | slots | ctx_lens | tables | positions (16-byte aligned).
  auto align = [](size_t x) { return (x + 15) & ~(size_t)15; };
  size_t off = 0;
  ctx->off_cu_q = off;
  off = align(off + ctx->cu_q.size() * 4);
  ctx->off_cu_k = off;
  off = align(off + ctx->cu_k.size() * 4);
  ctx->off_slots = off;
  off = align(off + ctx->slots.size() * 4);
  ctx->off_ctx = off;
  off = align(off + ctx->ctx_lens.size() * 4);
  ctx->off_tables = off;
  off = align(off + ctx->tables.size() * 4);
  ctx->off_pos = off;
  off = align(off + ctx->pos.size() * 4);
  const size_t bytes = std::max<size_t>(off, 16);
  HIP_TRY(ctx, ctx->step_stage.reserve(bytes), "step staging");
  HIP_TRY(ctx, ctx->d_step.reserve(bytes), "step buffer");
  char *h = static_cast<char *>(ctx->step_stage.ptr);
  auto put = [&](size_t o, const std::vector<int32_t> &v) {
    if (!v.empty()) memcpy(h + o, v.data(), v.size() * 4);
  };
  put(ctx->off_cu_q, ctx->cu_q);
  put(ctx->off_cu_k, ctx->cu_k);
  put(ctx->off_slots, ctx->slots);
  put(ctx->off_ctx, ctx->ctx_lens);
  put(ctx->off_tables, ctx->tables);
  put(ctx->off_pos, ctx->pos);
  HIP_TRY(ctx, ctx->step_stage.upload(ctx->d_step, bytes, ctx->stream), "step upload");
  return NVA_OK;
}

nva_status nva_step_positions(nva_ctx *ctx, const float *positions, int num_tokens) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (!ctx->has_step) return fail(ctx, NVA_E_NO_STEP, "no step metadata set on the context");
  if (num_tokens < 0 || (num_tokens > 0 && !positions))
    return fail(ctx, NVA_E_ARG, "positions required");
  std::vector<int32_t> pos(num_tokens);
  for (int t = 0; t < num_tokens; t++) pos[t] = java_round(positions[t]);
  if (ctx->has_pos && pos == ctx->pos) return NVA_OK;
  // Re-pack the step blob with the new positions at the end (the other arrays are unchanged).
  ctx->pos.swap(pos);
  ctx->has_pos = true;
  const size_t bytes = std::max<size_t>(ctx->off_pos + ctx->pos.size() * 4, 16);
  HIP_TRY(ctx, ctx->step_stage.reserve(bytes), "step staging");
  // reserve() may have reallocated the staging buffer: rebuild its content completely.
  char *h = static_cast<char *>(ctx->step_stage.ptr);
  auto put = [&](size_t o, const std::vector<int32_t> &v) {
    if (!v.empty()) memcpy(h + o, v.data(), v.size() * 4);
  };
  put(ctx->off_cu_q, ctx->cu_q);
  put(ctx->off_cu_k, ctx->cu_k);
  put(ctx->off_slots, ctx->slots);
  put(ctx->off_ctx, ctx->ctx_lens);
  put(ctx->off_tables, ctx->tables);
  put(ctx->off_pos, ctx->pos);
  if (ctx->d_step.cap < bytes) {
    // A larger blob needs a new device buffer; plans only hold offsets, so they stay valid.
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    HIP_TRY(ctx, ctx->d_step.reserve(bytes), "step buffer");
  }
  HIP_TRY(ctx, ctx->step_stage.upload(ctx->d_step, bytes, ctx->stream), "step upload");
  return NVA_OK;
}

nva_status nva_step_clear(nva_ctx *ctx) {
  if (!ctx) return NVA_E_ARG;
  ctx->has_step = false;
  for (Plan *p : ctx->plans) p->valid = false;
  return NVA_OK;
}

// ------------------------------------------------------------------------------- compute

nva_status nva_rope_forward(nva_ctx *ctx, const nva_rope *rope, const float *q, const float *k,
                            int num_tokens, int hq, int hk, float *q_out, float *k_out) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (!rope) return fail(ctx, NVA_E_ARG, "RoPE table is null");
  if (!ctx->has_step) return fail(ctx, NVA_E_NO_STEP, "no step metadata set on the context");
  if (num_tokens < 0 || hq < 0 || hk < 0) return fail(ctx, NVA_E_ARG, "negative shape");
  if (num_tokens == 0) return NVA_OK;  // empty batch: empty outputs, no pointers needed
  if (!q || !k || !q_out || !k_out) return fail(ctx, NVA_E_ARG, "q, k, q_out, k_out required");
  if (!aligned16(q) || !aligned16(k) || !aligned16(q_out) || !aligned16(k_out))
    return fail(ctx, NVA_E_ARG, "device pointers must be 16-byte aligned");
  nva_status st = check_positions(ctx, num_tokens, rope->max_pos);
  if (st != NVA_OK) return st;
  RopeStoreLaunch a{};
  a.xcd_hint = ctx->xcd_hint;
  a.q = q;
  a.k = k;
  a.v = nullptr;
  a.q_out = q_out;
  a.k_out = k_out;
  a.k_cache = nullptr;
  a.v_cache = nullptr;
  a.slots = nullptr;
  a.positions = ctx->dev_i32(ctx->off_pos);
  a.cos_sin = rope->table;
  a.tokens = num_tokens;
  a.hq = hq;
  a.hk = hk;
  a.head_dim = rope->head_size;
  Timed tm(ctx, "rope_store");
  HIP_TRY(ctx, launch_rope_store(a, ctx->stream, ctx->num_cus), "rope kernel launch");
  tm.done();
  return NVA_OK;
}

// Attention.forward: the store, then the attention kernels; scr selects the no-allocation
// workspace (null: the context's buffers).
static nva_status attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc *desc,
                                    const float *q, const float *k, const float *v,
                                    int num_tokens, float *out, Scratch *scr) {
  nva_status st = check_forward(ctx, kv, desc, num_tokens);
  if (st != NVA_OK) return st;
  if (num_tokens == 0) return NVA_OK;  // empty batch: an empty output, as Tensor.zeros(0, ...)
  if (!q || !out) return fail(ctx, NVA_E_ARG, "q and out are required");
  if (!aligned16(q) || !aligned16(out) || (k && !aligned16(k)) || (v && !aligned16(v)))
    return fail(ctx, NVA_E_ARG, "device pointers must be 16-byte aligned");
  const nva_attn_desc d = *desc;
  const int layer = d.kv_layer_index;
  if (scr) {
    st = noalloc_prepare(ctx, kv, d, num_tokens);
    if (st != NVA_OK) return st;
  }
  // Store first, Attention.java:157-160.
  if (d.write_kv && kv->k[layer] && ctx->has_slots && ctx->num_slots == num_tokens &&
      num_tokens > 0) {
    if (!k || !v) return fail(ctx, NVA_E_ARG, "k and v are required to store");
    st = check_slots(ctx, kv);
    if (st != NVA_OK) return st;
    RopeStoreLaunch a{};
    a.xcd_hint = ctx->xcd_hint;
    a.q = nullptr;
    a.k = k;
    a.v = v;
    a.k_cache = kv->k[layer];
    a.v_cache = kv->v[layer];
    a.slots = ctx->dev_i32(ctx->off_slots);
    a.positions = nullptr;
    a.tokens = num_tokens;
    a.hq = d.num_heads;
    a.hk = d.num_kv_heads;
    a.head_dim = d.head_dim;
    Timed tm(ctx, "store");
    HIP_TRY(ctx, launch_rope_store(a, ctx->stream, ctx->num_cus), "store kernel launch");
    tm.done();
  }
  return attention_after_store(ctx, kv, d, q, k, v, num_tokens, out, scr);
}

nva_status nva_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc *desc,
                                 const float *q, const float *k, const float *v, int num_tokens,
                                 float *out) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  return attention_forward(ctx, kv, desc, q, k, v, num_tokens, out, nullptr);
}

nva_status nva_attention_forward_noalloc(nva_ctx *ctx, nva_kv *kv, const nva_attn_desc *desc,
                                         const float *q, const float *k, const float *v,
                                         int num_tokens, float *out) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (!ctx->scratch)
    return fail(ctx, NVA_E_HIP, "device scratch array unavailable on device %d: %s",
                ctx->device, hipGetErrorString(ctx->scratch_err));
  Scratch scr;
  scr.base = ctx->scratch;
  return attention_forward(ctx, kv, desc, q, k, v, num_tokens, out, &scr);
}

nva_status nva_rope_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                      const nva_attn_desc *desc, const float *q,
                                      const float *k, const float *v, int num_tokens,
                                      float *q_out, float *k_out, float *out) {
  return nva_norm_rope_attention_forward(ctx, kv, rope, nullptr, nullptr, nullptr, desc, q, k, v,
                                         num_tokens, q_out, k_out, out);
}

// The head norms, RoPE, the store and attention with q, k, v rows read at token strides q_ld,
// k_ld, v_ld (floats): [T, heads, d] inputs, or the packed qkv_proj output.
static nva_status norm_rope_attention(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                      const nva_rms_norm *q_norm, const nva_rms_norm *k_norm,
                                      const nva_rms_norm *v_norm, const nva_attn_desc *desc,
                                      const float *q, const float *k, const float *v, int q_ld,
                                      int k_ld, int v_ld, int num_tokens, float *q_out,
                                      float *k_out, float *out) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  nva_status st = check_forward(ctx, kv, desc, num_tokens);
  if (st != NVA_OK) return st;
  if (!rope) return fail(ctx, NVA_E_ARG, "RoPE table is null");
  if (rope->head_size != desc->head_dim)
    return fail(ctx, NVA_E_ARG, "RoPE head size %d != headDim %d", rope->head_size,
                desc->head_dim);
  if (num_tokens == 0) return NVA_OK;  // empty batch
  if (!q || !k || !v || !out) return fail(ctx, NVA_E_ARG, "q, k, v and out are required");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      (q_out && !aligned16(q_out)) || (k_out && !aligned16(k_out)))
    return fail(ctx, NVA_E_ARG, "device pointers must be 16-byte aligned");
  for (const nva_rms_norm *n : {q_norm, k_norm, v_norm})
    if (n && n->weight && !aligned16(n->weight))
      return fail(ctx, NVA_E_ARG, "RMSNorm weights must be 16-byte aligned device pointers");
  st = check_positions(ctx, num_tokens, rope->max_pos);
  if (st != NVA_OK) return st;
  const nva_attn_desc d = *desc;
  const int layer = d.kv_layer_index;
  const size_t qn = (size_t)num_tokens * d.num_heads * d.head_dim;
  const size_t kn = (size_t)num_tokens * d.num_kv_heads * d.head_dim;
  if (!q_out) {
    HIP_TRY(ctx, ctx->d_q_rot.reserve(qn * 4 + 16), "rotated q scratch");
    q_out = static_cast<float *>(ctx->d_q_rot.ptr);
  }
  const bool dense = ctx->is_prefill && !ctx->has_tables;
  if (!k_out && dense) {
    HIP_TRY(ctx, ctx->d_k_rot.reserve(kn * 4 + 16), "rotated k scratch");
    k_out = static_cast<float *>(ctx->d_k_rot.ptr);
  }
  // Dense prefill attends over the step's own k/v rows, so a normalised v (or the v of packed
  // inputs) must exist as contiguous rows.
  const bool v_packed = v_ld != d.num_kv_heads * d.head_dim;
  float *v_out = nullptr;
  if ((v_norm || v_packed) && dense) {
    HIP_TRY(ctx, ctx->d_v_norm.reserve(kn * 4 + 16), "normalised v scratch");
    v_out = static_cast<float *>(ctx->d_v_norm.ptr);
  }
  const bool store = d.write_kv && kv->k[layer] && ctx->has_slots &&
                     ctx->num_slots == num_tokens;
  if (store) {
    st = check_slots(ctx, kv);
    if (st != NVA_OK) return st;
  }
  RopeStoreLaunch a{};
  a.xcd_hint = ctx->xcd_hint;
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_ld = q_ld;
  a.k_ld = k_ld;
  a.v_ld = v_ld;
  a.q_out = q_out;
  a.k_out = k_out;
  a.v_out = v_out;
  a.k_cache = store ? kv->k[layer] : nullptr;
  a.v_cache = store ? kv->v[layer] : nullptr;
  a.slots = store ? ctx->dev_i32(ctx->off_slots) : nullptr;
  a.positions = ctx->dev_i32(ctx->off_pos);
  a.cos_sin = rope->table;
  a.tokens = num_tokens;
  a.hq = d.num_heads;
  a.hk = d.num_kv_heads;
  a.head_dim = d.head_dim;
  a.qn = head_norm(q_norm);
  a.kn = head_norm(k_norm);
  a.vn = head_norm(v_norm);
  if (rope_store_norm_lds(a) > kRopeNormMaxLds)
    return fail(ctx, NVA_E_UNSUPPORTED, "head norms of %d+2*%d heads of %d floats exceed the "
                "kernel's %zu-byte LDS budget", a.hq, a.hk, a.head_dim, kRopeNormMaxLds);
  {
    Timed tm(ctx, "rope_store");
    HIP_TRY(ctx, launch_rope_store(a, ctx->stream, ctx->num_cus), "rope_store kernel launch");
    tm.done();
  }
  return attention_after_store(ctx, kv, d, q_out, k_out, v_out ? v_out : v, num_tokens, out);
}

nva_status nva_norm_rope_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                           const nva_rms_norm *q_norm,
                                           const nva_rms_norm *k_norm,
                                           const nva_rms_norm *v_norm,
                                           const nva_attn_desc *desc, const float *q,
                                           const float *k, const float *v, int num_tokens,
                                           float *q_out, float *k_out, float *out) {
  if (!ctx) return NVA_E_ARG;
  if (!desc) return fail(ctx, NVA_E_ARG, "attention descriptor is null");
  return norm_rope_attention(ctx, kv, rope, q_norm, k_norm, v_norm, desc, q, k, v,
                             desc->num_heads * desc->head_dim,
                             desc->num_kv_heads * desc->head_dim,
                             desc->num_kv_heads * desc->head_dim, num_tokens, q_out, k_out, out);
}

nva_status nva_qkv_norm_rope_attention_forward(nva_ctx *ctx, nva_kv *kv, const nva_rope *rope,
                                               const nva_rms_norm *q_norm,
                                               const nva_rms_norm *k_norm,
                                               const nva_rms_norm *v_norm,
                                               const nva_attn_desc *desc, const float *qkv,
                                               int num_tokens, float *q_out, float *k_out,
                                               float *out) {
  if (!ctx) return NVA_E_ARG;
  if (!desc) return fail(ctx, NVA_E_ARG, "attention descriptor is null");
  if (!qkv && num_tokens != 0) return fail(ctx, NVA_E_ARG, "qkv is required");
  const int64_t qs = (int64_t)desc->num_heads * desc->head_dim;
  const int64_t ks = (int64_t)desc->num_kv_heads * desc->head_dim;
  if (qs <= 0 || ks <= 0 || qs + 2 * ks > INT32_MAX)
    return fail(ctx, NVA_E_ARG, "bad head counts %d/%d x %d", desc->num_heads,
                desc->num_kv_heads, desc->head_dim);
  const int ld = (int)(qs + 2 * ks);
  if (!qkv)  // empty batch: checks only
    return norm_rope_attention(ctx, kv, rope, q_norm, k_norm, v_norm, desc, nullptr, nullptr,
                               nullptr, ld, ld, ld, 0, q_out, k_out, out);
  return norm_rope_attention(ctx, kv, rope, q_norm, k_norm, v_norm, desc, qkv, qkv + qs,
                             qkv + qs + ks, ld, ld, ld, num_tokens, q_out, k_out, out);
}

nva_status nva_linear_forward(nva_ctx *ctx, const float *x, int rows, int in,
                              const float *weight, int out, const float *bias, float *y) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (rows < 0 || in <= 0 || out <= 0)
    return fail(ctx, NVA_E_ARG, "bad linear shape rows=%d in=%d out=%d", rows, in, out);
  if (rows == 0) return NVA_OK;
  if (!x || !weight || !y) return fail(ctx, NVA_E_ARG, "x, weight and y are required");
  if (in % 4 != 0)
    return fail(ctx, NVA_E_UNSUPPORTED, "linear needs in %% 4 == 0 (got %d)", in);
  // The kernels address a tile's 128 rows with 32-bit byte offsets.
  if (in >= (1 << 22))
    return fail(ctx, NVA_E_UNSUPPORTED, "linear needs in < 4194304 (got %d)", in);
  if (!aligned16(x) || !aligned16(weight))
    return fail(ctx, NVA_E_ARG, "x and weight must be 16-byte aligned device pointers");
  const int cus = std::max(1, ctx->num_cus);
  const int64_t blocks = (int64_t)((out + 31) / 32) * ((rows + 31) / 32);
  if (rows <= linear_gemv_max_rows()) {
    // A few rows: stream W once (GEMV), no tiles, no K slices.
    LinearLaunch g{};
    g.x = x;
    g.w = weight;
    g.bias = bias;
    g.y = y;
    g.m = rows;
    g.n = out;
    g.k = in;
    g.splits = 1;
    g.k_per_split = in;
    Timed tm(ctx, "linear");
    HIP_TRY(ctx, launch_gemv(g, ctx->stream), "gemv kernel launch");
    tm.done();
    return NVA_OK;
  }
  const int64_t blocks16 = (int64_t)((out + 15) / 16) * ((rows + 15) / 16);
  if (2 * blocks <= cus && 2 * blocks16 >= cus && blocks16 <= 2 * (int64_t)cus) {
    // Decode batches whose 32 x 32 blocks would fill at most half the CUs: 16 x 16 blocks, one
    // or two per CU, K over each workgroup's waves and no slices, so no reduce launch (Qwen3
    // o_proj at 64 rows 6.2 + 3.0 us -> 5.9 us, at 128 rows 9.1 + 2.4 -> 9.1 us).
    LinearLaunch g{};
    g.x = x;
    g.w = weight;
    g.bias = bias;
    g.y = y;
    g.m = rows;
    g.n = out;
    g.k = in;
    g.splits = 1;
    g.k_per_split = in;
    Timed tm(ctx, "linear");
    HIP_TRY(ctx, launch_skinny16(g, ctx->stream), "skinny16 linear kernel launch");
    tm.done();
    return NVA_OK;
  }
  if (blocks <= cus) {
    // Decode batches: 32 x 32 blocks (one workgroup per CU, its LDS ring fills the CU), K
    // sliced only while the blocks leave CUs idle: the most slices s with blocks * s <= CUs
    // that keep a 32-k stage for every wave of a slice.
    const int kmin = linear_skinny_waves() * 32;
    int splits = 1;
    while (blocks * (splits + 1) <= cus && in / (splits + 1) >= kmin) splits++;
    const int kps = ((in + splits - 1) / splits + 31) / 32 * 32;
    LinearLaunch g{};
    g.x = x;
    g.w = weight;
    g.bias = bias;
    g.y = y;
    g.m = rows;
    g.n = out;
    g.k = in;
    g.splits = (in + kps - 1) / kps;
    g.k_per_split = kps;
    if (g.splits > 1) {
      HIP_TRY(ctx, ctx->d_lin.reserve((size_t)g.splits * rows * out * sizeof(float)),
              "linear partial buffer");
      g.part = static_cast<float *>(ctx->d_lin.ptr);
    }
    Timed tm(ctx, "linear");
    HIP_TRY(ctx, launch_skinny(g, ctx->stream), "skinny linear kernel launch");
    tm.done();
    return NVA_OK;
  }
  // K slices: the count s that minimises a per-CU cost model.  Two 128 x 64 workgroups share a
  // CU and run their K tiles together at about 1.8 us per pair of 128 x 64 x 32 tiles, so the
  // kernel takes ceil(tiles * s / (2 CUs)) rounds of ceil(K tiles / s) K tiles; s > 1 adds the
  // partial planes (written, then read by the reduce, at about 5 TB/s) and the reduce launch.
  // Every slice keeps at least 4 K tiles.
  const int64_t tiles = (int64_t)((out + linear_tile_cols() - 1) / linear_tile_cols()) *
                        ((rows + linear_tile_rows() - 1) / linear_tile_rows());
  const int bk = linear_k_tile();
  const int nkt = (in + bk - 1) / bk;
  const int64_t slots = 2 * (int64_t)cus;
  int splits = 1;
  double best = 0.0;
  for (int sl = 1; sl <= std::max(1, nkt / 4); sl++) {
    const int per = (nkt + sl - 1) / sl;
    if (sl > 1 && (nkt + per - 1) / per != sl) continue;  // same slices as a smaller count
    const double rounds = (double)((tiles * sl + slots - 1) / slots);
    double us = rounds * per * 1.8;
    if (sl > 1) us += 2.0 * sl * (double)rows * out * 4.0 / 5.0e6 + 3.0;
    if (sl == 1 || us < best) {
      best = us;
      splits = sl;
    }
  }
  const int kt_per = (nkt + splits - 1) / splits;
  splits = (nkt + kt_per - 1) / kt_per;
  LinearLaunch a{};
  a.x = x;
  a.w = weight;
  a.bias = bias;
  a.y = y;
  a.m = rows;
  a.n = out;
  a.k = in;
  a.splits = splits;
  a.k_per_split = kt_per * bk;
  if (splits > 1) {
    HIP_TRY(ctx, ctx->d_lin.reserve((size_t)splits * rows * out * sizeof(float)),
            "linear partial buffer");
    a.part = static_cast<float *>(ctx->d_lin.ptr);
  }
  Timed tm(ctx, "linear");
  HIP_TRY(ctx, launch_linear(a, ctx->stream), "linear kernel launch");
  tm.done();
  return NVA_OK;
}

nva_status nva_rms_norm_forward(nva_ctx *ctx, const nva_rms_norm *norm, const float *x, int rows,
                                int width, float *out) {
  if (!ctx) return NVA_E_ARG;
  DeviceGuard dg(ctx);
  if (!norm) return fail(ctx, NVA_E_ARG, "RMSNorm descriptor is null");
  if (rows < 0 || width <= 0) return fail(ctx, NVA_E_ARG, "bad shape [%d, %d]", rows, width);
  if (rows > 0 && (!x || !out)) return fail(ctx, NVA_E_ARG, "x and out are required");
  NormLaunch a{};
  a.x = x;
  a.out = out;
  a.norm = head_norm(norm);
  a.rows = rows;
  a.width = width;
  Timed tm(ctx, "rms_norm");
  HIP_TRY(ctx, launch_rms_norm(a, ctx->stream), "rms_norm kernel launch");
  tm.done();
  return NVA_OK;
}

}  // extern "C"
