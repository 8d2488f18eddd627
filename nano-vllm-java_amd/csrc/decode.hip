// Kernel (b): split-KV GQA/MQA attention of single query rows over the paged KV cache, and
// the merge of split partials.
//
// Semantics (layers/Attention.java:285-299 decode, :328-396 attendJobs): query row r of head
// h attends keys [kbeg, kend) of its sequence through the block table
// (slot(t) = table[t / BS] * BS + t % BS, Attention.java:131-137) with the KV head
// kvh = h / rep, score = dot(q, k) * scale, softmax over the keys, out = sum(w v) / sum(w),
// and out = 0 when no key is visible.  The reference's 64-key online softmax is replaced by a
// per-stream online softmax over 8-key groups and a final log-sum-exp merge of the streams, in
// the log2 domain (scores scaled by scale * log2 e, v_exp_f32); the result agrees with the
// reference to fp32 rounding.
//
// Mapping onto CDNA4 (wave64):
//   * one workgroup (4 waves) per (work item, KV head, group of HPW query heads); a work item
//     is one query row and a chunk of its key range (the host splits long rows so that every
//     workgroup reads about the same number of bytes and the grid has thousands of groups);
//   * a K/V row (D fp32) is read by LPT lanes, VPL float4 each (VPL = 2 from d = 32 on, with at
//     most 4 heads per workgroup): each wave load instruction fetches TPW = 64/LPT whole rows,
//     i.e. contiguous 128-byte lines, and all HPW query heads of the KV head reuse the registers
//     (K/V are read from HBM exactly once per KV head);
//   * paged K/V with power-of-two pages: a wave's rows of one register group lie in one page,
//     so their address is formed in scalar registers and the loads take a fixed per-lane offset
//     (the vector ALU does the attention arithmetic only);
//   * the dot products are reduced across the LPT lanes with DPP row ops and gfx950's row
//     swaps (no LDS traffic); each group of LPT lanes is an independent online-softmax stream;
//   * the TPW streams of a wave fold together with lane shuffles, the 4 waves' results merge
//     through LDS, and either the output row (unsplit item) or the partial (m, l, acc) of the
//     chunk is written;
//   * where the planner gives a workgroup 5 to 16 query heads of one KV head (d = 64 and 128,
//     power-of-two pages of >= 16 tokens), row_mfma_kernel runs the same units on fp32 MFMA.
// HBM bytes per work item: chunk * 2 * D * 4 per KV head (+ q, + the partial or output row).
#include "nva_internal.h"
#include "nva_device.h"

namespace nva {

// KV head of this workgroup's unit.  Workgroups go to the 8 XCDs in turn, continuing from the
// launch before, and with 2, 4 or 8 units per item each XCD reads one KV head (a 512-byte slice of
// every token row at d = 128, 256 bytes at d = 64).  Which parity of head index each XCD should read depends on the
// kernel (measured at the headline's rows and contexts): the row kernel runs 2.16-2.17 ms at
// 16 q / 8 KV heads when the head index has the parity of the XCD id and 2.22-2.25 ms with the
// other (1.098 against 1.133 ms at 8 q / 4 KV heads, 0.567 against 0.584 ms at 4 q / 2 KV
// heads), the MFMA row kernel the other way round
// (40 q / 8 KV heads 2.269 against 2.282-2.288 ms, 28 q / 4 KV heads 1.171 against 1.189 ms).
// At d = 64, where a head's rows start 256 bytes apart instead of 512, both flip (row kernel at
// 32 q / 8 KV heads 1.129 against 1.158 ms with the other parity, MFMA row kernel at 14 q / 2
// KV heads 0.319 against 0.323 ms with the same).
// The launch before (kernel (a)) recorded the XCD of its last workgroup, and this launch's
// first workgroup runs on the next one (checked with per-launch XCD stamps); every workgroup
// reads the same recorded value and rotates the heads by the same amount, so the units stay a
// bijection whatever the placement.
__device__ __forceinline__ int unit_kv_head(const RowLaunch &a, int kvh) {
  if (!a.rotate_heads || !a.xcd_hint) return kvh;
  const int first_xcd = (a.xcd_hint[0] + 1) & 7;  // XCD of block 0 under in-turn dispatch
  // block b: XCD (b + first_xcd) mod 8, and b mod hkv is the unit's KV head before rotation
  const int r = (first_xcd & 1) ^ (a.mfma ? 1 : 0) ^ (a.head_dim == 64 ? 1 : 0);
  return (kvh + r) & (a.hkv - 1);
}

namespace {

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

// K/V rows are read once per step: non-temporal loads stream them past the caches, which
// sustains a higher HBM read rate than ordinary loads.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4_stream(const float *p) {
  const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}
// The same non-temporal load from a wave-uniform base plus a 32-bit lane offset (floats), as a
// buffer load: the base stays in scalar registers, so no per-lane 64-bit address is formed
// (headline decode 2.160-2.162 against 2.166-2.171 ms with the pointer form).  The cache policy
// matters, the form little: without the non-temporal bit the same loads take 2.40 ms, and
// adding the L1-bypass (sc0) or device-scope (sc1) bits changes nothing.
__device__ __forceinline__ float4 ld4_stream_at(const float *base, uint32_t off) {
  constexpr int kNonTemporal = 2;  // the nt bit of the buffer instructions' cache policy
  const uint64_t b = (uint64_t)(size_t)base;
  const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void *)(size_t)u, (short)0, 0x7fffffff, kBufferWord3);
  const f32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, off * 4, 0, kNonTemporal);
  return make_float4(t.x, t.y, t.z, t.w);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_amdgcn_update_dpp(0.0f, x, CTRL, 0xF, 0xF, false);
}

// x[lane] + x[lane ^ 16] (resp. lane ^ 32) in every lane, by gfx950's row-swap instructions:
// the swap of x with itself leaves one of the two values in each output, and the sum of the
// two is the same bits in both lanes of a pair.  No LDS round trip, unlike ds_swizzle or
// ds_bpermute.
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Max and sum over the four lanes {l, l ^ 16, l ^ 32, l ^ 48}; every lane gets the same bits.
__device__ __forceinline__ float max4_lanes(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float m = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false,
                                                  false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float sum4_lanes(float x) { return add_xor32(add_xor16(x)); }

// Sum of x over aligned groups of LPT lanes; every lane of the group receives the sum.
template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (LPT >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (LPT >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (LPT >= 8) x += dpp<0x141>(x);  // row_half_mirror
  if constexpr (LPT >= 16) x += dpp<0x140>(x); // row_mirror
  if constexpr (LPT >= 32) x = add_xor16(x);
  if constexpr (LPT >= 64) x = add_xor32(x);
  return x;
}

__device__ __forceinline__ int page_of(const KvView &kv, int t) {
  return kv.bs_shift >= 0 ? t >> kv.bs_shift : t / kv.block_size;
}

// Row of key t: dense rows follow kbase; paged rows go through the LDS copy of the item's
// block ids, which starts at page blk0.
__device__ __forceinline__ int64_t kv_row(const KvView &kv, const int32_t *stab, int blk0,
                                          int kbase, int t) {
  if (!kv.paged) return (int64_t)kbase + t;
  const int blk = page_of(kv, t);
  const int off = t - blk * kv.block_size;
  return (int64_t)stab[blk - blk0] * kv.block_size + off;
}

}  // namespace

// Lane layout of the K/V rows, per head dim and heads per workgroup: a row is read by LPT lanes
// holding VPL float4 each, so a lane's part of a dot product is 4 * VPL fmas before the LPT-lane
// reduction; TPW rows per wave load instruction, UH rows per lane per register group and
// G = TPW * UH rows per wave per group.  VPL = 2 from d = 32 on halves the reduction steps per
// key against one float4 per lane (d = 128: 16 lanes per row, all within one DPP row); eight
// heads per workgroup keep one float4 per lane, as q and the accumulators then take 16
// registers per head.
template <int D, int HPW>
struct RowShape {
  static constexpr int VPL = D >= 512 ? 2 : (D >= 32 && HPW <= 4 ? 2 : 1);
  static constexpr int LPT = D / (4 * VPL);
  static constexpr int TPW = 64 / LPT;
  static constexpr int UH = 4 / VPL;
  static constexpr int G = TPW * UH;
};

// PAGED_ALIGNED: paged K/V whose block size is a power of two and a multiple of G.  A wave's
// register groups then start at multiples of G, so each group's G rows lie in one page and
// are consecutive there: the group's first row address is formed once in scalar registers
// (block id from the staged table, read only when the page changes) and every lane adds a
// fixed 32-bit offset, so a K/V load costs no vector instruction.  Other layouts (dense K/V,
// small pages) form each lane's row address from its key.
template <int D, int HPW, bool PAGED_ALIGNED>
__global__ void __launch_bounds__(256) row_attention_kernel(RowLaunch a) {
  using S = RowShape<D, HPW>;
  constexpr int LPT = S::LPT, VPL = S::VPL, TPW = S::TPW, UH = S::UH, G = S::G;
  // d = 512 with 8 heads: q lives in LDS (in registers its 64 values per lane left one wave per
  // SIMD), and the waves' final states merge in two passes of 4 heads to bound the LDS.
  constexpr bool QL = D >= 512 && HPW >= 8;
  constexpr int HA = QL ? HPW / 2 : HPW;  // heads per pass of the final merge
  __shared__ float sm_m[4][HPW];
  __shared__ float sm_l[4][HPW];
  __shared__ float4 sm_acc[4][HA][D / 4];
  __shared__ float4 sq[QL ? HPW : 1][QL ? D / 4 : 1];
  __shared__ int32_t stab[kRowTablePages];  // block ids of the pages this item touches

  const int rep = a.hq / a.hkv;
  const int groups = rep / HPW;
  const int per_item = a.hkv * groups;
  const int item = blockIdx.x / per_item;
  const int gy = blockIdx.x - item * per_item;
  const RowItem it = a.items[item];
  const int kvh = unit_kv_head(a, gy / groups);
  const int h0 = kvh * rep + (gy - (gy / groups) * groups) * HPW;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane / LPT;
  const int c = lane - sub * LPT;

  // Lane c holds dims [4c + 4*LPT*j, +4) for j < VPL, so each load instruction is contiguous.
  // q is pre-scaled by scale * log2(e): the dot products come out in log2 units.
  const float sl2 = a.scale * 1.4426950408889634f;
  float4 qv[QL ? 1 : HPW][VPL];
  if constexpr (QL) {
    for (int idx = threadIdx.x; idx < HPW * (D / 4); idx += blockDim.x) {
      const int h = idx / (D / 4);
      const int cc = idx - h * (D / 4);
      const float4 x = ld4(a.q + ((size_t)it.qrow * a.hq + h0 + h) * D + cc * 4);
      sq[h][cc] = make_float4(x.x * sl2, x.y * sl2, x.z * sl2, x.w * sl2);
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int h = 0; h < HPW; h++)
#pragma unroll
      for (int j = 0; j < VPL; j++) {
        const float4 x = ld4(a.q + ((size_t)it.qrow * a.hq + h0 + h) * D + (c + LPT * j) * 4);
        qv[h][j] = make_float4(x.x * sl2, x.y * sl2, x.z * sl2, x.w * sl2);
      }
  }

  const size_t rs = (size_t)a.hkv * D;
  // Stage the item's block ids in LDS once (the host caps items at kRowTablePages pages), so
  // a row address waits on an LDS read instead of on every K/V load issued before it.
  int blk0 = 0;
  // An item within at most two pages carries their block ids, so its first K/V loads wait on no
  // table read.
  const bool inl = a.kv.paged && it.blk_a != 0;
  if (a.kv.paged) blk0 = page_of(a.kv, it.kbeg);
  if (a.kv.paged && !inl) {
    const int32_t *table = a.kv.table + (size_t)it.seq * a.kv.bt_stride;
    const int npages = it.kend > it.kbeg ? page_of(a.kv, it.kend - 1) - blk0 + 1 : 0;
    for (int j = threadIdx.x; j < npages; j += blockDim.x) stab[j] = table[blk0 + j];
    __syncthreads();
  }

  float m[HPW], l[HPW];
  float4 acc[HPW][VPL];
#pragma unroll
  for (int h = 0; h < HPW; h++) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) acc[h][j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Aligned layouts start the groups at the multiple of G at or below the first key; the keys
  // before it are masked.
  const int gfirst = PAGED_ALIGNED ? (it.kbeg & ~(G - 1)) : it.kbeg;
  const uint32_t lane_off = (uint32_t)(sub * rs + c * 4);  // floats from the group's first row
  const float *kbase_h = a.kv.k + (size_t)kvh * D;
  const float *vbase_h = a.kv.v + (size_t)kvh * D;
  int cur_page = -1;      // page whose first row is cur_row0 (wave-uniform)
  int64_t cur_row0 = 0;

  // Two register groups of UH rows per stream: the loads of the next group are issued before
  // the current one is folded, so every wave keeps loads in flight while it computes.  The
  // issue is unconditional (a group past the end reloads the item's first group, masked),
  // which keeps the wait before each fold to exactly the current group's loads.
  float4 kra[UH][VPL], vra[UH][VPL], krb[UH][VPL], vrb[UH][VPL];
  bool oka[UH], okb[UH];
  auto issue = [&](int g0, float4(&kr)[UH][VPL], float4(&vr)[UH][VPL], bool(&ok)[UH]) {
    if constexpr (PAGED_ALIGNED) {
      const int gq = g0 < it.kend ? g0 : gfirst;
      const int p = gq >> a.kv.bs_shift;
      if (p != cur_page) {
        const int id = inl ? (p == blk0 ? it.blk_a - 1 : it.blk_b)
                           : __builtin_amdgcn_readfirstlane(stab[p - blk0]);
        cur_page = p;
        cur_row0 = (int64_t)id * a.kv.block_size - ((int64_t)p << a.kv.bs_shift);
      }
      const int64_t row = cur_row0 + gq;
      const float *kb = kbase_h + row * rs;
      const float *vb = vbase_h + row * rs;
      // Lane offsets (floats) of the group's rows.  In a partial group (the item's first or
      // last, or one past its end that reloads the first) masked keys may sit on page slots
      // never written (any bits, NaN included), so each lane reads the group's key nearest its
      // own inside [kbeg, kend) instead, whose finite V row adds exactly 0 at weight 0.
      uint32_t off[UH];
      if (g0 >= it.kbeg && g0 + G <= it.kend) {
#pragma unroll
        for (int u = 0; u < UH; u++) {
          ok[u] = true;
          off[u] = lane_off + (uint32_t)(u * TPW * rs);
        }
      } else {
#pragma unroll
        for (int u = 0; u < UH; u++) {
          const int t = g0 + u * TPW + sub;
          ok[u] = t >= it.kbeg && t < it.kend;
          // (A group past the end reads only the item's first key: its loads are never folded.)
          const int tq = gq + u * TPW + sub;
          const int tc = g0 >= it.kend ? it.kbeg : min(max(tq, it.kbeg), it.kend - 1);
          off[u] = (uint32_t)__mul24(tc - gq, (int)rs) + c * 4;
        }
      }
#pragma unroll
      for (int u = 0; u < UH; u++)
#pragma unroll
        for (int j = 0; j < VPL; j++) {
          kr[u][j] = ld4_stream_at(kb, off[u] + LPT * 4 * j);  // kb, vb: wave-uniform
          vr[u][j] = ld4_stream_at(vb, off[u] + LPT * 4 * j);
        }
    } else {
#pragma unroll
      for (int u = 0; u < UH; u++) {
        const int t = g0 + u * TPW + sub;
        ok[u] = t < it.kend;
        const int tt = ok[u] ? t : it.kbeg;
        int64_t row;
        if (inl) {
          const int blk = page_of(a.kv, tt);
          const int id = blk == blk0 ? it.blk_a - 1 : it.blk_b;
          row = (int64_t)id * a.kv.block_size + (tt - blk * a.kv.block_size);
        } else {
          row = kv_row(a.kv, stab, blk0, it.kbase, tt);
        }
#pragma unroll
        for (int j = 0; j < VPL; j++) {
          kr[u][j] = ld4_stream(kbase_h + row * rs + c * 4 + LPT * 4 * j);
          vr[u][j] = ld4_stream(vbase_h + row * rs + c * 4 + LPT * 4 * j);
        }
      }
    }
  };
  auto fold = [&](const float4(&kr)[UH][VPL], const float4(&vr)[UH][VPL], const bool(&ok)[UH]) {
    // With q in LDS, keep its reads in the loop: hoisted out of it they would take the
    // registers this layout frees.
    if constexpr (QL) asm volatile("" ::: "memory");
#pragma unroll
    for (int h = 0; h < HPW; h++) {
      float4 qh[VPL];
#pragma unroll
      for (int j = 0; j < VPL; j++) {
        if constexpr (QL) qh[j] = sq[h][c + LPT * j];
        else qh[j] = qv[h][j];
      }
      float s[UH];
#pragma unroll
      for (int u = 0; u < UH; u++) {
        float p = qh[0].x * kr[u][0].x;
        p = fmaf(qh[0].y, kr[u][0].y, p);
        p = fmaf(qh[0].z, kr[u][0].z, p);
        p = fmaf(qh[0].w, kr[u][0].w, p);
#pragma unroll
        for (int j = 1; j < VPL; j++) {
          p = fmaf(qh[j].x, kr[u][j].x, p);
          p = fmaf(qh[j].y, kr[u][j].y, p);
          p = fmaf(qh[j].z, kr[u][j].z, p);
          p = fmaf(qh[j].w, kr[u][j].w, p);
        }
        s[u] = group_sum<LPT>(p);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < UH; u++) {
        s[u] = ok[u] ? s[u] : -INFINITY;
        mx = fmaxf(mx, s[u]);
      }
      const float mn = fmaxf(m[h], mx);
      const float ms = mn == -INFINITY ? 0.0f : mn;
      const float alpha = __builtin_amdgcn_exp2f(m[h] - ms);
      float ls = 0.0f;
      float4 av[VPL];
#pragma unroll
      for (int j = 0; j < VPL; j++) av[j] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < UH; u++) {
        const float w = __builtin_amdgcn_exp2f(s[u] - ms);
        ls += w;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
          av[j].x = fmaf(w, vr[u][j].x, av[j].x);
          av[j].y = fmaf(w, vr[u][j].y, av[j].y);
          av[j].z = fmaf(w, vr[u][j].z, av[j].z);
          av[j].w = fmaf(w, vr[u][j].w, av[j].w);
        }
      }
      l[h] = fmaf(l[h], alpha, ls);
#pragma unroll
      for (int j = 0; j < VPL; j++) {
        acc[h][j].x = fmaf(acc[h][j].x, alpha, av[j].x);
        acc[h][j].y = fmaf(acc[h][j].y, alpha, av[j].y);
        acc[h][j].z = fmaf(acc[h][j].z, alpha, av[j].z);
        acc[h][j].w = fmaf(acc[h][j].w, alpha, av[j].w);
      }
      m[h] = mn;
    }
  };

  int g0 = gfirst + wave * G;
  if (g0 < it.kend) {
    issue(g0, kra, vra, oka);
    for (;;) {
      issue(g0 + 4 * G, krb, vrb, okb);
      fold(kra, vra, oka);
      g0 += 4 * G;
      if (g0 >= it.kend) break;
      issue(g0 + 4 * G, kra, vra, oka);
      fold(krb, vrb, okb);
      g0 += 4 * G;
      if (g0 >= it.kend) break;
    }
  }

  // The TPW streams of a wave fold into the lanes of stream 0 (each lane with the stream
  // LPT * 2^i lanes above it, lower stream first), then the waves' streams merge through LDS.
#pragma unroll
  for (int dist = LPT; dist < 64; dist <<= 1) {
#pragma unroll
    for (int h = 0; h < HPW; h++) {
      const float mo = __shfl_xor(m[h], dist);
      const float lo = __shfl_xor(l[h], dist);
      const float M = fmaxf(m[h], mo);
      const float Ms = M == -INFINITY ? 0.0f : M;
      const float ea = __builtin_amdgcn_exp2f(m[h] - Ms);
      const float eb = __builtin_amdgcn_exp2f(mo - Ms);
      l[h] = fmaf(lo, eb, l[h] * ea);
#pragma unroll
      for (int j = 0; j < VPL; j++) {
        float4 &x = acc[h][j];
        x.x = fmaf(__shfl_xor(x.x, dist), eb, x.x * ea);
        x.y = fmaf(__shfl_xor(x.y, dist), eb, x.y * ea);
        x.z = fmaf(__shfl_xor(x.z, dist), eb, x.z * ea);
        x.w = fmaf(__shfl_xor(x.w, dist), eb, x.w * ea);
      }
      m[h] = M;
    }
  }
#pragma unroll
  for (int pass = 0; pass < HPW / HA; pass++) {
  if (pass > 0) __syncthreads();  // the previous pass has read sm_acc
  if (sub == 0) {
#pragma unroll
    for (int h = 0; h < HPW; h++) {
      if (pass == 0 && c == 0) {
        sm_m[wave][h] = m[h];
        sm_l[wave][h] = l[h];
      }
      if (h / HA == pass) {
#pragma unroll
        for (int j = 0; j < VPL; j++) sm_acc[wave][h - pass * HA][c + LPT * j] = acc[h][j];
      }
    }
  }
  __syncthreads();

  // sm_acc[.][h - pass * HA][cc] holds dims [4cc, 4cc + 4) of head h.
  for (int idx = threadIdx.x; idx < HA * (D / 4); idx += blockDim.x) {
    const int hl = idx / (D / 4);
    const int h = pass * HA + hl;
    const int cc = idx - hl * (D / 4);
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < 4; s++) M = fmaxf(M, sm_m[s][h]);
    const float Ms = M == -INFINITY ? 0.0f : M;
    float L = 0.0f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const float e = __builtin_amdgcn_exp2f(sm_m[s][h] - Ms);
      L = fmaf(sm_l[s][h], e, L);
      const float4 x = sm_acc[s][hl][cc];
      A.x = fmaf(x.x, e, A.x);
      A.y = fmaf(x.y, e, A.y);
      A.z = fmaf(x.z, e, A.z);
      A.w = fmaf(x.w, e, A.w);
    }
    if (it.part < 0) {
      const float inv = L == 0.0f ? 0.0f : 1.0f / L;
      st4(a.out + ((size_t)it.qrow * a.hq + h0 + h) * D + cc * 4,
          make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv));
    } else {
      const size_t p = (size_t)it.part * a.hq + h0 + h;
      st4(a.part_acc + p * D + cc * 4, A);
      if (cc == 0) {
        a.part_m[p] = M;
        a.part_l[p] = L;
      }
    }
  }
  }  // passes
}

// Split-KV decode with several query heads per KV head on fp32 MFMA (v_mfma_f32_16x16x4_f32),
// for paged K/V whose pages are a power of two of at least 16 keys, at d = 64 and 128.  The
// unit of work is the row kernel's: one query row x one key chunk x one KV head x HPW query
// heads (HPW <= 16); each wave takes 16-key blocks of the chunk in turn (wave w: blocks w,
// w + 4, ...), so the 4 waves read 64 consecutive keys at a time.
//   S^T[key][head] = K Q^T  D/4 MFMAs per block: at step s = 4v + c lane (i, g) supplies
//                           K[t0 + i][16v + 4g + c] (A) and Q[h0 + i][16v + 4g + c] (B, zero
//                           for i >= HPW), i = lane % 16, g = lane / 16; lane (j, g) then holds
//                           the scores of head j for keys t0 + 4g + r in st[r];
//   O^T[dim][head] += V^T P^T  4 x D/16 MFMAs per block: step s contracts key t0 + 4g + s,
//                           whose probability is this lane's own p[s] (B), against V[that
//                           key][64w + 4i + c] (A) in block b = 4w + c, so P never leaves the
//                           registers.
// Each K load instruction reads 64 contiguous bytes of each of 16 rows and each V load 256
// contiguous bytes of each of 4 rows (whole 128-byte lines), from a wave-uniform page base plus
// fixed lane offsets.  The row max needs only the two lane swaps across the lane groups that
// hold a head, and the dot products need no cross-lane reduction (the row kernel's reductions
// grow with the heads per KV head).  The MFMA work is the same for any HPW <= 16 (unused
// columns are zero).
template <int D>
__global__ void __launch_bounds__(256) row_mfma_kernel(RowLaunch a, int hpw) {
  constexpr int DQ = D / 4;   // QK steps per block
  constexpr int NB = D / 16;  // O^T blocks; block b = 4w + c, row i is dim 64w + 4i + c
  constexpr int NQ = DQ / 4;  // float4 loads of a K row part per lane
  constexpr int NV = NB / 4;  // float4 loads of a V row part per lane per key (one per 64 dims)
  static_assert(NV >= 1, "d >= 64");
  constexpr int MAXH = kRowMfmaMaxHeads;
  __shared__ float sm_m[4][MAXH];
  __shared__ float sm_l[4][MAXH];
  __shared__ float4 sm_acc[4][MAXH][D / 4];
  __shared__ int32_t stab[kRowTablePages];

  const int rep = a.hq / a.hkv;
  const int groups = rep / hpw;
  const int per_item = a.hkv * groups;
  const int item = blockIdx.x / per_item;
  const int gy = blockIdx.x - item * per_item;
  const RowItem it = a.items[item];
  const int kvh = unit_kv_head(a, gy / groups);
  const int h0 = kvh * rep + (gy - (gy / groups) * groups) * hpw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15;
  const int g = lane >> 4;

  // B operand of QK: this lane's head i, dims 16v + 4g + [0, 4), pre-scaled to log2 units.
  const float sl2 = a.scale * 1.4426950408889634f;
  float q[DQ];
  if (i < hpw) {
    const float *qp = a.q + ((size_t)it.qrow * a.hq + h0 + i) * D + 4 * g;
#pragma unroll
    for (int v = 0; v < NQ; v++) {
      const float4 x = ld4(qp + 16 * v);
      q[4 * v] = x.x * sl2;
      q[4 * v + 1] = x.y * sl2;
      q[4 * v + 2] = x.z * sl2;
      q[4 * v + 3] = x.w * sl2;
    }
  } else {
#pragma unroll
    for (int s = 0; s < DQ; s++) q[s] = 0.0f;
  }

  const size_t rs = (size_t)a.hkv * D;
  const int bs_shift = a.kv.bs_shift;
  const int blk0 = it.kbeg >> bs_shift;
  const bool inl = it.blk_a != 0;
  if (!inl) {
    const int32_t *table = a.kv.table + (size_t)it.seq * a.kv.bt_stride;
    const int npages = it.kend > it.kbeg ? ((it.kend - 1) >> bs_shift) - blk0 + 1 : 0;
    for (int j = threadIdx.x; j < npages; j += blockDim.x) stab[j] = table[blk0 + j];
    __syncthreads();
  }
  const float *kbase_h = a.kv.k + (size_t)kvh * D;
  const float *vbase_h = a.kv.v + (size_t)kvh * D;
  const int tfirst = it.kbeg & ~15;
  // Fixed lane offsets (floats) from a block's first row: K row i, dims 16v + 4g; V rows
  // 4g + s, dims 64w + 4i.
  const uint32_t koff = (uint32_t)(i * rs + 4 * g);
  const uint32_t voff = (uint32_t)(4 * g * rs + 4 * i);

  float kra[DQ], krb[DQ];
  float vra[4][NB], vrb[4][NB];
  auto issue = [&](int t0, float(&kr)[DQ], float(&vr)[4][NB]) {
    // A block past the chunk's end reloads its first block (never folded).
    const int tb = t0 < it.kend ? t0 : tfirst;
    const int p = tb >> bs_shift;
    const int id = inl ? (p == blk0 ? it.blk_a - 1 : it.blk_b)
                       : __builtin_amdgcn_readfirstlane(stab[p - blk0]);
    const int64_t row = (int64_t)id * a.kv.block_size + (tb - (p << bs_shift));
    const float *kb = kbase_h + row * rs;
    const float *vb = vbase_h + row * rs;
    uint32_t ko = koff, vo[4];
#pragma unroll
    for (int s = 0; s < 4; s++) vo[s] = voff + (uint32_t)(s * rs);
    if (tb < it.kbeg || tb + 16 > it.kend) {
      // A partial block: every lane reads the block's key nearest its own inside the chunk (an
      // unwritten slot could hold any bits, NaN included; a finite V row adds 0 at weight 0).
      const int tk = min(max(tb + i, it.kbeg), it.kend - 1);
      ko = (uint32_t)((tk - tb) * rs + 4 * g);
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const int tv = min(max(tb + 4 * g + s, it.kbeg), it.kend - 1);
        vo[s] = (uint32_t)((tv - tb) * rs + 4 * i);
      }
    }
#pragma unroll
    for (int v = 0; v < NQ; v++) {
      const float4 x = ld4_stream_at(kb, ko + 16 * v);
      kr[4 * v] = x.x;
      kr[4 * v + 1] = x.y;
      kr[4 * v + 2] = x.z;
      kr[4 * v + 3] = x.w;
    }
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const float4 x = ld4_stream_at(vb, vo[s] + 64 * v);
        vr[s][4 * v] = x.x;
        vr[s][4 * v + 1] = x.y;
        vr[s][4 * v + 2] = x.z;
        vr[s][4 * v + 3] = x.w;
      }
  };

  f32x4 o[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) o[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;  // head i's running max (log2 units), the same in its 4 lanes
  float l_run = 0.0f;       // this lane's part of head i's running sum (its keys 4g + r)
  auto fold = [&](int t0, const float(&kr)[DQ], const float(&vr)[4][NB]) {
    f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < DQ; s++)
      st = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[s], q[s], st, 0, 0, 0);
    float p[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int key = t0 + 4 * g + r;
      p[r] = (key >= it.kbeg && key < it.kend) ? st[r] : -INFINITY;
      mx = fmaxf(mx, p[r]);
    }
    mx = max4_lanes(mx);
    const bool need = mx > m_run + 8.0f;
    if (__any(need)) {
      const float mn = need ? mx : m_run;
      const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - mn);
      l_run *= alpha;
#pragma unroll
      for (int b = 0; b < NB; b++) o[b] *= alpha;
      m_run = mn;
    }
    const float ms = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      p[r] = __builtin_amdgcn_exp2f(p[r] - ms);
      l_run += p[r];
    }
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int b = 0; b < NB; b++)
        o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[s][b], p[s], o[b], 0, 0, 0);
  };

  int t0 = tfirst + 16 * wave;
  if (t0 < it.kend) {
    issue(t0, kra, vra);
    for (;;) {
      issue(t0 + 64, krb, vrb);
      fold(t0, kra, vra);
      t0 += 64;
      if (t0 >= it.kend) break;
      issue(t0 + 64, kra, vra);
      fold(t0, krb, vrb);
      t0 += 64;
      if (t0 >= it.kend) break;
    }
  }

  // Head i's sum over its 4 lanes; the waves' states merge through LDS.
  const float l_tot = sum4_lanes(l_run);
  if (i < hpw) {
    if (g == 0) {
      sm_m[wave][i] = m_run;
      sm_l[wave][i] = l_tot;
    }
    // Lane (i, g) holds row 4g + r of block 4w + c: dim 64w + 16g + 4r + c.
#pragma unroll
    for (int w = 0; w < NV; w++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        sm_acc[wave][i][16 * w + 4 * g + r] =
            make_float4(o[4 * w][r], o[4 * w + 1][r], o[4 * w + 2][r], o[4 * w + 3][r]);
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < hpw * (D / 4); idx += blockDim.x) {
    const int h = idx / (D / 4);
    const int cc = idx - h * (D / 4);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++) M = fmaxf(M, sm_m[w][h]);
    const float Ms = M == -INFINITY ? 0.0f : M;
    float L = 0.0f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float e = __builtin_amdgcn_exp2f(sm_m[w][h] - Ms);
      L = fmaf(sm_l[w][h], e, L);
      const float4 x = sm_acc[w][h][cc];
      A.x = fmaf(x.x, e, A.x);
      A.y = fmaf(x.y, e, A.y);
      A.z = fmaf(x.z, e, A.z);
      A.w = fmaf(x.w, e, A.w);
    }
    if (it.part < 0) {
      const float inv = L == 0.0f ? 0.0f : 1.0f / L;
      st4(a.out + ((size_t)it.qrow * a.hq + h0 + h) * D + cc * 4,
          make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv));
    } else {
      const size_t pi = (size_t)it.part * a.hq + h0 + h;
      st4(a.part_acc + pi * D + cc * 4, A);
      if (cc == 0) {
        a.part_m[pi] = M;
        a.part_l[pi] = L;
      }
    }
  }
}

// Row-wide merge for plans whose split rows have at most MP (4 or 8, kMergeRowsMaxParts)
// partials (prefill segments): one workgroup per row covers all heads, each thread folding the
// partials of one float4 of one head in order.  All of a thread's partial loads are issued
// before the first is used, so the merge costs one memory round trip instead of two per
// partial.
template <int MP>
__global__ void __launch_bounds__(256) merge_rows_kernel(MergeLaunch a) {
  const MergeItem it = a.items[blockIdx.x];
  const int d4 = a.head_dim >> 2;
  const int n = it.nparts;  // 0 .. MP
  for (int idx = threadIdx.x; idx < a.hq * d4; idx += blockDim.x) {
    const int h = idx / d4;
    const int cc = idx - h * d4;
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n > 0) {
      float pm[MP], pl[MP];
      float4 px[MP];
#pragma unroll
      for (int p = 0; p < MP; p++) {
        if (p < n) {
          const size_t pi = (size_t)(it.first + p) * a.hq + h;
          pm[p] = a.part_m[pi];
          pl[p] = a.part_l[pi];
          px[p] = ld4(a.part_acc + pi * a.head_dim + cc * 4);
        }
      }
      float M = -INFINITY;
#pragma unroll
      for (int p = 0; p < MP; p++)
        if (p < n) M = fmaxf(M, pm[p]);
      const float Ms = M == -INFINITY ? 0.0f : M;
      float L = 0.0f;
      float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int p = 0; p < MP; p++) {
        if (p < n) {
          const float e = __builtin_amdgcn_exp2f(pm[p] - Ms);
          L = fmaf(pl[p], e, L);
          A.x = fmaf(px[p].x, e, A.x);
          A.y = fmaf(px[p].y, e, A.y);
          A.z = fmaf(px[p].z, e, A.z);
          A.w = fmaf(px[p].w, e, A.w);
        }
      }
      const float inv = L == 0.0f ? 0.0f : 1.0f / L;
      r = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
    }
    st4(a.out + ((size_t)it.qrow * a.hq + h) * a.head_dim + cc * 4, r);
  }
}

// Log-sum-exp merge of the chunk partials of split rows; rows with no visible key get zeros.
// One workgroup of NW waves per (row, head): wave w folds partials w, w + NW, ... in batches of
// four whose loads are all issued before any is used (an online fold: the running sums are
// rescaled when a batch raises the maximum), lane c holding float4 c (and c + 64 at d = 512)
// of the head; the waves' (m, l, acc) are then combined in wave order through LDS, so the
// result is deterministic.
template <int NW>
__global__ void __launch_bounds__(NW * 64) merge_kernel(MergeLaunch a) {
  __shared__ float sm[NW], sl[NW];
  __shared__ float4 sacc[NW][128];
  const MergeItem it = a.items[blockIdx.x];
  const int h = blockIdx.y;
  const int d4 = a.head_dim >> 2;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  float4 *out = reinterpret_cast<float4 *>(a.out + ((size_t)it.qrow * a.hq + h) * a.head_dim);
  if (it.nparts <= 0) {
    for (int c = threadIdx.x; c < d4; c += blockDim.x) out[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    return;
  }
  float M = -INFINITY, L = 0.0f;
  float4 A0 = make_float4(0.f, 0.f, 0.f, 0.f), A1 = A0;
  const bool c0 = lane < d4, c1 = lane + 64 < d4;
  for (int p0 = wave; p0 < it.nparts; p0 += 4 * NW) {
    float pm[4], pl[4];
    float4 x0[4], x1[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int p = p0 + NW * u;
      const bool ok = p < it.nparts;
      const size_t pi = (size_t)(it.first + (ok ? p : p0)) * a.hq + h;  // p0 < nparts
      const float4 *src = reinterpret_cast<const float4 *>(a.part_acc + pi * a.head_dim);
      pm[u] = ok ? a.part_m[pi] : -INFINITY;
      pl[u] = ok ? a.part_l[pi] : 0.0f;
      x0[u] = ok && c0 ? src[lane] : make_float4(0.f, 0.f, 0.f, 0.f);
      x1[u] = ok && c1 ? src[lane + 64] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float Mn = fmaxf(fmaxf(M, fmaxf(pm[0], pm[1])), fmaxf(pm[2], pm[3]));
    const float Ms = Mn == -INFINITY ? 0.0f : Mn;
    const float alpha = __builtin_amdgcn_exp2f(M - Ms);  // 0 while M is -inf
    L *= alpha;
    A0 = make_float4(A0.x * alpha, A0.y * alpha, A0.z * alpha, A0.w * alpha);
    A1 = make_float4(A1.x * alpha, A1.y * alpha, A1.z * alpha, A1.w * alpha);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const float e = __builtin_amdgcn_exp2f(pm[u] - Ms);  // 0 for the unused slots
      L = fmaf(pl[u], e, L);
      A0.x = fmaf(x0[u].x, e, A0.x);
      A0.y = fmaf(x0[u].y, e, A0.y);
      A0.z = fmaf(x0[u].z, e, A0.z);
      A0.w = fmaf(x0[u].w, e, A0.w);
      A1.x = fmaf(x1[u].x, e, A1.x);
      A1.y = fmaf(x1[u].y, e, A1.y);
      A1.z = fmaf(x1[u].z, e, A1.z);
      A1.w = fmaf(x1[u].w, e, A1.w);
    }
    M = Mn;
  }
  if (lane == 0) {
    sm[wave] = M;
    sl[wave] = L;
  }
  if (c0) sacc[wave][lane] = A0;
  if (c1) sacc[wave][lane + 64] = A1;
  __syncthreads();
  float G = -INFINITY;
  for (int w = 0; w < NW; w++) G = fmaxf(G, sm[w]);
  const float Gs = G == -INFINITY ? 0.0f : G;
  float LT = 0.0f;
  for (int w = 0; w < NW; w++) LT = fmaf(sl[w], __builtin_amdgcn_exp2f(sm[w] - Gs), LT);
  const float inv = LT == 0.0f ? 0.0f : 1.0f / LT;
  for (int c = threadIdx.x; c < d4; c += blockDim.x) {
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = 0; w < NW; w++) {
      const float ew = __builtin_amdgcn_exp2f(sm[w] - Gs);
      const float4 x = sacc[w][c];
      r.x = fmaf(x.x, ew, r.x);
      r.y = fmaf(x.y, ew, r.y);
      r.z = fmaf(x.z, ew, r.z);
      r.w = fmaf(x.w, ew, r.w);
    }
    out[c] = make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
  }
}

namespace {

template <int D, int HPW>
void launch_row_dh(const RowLaunch &a, const dim3 &grid, hipStream_t s) {
  constexpr int G = RowShape<D, HPW>::G;
  if (a.kv.paged && a.kv.bs_shift >= 0 && a.kv.block_size % G == 0)
    hipLaunchKernelGGL((row_attention_kernel<D, HPW, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((row_attention_kernel<D, HPW, false>), grid, dim3(256), 0, s, a);
}

// Head counts that are not powers of two (GQA ratios 3, 5, 6, 7, e.g. 40 query heads over 8 KV
// heads) are built for the head dims of real models only.
constexpr bool row_odd_heads(int d) { return d >= 32 && d <= 256; }

template <int D>
hipError_t launch_row_d(const RowLaunch &a, int hpw, hipStream_t s) {
  const dim3 grid(a.num_items * (a.hkv * ((a.hq / a.hkv) / hpw)));
  if constexpr (D == 64 || D == 128) {
    if (a.mfma && hpw >= 1 && hpw <= kRowMfmaMaxHeads &&
        row_mfma_supports(D, a.kv.paged, a.kv.block_size)) {
      hipLaunchKernelGGL((row_mfma_kernel<D>), grid, dim3(256), 0, s, a, hpw);
      return hipGetLastError();
    }
  }
  switch (hpw) {
    case 1: launch_row_dh<D, 1>(a, grid, s); break;
    case 2: launch_row_dh<D, 2>(a, grid, s); break;
    case 4: launch_row_dh<D, 4>(a, grid, s); break;
    case 8: launch_row_dh<D, 8>(a, grid, s); break;
    case 3:
    case 5:
    case 6:
    case 7:
      if constexpr (row_odd_heads(D)) {
        if (hpw == 3) launch_row_dh<D, 3>(a, grid, s);
        else if (hpw == 5) launch_row_dh<D, 5>(a, grid, s);
        else if (hpw == 6) launch_row_dh<D, 6>(a, grid, s);
        else launch_row_dh<D, 7>(a, grid, s);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool row_mfma_supports(int head_dim, int paged, int block_size) {
  return (head_dim == 64 || head_dim == 128) && paged && block_size >= 16 &&
         (block_size & (block_size - 1)) == 0;
}

bool row_kernel_supports(int head_dim, int heads_per_wg) {
  const bool d_ok = head_dim == 4 || head_dim == 8 || head_dim == 16 || head_dim == 32 ||
                    head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512;
  const bool h_ok = heads_per_wg == 1 || heads_per_wg == 2 || heads_per_wg == 4 ||
                    heads_per_wg == 8 ||
                    ((heads_per_wg == 3 || (heads_per_wg >= 5 && heads_per_wg <= 7)) &&
                     row_odd_heads(head_dim));
  return d_ok && h_ok;
}

// Eight heads at every head dim: at d = 512 (256 VGPRs, one wave per SIMD) they still beat two
// 4-head workgroups that each read the K/V (Gemma 4 global-layer decode, 8 query heads over
// one KV head: 2.27 -> 1.66 ms for 256 rows, 163 -> 141 us for 32 rows after a flush).
int row_kernel_max_heads(int /*head_dim*/) { return 8; }

hipError_t launch_row_attention(const RowLaunch &a, int hpw, hipStream_t s) {
  if (a.num_items <= 0) return hipSuccess;
  switch (a.head_dim) {
    case 4: return launch_row_d<4>(a, hpw, s);
    case 8: return launch_row_d<8>(a, hpw, s);
    case 16: return launch_row_d<16>(a, hpw, s);
    case 32: return launch_row_d<32>(a, hpw, s);
    case 64: return launch_row_d<64>(a, hpw, s);
    case 128: return launch_row_d<128>(a, hpw, s);
    case 256: return launch_row_d<256>(a, hpw, s);
    case 512: return launch_row_d<512>(a, hpw, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_merge(const MergeLaunch &a, int max_parts, hipStream_t s) {
  if (a.num_items <= 0) return hipSuccess;
  if (a.head_dim > 512 || (a.head_dim & 3)) return hipErrorInvalidValue;
  // Few partials per row: one row-wide workgroup per row; many: spread them over 4 or 16 waves.
  // Rows with 5..8 partials take the row-wide form only when there are enough rows to fill the
  // chip (prefill segments); a decode step's few rows merge faster with a workgroup per (row,
  // head) (Qwen3 decode of 8 rows: 6.3-6.7 against 6.2-6.3 us after a flush).
  if (max_parts <= 4)
    hipLaunchKernelGGL(merge_rows_kernel<4>, dim3(a.num_items), dim3(256), 0, s, a);
  else if (max_parts <= kMergeRowsMaxParts && a.num_items >= 512)
    hipLaunchKernelGGL(merge_rows_kernel<kMergeRowsMaxParts>, dim3(a.num_items), dim3(256), 0,
                       s, a);
  else if (max_parts <= 32)
    hipLaunchKernelGGL((merge_kernel<4>), dim3(a.num_items, a.hq), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((merge_kernel<16>), dim3(a.num_items, a.hq), dim3(1024), 0, s, a);
  return hipGetLastError();
}

}  // namespace nva
