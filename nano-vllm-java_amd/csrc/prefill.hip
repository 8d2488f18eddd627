// Kernel (c): varlen causal prefill on fp32 MFMA over dense K/V or the paged KV cache.
//
// Semantics (layers/Attention.java:245-280 prefillDense / prefillWithCache, :328-396
// attendJobs): query qi of a sequence with qLen queries and kLen keys sits at absolute
// position aq = kLen - qLen + qi and sees keys [max(0, aq - W + 1) (window W > 0, else 0),
// aq]; KV head kvh = h / rep; score = dot(q, k) * scale; out = softmax-weighted sum of v.
// Keys come from dense k/v rows (prefillDense) or from the cache through the block table
// (prefillWithCache).
//
// Mapping onto CDNA4: a workgroup (4 waves) owns a tile of queries of one sequence for one
// KV head and HPW of its query heads; wave w handles 32 queries of one head.  Key tiles of 32
// rows of K and V are staged in LDS (coalesced 512-byte row loads, prefetched into registers
// one tile ahead) and shared by the 4 waves.  Per key tile each wave computes
//   S^T[key][query] = K Q^T      64 x v_mfma_f32_32x32x2_f32 (D = 128)
//   O^T[dim][query] += V^T P^T   64 x v_mfma_f32_32x32x2_f32
// With S transposed, each lane holds 16 keys of ONE query, so the softmax row max is an
// in-lane max plus one exchange with lane^32, and the running sum needs no exchange until the
// end.  The P^T values land in exactly the registers the PV MFMA reads as its B operand (the
// contraction order over keys is permuted to match), so P never goes through LDS.  Only tiles
// that cross the causal diagonal, the window edge or the end of the keys are masked; all
// others run unmasked.  Q (32 x D/2 per lane) stays in registers for the whole key loop.
#include "nva_internal.h"

namespace nva {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

__device__ __forceinline__ int64_t tile_row(const KvView &kv, const int32_t *table, int kbase,
                                            int t) {
  if (!kv.paged) return (int64_t)kbase + t;
  int blk, off;
  if (kv.bs_shift >= 0) {
    blk = t >> kv.bs_shift;
    off = t & (kv.block_size - 1);
  } else {
    blk = t / kv.block_size;
    off = t - blk * kv.block_size;
  }
  return (int64_t)table[blk] * kv.block_size + off;
}

}  // namespace

template <int D, int HPW>
__global__ void __launch_bounds__(256) prefill_kernel(TileLaunch a) {
  constexpr int KT = 32;          // keys per tile
  constexpr int DP = D + 4;       // padded LDS row (conflict-free b128 column reads)
  constexpr int DH = D / 2;       // QK contraction steps per lane half
  constexpr int NB = D / 32;      // 32-wide output blocks of O^T
  constexpr int C4 = D / 4;       // float4 per K/V row
  constexpr int RPP = 256 / C4;   // rows loaded per pass by the workgroup
  constexpr int LP = KT / RPP;    // load passes per tile
  __shared__ __attribute__((aligned(16))) float sk[KT * DP];
  __shared__ __attribute__((aligned(16))) float sv[KT * DP];

  const TileItem it = a.items[blockIdx.x];
  const int rep = a.hq / a.hkv;
  const int groups = rep / HPW;
  const int kvh = blockIdx.y / groups;
  const int h = kvh * rep + (blockIdx.y - kvh * groups) * HPW + (threadIdx.x >> 6) % HPW;
  const int qb = (threadIdx.x >> 6) / HPW;
  const int lane = threadIdx.x & 63;
  const int i = lane & 31;
  const int half = lane >> 5;
  const int W = a.window;
  const int off = it.klen - it.qlen;  // absolute position of query 0

  // This lane's query (column i of S^T) and its visible key range.
  const int qi = it.q0 + qb * 32 + i;
  const bool qvalid = qi < it.qlen;
  const int qic = qvalid ? qi : it.qlen - 1;
  const int aq = off + qic;
  const int vis_lo = W > 0 ? max(0, aq - W + 1) : 0;
  const int vis_hi = aq + 1;
  // The wave's queries: union and intersection of their visible ranges.
  const int wq0 = it.q0 + qb * 32;
  const bool wave_active = wq0 < it.qlen;
  const int wq1 = min(wq0 + 31, it.qlen - 1);
  const int wlo_min = W > 0 ? max(0, off + wq0 - W + 1) : 0;  // earliest key any query sees
  const int wlo_max = W > 0 ? max(0, off + wq1 - W + 1) : 0;  // latest first-visible key
  const int whi_min = off + wq0 + 1;                            // every query sees < this
  const int whi_max = off + wq1 + 1;

  float qr[DH];
  {
    const float *qp = a.q + ((size_t)(it.qstart + qic) * a.hq + h) * D + half * DH;
#pragma unroll
    for (int s = 0; s < DH; s += 4) {
      const float4 x = ld4(qp + s);
      qr[s] = x.x;
      qr[s + 1] = x.y;
      qr[s + 2] = x.z;
      qr[s + 3] = x.w;
    }
  }

  f32x16 o[NB];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int v = 0; v < 16; v++) o[b][v] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const size_t rs = (size_t)a.hkv * D;
  const float *kbase = a.kv.k + (size_t)kvh * D;
  const float *vbase = a.kv.v + (size_t)kvh * D;
  const int32_t *table = a.kv.paged ? a.kv.table + (size_t)it.seq * a.kv.bt_stride : nullptr;
  const int lrow = threadIdx.x / C4;
  const int lcol = (threadIdx.x - lrow * C4) * 4;

  float4 pk[LP], pv[LP];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int p = 0; p < LP; p++) {
      const int key = kt + lrow + p * RPP;
      if (key < it.klen) {
        const int64_t row = tile_row(a.kv, table, it.kbase, key);
        pk[p] = ld4(kbase + row * rs + lcol);
        pv[p] = ld4(vbase + row * rs + lcol);
      } else {
        pk[p] = make_float4(0.f, 0.f, 0.f, 0.f);
        pv[p] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };

  load_tile(it.ks);
  for (int kt = it.ks; kt < it.ke; kt += KT) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < LP; p++) {
      *reinterpret_cast<float4 *>(&sk[(lrow + p * RPP) * DP + lcol]) = pk[p];
      *reinterpret_cast<float4 *>(&sv[(lrow + p * RPP) * DP + lcol]) = pv[p];
    }
    if (kt + KT < it.ke) load_tile(kt + KT);
    __syncthreads();

    // Skip tiles no query of this wave sees.
    if (!wave_active || kt >= whi_max || kt + KT <= wlo_min) continue;
    const bool full = (kt + KT <= whi_min) && (kt >= wlo_max);

    // S^T = K Q^T: A[key][k] = K[key][half*DH + s], B[k][query] = Q[query][half*DH + s].
    f32x16 st;
#pragma unroll
    for (int v = 0; v < 16; v++) st[v] = 0.0f;
    const float *krow = &sk[i * DP + half * DH];
#pragma unroll
    for (int s = 0; s < DH; s += 4) {
      const float4 kk = *reinterpret_cast<const float4 *>(krow + s);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.x, qr[s], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.y, qr[s + 1], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.z, qr[s + 2], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.w, qr[s + 3], st, 0, 0, 0);
    }

    // st[v] holds key kt + 8*(v/4) + 4*half + v%4 for query i.
    float mx = -INFINITY;
    if (full) {
#pragma unroll
      for (int v = 0; v < 16; v++) {
        st[v] *= a.scale;
        mx = fmaxf(mx, st[v]);
      }
    } else {
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int key = kt + 8 * (v >> 2) + 4 * half + (v & 3);
        const bool vis = key >= vis_lo && key < vis_hi;
        st[v] = vis ? st[v] * a.scale : -INFINITY;
        mx = fmaxf(mx, st[v]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m_run, mx);
    const float ms = mn == -INFINITY ? 0.0f : mn;
    const float alpha = expf(m_run - ms);
    float ls = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      st[v] = expf(st[v] - ms);
      ls += st[v];
    }
    l_run = fmaf(l_run, alpha, ls);
    m_run = mn;
#pragma unroll
    for (int b = 0; b < NB; b++) o[b] *= alpha;

    // O^T += V^T P^T: step s contracts key 8*(s/4) + 4*half + s%4, which is st[s] in this lane.
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int key = 8 * (s >> 2) + 4 * half + (s & 3);
        const float vv = sv[key * DP + b * 32 + i];
        o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, st[s], o[b], 0, 0, 0);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot == 0.0f ? 0.0f : 1.0f / l_tot;
  if (qvalid) {
    float *op = a.out + ((size_t)(it.qstart + qi) * a.hq + h) * D + 4 * half;
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        st4(op + b * 32 + 8 * g, make_float4(o[b][4 * g] * inv, o[b][4 * g + 1] * inv,
                                             o[b][4 * g + 2] * inv, o[b][4 * g + 3] * inv));
  }
}

namespace {

template <int D>
hipError_t launch_prefill_d(const TileLaunch &a, int hpw, hipStream_t s) {
  const dim3 grid(a.num_items, a.hkv * ((a.hq / a.hkv) / hpw));
  switch (hpw) {
    case 1: hipLaunchKernelGGL((prefill_kernel<D, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<D, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<D, 4>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool prefill_kernel_supports(int head_dim, int heads_per_wg) {
  return (head_dim == 64 || head_dim == 128) &&
         (heads_per_wg == 1 || heads_per_wg == 2 || heads_per_wg == 4);
}

hipError_t launch_prefill_tiles(const TileLaunch &a, int hpw, hipStream_t s) {
  if (a.num_items <= 0) return hipSuccess;
  switch (a.head_dim) {
    case 64: return launch_prefill_d<64>(a, hpw, s);
    case 128: return launch_prefill_d<128>(a, hpw, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nva
