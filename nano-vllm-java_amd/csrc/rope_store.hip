// Kernel (a): per-head RMSNorm of q/k/v, RoPE on q/k and the slot-mapped K/V store, fused
// into one pass over the token's rows; also the plain store, the gather and a standalone RMSNorm.
//
// RMSNorm restates Ops.rmsNorm (tensor/Ops.java:444-500) as the model layers apply it per head
// (normHeads, models/internal/Qwen3ForCausalLM.java:215-227; Gemma3ForCausalLM.java:146-157;
// Gemma4ForCausalLM.java:164-197): sum = ScalarFloatKernels.sumSquares (groups of four added
// left to right, each group added to the running sum in order, then the tail; no FMA),
// var = sum / d, inv = (float)(1.0 / Math.sqrt(var + eps)) in double, and
// out = x * inv [* w | * (1 + w)].  The per-group sums run in parallel; one lane per row then
// adds them in the reference's order, so the result is bit-identical to the scalar backend.
// RoPE restates RotaryEmbedding.apply (layers/Norms.java:337-345): for each head,
//   o[i] = x1*cos - x2*sin,  o[h+i] = x2*cos + x1*sin,  h = d/2 (rotate-half)
// with the cos|sin row of the token's position taken from the caller's table.  Java never
// contracts these into FMAs, so contraction is switched off here: each product and sum is a
// separately rounded fp32 op and the result is bit-identical to the reference.
// The store restates Attention.storeKvCache (layers/Attention.java:221-240): the token's
// Hkv*d floats of rotated k and of v go to cache[slot*Hkv*d ...]; negative slots are skipped.
//
// HBM traffic per token: read q,k,v and the table row, write q_out (+k_out) and the two
// cache rows (the norm re-reads the rows it has just read, from L1/L2).  One workgroup per
// token; every access is a 16-byte vector access when d % 8 == 0 (all shapes of interest),
// scalar otherwise.
#include "nva_internal.h"
#include "nva_device.h"

namespace nva {

#pragma clang fp contract(off)

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

namespace {

// Separately rounded fp32 ops.  They are defined here, under the file's contract(off) pragma, so
// no product is ever fused into an FMA after inlining (the header versions of __fmul_rn and
// __fadd_rn are plain operators compiled under the default contraction mode).
__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }

// x * inv, then * w or * (1 + w): the products of Ops.rmsNorm, separately rounded.
__device__ __forceinline__ float norm1(float x, float inv, const HeadNorm &n, int j) {
  float y = mul_rn(x, inv);
  if (n.weight) y = mul_rn(y, n.one_plus ? add_rn(1.0f, n.weight[j]) : n.weight[j]);
  return y;
}

// Four consecutive elements starting at j (j % 4 == 0; the weight is 16-byte aligned).
__device__ __forceinline__ float4 norm4(float4 x, float inv, const HeadNorm &n, int j) {
  float4 y = make_float4(mul_rn(x.x, inv), mul_rn(x.y, inv), mul_rn(x.z, inv), mul_rn(x.w, inv));
  if (n.weight) {
    float4 w = ld4(n.weight + j);
    if (n.one_plus)
      w = make_float4(add_rn(1.0f, w.x), add_rn(1.0f, w.y), add_rn(1.0f, w.z), add_rn(1.0f, w.w));
    y = make_float4(mul_rn(y.x, w.x), mul_rn(y.y, w.y), mul_rn(y.z, w.z), mul_rn(y.w, w.w));
  }
  return y;
}

// ((x0*x0 + x1*x1) + x2*x2) + x3*x3, the group sum of ScalarFloatKernels.sumSquares.
__device__ __forceinline__ float group_sq(float x0, float x1, float x2, float x3) {
  float s = mul_rn(x0, x0);
  s = add_rn(s, mul_rn(x1, x1));
  s = add_rn(s, mul_rn(x2, x2));
  return add_rn(s, mul_rn(x3, x3));
}

// Folds the group sums in order, adds the tail, and returns (float)(1 / sqrt(sum/d + eps)).
__device__ __forceinline__ float rms_inv(const float *groups, int ngroups, const float *x, int d,
                                         float eps) {
  float sum = 0.0f;
  for (int c = 0; c < ngroups; c++) sum = add_rn(sum, groups[c]);
  for (int i = 4 * ngroups; i < d; i++) sum = add_rn(sum, mul_rn(x[i], x[i]));
  const float var = sum / (float)d;  // correctly rounded (HIP default)
  return (float)(1.0 / sqrt((double)add_rn(var, eps)));
}

// The value of lane ^ X (X = half a row group): DPP within a quad or row, a bit-mode swizzle
// across the two 16-lane rows of a 32-lane half, a lane permute for the two halves of a wave.
template <int X>
__device__ __forceinline__ float partner(float v) {
  if constexpr (X == 1) return __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);
  if constexpr (X == 2) return __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);
  if constexpr (X == 16)
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  return __shfl_xor(v, X);
}

}  // namespace

__global__ void __launch_bounds__(256) rope_store_kernel(RopeStoreLaunch a) {
  extern __shared__ float norm_lds[];  // [rows][d/4] group sums, then [rows] inverse RMS
  record_last_xcd(a.xcd_hint);
  const int t = blockIdx.x;
  const int d = a.head_dim;
  const int half = d >> 1;
  // Norm rows of the token: q heads [0, hq), k heads [hq, hq + hk), v heads [hq + hk, hq + 2hk).
  const int nrows = a.hq + 2 * a.hk;
  const int ngroups = d >> 2;
  float *inv_lds = norm_lds + (size_t)nrows * ngroups;
  auto row_ptr = [&](int r) -> const float * {
    if (r < a.hq) return a.q + (size_t)t * a.q_ld + (size_t)r * d;
    if (r < a.hq + a.hk) return a.k + (size_t)t * a.k_ld + (size_t)(r - a.hq) * d;
    return a.v + (size_t)t * a.v_ld + (size_t)(r - a.hq - a.hk) * d;
  };
  auto row_norm = [&](int r) -> const HeadNorm & {
    return r < a.hq ? a.qn : (r < a.hq + a.hk ? a.kn : a.vn);
  };
  if (a.qn.enabled | a.kn.enabled | a.vn.enabled) {
    for (int it = threadIdx.x; it < nrows * ngroups; it += blockDim.x) {
      const int r = it / ngroups;
      if (!row_norm(r).enabled) continue;
      const float *x = row_ptr(r) + 4 * (it - r * ngroups);
      norm_lds[it] = group_sq(x[0], x[1], x[2], x[3]);
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
      const HeadNorm &n = row_norm(r);
      if (n.enabled) inv_lds[r] = rms_inv(norm_lds + (size_t)r * ngroups, ngroups, row_ptr(r), d,
                                          n.eps);
    }
    __syncthreads();
  }
  const int pos = a.positions ? a.positions[t] : -1;
  const float *cs = a.positions ? a.cos_sin + (size_t)pos * d : nullptr;
  const int32_t slot = a.slots ? a.slots[t] : -1;
  const bool store = a.k_cache != nullptr && slot >= 0;
  const size_t krow = (size_t)a.hk * d;
  float *kc = store ? a.k_cache + (size_t)slot * krow : nullptr;
  float *vc = store ? a.v_cache + (size_t)slot * krow : nullptr;
  const bool vec = (half & 3) == 0;

  if (cs != nullptr) {
    // Rotation: items are (head, i) pairs over q heads then k heads.
    const int step = vec ? 4 : 1;
    const int per_head = half / step;
    const int items = (a.hq + a.hk) * per_head;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
      const int hh = it / per_head;
      const int i = (it - hh * per_head) * step;
      const bool isq = hh < a.hq;
      const int h = isq ? hh : hh - a.hq;
      const size_t base = ((size_t)t * (isq ? a.hq : a.hk) + h) * d;  // output row
      const float *in = (isq ? a.q + (size_t)t * a.q_ld : a.k + (size_t)t * a.k_ld) + (size_t)h * d;
      const HeadNorm &nm = isq ? a.qn : a.kn;
      const float inv = nm.enabled ? inv_lds[hh] : 1.0f;
      if (vec) {
        float4 x1 = ld4(in + i), x2 = ld4(in + half + i);
        if (nm.enabled) {
          x1 = norm4(x1, inv, nm, i);
          x2 = norm4(x2, inv, nm, half + i);
        }
        const float4 c = ld4(cs + i), s = ld4(cs + half + i);
        float4 o1, o2;
        o1.x = x1.x * c.x - x2.x * s.x;
        o1.y = x1.y * c.y - x2.y * s.y;
        o1.z = x1.z * c.z - x2.z * s.z;
        o1.w = x1.w * c.w - x2.w * s.w;
        o2.x = x2.x * c.x + x1.x * s.x;
        o2.y = x2.y * c.y + x1.y * s.y;
        o2.z = x2.z * c.z + x1.z * s.z;
        o2.w = x2.w * c.w + x1.w * s.w;
        if (isq) {
          st4(a.q_out + base + i, o1);
          st4(a.q_out + base + half + i, o2);
        } else {
          if (a.k_out) {
            st4(a.k_out + base + i, o1);
            st4(a.k_out + base + half + i, o2);
          }
          if (store) {
            st4(kc + (size_t)h * d + i, o1);
            st4(kc + (size_t)h * d + half + i, o2);
          }
        }
      } else {
        float x1 = in[i], x2 = in[half + i];
        if (nm.enabled) {
          x1 = norm1(x1, inv, nm, i);
          x2 = norm1(x2, inv, nm, half + i);
        }
        const float c = cs[i], s = cs[half + i];
        const float o1 = x1 * c - x2 * s;
        const float o2 = x2 * c + x1 * s;
        if (isq) {
          a.q_out[base + i] = o1;
          a.q_out[base + half + i] = o2;
        } else {
          if (a.k_out) {
            a.k_out[base + i] = o1;
            a.k_out[base + half + i] = o2;
          }
          if (store) {
            kc[(size_t)h * d + i] = o1;
            kc[(size_t)h * d + half + i] = o2;
          }
        }
      }
    }
  } else if (store) {
    // Store without rotation (Attention.forward's own store of already-rotated k).
    const float *kin = a.k + (size_t)t * a.k_ld;
    if ((krow & 3) == 0) {
      for (int i = threadIdx.x * 4; i < (int)krow; i += blockDim.x * 4) st4(kc + i, ld4(kin + i));
    } else {
      for (int i = threadIdx.x; i < (int)krow; i += blockDim.x) kc[i] = kin[i];
    }
  }
  if (a.vn.enabled && (store || a.v_out)) {
    // Normalised v rows (Gemma 4's weightless v norm) to the pages and/or v_out; a float4 never
    // straddles two heads.
    const float *vin = a.v + (size_t)t * a.v_ld;
    float *vo = a.v_out ? a.v_out + (size_t)t * krow : nullptr;
    const int step = (d & 3) == 0 ? 4 : 1;
    for (int i = threadIdx.x * step; i < (int)krow; i += blockDim.x * step) {
      const int h = i / d;
      const float inv = inv_lds[a.hq + a.hk + h];
      if (step == 4) {
        const float4 y = norm4(ld4(vin + i), inv, a.vn, i - h * d);
        if (store) st4(vc + i, y);
        if (vo) st4(vo + i, y);
      } else {
        const float y = norm1(vin[i], inv, a.vn, i - h * d);
        if (store) vc[i] = y;
        if (vo) vo[i] = y;
      }
    }
  } else if (store || a.v_out) {
    // v rows to the pages and/or as contiguous rows (v_out: packed inputs, dense prefill).
    const float *vin = a.v + (size_t)t * a.v_ld;
    float *vo = a.v_out ? a.v_out + (size_t)t * krow : nullptr;
    if ((krow & 3) == 0) {
      for (int i = threadIdx.x * 4; i < (int)krow; i += blockDim.x * 4) {
        const float4 y = ld4(vin + i);
        if (store) st4(vc + i, y);
        if (vo) st4(vo + i, y);
      }
    } else {
      for (int i = threadIdx.x; i < (int)krow; i += blockDim.x) {
        if (store) vc[i] = vin[i];
        if (vo) vo[i] = vin[i];
      }
    }
  }
}

// Row iterations a workgroup of rope_rows_kernel loads together.
constexpr int kRopeRowsPerLoad = 4;

// The same work with one group of LPR lanes per head row (q, k or v row of one token) and no
// LDS or barriers.  Workgroup (t, s) handles token t's rows: row group g takes rows
// g + RPB * i for the iterations i of slice s (the host sizes the slices so that small batches
// still fill the chip), loading four rows at a time.  The token's cos|sin row, position and
// slot are loaded once per lane and reused by every row.  Lane c of a group holds the float4
// groups c + LPR * j (j < VPL) of the row.  The norm's group sums are folded in index order with
// DPP shifts; the rotation partner of a first-half element sits LPR / 2 lanes away (VPL = 1) or
// in the lane's own column VPL/2 further on (VPL > 1).
template <int LPR, int VPL>
__global__ void __launch_bounds__(256) rope_rows_kernel(RopeStoreLaunch a) {
  constexpr int D = 4 * LPR * VPL;
  record_last_xcd(a.xcd_hint);
  constexpr int HALF = D / 2;
  constexpr int RPB = 256 / LPR;  // row groups per workgroup
  constexpr int NR = kRopeRowsPerLoad;  // rows loaded together
  const int t = blockIdx.x;
  const int c = threadIdx.x % LPR;
  const int grp = threadIdx.x / LPR;
  const int base = (threadIdx.x & 63) - c;  // first lane of this row group in the wave
  const int rq = a.q ? a.hq : 0;
  const int rk = a.k ? a.hk : 0;
  const bool store_any = a.k_cache != nullptr;
  const int rv = (a.v && (store_any || a.v_out)) ? a.hk : 0;
  const int rows = rq + rk + rv;
  const int iters = (rows + RPB - 1) / RPB;
  const int it0 = blockIdx.y * a.iters_per_wg;
  const int it1 = min(iters, it0 + a.iters_per_wg);
  const size_t krow = (size_t)a.hk * D;

  const bool rotate = a.positions != nullptr;
  constexpr int H2 = VPL > 1 ? VPL / 2 : 1;  // cos|sin float4s a lane needs
  static_assert(VPL == 1 || VPL % 2 == 0, "a split row holds both halves in its own lanes");
  float4 cv[H2], sv[H2];
  if (rotate) {
    const float *cs = a.cos_sin + (size_t)a.positions[t] * D;
    if constexpr (VPL == 1) {
      // Lane c < LPR/2 rotates x1 = elements 4c.., the others x2 = HALF + 4(c - LPR/2).
      const int i0 = 4 * (c < LPR / 2 ? c : c - LPR / 2);
      cv[0] = ld4(cs + i0);
      sv[0] = ld4(cs + HALF + i0);
    } else {
      // Columns j < VPL/2 hold first-half elements 4(c + LPR j); column j + VPL/2 holds their
      // partners HALF elements on.
#pragma unroll
      for (int j = 0; j < H2; j++) {
        cv[j] = ld4(cs + 4 * (c + LPR * j));
        sv[j] = ld4(cs + HALF + 4 * (c + LPR * j));
      }
    }
  }
  const int32_t slot = a.slots ? a.slots[t] : -1;
  const bool store = store_any && slot >= 0;

  for (int ib = it0; ib < it1; ib += NR) {
    int kind[NR], h[NR];
    bool live[NR];
    float4 x[NR][VPL];
#pragma unroll
    for (int i = 0; i < NR; i++) {
      const int r = grp + RPB * (ib + i);
      live[i] = ib + i < it1 && r < rows;  // uniform over the row group
      const int rc = live[i] ? r : 0;
      kind[i] = rc < rq ? 0 : (rc < rq + rk ? 1 : 2);  // q, k, v
      h[i] = kind[i] == 0 ? rc : (kind[i] == 1 ? rc - rq : rc - rq - rk);
      const int ld = kind[i] == 0 ? a.q_ld : (kind[i] == 1 ? a.k_ld : a.v_ld);
      const float *src = (kind[i] == 0 ? a.q : (kind[i] == 1 ? a.k : a.v)) + (size_t)t * ld +
                         (size_t)h[i] * D;
#pragma unroll
      for (int j = 0; j < VPL; j++)
        x[i][j] = live[i] ? ld4(src + 4 * (c + LPR * j)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }

#pragma unroll
    for (int i = 0; i < NR; i++) {
      if (ib + i >= it1) break;  // uniform over the workgroup (the DPP fold spans the wave)
      const HeadNorm &nm = kind[i] == 0 ? a.qn : (kind[i] == 1 ? a.kn : a.vn);
      if (nm.enabled) {
        // ScalarFloatKernels.sumSquares order: group sums added in group-index order, as a
        // shift-and-add chain per float4 column j: after step s, lane l holds the in-order sum
        // of the s group sums ending at lane l, starting from 0 (lane 0 shifts in 0), so after
        // LPR steps the group's last lane holds ((0 + p0) + p1) + ... + p[LPR-1] -- the same
        // additions in the same order, with no LDS traffic.  Column j > 0 continues the total
        // of the columns before it: the group's first lane adds that total to its own group
        // sum first, which is the chain's first addition (0 + that sum is exact).
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
          float p = group_sq(x[i][j].x, x[i][j].y, x[i][j].z, x[i][j].w);
          if (j > 0 && c == 0) p = add_rn(sum, p);
          float acc = 0.0f;
#pragma unroll
          for (int l = 0; l < LPR; l++)
            acc = add_rn(__builtin_amdgcn_update_dpp(0.0f, acc, 0x138, 0xF, 0xF, false), p);
          sum = __shfl(acc, base + LPR - 1);
        }
        const float var = sum / (float)D;  // correctly rounded (HIP default)
        const float inv = (float)(1.0 / sqrt((double)add_rn(var, nm.eps)));
#pragma unroll
        for (int j = 0; j < VPL; j++) x[i][j] = norm4(x[i][j], inv, nm, 4 * (c + LPR * j));
      }

      float4 o[VPL];
      if (kind[i] != 2 && rotate) {
        if constexpr (VPL == 1) {
          // Partner = the other half of the row.
          float4 y;
          y.x = partner<LPR / 2>(x[i][0].x);
          y.y = partner<LPR / 2>(x[i][0].y);
          y.z = partner<LPR / 2>(x[i][0].z);
          y.w = partner<LPR / 2>(x[i][0].w);
          if (c < LPR / 2) {  // o[i] = x1*cos - x2*sin
            o[0].x = x[i][0].x * cv[0].x - y.x * sv[0].x;
            o[0].y = x[i][0].y * cv[0].y - y.y * sv[0].y;
            o[0].z = x[i][0].z * cv[0].z - y.z * sv[0].z;
            o[0].w = x[i][0].w * cv[0].w - y.w * sv[0].w;
          } else {            // o[h+i] = x2*cos + x1*sin
            o[0].x = x[i][0].x * cv[0].x + y.x * sv[0].x;
            o[0].y = x[i][0].y * cv[0].y + y.y * sv[0].y;
            o[0].z = x[i][0].z * cv[0].z + y.z * sv[0].z;
            o[0].w = x[i][0].w * cv[0].w + y.w * sv[0].w;
          }
        } else {
          // Column j (first half) and column j + VPL/2 (its partners).
#pragma unroll
          for (int j = 0; j < H2; j++) {
            const float4 u = x[i][j], w = x[i][j + H2];
            o[j].x = u.x * cv[j].x - w.x * sv[j].x;
            o[j].y = u.y * cv[j].y - w.y * sv[j].y;
            o[j].z = u.z * cv[j].z - w.z * sv[j].z;
            o[j].w = u.w * cv[j].w - w.w * sv[j].w;
            o[j + H2].x = w.x * cv[j].x + u.x * sv[j].x;
            o[j + H2].y = w.y * cv[j].y + u.y * sv[j].y;
            o[j + H2].z = w.z * cv[j].z + u.z * sv[j].z;
            o[j + H2].w = w.w * cv[j].w + u.w * sv[j].w;
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) o[j] = x[i][j];
      }
      if (!live[i]) continue;
      const int heads = kind[i] == 0 ? a.hq : a.hk;
      const size_t row = ((size_t)t * heads + h[i]) * D;
#pragma unroll
      for (int j = 0; j < VPL; j++) {
        const int e = 4 * (c + LPR * j);
        if (kind[i] == 0) {
          st4(a.q_out + row + e, o[j]);
        } else if (kind[i] == 1) {
          if (a.k_out) st4(a.k_out + row + e, o[j]);
          if (store) st4(a.k_cache + (size_t)slot * krow + (size_t)h[i] * D + e, o[j]);
        } else {
          if (store) st4(a.v_cache + (size_t)slot * krow + (size_t)h[i] * D + e, o[j]);
          if (a.v_out) st4(a.v_out + row + e, o[j]);
        }
      }
    }
  }
}

// RMSNorm.forward over rows of any width (Ops.java:444-500): one workgroup per row; the group
// sums of each 1024-group chunk go through LDS and one lane adds them in the reference's order.
__global__ void __launch_bounds__(256) rms_norm_kernel(NormLaunch a) {
  __shared__ float groups[1024];
  __shared__ float s_inv;
  const float *x = a.x + (size_t)blockIdx.x * a.width;
  float *o = a.out + (size_t)blockIdx.x * a.width;
  const int ng = a.width >> 2;
  float sum = 0.0f;  // lane 0 only
  for (int c0 = 0; c0 < ng; c0 += 1024) {
    const int n = min(1024, ng - c0);
    for (int c = threadIdx.x; c < n; c += blockDim.x) {
      const float *p = x + 4 * (c0 + c);
      groups[c] = group_sq(p[0], p[1], p[2], p[3]);
    }
    __syncthreads();
    if (threadIdx.x == 0)
      for (int c = 0; c < n; c++) sum = add_rn(sum, groups[c]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    for (int i = 4 * ng; i < a.width; i++) sum = add_rn(sum, mul_rn(x[i], x[i]));
    const float var = sum / (float)a.width;
    s_inv = (float)(1.0 / sqrt((double)add_rn(var, a.norm.eps)));
  }
  __syncthreads();
  const float inv = s_inv;
  for (int i = threadIdx.x; i < a.width; i += blockDim.x) o[i] = norm1(x[i], inv, a.norm, i);
}

// out[0 .. n) = 0 (rows no sequence covers stay zero, as Tensor.zeros in the reference).  A
// kernel rather than hipMemsetAsync so that a caller may capture the call in a graph.
__global__ void __launch_bounds__(256) zero_kernel(float *out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = 0.0f;
}

// gatherKvCache (layers/Attention.java:201-216): rows of the producer layer's pages at the
// step's slots into dense [T, Hkv, d]; negative slots give zero rows.
__global__ void __launch_bounds__(256) gather_kernel(GatherLaunch a) {
  const int t = blockIdx.x;
  const int32_t slot = a.slots[t];
  float *ko = a.k_out + (size_t)t * a.row;
  float *vo = a.v_out + (size_t)t * a.row;
  for (int i = threadIdx.x; i < a.row; i += blockDim.x) {
    ko[i] = slot >= 0 ? a.k_cache[(size_t)slot * a.row + i] : 0.0f;
    vo[i] = slot >= 0 ? a.v_cache[(size_t)slot * a.row + i] : 0.0f;
  }
}

size_t rope_store_norm_lds(const RopeStoreLaunch &a) {
  if (!(a.qn.enabled | a.kn.enabled | a.vn.enabled)) return 0;
  const size_t rows = (size_t)a.hq + 2 * (size_t)a.hk;
  return rows * ((size_t)(a.head_dim >> 2) + 1) * sizeof(float);
}

namespace {

template <int LPR, int VPL>
hipError_t launch_rows(const RopeStoreLaunch &a, hipStream_t s, int num_cus) {
  const int rq = a.q ? a.hq : 0;
  const int rk = a.k ? a.hk : 0;
  const int rv = (a.v && (a.k_cache || a.v_out)) ? a.hk : 0;
  const int rows = rq + rk + rv;
  if (rows <= 0) return hipSuccess;
  constexpr int RPB = 256 / LPR;
  const int iters = (rows + RPB - 1) / RPB;
  // Split a token's rows over several workgroups when the batch alone would leave the chip
  // short of about four workgroups per CU, and so that no workgroup loads more than one batch
  // of row iterations (Qwen3-4B-like heads, 48 rows per token: 38.4 -> 36.8 us for 2112 tokens).
  int slices = (iters + kRopeRowsPerLoad - 1) / kRopeRowsPerLoad;
  while (slices < iters && (int64_t)a.tokens * slices < 4LL * num_cus) slices++;
  RopeStoreLaunch b = a;
  b.iters_per_wg = (iters + slices - 1) / slices;
  const int grid_y = (iters + b.iters_per_wg - 1) / b.iters_per_wg;
  hipLaunchKernelGGL((rope_rows_kernel<LPR, VPL>), dim3(a.tokens, grid_y), dim3(256), 0, s, b);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rope_store(const RopeStoreLaunch &in, hipStream_t s, int num_cus) {
  if (in.tokens <= 0) return hipSuccess;
  RopeStoreLaunch a = in;  // inputs with no stride given are contiguous [T, heads, d]
  if (!a.q_ld) a.q_ld = a.hq * a.head_dim;
  if (!a.k_ld) a.k_ld = a.hk * a.head_dim;
  if (!a.v_ld) a.v_ld = a.hk * a.head_dim;
  // Row kernel for the head dims it is instantiated for; the per-token kernel otherwise.
  switch (a.head_dim) {
    case 8: return launch_rows<2, 1>(a, s, num_cus);
    case 16: return launch_rows<4, 1>(a, s, num_cus);
    case 32: return launch_rows<8, 1>(a, s, num_cus);
    case 64: return launch_rows<16, 1>(a, s, num_cus);
    case 128: return launch_rows<32, 1>(a, s, num_cus);
    case 256: return launch_rows<64, 1>(a, s, num_cus);
    case 512: return launch_rows<64, 2>(a, s, num_cus);
    default: break;
  }
  const size_t lds = rope_store_norm_lds(a);
  if (lds > kRopeNormMaxLds) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rope_store_kernel, dim3(a.tokens), dim3(128), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const NormLaunch &a, hipStream_t s) {
  if (a.rows <= 0 || a.width <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_kernel, dim3(a.rows), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_zero(float *out, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(zero_kernel, dim3(blocks), dim3(256), 0, s, out, n);
  return hipGetLastError();
}

hipError_t launch_gather(const GatherLaunch &a, hipStream_t s) {
  if (a.tokens <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(a.tokens), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace nva
