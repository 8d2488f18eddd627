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

__device__ __forceinline__ float4 norm4(float4 x, float inv, const HeadNorm &n, int j) {
  return make_float4(norm1(x.x, inv, n, j), norm1(x.y, inv, n, j + 1), norm1(x.z, inv, n, j + 2),
                     norm1(x.w, inv, n, j + 3));
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

}  // namespace

__global__ void __launch_bounds__(256) rope_store_kernel(RopeStoreLaunch a) {
  extern __shared__ float norm_lds[];  // [rows][d/4] group sums, then [rows] inverse RMS
  const int t = blockIdx.x;
  const int d = a.head_dim;
  const int half = d >> 1;
  // Norm rows of the token: q heads [0, hq), k heads [hq, hq + hk), v heads [hq + hk, hq + 2hk).
  const int nrows = a.hq + 2 * a.hk;
  const int ngroups = d >> 2;
  float *inv_lds = norm_lds + (size_t)nrows * ngroups;
  auto row_ptr = [&](int r) -> const float * {
    if (r < a.hq) return a.q + ((size_t)t * a.hq + r) * d;
    if (r < a.hq + a.hk) return a.k + ((size_t)t * a.hk + (r - a.hq)) * d;
    return a.v + ((size_t)t * a.hk + (r - a.hq - a.hk)) * d;
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
      const size_t base = ((size_t)t * (isq ? a.hq : a.hk) + h) * d;
      const float *in = (isq ? a.q : a.k) + base;
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
    const float *kin = a.k + (size_t)t * krow;
    if ((krow & 3) == 0) {
      for (int i = threadIdx.x * 4; i < (int)krow; i += blockDim.x * 4) st4(kc + i, ld4(kin + i));
    } else {
      for (int i = threadIdx.x; i < (int)krow; i += blockDim.x) kc[i] = kin[i];
    }
  }
  if (a.vn.enabled && (store || a.v_out)) {
    // Normalised v rows (Gemma 4's weightless v norm) to the pages and/or v_out; a float4 never
    // straddles two heads.
    const float *vin = a.v + (size_t)t * krow;
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
  } else if (store) {
    const float *vin = a.v + (size_t)t * krow;
    if ((krow & 3) == 0) {
      for (int i = threadIdx.x * 4; i < (int)krow; i += blockDim.x * 4) st4(vc + i, ld4(vin + i));
    } else {
      for (int i = threadIdx.x; i < (int)krow; i += blockDim.x) vc[i] = vin[i];
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

hipError_t launch_rope_store(const RopeStoreLaunch &a, hipStream_t s) {
  if (a.tokens <= 0) return hipSuccess;
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

hipError_t launch_gather(const GatherLaunch &a, hipStream_t s) {
  if (a.tokens <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(a.tokens), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace nva
