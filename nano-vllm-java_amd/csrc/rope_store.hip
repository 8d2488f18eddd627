// Kernel (a): RoPE on q/k fused with the slot-mapped K/V store, and the plain store/gather.
//
// RoPE restates RotaryEmbedding.apply (layers/Norms.java:337-345): for each head,
//   o[i] = x1*cos - x2*sin,  o[h+i] = x2*cos + x1*sin,  h = d/2 (rotate-half)
// with the cos|sin row of the token's position taken from the caller's table.  Java never
// contracts these into FMAs, so contraction is switched off here: each product and sum is a
// separately rounded fp32 op and the result is bit-identical to the reference.
// The store restates Attention.storeKvCache (layers/Attention.java:221-240): the token's
// Hkv*d floats of rotated k and of v go to cache[slot*Hkv*d ...]; negative slots are skipped.
//
// HBM traffic per token: read q,k,v and the table row, write q_out (+k_out) and the two
// cache rows.  One workgroup per token; every access is a 16-byte vector access when
// d % 8 == 0 (all shapes of interest), scalar otherwise.
#include "nva_internal.h"

namespace nva {

#pragma clang fp contract(off)

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

__global__ void __launch_bounds__(256) rope_store_kernel(RopeStoreLaunch a) {
  const int t = blockIdx.x;
  const int d = a.head_dim;
  const int half = d >> 1;
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
      if (vec) {
        const float4 x1 = ld4(in + i), x2 = ld4(in + half + i);
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
        const float x1 = in[i], x2 = in[half + i];
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
  if (store) {
    const float *vin = a.v + (size_t)t * krow;
    if ((krow & 3) == 0) {
      for (int i = threadIdx.x * 4; i < (int)krow; i += blockDim.x * 4) st4(vc + i, ld4(vin + i));
    } else {
      for (int i = threadIdx.x; i < (int)krow; i += blockDim.x) vc[i] = vin[i];
    }
  }
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

hipError_t launch_rope_store(const RopeStoreLaunch &a, hipStream_t s) {
  if (a.tokens <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_store_kernel, dim3(a.tokens), dim3(128), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gather(const GatherLaunch &a, hipStream_t s) {
  if (a.tokens <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(a.tokens), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace nva
