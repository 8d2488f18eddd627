// Linear.Row (o_proj): y[M, N] = x[M, K] W[N, K]^T (+ bias) in fp32 on MFMA.
//
// Semantics (tensor/Ops.java:84-124 linear, tensor/MatmulRuntime.java:234-255): W is the
// row-major [out, in] weight, x the [rows, in] activations (the attention output
// [T, Hq * d], used in place), y a fresh [rows, out]; y = x W^T + bias.  The reference sums each
// output in its gemv panel order; here the sum runs over MFMA steps and split-K slices, so the
// result agrees to fp32 rounding (checked against the oracle within the attention tolerance).
//
// Mapping onto CDNA4.  Three kernels by shape:
//   * gemv_kernel for at most 8 rows (a weight-streaming GEMV, below);
//   * skinny_kernel when the 32 x 32 blocks of y number at most one per CU (decode batches of
//     tens to a few hundred rows): one block per workgroup, K split over its eight waves, each
//     streaming its own K range through a private LDS ring (below);
//   * linear_kernel otherwise.  A workgroup owns a 128 x 128 tile of y and one K slice: four
//     waves of 64 x 64 (2 x 2 blocks of v_mfma_f32_32x32x2_f32), or, when the grid has no more
//     workgroups than CUs, eight waves of 32 x 64, so each SIMD still has two waves to switch
//     between.
//   * x and W are both K-contiguous, so the A operand (x rows) and the B operand (W rows) are
//     read the same way: for each 8-wide K chunk a lane (i, h) reads one float4 of its row
//     (elements 4h .. 4h + 3), which feeds 4 MFMA steps -- step s contracts k = 4h + s, a
//     permutation of the chunk that A and B share.
//   * K tiles of 32 are copied HBM -> LDS with 16-byte loads that write LDS directly (buffer
//     loads from a uniform descriptor for interior tiles), double-buffered, one barrier per
//     tile; each 128-byte row of a tile has its 16-byte chunks XOR-swizzled by ((row >> 1) & 7):
//     measured free of LDS bank conflicts (row & 7: half of the LDS-active cycles were conflict
//     stalls).
//   * Output block layout (32 x 32, 16 values per lane): value r of lane (i, h) is row
//     8 * (r / 4) + 4 * h + r % 4, column i -- lanes 0..31 write 128 contiguous bytes.
//   * When the grid alone cannot fill the chip, K is split over blockIdx.z (both MFMA
//     kernels); slices write partial sums and linear_reduce_kernel adds them in slice order,
//     plus the bias.  (Letting the last slice of a tile reduce in place needs a device-scope
//     release per slice, which on this multi-XCD part writes back L2 and cost more than the
//     separate launch.)
// Algorithmic work: 2 * M * N * K flops; HBM bytes (once): 4 * (M * K + N * K + M * N).
#include "nva_internal.h"
#include "nva_device.h"

namespace nva {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int kSkinnyWaves = 8;  // waves of a skinny_kernel workgroup (two per SIMD)

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

typedef float f4v __attribute__((ext_vector_type(4)));

// ds_read_b128 the compiler does not see as an LDS read, so it adds no wait for every
// outstanding LDS copy before it (it cannot tell a ring's stages apart); the caller waits
// (lgkmcnt) before using the value, tying the wait to the registers.
__device__ __forceinline__ f4v lds_read4(const float *p) {
  const unsigned addr = (unsigned)(size_t)(const __attribute__((address_space(3))) float *)p;
  f4v v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Wait until at most N vector memory operations are outstanding.
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace

// WM x 2 waves; wave (wm, wn) owns 128/WM rows x 64 columns of the tile as MB x 2 blocks of
// 32 x 32.  WM = 2: four waves of 64 x 64 (64 accumulators), two workgroups per CU; WM = 4:
// eight waves of 32 x 64 (32 accumulators), two workgroups per CU and four waves per SIMD.
template <int WM>
__global__ void __launch_bounds__(64 * WM * 2) __attribute__((amdgpu_waves_per_eu(WM == 4 ? 4 : 2)))
linear_kernel(LinearLaunch a) {
  constexpr int NW = WM * 2;       // waves
  constexpr int MB = BM / WM / 32; // 32-row blocks per wave
  constexpr int LPW = 16 / NW;     // tile-copy instructions per wave per operand
  // Two buffers of the A (x) and B (W) tiles, as separate arrays so the compiler sees that the
  // copies into one never alias the reads of the other.
  __shared__ __attribute__((aligned(16))) float sa0[BM * BK];
  __shared__ __attribute__((aligned(16))) float sb0[BN * BK];
  __shared__ __attribute__((aligned(16))) float sa1[BM * BK];
  __shared__ __attribute__((aligned(16))) float sb1[BN * BK];

  const int n0 = blockIdx.x * BN;
  const int m0 = blockIdx.y * BM;
  const int kb = blockIdx.z * a.k_per_split;
  const int ke = min(a.k, kb + a.k_per_split);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform per wave
  const int lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;  // wave = 2 * wm + wn
  const int i = lane & 31;  // MFMA row (A) / column (B) index of this lane
  const int h = lane >> 5;  // which half of an 8-wide K chunk this lane supplies

  f32x16 acc[MB][2];
#pragma unroll
  for (int bm = 0; bm < MB; bm++)
#pragma unroll
    for (int bn = 0; bn < 2; bn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[bm][bn][r] = 0.0f;

  // Copy instruction p of wave w moves rows [8g, 8g + 8) of a tile, g = 4p + w: lane l takes
  // row 8g + l / 8, LDS chunk position l % 8, i.e. global chunk (l % 8) ^ ((row >> 1) & 7).
  const int lrow = lane >> 3;
  const int lpos = lane & 7;
  // An interior tile (all 128 rows of x and of W exist, and the K tile lies inside the slice)
  // is copied from a wave-uniform base at (row m0 or n0, column kt) plus these fixed byte
  // offsets, through buffer descriptors: no per-lane address arithmetic.
  // (Offsets and the descriptor size are 32-bit: 128 rows of k floats must stay below 2 GiB.)
  const bool interior = m0 + BM <= a.m && n0 + BN <= a.n && a.k < (1 << 22);
  uint32_t loff[LPW];
#pragma unroll
  for (int p = 0; p < LPW; p++) {
    const int r = 8 * (NW * p + wave) + lrow;
    loff[p] = (uint32_t)r * (uint32_t)a.k * 4u + (uint32_t)(lpos ^ ((r >> 1) & 7)) * 16u;
  }
  const int span_bytes = ((BM - 1) * a.k + BK) * 4;  // rows m0.. (n0..), columns kt..kt+BK-1
  auto issue = [&](int kt, float *da, float *db) {
    if (interior && kt + BK <= ke) {
      const float *xb = a.x + (size_t)m0 * a.k + kt;
      const float *wb = a.w + (size_t)n0 * a.k + kt;
#pragma unroll
      for (int p = 0; p < LPW; p++) {
        const int g = NW * p + wave;
        copy16_to_lds(xb, span_bytes, loff[p], da + g * 8 * BK);
        copy16_to_lds(wb, span_bytes, loff[p], db + g * 8 * BK);
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < LPW; p++) {
      const int g = NW * p + wave;
      const int r = 8 * g + lrow;
      int kc = kt + 4 * (lpos ^ ((r >> 1) & 7));
      kc = kc < ke ? kc : kb;  // past the slice: a valid address, zeroed at use
      const int xr = min(m0 + r, a.m - 1);
      const int wr = min(n0 + r, a.n - 1);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)(a.x + (size_t)xr * a.k + kc),
          (__attribute__((address_space(3))) void *)(da + g * 8 * BK), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)(a.w + (size_t)wr * a.k + kc),
          (__attribute__((address_space(3))) void *)(db + g * 8 * BK), 16, 0, 0);
    }
  };

  // full: every chunk of the tile lies inside the slice (all but a ragged last tile); the
  // chunks of a ragged tile past the slice end are zeroed.
  auto compute = [&](int kt, const float *sa, const float *sb, bool full) {
#pragma unroll
    for (int kk = 0; kk < BK / 8; kk++) {
      const int c = 2 * kk + h;  // this lane's 16-byte chunk of the row
      float4 av[MB], bv[2];
#pragma unroll
      for (int b = 0; b < MB; b++) {
        const int ra = wm * 32 * MB + b * 32 + i;
        av[b] = ld4(sa + ra * BK + 4 * (c ^ ((ra >> 1) & 7)));
      }
#pragma unroll
      for (int b = 0; b < 2; b++) {
        const int rb = wn * 64 + b * 32 + i;
        bv[b] = ld4(sb + rb * BK + 4 * (c ^ ((rb >> 1) & 7)));
      }
      if (!full && !(kt + 4 * c < ke)) {
#pragma unroll
        for (int b = 0; b < MB; b++) av[b] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int b = 0; b < 2; b++) bv[b] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int bm = 0; bm < MB; bm++)
#pragma unroll
        for (int bn = 0; bn < 2; bn++) {
          acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[bm].x, bv[bn].x, acc[bm][bn], 0, 0, 0);
          acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[bm].y, bv[bn].y, acc[bm][bn], 0, 0, 0);
          acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[bm].z, bv[bn].z, acc[bm][bn], 0, 0, 0);
          acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[bm].w, bv[bn].w, acc[bm][bn], 0, 0, 0);
        }
    }
  };

  // Double-buffered K loop with one barrier per tile: at the barrier of tile t every wave has
  // finished tile t-1, whose buffer is then refilled with tile t+1.
  const int ntiles = (ke - kb + BK - 1) / BK;
  if (ntiles > 0) issue(kb, sa0, sb0);
  for (int t = 0; t < ntiles; t += 2) {
    const int kt = kb + t * BK;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of tile t landed
    __syncthreads();
    if (t + 1 < ntiles) issue(kt + BK, sa1, sb1);
    compute(kt, sa0, sb0, kt + BK <= ke);
    // A conditional block rather than a mid-loop exit, so the accumulators leave the loop
    // from one place and keep one set of registers.
    if (t + 1 < ntiles) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (t + 2 < ntiles) issue(kt + 2 * BK, sa0, sb0);
      compute(kt + BK, sa1, sb1, kt + 2 * BK <= ke);
    }
  }

  const bool direct = a.splits == 1;
  float *dst = direct ? a.y : a.part + (size_t)blockIdx.z * a.m * a.n;
#pragma unroll
  for (int bm = 0; bm < MB; bm++)
#pragma unroll
    for (int bn = 0; bn < 2; bn++) {
      const int col = n0 + wn * 64 + bn * 32 + i;
      if (col >= a.n) continue;
      const float bias = direct && a.bias ? a.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * 32 * MB + bm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < a.m) dst[(size_t)row * a.n + col] = acc[bm][bn][r] + bias;
      }
    }
}

// y = bias + sum over slices of the partials, slices added in order; four outputs per thread
// when a row is a multiple of 4 floats, so every load is a float4 and the slices' loads are
// independent.
__global__ void __launch_bounds__(256) linear_reduce_kernel(LinearLaunch a) {
  const size_t plane = (size_t)a.m * a.n;
  const bool vec = (a.n & 3) == 0;
  const size_t units = vec ? plane / 4 : plane;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += stride) {
    if (vec) {
      const size_t idx = 4 * u;
      float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int z = 0; z < a.splits; z++) {
        const float4 p = *reinterpret_cast<const float4 *>(a.part + (size_t)z * plane + idx);
        s.x += p.x;
        s.y += p.y;
        s.z += p.z;
        s.w += p.w;
      }
      if (a.bias) {
        const int col = (int)(idx % a.n);
        s.x += a.bias[col];
        s.y += a.bias[col + 1];
        s.z += a.bias[col + 2];
        s.w += a.bias[col + 3];
      }
      *reinterpret_cast<float4 *>(a.y + idx) = s;
    } else {
      float s = 0.0f;
      for (int z = 0; z < a.splits; z++) s += a.part[(size_t)z * plane + u];
      a.y[u] = a.bias ? s + a.bias[u % a.n] : s;
    }
  }
}

// Tens to a few hundred rows (decode batches): one 32 x 32 block of y per workgroup, so the
// 256-row, 1024-column o_proj alone has 256 workgroups, and the K slice split over the
// workgroup's NW waves.  No operand is shared between the waves, so each wave streams its own
// K range through a private ring of PF LDS stages (32 x rows and 32 W rows of 32 k each),
// copied with global_load_lds_dwordx4 so that every copy instruction reads whole 128-byte
// rows, with the chunk swizzle of the tiled kernel; no barrier until the end.  A stage is read
// into registers whole, its refill issued, then its 16 MFMAs run: lane (i, h) holds
// k = kt + 16h .. kt + 16h + 15 of row i as four float4, and MFMA step j contracts
// k = kt + 16h + j (the same permutation for A and B).  The waves' blocks meet in LDS and are
// added in wave order (plus the bias, or into the slice's partial plane).  Eight waves with two
// stages each (128 KB of LDS, one workgroup per CU) measured faster than four waves with four
// (one wave per SIMD), and than staging through registers instead of LDS.
template <int NW, int PF>
__global__ void __launch_bounds__(64 * NW) skinny_kernel(LinearLaunch a) {
  constexpr int KI = 32;       // k per stage
  constexpr int ST = 32 * KI;  // floats per operand per stage
  __shared__ __attribute__((aligned(16))) float ring[NW][PF][2][ST];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  const int kb = blockIdx.z * a.k_per_split;
  const int ke = min(a.k, kb + a.k_per_split);
  const int per = (ke - kb + NW * KI - 1) / (NW * KI) * KI;
  const int wk0 = kb + w * per, wk1 = min(ke, wk0 + per);
  const int iters = wk1 > wk0 ? (wk1 - wk0 + KI - 1) / KI : 0;

  // Copy instruction g moves rows [8g, 8g + 8) of a stage: lane l takes row 8g + l / 8, LDS
  // chunk position l % 8, i.e. global chunk (l % 8) ^ ((row >> 1) & 7).  Rows and columns past
  // the edge copy the last valid row (their sums are not stored); chunks past the wave's K
  // range copy a valid address and are zeroed at use.
  const int lrow = lane >> 3, lpos = lane & 7;
  // A full block (32 rows of x and of W) and a stage inside the wave's K range: copied from
  // wave-uniform bases (row m0 / n0, column kt) plus fixed byte offsets, shared by x and W
  // (both K-contiguous with row stride k), through buffer descriptors.
  const bool full_block = m0 + 32 <= a.m && n0 + 32 <= a.n && a.k < (1 << 22);
  uint32_t soff[4];
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int r = 8 * g + lrow;
    soff[g] = (uint32_t)r * (uint32_t)a.k * 4u + (uint32_t)(lpos ^ ((r >> 1) & 7)) * 16u;
  }
  const int span_bytes = (31 * a.k + KI) * 4;
  auto issue = [&](int it, int st) {
    const int kt = wk0 + it * KI;
    if (full_block && kt + KI <= wk1) {
      const float *xb = a.x + (size_t)m0 * a.k + kt;
      const float *wb = a.w + (size_t)n0 * a.k + kt;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        copy16_to_lds(xb, span_bytes, soff[g], &ring[w][st][0][g * 8 * KI]);
        copy16_to_lds(wb, span_bytes, soff[g], &ring[w][st][1][g * 8 * KI]);
      }
      return;
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int r = 8 * g + lrow;
      int kc = kt + 4 * (lpos ^ ((r >> 1) & 7));
      kc = kc < wk1 ? kc : 0;
      const int xr = min(m0 + r, a.m - 1);
      const int wr = min(n0 + r, a.n - 1);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)(a.x + (size_t)xr * a.k + kc),
          (__attribute__((address_space(3))) void *)(&ring[w][st][0][g * 8 * KI]), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)(a.w + (size_t)wr * a.k + kc),
          (__attribute__((address_space(3))) void *)(&ring[w][st][1][g * 8 * KI]), 16, 0, 0);
    }
  };
  constexpr int OPS = 8;  // copy instructions per stage
  f32x16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    acc0[r] = 0.0f;
    acc1[r] = 0.0f;
  }
#pragma unroll
  for (int p = 0; p < PF; p++)
    if (p < iters) issue(p, p);
  for (int it = 0; it < iters; it += PF) {
#pragma unroll
    for (int p = 0; p < PF; p++) {
      if (it + p < iters) {
        // Stage p landed: every later stage issued so far (OPS operations each) may still be in
        // flight.
        if (it + p + PF - 1 < iters)
          wait_vm<OPS * (PF - 1)>();
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const int kt = wk0 + (it + p) * KI;
        const float *sa = ring[w][p][0], *sb = ring[w][p][1];
        const int sw = i * KI, sx = (i >> 1) & 7;
        // The whole stage goes to registers first, so its refill is issued before the MFMAs.
        f4v av[4], bv[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          av[q] = lds_read4(sa + sw + 4 * ((4 * h + q) ^ sx));
          bv[q] = lds_read4(sb + sw + 4 * ((4 * h + q) ^ sx));
        }
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]), "+v"(bv[0]),
                       "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3])::"memory");
        if (it + p + PF < iters) issue(it + p + PF, p);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          if (kt + 4 * (4 * h + q) >= wk1) {
            av[q] = f4v{0.f, 0.f, 0.f, 0.f};
            bv[q] = f4v{0.f, 0.f, 0.f, 0.f};
          }
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][0], bv[q][0], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][1], bv[q][1], acc1, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][2], bv[q][2], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][3], bv[q][3], acc1, 0, 0, 0);
        }
      }
    }
  }
  // The wave's block goes to its own first stage (its copies have all landed and been read).
  // Value r of lane (i, h): row 8 * (r / 4) + 4 * h + r % 4, column i.
  float *red = ring[w][0][0];
#pragma unroll
  for (int r = 0; r < 16; r++) red[(8 * (r >> 2) + 4 * h + (r & 3)) * 32 + i] = acc0[r] + acc1[r];
  __syncthreads();
  const bool direct = a.splits == 1;
  float *dst = direct ? a.y : a.part + (size_t)blockIdx.z * a.m * a.n;
  for (int u = threadIdx.x; u < 256; u += 64 * NW) {
    const int row = u >> 3, c = 4 * (u & 7);
    float4 s = ld4(&ring[0][0][0][row * 32 + c]);
#pragma unroll
    for (int v = 1; v < NW; v++) {
      const float4 t = ld4(&ring[v][0][0][row * 32 + c]);
      s.x += t.x;
      s.y += t.y;
      s.z += t.z;
      s.w += t.w;
    }
    if (m0 + row >= a.m) continue;
    float *yr = dst + (size_t)(m0 + row) * a.n;
    const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int col = n0 + c + e;
      if (col < a.n) yr[col] = direct && a.bias ? sv[e] + a.bias[col] : sv[e];
    }
  }
}

// Few rows (decode batches): y = x W^T + bias as a weight-streaming GEMV.  Wave w of
// workgroup b owns output columns n0 = (4b + w) * CPW .. n0 + CPW - 1 for all M rows: lane l
// reads the 16-byte chunks l, l + 64, ... of those W rows (non-temporal loads: W is read once)
// and the same chunks of the M x rows (cached: every wave reads them), keeps M * CPW partial
// dot products, and folds them across the wave in a fixed DPP order.  HBM bytes: W once, plus
// x and y; the MFMA tiles would compute 128-row blocks for a handful of rows.
namespace {

typedef float gv4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4_stream(const float *p) {
  const gv4 t = __builtin_nontemporal_load(reinterpret_cast<const gv4 *>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}

// Sum over the 64 lanes; lane 63 holds the total.
__device__ __forceinline__ float wave_sum(float v) {
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x114, 0xF, 0xE, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x118, 0xF, 0xC, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

}  // namespace

template <int M, int CPW>
__global__ void __launch_bounds__(256) gemv_kernel(LinearLaunch a) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + wave) * CPW;
  if (n0 >= a.n) return;  // uniform per wave
  const int chunks = a.k >> 2;
  float acc[M][CPW];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < CPW; j++) acc[m][j] = 0.0f;
  const float *wr[CPW];
#pragma unroll
  for (int j = 0; j < CPW; j++) wr[j] = a.w + (size_t)min(n0 + j, a.n - 1) * a.k;
  const int rows = min(M, a.m);
  // U chunks per lane in flight, W and x loads issued together before any arithmetic; chunks
  // past the end (and x rows past M) load chunk 0 / row 0 and are skipped.
  constexpr int U = M <= 2 ? 4 : 2;
  for (int c0 = lane; c0 < chunks; c0 += U * 64) {
    float4 wv[U][CPW], xv[U][M];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      ok[u] = c0 + 64 * u < chunks;
      const int c = ok[u] ? c0 + 64 * u : 0;
#pragma unroll
      for (int j = 0; j < CPW; j++) wv[u][j] = ld4_stream(wr[j] + 4 * c);
#pragma unroll
      for (int m = 0; m < M; m++)
        xv[u][m] = *reinterpret_cast<const float4 *>(a.x + (size_t)(m < rows ? m : 0) * a.k + 4 * c);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (!ok[u]) break;
#pragma unroll
      for (int m = 0; m < M; m++) {
        if (m < rows) {
#pragma unroll
          for (int j = 0; j < CPW; j++) {
            acc[m][j] = fmaf(xv[u][m].x, wv[u][j].x, acc[m][j]);
            acc[m][j] = fmaf(xv[u][m].y, wv[u][j].y, acc[m][j]);
            acc[m][j] = fmaf(xv[u][m].z, wv[u][j].z, acc[m][j]);
            acc[m][j] = fmaf(xv[u][m].w, wv[u][j].w, acc[m][j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++) {
    if (m >= rows) break;
#pragma unroll
    for (int j = 0; j < CPW; j++) {
      const float t = wave_sum(acc[m][j]);
      const int n = n0 + j;
      if (lane == 63 && n < a.n) a.y[(size_t)m * a.n + n] = a.bias ? t + a.bias[n] : t;
    }
  }
}

int linear_gemv_max_rows() { return 8; }

hipError_t launch_gemv(const LinearLaunch &a, hipStream_t s) {
  constexpr int CPW = 2;
  const dim3 grid((a.n + 4 * CPW - 1) / (4 * CPW));
  if (a.m <= 1) hipLaunchKernelGGL((gemv_kernel<1, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 2) hipLaunchKernelGGL((gemv_kernel<2, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 4) hipLaunchKernelGGL((gemv_kernel<4, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 8) hipLaunchKernelGGL((gemv_kernel<8, CPW>), grid, dim3(256), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

namespace {

hipError_t launch_reduce(const LinearLaunch &a, hipStream_t s) {
  const size_t units = (a.n & 3) == 0 ? (size_t)a.m * a.n / 4 : (size_t)a.m * a.n;
  const unsigned blocks = (unsigned)std::min<size_t>((units + 255) / 256, 8192);
  hipLaunchKernelGGL(linear_reduce_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_linear(const LinearLaunch &a, hipStream_t s) {
  if (a.m <= 0 || a.n <= 0) return hipSuccess;
  const dim3 grid((a.n + BN - 1) / BN, (a.m + BM - 1) / BM, a.splits);
  if (a.waves_m == 4)
    hipLaunchKernelGGL(linear_kernel<4>, grid, dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(linear_kernel<2>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  return launch_reduce(a, s);
}

hipError_t launch_skinny(const LinearLaunch &a, hipStream_t s) {
  if (a.m <= 0 || a.n <= 0) return hipSuccess;
  const dim3 grid((a.n + 31) / 32, (a.m + 31) / 32, a.splits);
  hipLaunchKernelGGL((skinny_kernel<kSkinnyWaves, 2>), grid, dim3(64 * kSkinnyWaves), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  return launch_reduce(a, s);
}

int linear_tile_rows() { return BM; }
int linear_tile_cols() { return BN; }
int linear_k_tile() { return BK; }
int linear_skinny_waves() { return kSkinnyWaves; }

}  // namespace nva
