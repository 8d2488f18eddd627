// Linear.Row (o_proj): y[M, N] = x[M, K] W[N, K]^T (+ bias) in fp32 on MFMA.
//
// Semantics (tensor/Ops.java:84-124 linear, tensor/MatmulRuntime.java:234-255): W is the
// row-major [out, in] weight, x the [rows, in] activations (the attention output
// [T, Hq * d], used in place), y a fresh [rows, out]; y = x W^T + bias.  The reference sums each
// output in its gemv panel order; here the sum runs over MFMA steps and split-K slices, so the
// result agrees to fp32 rounding (checked against the oracle within the attention tolerance).
//
// Mapping onto CDNA4.  Four kernels by shape:
//   * gemv_kernel for at most 16 rows (a weight-streaming GEMV, below);
//   * skinny16_kernel when 32 x 32 blocks would fill at most half the CUs but 16 x 16 blocks
//     fill at least half (tens to ~128 rows at 1024 columns): one 16 x 16 block per
//     workgroup, K split over its eight waves, no K slices (below);
//   * skinny_kernel when the 32 x 32 blocks of y number at most one per CU (decode batches of
//     tens to a few hundred rows): one block per workgroup, K split over its eight waves, each
//     streaming its own K range through a private LDS ring (below);
//   * linear_kernel otherwise.  A workgroup owns a 128 x 64 tile of y and one K slice; its four
//     waves own 32 rows x 64 columns each (2 blocks of v_mfma_f32_32x32x2_f32).  Two workgroups
//     share a CU (48 KB of LDS, 88 VGPRs each), so while one waits at its barrier the other's
//     MFMAs run on every SIMD: with one 128 x 128 workgroup of eight waves per CU, both waves of
//     a SIMD stopped at the same barrier every tile (28% of wave cycles waiting, MFMA busy 0.77,
//     against 0.93 of the fp32 peak here on large GEMMs).
//   * x and W are both K-contiguous, so the A operand (x rows) and the B operand (W rows) are
//     read the same way: for each 8-wide K step a lane (i, h) reads one float4 of its row
//     (elements 4h .. 4h + 3 of the step), which feeds 4 MFMAs -- MFMA s contracts
//     k = {s, 4 + s} of the step, a permutation that A and B share.
//   * K tiles of 32 are copied HBM -> LDS with buffer loads that write LDS directly, from a
//     wave-uniform base (row m0 / n0, column kt) plus fixed 32-bit lane offsets (rows past the
//     matrix edge repeat its last row; their sums are never stored).  Each 128-byte row of a
//     tile has its 16-byte chunks XOR-swizzled by ((row >> 1) & 7): measured free of LDS bank
//     conflicts.  The copies are issued through copy16_to_lds_async, so the compiler adds no wait
//     on them before the LDS reads of another stage.
//   * Double-buffered, one barrier per K tile, placed before the tile's last 8-k step: the last
//     step's fragments are already in registers, so the barrier (every wave has read this
//     stage, and the next tile has landed) is followed at once by the next tile's copies into
//     this stage and by MFMAs.  The next step's fragments are read while the current step's 8
//     MFMAs run.
//   * Output block layout (32 x 32, 16 values per lane): value r of lane (i, h) is row
//     8 * (r / 4) + 4 * h + r % 4, column i -- lanes 0..31 write 128 contiguous bytes.
//   * Tiles are assigned so that each XCD's workgroups cover one rectangle of the tile grid
//     (xcd_tile below): each XCD's L2 then fetches only its share of x and of W.
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
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BM = 128, BN = 64, BK = 32;  // linear_kernel tile
constexpr int kSkinnyWaves = 8;  // waves of a skinny_kernel workgroup (two per SIMD)

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// Tile (column tile tn, row band tm) of this workgroup within its K slice.  Workgroups are
// handed to the 8 XCDs round-robin by linear block id, so consecutive ids would spread every
// 128-row band of x over all eight L2s, each fetching it again.  When the tile grid divides
// into 8 equal rectangles of gm row bands x gn column tiles (gm * gn = 8), XCD slot t % 8 runs
// rectangle t % 8 and t / 8 walks it row-major: each L2 then fetches 1/gm of x and 1/gn of W.
// gm minimises that sum (x bands are BM rows, W tiles BN rows; ties go to the smaller gm: at
// 4096 x 2048 -> 1024, 4 x 2 rectangles fetched 65 MB against 81 MB as 8 x 1 bands and 142 MB
// in launch order, in the same time).  Any other grid keeps the launch order.  A bijection
// either way, so the result does not depend on where a workgroup actually runs.
__device__ __forceinline__ void xcd_tile(int &tn, int &tm) {
  const int nt = gridDim.x, mt = gridDim.y;
  int gm = 0, best = 0x7fffffff;
  for (int c = 1; c <= 8; c <<= 1) {
    if (mt % c != 0 || nt % (8 / c) != 0) continue;
    const int cost = mt / c * BM + nt / (8 / c) * BN;
    if (cost < best) {
      best = cost;
      gm = c;
    }
  }
  const int t = blockIdx.y * nt + blockIdx.x;
  if (gm == 0) {
    tm = blockIdx.y;
    tn = blockIdx.x;
    return;
  }
  const int gn = 8 / gm, rh = mt / gm, cw = nt / gn;
  const int x = t & 7, r = t >> 3;
  const int lr = r / cw;
  tm = (x / gn) * rh + lr;
  tn = (x % gn) * cw + (r - lr * cw);
}

template <int N> struct IntC { static constexpr int value = N; };
template <bool B> struct BoolC { static constexpr bool value = B; };

}  // namespace

// One 128 x 64 tile of y (or of a K slice's partial plane) per workgroup; wave w owns rows
// 32 w .. 32 w + 31 as two 32 x 32 blocks.
__global__ void __launch_bounds__(256) linear_kernel(LinearLaunch a) {
  constexpr int LA = BM / 32, LB = BN / 32;  // copy instructions per wave per tile (8 rows each)
  constexpr int OPS = LA + LB;
  constexpr int STAGE = (BM + BN) * BK;      // floats: A rows, then B rows
  __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];

  int tn, tm;
  xcd_tile(tn, tm);
  const int n0 = tn * BN;
  const int m0 = tm * BM;
  const int kb = blockIdx.z * a.k_per_split;
  const int ke = min(a.k, kb + a.k_per_split);
  const int ntiles = (ke - kb + BK - 1) / BK;
  const bool ragged = (ke - kb) % BK != 0;  // the last tile ends inside a K tile
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int i = lane & 31;  // MFMA row (A) / column (B) index of this lane
  const int h = lane >> 5;  // which float4 of an 8-wide K step this lane supplies

  f32x16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    acc0[r] = 0.0f;
    acc1[r] = 0.0f;
  }

  // Copy instruction p of wave w moves rows [8g, 8g + 8), g = 4p + w, of A (p < LA) or of B:
  // lane l takes row 8g + l / 8 at LDS chunk position l % 8, i.e. global chunk
  // (l % 8) ^ ((row >> 1) & 7).  Offsets are 32-bit: 128 rows of k floats stay below 2 GiB.
  const int lrow = lane >> 3, lpos = lane & 7;
  const int rows_a = min(BM, a.m - m0), rows_b = min(BN, a.n - n0);
  uint32_t off[OPS];
#pragma unroll
  for (int p = 0; p < OPS; p++) {
    const int r = 8 * (4 * (p < LA ? p : p - LA) + wave) + lrow;
    const int rows = p < LA ? rows_a : rows_b;
    off[p] = (uint32_t)min(r, rows - 1) * (uint32_t)a.k * 4u +
             (uint32_t)(lpos ^ ((r >> 1) & 7)) * 16u;
  }
  const uint32_t lds0 = lds_address(lds);
  auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
    // The descriptors end at the last row's column min(kt + BK, k): nothing past the matrix.
    const int cols = min(BK, a.k - kt);
    const float *xb = a.x + (size_t)m0 * a.k + kt;
    const float *wb = a.w + (size_t)n0 * a.k + kt;
    const uint32_t dst = lds0 + (uint32_t)(stage * STAGE) * 4u;
#pragma unroll
    for (int p = 0; p < LA; p++)
      copy16_to_lds_async(xb, ((rows_a - 1) * a.k + cols) * 4, off[p],
                          dst + (uint32_t)((4 * p + wave) * 8 * BK) * 4u);
#pragma unroll
    for (int p = 0; p < LB; p++)
      copy16_to_lds_async(wb, ((rows_b - 1) * a.k + cols) * 4, off[LA + p],
                          dst + (uint32_t)((BM + (4 * p + wave) * 8) * BK) * 4u);
  };

  // Fragments of 8-k step kk of a stage: A rows 32 w + i, B rows i and 32 + i, chunk 2 kk + h.
  const int ra = 32 * wave + i;
  const int xa = 4 * ((ra >> 1) & 7), xb = 4 * ((i >> 1) & 7);  // chunk swizzles (B: same for i, 32 + i)
  auto frag = [&](int stage, int kk, float4 &av, float4 &b0, float4 &b1) __attribute__((always_inline)) {
    const float *s = lds + stage * STAGE;
    const int c = 4 * (2 * kk + h);
    av = ld4(s + ra * BK + (c ^ xa));
    b0 = ld4(s + (BM + i) * BK + (c ^ xb));
    b1 = ld4(s + (BM + 32 + i) * BK + (c ^ xb));
  };
  // Chunks of a ragged last tile past the slice end are zero in both operands.
  auto mask = [&](int kt, int kk, float4 &av, float4 &b0, float4 &b1) __attribute__((always_inline)) {
    if (kt + 4 * (2 * kk + h) >= ke) {
      av = make_float4(0.f, 0.f, 0.f, 0.f);
      b0 = av;
      b1 = av;
    }
  };
  // The two blocks' accumulations alternate, so no MFMA waits on the one before it.
  auto mma = [&](const float4 &av, const float4 &b0, const float4 &b1) __attribute__((always_inline)) {
    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, b0.x, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, b1.x, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, b0.y, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, b1.y, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, b0.z, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, b1.z, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, b0.w, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, b1.w, acc1, 0, 0, 0);
  };

  float4 fa0, fb00, fb01, fa1, fb10, fb11;  // two fragment sets: steps 0/2 and 1/3
  if (ntiles > 0) {
    issue(kb, 0);
    if (ntiles > 1) {
      issue(kb + BK, 1);
      wait_copies<OPS>();
    } else {
      wait_copies<0>();
    }
    lds_barrier();
    frag(0, 0, fa0, fb00, fb01);
  }
  // Tile t in stage s (a constant: two tiles per loop iteration).  RAGGED (the last tile of a
  // slice that ends inside it) zeroes the chunks past the slice end; it is a separate copy of
  // the body, so the common body is straight-line code the compiler can interleave.
  auto tile = [&](int t, auto s_, auto ragged_) __attribute__((always_inline)) {
    constexpr int s = decltype(s_)::value;
    constexpr bool RAGGED = decltype(ragged_)::value;
    const int kt = kb + t * BK;
    frag(s, 1, fa1, fb10, fb11);
    if (RAGGED) mask(kt, 0, fa0, fb00, fb01);
    mma(fa0, fb00, fb01);
    frag(s, 2, fa0, fb00, fb01);
    if (RAGGED) mask(kt, 1, fa1, fb10, fb11);
    mma(fa1, fb10, fb11);
    frag(s, 3, fa1, fb10, fb11);
    if (RAGGED) mask(kt, 2, fa0, fb00, fb01);
    mma(fa0, fb00, fb01);
    if (t + 1 < ntiles) {
      // This wave's reads of stage s have returned (step 3 is in registers) and its copies of
      // tile t + 1 have landed (tile t + 2's are not issued yet); after the barrier the same
      // holds for every wave, so stage s takes tile t + 2 and tile t + 1 is read.
      wait_lds_reads();
      wait_copies<0>();
      lds_barrier();
      if (t + 2 < ntiles) issue(kt + 2 * BK, s);
      frag(s ^ 1, 0, fa0, fb00, fb01);
    }
    if (RAGGED) mask(kt, 3, fa1, fb10, fb11);
    mma(fa1, fb10, fb11);
  };
  const int full_tiles = ragged ? ntiles - 1 : ntiles;
  int t = 0;
  for (; t + 1 < full_tiles; t += 2) {
    tile(t, IntC<0>{}, BoolC<false>{});
    tile(t + 1, IntC<1>{}, BoolC<false>{});
  }
  if (t < full_tiles) {
    tile(t, IntC<0>{}, BoolC<false>{});
    t++;
  }
  if (t < ntiles) {  // the ragged last tile, in stage t % 2
    if (t & 1)
      tile(t, IntC<1>{}, BoolC<true>{});
    else
      tile(t, IntC<0>{}, BoolC<true>{});
  }

  const bool direct = a.splits == 1;
  float *dst = direct ? a.y : a.part + (size_t)blockIdx.z * a.m * a.n;
#pragma unroll
  for (int bn = 0; bn < 2; bn++) {
    const int col = n0 + bn * 32 + i;
    if (col >= a.n) continue;
    const float bias = direct && a.bias ? a.bias[col] : 0.0f;
    const f32x16 &acc = bn == 0 ? acc0 : acc1;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m0 + 32 * wave + 8 * (r >> 2) + 4 * h + (r & 3);
      if (row < a.m) dst[(size_t)row * a.n + col] = acc[r] + bias;
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
// copied with buffer loads that write LDS directly so that every copy instruction reads whole
// 128-byte rows, with the tiled kernel's chunk swizzle; no barrier until the end.  A stage is
// read into registers whole, its refill issued, then its 16 MFMAs run: lane (i, h) holds
// k = kt + 16h .. kt + 16h + 15 of row i as four float4, and MFMA step j contracts
// k = kt + 16h + j (the same permutation for A and B).  The waves' blocks meet in LDS and are
// added in wave order (plus the bias, or into the slice's partial plane).  Eight waves with two
// stages each (128 KB of LDS, one workgroup per CU) measured faster than four waves with four
// (one wave per SIMD), and than staging through registers instead of LDS.
template <int NW, int PF>
__global__ void __launch_bounds__(64 * NW) skinny_kernel(LinearLaunch a) {
  constexpr int KI = 32;       // k per stage
  constexpr int ST = 32 * KI;  // floats per operand per stage
  constexpr int OPS = 8;       // copy instructions per stage
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

  // Copy instruction g moves rows [8g, 8g + 8) of a stage: lane l takes row 8g + l / 8 (rows
  // past the edge repeat the last valid row; their sums are not stored), LDS chunk position
  // l % 8, i.e. global chunk (l % 8) ^ ((row >> 1) & 7), from wave-uniform bases (row m0 / n0,
  // column kt).  Chunks past the wave's K range are zeroed at use.
  const int lrow = lane >> 3, lpos = lane & 7;
  const int rows_x = min(32, a.m - m0), rows_w = min(32, a.n - n0);
  uint32_t offx[4], offw[4];
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int r = 8 * g + lrow;
    const uint32_t c = (uint32_t)(lpos ^ ((r >> 1) & 7)) * 16u;
    offx[g] = (uint32_t)min(r, rows_x - 1) * (uint32_t)a.k * 4u + c;
    offw[g] = (uint32_t)min(r, rows_w - 1) * (uint32_t)a.k * 4u + c;
  }
  const uint32_t ring0 = lds_address(&ring[w][0][0][0]);
  auto issue = [&](int it, int st) __attribute__((always_inline)) {
    const int kt = wk0 + it * KI;
    const int cols = min(KI, a.k - kt);  // the descriptors end inside the matrix
    const float *xb = a.x + (size_t)m0 * a.k + kt;
    const float *wb = a.w + (size_t)n0 * a.k + kt;
    const uint32_t dst = ring0 + (uint32_t)(st * 2 * ST) * 4u;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      copy16_to_lds_async(xb, ((rows_x - 1) * a.k + cols) * 4, offx[g], dst + g * 8 * KI * 4);
      copy16_to_lds_async(wb, ((rows_w - 1) * a.k + cols) * 4, offw[g],
                          dst + (ST + g * 8 * KI) * 4);
    }
  };
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
        // Stage p landed: every later stage issued so far (OPS copies each) may still be in
        // flight.
        if (it + p + PF - 1 < iters)
          wait_copies<OPS * (PF - 1)>();
        else
          wait_copies<0>();
        const int kt = wk0 + (it + p) * KI;
        const float *sa = ring[w][p][0], *sb = ring[w][p][1];
        const int sw = i * KI, sx = (i >> 1) & 7;
        // The whole stage goes to registers first, so its refill is issued before the MFMAs.
        float4 av[4], bv[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          av[q] = ld4(sa + sw + 4 * ((4 * h + q) ^ sx));
          bv[q] = ld4(sb + sw + 4 * ((4 * h + q) ^ sx));
        }
        if (it + p + PF < iters) {
          wait_lds_reads();  // the refill overwrites this stage
          issue(it + p + PF, p);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          if (kt + 4 * (4 * h + q) >= wk1) {
            av[q] = make_float4(0.f, 0.f, 0.f, 0.f);
            bv[q] = av[q];
          }
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q].x, bv[q].x, acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q].y, bv[q].y, acc1, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q].z, bv[q].z, acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q].w, bv[q].w, acc1, 0, 0, 0);
        }
      }
    }
  }
  // The wave's block goes to its own first stage (its copies have all landed and been read).
  // Value r of lane (i, h): row 8 * (r / 4) + 4 * h + r % 4, column i.
  wait_lds_reads();
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

// Decode batches whose 32 x 32 blocks would leave half the CUs idle (tens to ~128 rows at
// 1024 columns): one 16 x 16 block of y per workgroup on v_mfma_f32_16x16x4_f32, four times the
// workgroups, so K needs no slices and no reduce launch.  As in skinny_kernel, K is split over
// the workgroup's NW waves, each streaming its own K range through a private LDS ring (16 x
// rows and 16 W rows of 32 k per stage, chunk-swizzled), and the waves' blocks are added in
// wave order through LDS.  Lane (i, g) supplies row i's chunks g and g + 4 of a stage (4 k
// each) to both operands; MFMA (t, e) contracts component e of chunk g + 4t over g, a k order
// A and B share.
template <int NW, int PF>
__global__ void __launch_bounds__(64 * NW) skinny16_kernel(LinearLaunch a) {
  constexpr int KI = 32;       // k per stage
  constexpr int ST = 16 * KI;  // floats per operand per stage
  constexpr int OPS = 4;       // copy instructions per stage
  __shared__ __attribute__((aligned(16))) float ring[NW][PF][2][ST];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int kb = blockIdx.z * a.k_per_split;
  const int ke = min(a.k, kb + a.k_per_split);
  const int per = (ke - kb + NW * KI - 1) / (NW * KI) * KI;
  const int wk0 = kb + w * per, wk1 = min(ke, wk0 + per);
  const int iters = wk1 > wk0 ? (wk1 - wk0 + KI - 1) / KI : 0;

  // Copy instruction c moves rows [8c, 8c + 8) of an operand: lane l takes row 8c + l / 8 (rows
  // past the edge repeat the last valid row; their sums are not stored), LDS chunk position
  // l % 8, i.e. global chunk (l % 8) ^ ((row >> 1) & 7).  Chunks past the wave's K range are
  // zeroed at use.
  const int lrow = lane >> 3, lpos = lane & 7;
  const int rows_x = min(16, a.m - m0), rows_w = min(16, a.n - n0);
  uint32_t offx[2], offw[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int r = 8 * c + lrow;
    const uint32_t ch = (uint32_t)(lpos ^ ((r >> 1) & 7)) * 16u;
    offx[c] = (uint32_t)min(r, rows_x - 1) * (uint32_t)a.k * 4u + ch;
    offw[c] = (uint32_t)min(r, rows_w - 1) * (uint32_t)a.k * 4u + ch;
  }
  const uint32_t ring0 = lds_address(&ring[w][0][0][0]);
  auto issue = [&](int it, int st) __attribute__((always_inline)) {
    const int kt = wk0 + it * KI;
    const int cols = min(KI, a.k - kt);  // the descriptors end inside the matrix
    const float *xb = a.x + (size_t)m0 * a.k + kt;
    const float *wb = a.w + (size_t)n0 * a.k + kt;
    const uint32_t dst = ring0 + (uint32_t)(st * 2 * ST) * 4u;
#pragma unroll
    for (int c = 0; c < 2; c++) {
      copy16_to_lds_async(xb, ((rows_x - 1) * a.k + cols) * 4, offx[c], dst + c * 8 * KI * 4);
      copy16_to_lds_async(wb, ((rows_w - 1) * a.k + cols) * 4, offw[c],
                          dst + (ST + c * 8 * KI) * 4);
    }
  };
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int p = 0; p < PF; p++)
    if (p < iters) issue(p, p);
  for (int it = 0; it < iters; it += PF) {
#pragma unroll
    for (int p = 0; p < PF; p++) {
      if (it + p < iters) {
        if (it + p + PF - 1 < iters)
          wait_copies<OPS * (PF - 1)>();
        else
          wait_copies<0>();
        const int kt = wk0 + (it + p) * KI;
        const float *sa = ring[w][p][0], *sb = ring[w][p][1];
        const int sw = i * KI, sx = (i >> 1) & 7;
        float4 av[2], bv[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
          av[t] = ld4(sa + sw + 4 * ((g + 4 * t) ^ sx));
          bv[t] = ld4(sb + sw + 4 * ((g + 4 * t) ^ sx));
        }
        if (it + p + PF < iters) {
          wait_lds_reads();  // the refill overwrites this stage
          issue(it + p + PF, p);
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
          if (kt + 4 * (g + 4 * t) >= wk1) {
            av[t] = make_float4(0.f, 0.f, 0.f, 0.f);
            bv[t] = av[t];
          }
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t].x, bv[t].x, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t].y, bv[t].y, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t].z, bv[t].z, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t].w, bv[t].w, acc, 0, 0, 0);
        }
      }
    }
  }
  // The wave's block goes to its own first stage.  Value r of lane (j, g): row 4g + r, column j.
  wait_lds_reads();
  float *red = ring[w][0][0];
#pragma unroll
  for (int r = 0; r < 4; r++) red[(4 * g + r) * 16 + i] = acc[r];
  __syncthreads();
  for (int u = threadIdx.x; u < 64; u += 64 * NW) {
    const int row = u >> 2, c = 4 * (u & 3);
    float4 sacc = ld4(&ring[0][0][0][row * 16 + c]);
#pragma unroll
    for (int v = 1; v < NW; v++) {
      const float4 t = ld4(&ring[v][0][0][row * 16 + c]);
      sacc.x += t.x;
      sacc.y += t.y;
      sacc.z += t.z;
      sacc.w += t.w;
    }
    if (m0 + row >= a.m) continue;
    float *yr = a.y + (size_t)(m0 + row) * a.n;
    const float sv[4] = {sacc.x, sacc.y, sacc.z, sacc.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int col = n0 + c + e;
      if (col < a.n) yr[col] = a.bias ? sv[e] + a.bias[col] : sv[e];
    }
  }
}

// Few rows (decode batches): y = x W^T + bias as a weight-streaming GEMV.  Workgroup b owns
// output columns n0 = b * CPW .. n0 + CPW - 1 for all M rows, and its wave w the w-th quarter
// of K: lane l reads the 16-byte chunks l, l + 64, ... of that quarter of those W rows
// (non-temporal loads: W is read once) and the same chunks of the M x rows (cached: every
// workgroup reads them), keeps M * CPW partial dot products, folds them across the wave in a
// fixed DPP order, and the four quarters are added in wave order through LDS.  With K split,
// a 2048-wide row takes one round of loads per wave and the grid has four times the waves
// (8 per CU at 1024 columns), so the latency of the load rounds is paid once.  HBM bytes: W
// once, plus x and y; the MFMA tiles would compute 128-row blocks for a handful of rows.
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
  __shared__ float red[4][M][CPW];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n0 = blockIdx.x * CPW;  // the workgroup's columns; K is split over its 4 waves
  const int chunks = a.k >> 2;
  const int per = (chunks + 3) >> 2;
  const int cb = wave * per;
  const int ce = min(chunks, cb + per);
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
  // past the wave's range (and x rows past M) load the lane's first chunk / row 0 and are
  // skipped.
  constexpr int U = M <= 2 ? 4 : 2;
  for (int c0 = cb + lane; c0 < ce; c0 += U * 64) {
    float4 wv[U][CPW], xv[U][M];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      ok[u] = c0 + 64 * u < ce;
      const int c = ok[u] ? c0 + 64 * u : c0;
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
  // Each wave's sums (left in lane 63), then the four K quarters added in wave order.
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < CPW; j++) {
      const float t = wave_sum(acc[m][j]);
      if (lane == 63) red[wave][m][j] = t;
    }
  __syncthreads();
  if (threadIdx.x < M * CPW) {
    const int m = threadIdx.x / CPW;
    const int j = threadIdx.x - m * CPW;
    const int n = n0 + j;
    if (m < rows && n < a.n) {
      const float t = (red[0][m][j] + red[1][m][j]) + (red[2][m][j] + red[3][m][j]);
      a.y[(size_t)m * a.n + n] = a.bias ? t + a.bias[n] : t;
    }
  }
}

int linear_gemv_max_rows() { return 16; }

hipError_t launch_gemv(const LinearLaunch &a, hipStream_t s) {
  constexpr int CPW = 2;
  const dim3 grid((a.n + CPW - 1) / CPW);
  if (a.m <= 1) hipLaunchKernelGGL((gemv_kernel<1, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 2) hipLaunchKernelGGL((gemv_kernel<2, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 4) hipLaunchKernelGGL((gemv_kernel<4, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 8) hipLaunchKernelGGL((gemv_kernel<8, CPW>), grid, dim3(256), 0, s, a);
  else if (a.m <= 16) hipLaunchKernelGGL((gemv_kernel<16, CPW>), grid, dim3(256), 0, s, a);
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
  hipLaunchKernelGGL(linear_kernel, grid, dim3(256), 0, s, a);
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

hipError_t launch_skinny16(const LinearLaunch &a, hipStream_t s) {
  if (a.m <= 0 || a.n <= 0) return hipSuccess;
  if (a.splits != 1) return hipErrorInvalidValue;  // one K range per block (no partial planes)
  const dim3 grid((a.n + 15) / 16, (a.m + 15) / 16, 1);
  hipLaunchKernelGGL((skinny16_kernel<kSkinnyWaves, 2>), grid, dim3(64 * kSkinnyWaves), 0, s, a);
  return hipGetLastError();
}

int linear_tile_rows() { return BM; }
int linear_tile_cols() { return BN; }
int linear_k_tile() { return BK; }
int linear_skinny_waves() { return kSkinnyWaves; }

}  // namespace nva
