// Kernel (c): varlen causal prefill on fp32 MFMA over dense K/V or the paged KV cache.
//
// Semantics (layers/Attention.java:245-280 prefillDense / prefillWithCache, :328-396
// attendJobs): query qi of a sequence with qLen queries and kLen keys sits at absolute
// position aq = kLen - qLen + qi and sees keys [max(0, aq - W + 1) (window W > 0, else 0),
// aq]; KV head kvh = h / rep; score = dot(q, k) * scale; out = softmax-weighted sum of v.
// Keys come from dense k/v rows (prefillDense) or from the cache through the block table
// (prefillWithCache).
//
// Mapping onto CDNA4.  The grid is exactly as many workgroups per head group as can be
// resident at once; each runs the segments of its slot of a stream-K schedule (equal numbers
// of 32-key tiles per slot; a query tile whose keys straddle slots is split and its partials
// merged).  The whole step's K/V (tens of MB) stays in the 256 MB Infinity Cache, which all
// XCDs share, so slots need no XCD-aware placement.  A segment is a tile of 16 * 8 / HPW queries of one
// sequence for HPW query heads of one KV head, over a key range [ks, ke).  The 8 waves of the
// workgroup each own 16 queries of one head.
//   * Key tiles of 32 rows of K and V are copied HBM -> LDS with 16-byte loads that write LDS
//     directly (no register staging), double-buffered so the next tile streams in while this
//     one is used; one barrier per tile.  A full tile inside one page (or of dense rows) is 32
//     consecutive rows: its copies are buffer loads from a wave-uniform descriptor plus fixed
//     32-bit lane offsets, no per-lane address arithmetic; the last tile of a chunk and tiles
//     that cross a page compute each row's address (rows past the chunk clamped).  Rows are
//     stored unpadded; K rows have their 16-byte chunks XOR-swizzled (kswz) so the column
//     reads of QK are conflict-free, V rows are read along the row and need no swizzle.  The
//     block ids of the segment's pages are staged in LDS once, so a paged tile load never
//     waits on a global table read.
//   * Per tile each wave computes (D = 128)
//       S^T[key][query] = K Q^T      64 x v_mfma_f32_16x16x4_f32, K from LDS (ds_read_b128),
//                                    Q (16 queries x D/4 per lane) resident in registers;
//       O^T[dim][query] += V^T P^T   64 x v_mfma_f32_16x16x4_f32, one ds_read_b128 of V feeds
//                                    4 MFMAs (output block 4*hh + b holds dims 64*hh + 4r + b).
//     With S transposed each lane holds 8 keys of ONE query: the row max is an in-lane max plus
//     exchanges with lane^16 and lane^32, and P^T lands exactly in the registers the PV MFMA
//     reads as its B operand (the key order of the contraction is permuted to match), so P
//     never touches LDS.
//   * Softmax runs in the log2 domain (scale * log2 e folded into the score, v_exp_f32), and the
//     running max is only moved -- and O rescaled -- when a tile's max exceeds it by more than
//     2^8, which after the first tiles almost never happens.
//   * Only tiles that cross the causal diagonal, the window edge or the end of the keys are
//     masked.
#include "nva_internal.h"
#include "nva_device.h"

namespace nva {

typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyRescale = 8.0f;  // log2 units

}  // namespace

// Pages of one key chunk whose block ids are staged in LDS (the host splits chunks to fit).
constexpr int kTablePages = kPrefillTablePages;

namespace {

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// The pair {x[lane], x[lane ^ 16]} (resp. lane ^ 32) in every lane, by gfx950's row-swap
// instructions: both outputs of the swap of x with itself hold one of the two values.
struct Pair {
  float a, b;
};
__device__ __forceinline__ Pair pair_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ Pair pair_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
// Max and sum over the four lanes {i, i+16, i+32, i+48}; every lane gets the same bits.
__device__ __forceinline__ float max4_lanes(float x) {
  const Pair p = pair_xor16(x);
  const Pair q = pair_xor32(fmaxf(p.a, p.b));
  return fmaxf(q.a, q.b);
}
__device__ __forceinline__ float sum4_lanes(float x) {
  const Pair p = pair_xor16(x);
  const Pair q = pair_xor32(p.a + p.b);
  return q.a + q.b;
}
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

// LDS position of chunk c of K row r (and, being an involution, the chunk at position c):
// the low three bits are XORed with r & 7; from d = 256 on, where a lane group's 16 or more
// chunks span a whole 256-byte bank period, bit 3 is also XORed with bit 4 of the chunk, which
// tells adjacent lane groups apart (a lane group reads chunks 16g + j at d = 256 and, in the
// half-row waves of d = 512, 64 half + 16g + j).  Measured with SQ_LDS_BANK_CONFLICT: zero
// conflicts for d = 128, 256 and 512 (r & 15 alone: 33% of the LDS-active cycles at d = 128;
// at d = 512, bit 3 from the parity of c / 32: 30%).
template <int D>
__device__ __forceinline__ int kswz(int c, int r) {
  constexpr int GS = D / 16;  // chunks per lane group of a full-row read
  int x = r & 7;
  if constexpr (GS >= 16) x |= ((c >> 4) & 1) << 3;
  return c ^ x;
}

// Row of key t: dense rows follow kbase; paged rows go through the LDS copy of the block
// table, which starts at page blk0.
__device__ __forceinline__ int64_t tile_row(const KvView &kv, const int32_t *stab, int blk0,
                                            int kbase, int t) {
  if (!kv.paged) return (int64_t)kbase + t;
  int blk, off;
  if (kv.bs_shift >= 0) {
    blk = t >> kv.bs_shift;
    off = t & (kv.block_size - 1);
  } else {
    blk = t / kv.block_size;
    off = t - blk * kv.block_size;
  }
  return (int64_t)stab[blk - blk0] * kv.block_size + off;
}

}  // namespace

// NW waves per workgroup, KT keys per tile.  Four waves per SIMD (at most 128 VGPRs) for
// d <= 128; d = 256 needs more than 128 registers for its Q and O blocks, and d = 512 keeps
// its O blocks in AGPRs (one wave per SIMD).
template <int D, int HPW, int KT, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 4 : 1)))
prefill_kernel(TileLaunch a) {
  constexpr int KB = KT / 16;      // 16-key MFMA blocks per key tile
  constexpr int DQ = D / 4;        // QK contraction steps per lane group g: dims [DQ*g, DQ*g+DQ)
  constexpr int NB = D / 16;       // O^T blocks of 16 dims: block 4*hh+bb holds dims 64*hh+4r+bb
  constexpr int H64 = D / 64;      // 64-dim halves of a V row (one ds_read_b128 each)
  constexpr int C4 = D / 4;        // 16-byte chunks per K/V row
  constexpr int NI = KT * C4 / 64;  // load instructions per tensor per tile (64 chunks each)
  constexpr int LPW = NI / NW;     // load instructions per wave per tensor per tile
  constexpr int TILE = KT * D;     // floats per K (or V) tile
  static_assert(LPW >= 1 && NI % NW == 0, "tile does not split evenly over the waves");
  __shared__ __attribute__((aligned(16))) float sk0[TILE];
  __shared__ __attribute__((aligned(16))) float sv0[TILE];
  __shared__ __attribute__((aligned(16))) float sk1[TILE];
  __shared__ __attribute__((aligned(16))) float sv1[TILE];
  __shared__ int32_t stab[kTablePages];  // block ids of the pages this chunk touches

  const int slot = blockIdx.x;
  const int seg_end = a.seg_off[slot + 1];
  // Byte offsets of this lane's copies within a tile whose 32 rows are consecutive rows of the
  // K/V arrays (every full tile of a dense step, and of a paged one when it lies in one page):
  // such a tile is copied from one wave-uniform base plus these fixed offsets.
  uint32_t koff[LPW], voff[LPW];
  {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rsb = (uint32_t)(a.hkv * D) * 4u;
#pragma unroll
    for (int p = 0; p < LPW; p++) {
      const int q = (p * NW + wave) * 64 + lane;  // chunk q of the tile, row-major
      const int r = q / C4, pos = q - r * C4;
      koff[p] = (uint32_t)r * rsb + (uint32_t)kswz<D>(pos, r) * 16u;
      voff[p] = (uint32_t)r * rsb + (uint32_t)pos * 16u;
    }
  }
  for (int seg = a.seg_off[slot]; seg < seg_end; seg++) {
  // Every wave is done with the previous segment's LDS tiles and table before they are reused.
  __syncthreads();
  const TileItem it = a.items[seg];
  const int rep = a.hq / a.hkv;
  const int groups = rep / HPW;
  const int kvh = blockIdx.y / groups;
  // Wave-uniform, and known to be: every value derived from it lives in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = kvh * rep + (blockIdx.y - kvh * groups) * HPW + wave % HPW;
  const int qb = wave / HPW;
  const int lane = threadIdx.x & 63;
  const int i = lane & 15;   // MFMA row/column index of this lane
  const int g = lane >> 4;   // MFMA k-slot (lane group)
  const int W = a.window;
  const int off = it.klen - it.qlen;  // absolute position of query 0
  const float sl2 = a.scale * kLog2e;

  // This lane's query (column i of S^T) and its visible key range.
  const int qi = it.q0 + qb * 16 + i;
  const bool qvalid = qi < it.qlen;
  const int qic = qvalid ? qi : it.qlen - 1;
  const int aq = off + qic;
  const int vis_lo = W > 0 ? max(0, aq - W + 1) : 0;
  const int vis_hi = aq + 1;
  // The wave's 16 queries: bounds of their visible ranges.
  const int wq0 = it.q0 + qb * 16;
  const bool wave_active = wq0 < it.qlen;
  const int wq1 = min(wq0 + 15, it.qlen - 1);
  const int wlo_min = W > 0 ? max(0, off + wq0 - W + 1) : 0;
  const int wlo_max = W > 0 ? max(0, off + wq1 - W + 1) : 0;
  const int whi_min = off + wq0 + 1;
  const int whi_max = off + wq1 + 1;

  // Q^T operand: lane (i, g) holds Q[query i][DQ*g + s], s < DQ, for the whole key loop.
  // Read from a wave-uniform row base plus a 32-bit lane offset (queries past the sequence
  // read its last one; a wave with none reads that one too).
  float qr[DQ];
  {
    const int wq0c = min(wq0, it.qlen - 1);
    const float *qw = a.q + ((size_t)(it.qstart + wq0c) * a.hq + h) * D;
    const uint32_t lo = (uint32_t)(qic - wq0c) * (uint32_t)(a.hq * D) + (uint32_t)(DQ * g);
#pragma unroll
    for (int s = 0; s < DQ; s += 4) {
      const float4 x = ld4(qw + lo + s);
      qr[s] = x.x;
      qr[s + 1] = x.y;
      qr[s + 2] = x.z;
      qr[s + 3] = x.w;
    }
  }

  f32x4 o[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) o[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;  // log2 units
  float l_run = 0.0f;

  const size_t rs = (size_t)a.hkv * D;
  const float *kbase = a.kv.k + (size_t)kvh * D;
  const float *vbase = a.kv.v + (size_t)kvh * D;
  // Stage the chunk's block ids in LDS once, so the tile loads never wait on a global load.
  int blk0 = 0;
  if (a.kv.paged) {
    const int bs = a.kv.block_size;
    blk0 = it.ks / bs;
    const int npages = (it.ke - 1) / bs - blk0 + 1;
    const int32_t *table = a.kv.table + (size_t)it.seq * a.kv.bt_stride + blk0;
    for (int j = threadIdx.x; j < npages; j += blockDim.x) stab[j] = table[j];
    __syncthreads();
  }
  // Load instruction gi copies chunks [64 gi, 64 gi + 64) of the tile in row-major order (a
  // whole number of rows for d <= 256, half a row at d = 512): lane l takes chunk q = 64 gi + l,
  // i.e. position q % C4 of tile row q / C4.
  const int lrow = C4 <= 64 ? lane / C4 : 0;  // rows within one instruction (d <= 256)
  const int lpos = C4 <= 64 ? lane - lrow * C4 : 0;
  int cur_page = -1;  // page whose block id cur_id holds (wave-uniform)
  int cur_id = 0;
  auto issue_tile = [&](int kt, float *dk, float *dv) {
    // A full tile inside one page (or of dense rows): one uniform row base, fixed offsets
    // (32-bit: the tile's rows must span less than 2 GiB).
    if (kt + KT <= it.ke && rs < (size_t)(1 << 22) &&
        (!a.kv.paged || (a.kv.bs_shift >= 0 && (kt >> a.kv.bs_shift) ==
                                                   ((kt + KT - 1) >> a.kv.bs_shift)))) {
      int64_t row0;
      if (!a.kv.paged) {
        row0 = (int64_t)it.kbase + kt;
      } else {
        const int pg = kt >> a.kv.bs_shift;
        if (pg != cur_page) {
          cur_id = __builtin_amdgcn_readfirstlane(stab[pg - blk0]);
          cur_page = pg;
        }
        row0 = (int64_t)cur_id * a.kv.block_size + (kt - (pg << a.kv.bs_shift));
      }
      const int tile_bytes = KT * (int)rs * 4;
      const float *gk0 = kbase + row0 * (int64_t)rs;
      const float *gv0 = vbase + row0 * (int64_t)rs;
#pragma unroll
      for (int p = 0; p < LPW; p++) {
        const int gi = p * NW + wave;
        copy16_to_lds(gk0, tile_bytes, koff[p], dk + gi * 256);
        copy16_to_lds(gv0, tile_bytes, voff[p], dv + gi * 256);
      }
      return;
    }
    // Last (partial) tile, or one that crosses a page: per-row addresses, rows past the chunk
    // clamped to its last key.
#pragma unroll
    for (int p = 0; p < LPW; p++) {
      const int gi = p * NW + wave;
      int r, pos;
      if constexpr (C4 <= 64) {
        r = gi * (64 / C4) + lrow;
        pos = lpos;
      } else {
        const int q = gi * 64 + lane;
        r = q / C4;
        pos = q - r * C4;
      }
      const int key = min(kt + r, it.ke - 1);  // rows past the chunk are loaded but masked
      const int64_t row = tile_row(a.kv, stab, blk0, it.kbase, key);
      // K chunks are XOR-swizzled (kswz) for the column reads of QK; V rows are read
      // along the row, which is conflict-free unswizzled.
      const float *gk = kbase + row * rs + kswz<D>(pos, r) * 4;
      const float *gv = vbase + row * rs + pos * 4;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)gk,
          (__attribute__((address_space(3))) void *)(dk + gi * 256), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)gv,
          (__attribute__((address_space(3))) void *)(dv + gi * 256), 16, 0, 0);
    }
  };

  auto compute_tile = [&](int kt, const float *sk, const float *sv) {
    if (!wave_active || kt >= whi_max || kt + KT <= wlo_min) return;
    const bool full = (kt + KT <= whi_min) && (kt >= wlo_max);

    // S^T = K Q^T per 16-key block kb: A[key][k] = K[16kb + i][DQ*g + s] (lane i, g),
    // B[k][query] = qr[s].  Chunk c = (DQ/4)*g + j of row 16kb+i sits at kswz(c, i).  Chunk
    // j of every block is read at once, so each LDS wait is followed by 4 * KB MFMAs that
    // alternate between the blocks' accumulators.
    f32x4 st[KB];
#pragma unroll
    for (int blk = 0; blk < KB; blk++) st[blk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const float *kb[DQ / 4];
#pragma unroll
    for (int j = 0; j < DQ / 4; j++) kb[j] = sk + i * D + 4 * kswz<D>((DQ / 4) * g + j, i);
#pragma unroll
    for (int s = 0; s < DQ; s += 4) {
      float4 kk[KB];
#pragma unroll
      for (int blk = 0; blk < KB; blk++) kk[blk] = ld4(kb[s >> 2] + blk * 16 * D);
#pragma unroll
      for (int blk = 0; blk < KB; blk++)
        st[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[blk].x, qr[s], st[blk], 0, 0, 0);
#pragma unroll
      for (int blk = 0; blk < KB; blk++)
        st[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[blk].y, qr[s + 1], st[blk], 0, 0, 0);
#pragma unroll
      for (int blk = 0; blk < KB; blk++)
        st[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[blk].z, qr[s + 2], st[blk], 0, 0, 0);
#pragma unroll
      for (int blk = 0; blk < KB; blk++)
        st[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[blk].w, qr[s + 3], st[blk], 0, 0, 0);
    }

    // p[4*blk + v] holds key kt + 16*blk + 4*g + v for query i (log2-scaled).
    float p[4 * KB];
    float mx = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < KB; blk++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        float x = st[blk][v] * sl2;
        if (!full) {
          const int key = kt + 16 * blk + 4 * g + v;
          x = (key >= vis_lo && key < vis_hi) ? x : -INFINITY;
        }
        p[4 * blk + v] = x;
        mx = fmaxf(mx, x);
      }
    mx = max4_lanes(mx);
    const bool need = mx > m_run + kLazyRescale;
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
    for (int s = 0; s < 4 * KB; s++) {
      p[s] = __builtin_amdgcn_exp2f(p[s] - ms);
      l_run += p[s];
    }

    // O^T += V^T P^T: step s contracts key 16*(s/4) + 4*g + s%4 (= p[s] in this lane).  The A
    // operand of block 4*hh + bb is V[key][64*hh + 4*i + bb], one ds_read_b128 per hh.
    const float *vrow = sv + 4 * g * D + 4 * i;
#pragma unroll
    for (int s = 0; s < 4 * KB; s++) {
      const float *vp = vrow + (16 * (s >> 2) + (s & 3)) * D;
#pragma unroll
      for (int hh = 0; hh < H64; hh++) {
        const float4 vv = ld4(vp + 64 * hh);
        o[4 * hh + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, p[s], o[4 * hh + 0], 0, 0, 0);
        o[4 * hh + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, p[s], o[4 * hh + 1], 0, 0, 0);
        o[4 * hh + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, p[s], o[4 * hh + 2], 0, 0, 0);
        o[4 * hh + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, p[s], o[4 * hh + 3], 0, 0, 0);
      }
    }
  };

  // Double-buffered key loop with one barrier per tile: at the barrier of tile t every wave
  // has finished tile t-1 (so its buffer can be refilled with tile t+1) and tile t has landed.
  const int ntiles = (it.ke - it.ks + KT - 1) / KT;
  issue_tile(it.ks, sk0, sv0);
  for (int t = 0; t < ntiles; t += 2) {
    const int kt = it.ks + t * KT;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of tile t landed
    __syncthreads();
    if (t + 1 < ntiles) issue_tile(kt + KT, sk1, sv1);
    compute_tile(kt, sk0, sv0);
    if (t + 1 >= ntiles) break;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 2 < ntiles) issue_tile(kt + 2 * KT, sk0, sv0);
    compute_tile(kt + KT, sk1, sv1);
  }

  const float l_tot = sum4_lanes(l_run);
  if (!qvalid || !wave_active) continue;
  // Lane (i, g) holds O^T rows r = 4g + v of every block: dims 64*hh + 4r + bb.
  float *op;
  float inv = 1.0f;
  const bool partial = it.part >= 0;
  size_t pidx = 0;
  if (!partial) {
    inv = l_tot == 0.0f ? 0.0f : 1.0f / l_tot;
    op = a.out + ((size_t)(it.qstart + qi) * a.hq + h) * D;
  } else {
    // Partial of one key chunk: rows of the tile are laid out query-major, chunk-minor.
    pidx = ((size_t)it.part + (size_t)(qi - it.q0) * it.nsplit + it.split) * a.hq + h;
    op = a.part_acc + pidx * D;
  }
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int r = 4 * g + v;
#pragma unroll
    for (int hh = 0; hh < H64; hh++)
      st4(op + 64 * hh + 4 * r, make_float4(o[4 * hh][v] * inv, o[4 * hh + 1][v] * inv,
                                          o[4 * hh + 2][v] * inv, o[4 * hh + 3][v] * inv));
  }
  if (partial && g == 0) {
    a.part_m[pidx] = m_run;
    a.part_l[pidx] = l_tot;
  }
  }  // segments
}

// Head dim 512 (Gemma 4 global layers) with the head split over a wave pair: one 8-wave
// workgroup per CU, waves w and w + 4 own the same 16 queries and the dims [256 h, 256 h + 256)
// of half h = w / 4.  Each wave forms the partial S^T of its half (64 MFMAs per 16-key tile),
// the pair adds the two partials through LDS in a fixed order (S = S_0 + S_1 in both waves, so
// both hold the same scores and run the same softmax) and each accumulates O^T for its own
// 256 dims.  Q and O take 64 registers each instead of 128, so two waves fit per SIMD and
// one covers the other's LDS waits (one 256-dim wave per SIMD left the matrix pipe idle for
// every LDS read).  Every wave executes the exchange barrier of every tile, active or not.
template <int HPW>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
prefill512_kernel(TileLaunch a) {
  constexpr int D = 512, DH = 256, KT = 16, NW = 8;
  constexpr int DQ = DH / 4;         // QK steps per lane group: dims DH*half + DQ*g + [0, DQ)
  constexpr int NB = DH / 16;        // O^T blocks of the half: block 4*hh+bb, dims 64*hh+4r+bb
  constexpr int H64 = DH / 64;
  constexpr int C4 = D / 4;          // 16-byte chunks per K/V row
  constexpr int NI = KT * C4 / 64;   // load instructions per tensor per tile
  constexpr int LPW = NI / NW;
  constexpr int TILE = KT * D;
  static_assert(HPW == 1, "one query head per workgroup");
  static_assert(LPW >= 1 && NI % NW == 0, "tile does not split evenly over the waves");
  __shared__ __attribute__((aligned(16))) float sk0[TILE];
  __shared__ __attribute__((aligned(16))) float sv0[TILE];
  __shared__ __attribute__((aligned(16))) float sk1[TILE];
  __shared__ __attribute__((aligned(16))) float sv1[TILE];
  __shared__ f32x4 spart[NW][64];  // each wave's partial S^T of the current tile
  __shared__ int32_t stab[kTablePages];

  const int slot = blockIdx.x;
  const int seg_end = a.seg_off[slot + 1];
  for (int seg = a.seg_off[slot]; seg < seg_end; seg++) {
  __syncthreads();
  const TileItem it = a.items[seg];
  const int rep = a.hq / a.hkv;
  const int kvh = blockIdx.y / rep;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.y;  // one head per workgroup: grid y runs over the query heads
  const int half = wave >> 2;
  const int qb = wave & 3;
  const int lane = threadIdx.x & 63;
  const int i = lane & 15;
  const int g = lane >> 4;
  const int W = a.window;
  const int off = it.klen - it.qlen;
  const float sl2 = a.scale * kLog2e;

  const int qi = it.q0 + qb * 16 + i;
  const bool qvalid = qi < it.qlen;
  const int qic = qvalid ? qi : it.qlen - 1;
  const int aq = off + qic;
  const int vis_lo = W > 0 ? max(0, aq - W + 1) : 0;
  const int vis_hi = aq + 1;
  const int wq0 = it.q0 + qb * 16;
  const bool wave_active = wq0 < it.qlen;
  const int wq1 = min(wq0 + 15, it.qlen - 1);
  const int wlo_min = W > 0 ? max(0, off + wq0 - W + 1) : 0;
  const int wlo_max = W > 0 ? max(0, off + wq1 - W + 1) : 0;
  const int whi_min = off + wq0 + 1;
  const int whi_max = off + wq1 + 1;

  float qr[DQ];
  {
    const float *qp = a.q + ((size_t)(it.qstart + qic) * a.hq + h) * D + DH * half + DQ * g;
#pragma unroll
    for (int s = 0; s < DQ; s += 4) {
      const float4 x = ld4(qp + s);
      qr[s] = x.x;
      qr[s + 1] = x.y;
      qr[s + 2] = x.z;
      qr[s + 3] = x.w;
    }
  }
  f32x4 o[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) o[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const size_t rs = (size_t)a.hkv * D;
  const float *kbase = a.kv.k + (size_t)kvh * D;
  const float *vbase = a.kv.v + (size_t)kvh * D;
  int blk0 = 0;
  if (a.kv.paged) {
    const int bs = a.kv.block_size;
    blk0 = it.ks / bs;
    const int npages = (it.ke - 1) / bs - blk0 + 1;
    const int32_t *table = a.kv.table + (size_t)it.seq * a.kv.bt_stride + blk0;
    for (int j = threadIdx.x; j < npages; j += blockDim.x) stab[j] = table[j];
    __syncthreads();
  }
  auto issue_tile = [&](int kt, float *dk, float *dv) {
#pragma unroll
    for (int p = 0; p < LPW; p++) {
      const int gi = p * NW + wave;
      const int q = gi * 64 + lane;
      const int r = q / C4;
      const int pos = q - r * C4;
      const int key = min(kt + r, it.ke - 1);
      const int64_t row = tile_row(a.kv, stab, blk0, it.kbase, key);
      const float *gk = kbase + row * rs + kswz<D>(pos, r) * 4;
      const float *gv = vbase + row * rs + pos * 4;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)gk,
          (__attribute__((address_space(3))) void *)(dk + gi * 256), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)gv,
          (__attribute__((address_space(3))) void *)(dv + gi * 256), 16, 0, 0);
    }
  };

  auto compute_tile = [&](int kt, const float *sk, const float *sv) {
    const bool active = wave_active && kt < whi_max && kt + KT > wlo_min;
    f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (active) {
      // Partial S^T over this half: A[key][k] = K[i][DH*half + DQ*g + s], chunk
      // 64*half + 16*g + s/4 of row i, at kswz(chunk, i).
      const float *kr = sk + i * D;
#pragma unroll
      for (int s = 0; s < DQ; s += 4) {
        const float4 kk = ld4(kr + 4 * kswz<D>(64 * half + 16 * g + (s >> 2), i));
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.x, qr[s], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.y, qr[s + 1], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.z, qr[s + 2], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.w, qr[s + 3], st, 0, 0, 0);
      }
      spart[wave][lane] = st;
    }
    __syncthreads();
    if (!active) return;
    const f32x4 other = spart[wave ^ 4][lane];
    st = half == 0 ? st + other : other + st;  // S_0 + S_1 in both waves of the pair
    const bool full = (kt + KT <= whi_min) && (kt >= wlo_max);

    // p[v] holds key kt + 4*g + v for query i (log2-scaled).
    float p[4];
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float x = st[v] * sl2;
      if (!full) {
        const int key = kt + 4 * g + v;
        x = (key >= vis_lo && key < vis_hi) ? x : -INFINITY;
      }
      p[v] = x;
      mx = fmaxf(mx, x);
    }
    mx = max4_lanes(mx);
    const bool need = mx > m_run + kLazyRescale;
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
    for (int v = 0; v < 4; v++) {
      p[v] = __builtin_amdgcn_exp2f(p[v] - ms);
      l_run += p[v];
    }

    // O^T += V^T P^T over this half's dims: step s contracts key 4*g + s (= p[s] in this lane).
    const float *vrow = sv + 4 * g * D + DH * half + 4 * i;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const float *vp = vrow + s * D;
#pragma unroll
      for (int hh = 0; hh < H64; hh++) {
        const float4 vv = ld4(vp + 64 * hh);
        o[4 * hh + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, p[s], o[4 * hh + 0], 0, 0, 0);
        o[4 * hh + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, p[s], o[4 * hh + 1], 0, 0, 0);
        o[4 * hh + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, p[s], o[4 * hh + 2], 0, 0, 0);
        o[4 * hh + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, p[s], o[4 * hh + 3], 0, 0, 0);
      }
    }
  };

  const int ntiles = (it.ke - it.ks + KT - 1) / KT;
  issue_tile(it.ks, sk0, sv0);
  for (int t = 0; t < ntiles; t += 2) {
    const int kt = it.ks + t * KT;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 1 < ntiles) issue_tile(kt + KT, sk1, sv1);
    compute_tile(kt, sk0, sv0);
    if (t + 1 >= ntiles) break;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 2 < ntiles) issue_tile(kt + 2 * KT, sk0, sv0);
    compute_tile(kt + KT, sk1, sv1);
  }

  const float l_tot = sum4_lanes(l_run);
  if (!qvalid || !wave_active) continue;
  float *op;
  float inv = 1.0f;
  const bool partial = it.part >= 0;
  size_t pidx = 0;
  if (!partial) {
    inv = l_tot == 0.0f ? 0.0f : 1.0f / l_tot;
    op = a.out + ((size_t)(it.qstart + qi) * a.hq + h) * D + DH * half;
  } else {
    pidx = ((size_t)it.part + (size_t)(qi - it.q0) * it.nsplit + it.split) * a.hq + h;
    op = a.part_acc + pidx * D + DH * half;
  }
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int r = 4 * g + v;
#pragma unroll
    for (int hh = 0; hh < H64; hh++)
      st4(op + 64 * hh + 4 * r, make_float4(o[4 * hh][v] * inv, o[4 * hh + 1][v] * inv,
                                          o[4 * hh + 2][v] * inv, o[4 * hh + 3][v] * inv));
  }
  if (partial && g == 0 && half == 0) {
    a.part_m[pidx] = m_run;
    a.part_l[pidx] = l_tot;
  }
  }  // segments
}

namespace {

// Keys per tile and waves per workgroup for head dim D.
template <int D>
constexpr int key_tile() {
  return D == 512 ? 16 : 32;
}
template <int D>
constexpr int tile_waves() {
  return 8;
}

template <int D>
hipError_t launch_prefill_d(const TileLaunch &a, int hpw, hipStream_t s) {
  constexpr int KT = key_tile<D>(), NW = tile_waves<D>();
  const dim3 grid(a.num_slots, a.hkv * ((a.hq / a.hkv) / hpw)), block(64 * NW);
  switch (hpw) {
    case 1: hipLaunchKernelGGL((prefill_kernel<D, 1, KT, NW>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<D, 2, KT, NW>), grid, block, 0, s, a); break;
    case 4:
      if constexpr (NW >= 4) {
        hipLaunchKernelGGL((prefill_kernel<D, 4, KT, NW>), grid, block, 0, s, a);
        break;
      }
      return hipErrorInvalidValue;
    case 8:
      if constexpr (NW >= 8) {
        hipLaunchKernelGGL((prefill_kernel<D, 8, KT, NW>), grid, block, 0, s, a);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

int prefill_waves(int head_dim) {
  if (head_dim == 64) return tile_waves<64>();
  if (head_dim == 256) return tile_waves<256>();
  if (head_dim == 512) return tile_waves<512>();
  return tile_waves<128>();
}

// At d = 512 a wave pair shares 16 queries (prefill512_kernel), one query head per workgroup;
// otherwise each wave owns 16 queries and up to a quarter of the waves share a head group.
int prefill_max_heads(int head_dim) {
  return head_dim == 512 ? 1 : std::max(1, prefill_waves(head_dim) / 4);
}

int prefill_tile_queries(int head_dim, int heads_per_wg) {
  const int query_blocks = head_dim == 512 ? prefill_waves(head_dim) / 2 : prefill_waves(head_dim);
  return 16 * (query_blocks / heads_per_wg);
}

bool prefill_kernel_supports(int head_dim, int heads_per_wg) {
  return (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512) &&
         (heads_per_wg == 1 || heads_per_wg == 2 || heads_per_wg == 4 || heads_per_wg == 8) &&
         heads_per_wg <= prefill_max_heads(head_dim);
}

namespace {

// Uncached: the caller (one context per device) keeps the answer.  The query reads the
// current device's properties, so the caller makes its device current first.
template <int D, int HPW>
int blocks_per_cu() {
  constexpr int NW = tile_waves<D>();
  int b = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &b, prefill_kernel<D, HPW, key_tile<D>(), NW>, 64 * NW, 0) != hipSuccess ||
      b < 1)
    b = 1;
  return b;
}

template <int D>
int blocks_per_cu_d(int hpw) {
  constexpr int NW = tile_waves<D>();
  switch (hpw) {
    case 1: return blocks_per_cu<D, 1>();
    case 2: return blocks_per_cu<D, 2>();
    case 4: return blocks_per_cu<D, NW >= 4 ? 4 : 1>();
    default: return blocks_per_cu<D, NW >= 8 ? 8 : 1>();
  }
}

}  // namespace

int prefill_blocks_per_cu(int head_dim, int heads_per_wg) {
  if (head_dim == 64) return blocks_per_cu_d<64>(heads_per_wg);
  if (head_dim == 256) return blocks_per_cu_d<256>(heads_per_wg);
  if (head_dim == 512) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, prefill512_kernel<1>, 512, 0) !=
            hipSuccess ||
        b < 1)
      b = 1;
    return b;
  }
  return blocks_per_cu_d<128>(heads_per_wg);
}

hipError_t launch_prefill_tiles(const TileLaunch &a, int hpw, hipStream_t s) {
  if (a.num_items <= 0 || a.num_slots <= 0) return hipSuccess;
  switch (a.head_dim) {
    case 64: return launch_prefill_d<64>(a, hpw, s);
    case 128: return launch_prefill_d<128>(a, hpw, s);
    case 256: return launch_prefill_d<256>(a, hpw, s);
    case 512:
      if (hpw != 1) return hipErrorInvalidValue;
      hipLaunchKernelGGL((prefill512_kernel<1>), dim3(a.num_slots, a.hq), dim3(512), 0, s, a);
      return hipGetLastError();
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nva
