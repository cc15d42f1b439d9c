// Panel kernel: out[M,N] = x1[M,K] · x2[K,N] for M <= 4 with a row-major x2
// (fp32 or bf16 in, fp32 out) — the GEMV regime of tilec's matmul, where the
// whole cost is streaming x2 from HBM once.
//
// Replaces, for small M, the reference's threadgroup-split dot product with a
// SIMD-group reduction (the legacy `_matrix_mul`, README.md:57,73, config
// space tilec/ext.py:29-51) and the 64x64 tile kernel's mostly empty tiles
// (tilec/ext.py:13-24).  It is output-stationary: a workgroup owns one panel
// of output columns — 512 bytes of each x2 row, 128 fp32 or 256 bf16
// columns — and one K split; the grid is panels fastest, splits slowest.
//
// What sets the rate at the GEMV sizes (x2 of 64 MiB; MI355X, x2 rotated over
// 512 MiB so every launch reads HBM), measured with per-workgroup
// s_memrealtime timelines and plain-read probes:
//   * the workgroups in flight must read the same rows of x2 side by side.
//     K is cut into batches of R = 64 rows and split s of S takes batches
//     s, s + S, s + 2S, ...; with panels fastest in the grid the chip then
//     reads one window of S batches of whole 16 KiB rows at a time.  A plain
//     read of 64 MiB in that order took 10.6-11.0 us against 11.6 us with
//     each workgroup reading one contiguous K chunk, and 12.5 us or more
//     with pieces of 256 bytes or less per row;
//   * a workgroup's waves sweep down each batch together: wave w takes row
//     pairs w, w + W, ..., 32 lanes x 16 bytes per row;
//   * about one workgroup of 8 waves per CU keeps the K split small, and
//     the split's tail short: after its last row the workgroup adds its
//     waves in LDS once, then wave 0 alone publishes the partial, counts
//     itself in and, if last, adds the partials with every load issued at
//     once.  That tail is three memory round trips (publish, count, read
//     back), about 1.8 us after the last row at K = N = 4096.
//
// Lane l: row rr = l / 32 of each row pair, 16-byte group cq = l % 32 of the
// panel (CPL = 4 fp32 / 8 bf16 columns).  It accumulates out[m][col] for its
// columns over its rows in plain FMAs (bf16 widened exactly, a 16-bit
// shift), x1[m][row] coming from the cache.  Masking is on addresses: rows
// past K, columns past N and x1 rows past M load zeros without
// touching memory, from both operands.
//
// Split K: the workgroup publishes its partial with agent-coherent (sc1)
// stores, waits for them, and counts itself in on the panel's counter
// (relaxed, agent scope); the workgroup that brings the count to S resets it
// and adds the S partials in split order (its own from registers), so
// results do not depend on scheduling.  No workgroup waits for another, so
// the grid needs no co-residency.
#include <algorithm>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;  // bf16 bit pattern

constexpr int kRows = 16;           // partial slots reserve 16 rows (the streaming kernel's block)
constexpr int kKcMax = 1024;        // rows of K per workgroup at most
constexpr int kCounterStride = 64;  // uint32s between panel counters (own 256-byte line each)
constexpr int kCpolX2 = 2;          // x2 is streamed once: non-temporal loads

template <typename T>
struct PE;
template <>
struct PE<float> {
  static constexpr int CPL = 4, BYTES = 4;
  typedef f32x4 V;
};
template <>
struct PE<u16> {
  static constexpr int CPL = 8, BYTES = 2;
  typedef i32x4 V;
};

template <typename T>
constexpr int kPanelOf = 32 * PE<T>::CPL;  // 128 fp32 / 256 bf16 columns = 512 bytes

__device__ __forceinline__ float bf_lo(int w) { return __int_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(int w) { return __int_as_float(w & (int)0xffff0000u); }

// Element e of a 16-byte group.
template <typename T>
__device__ __forceinline__ float elem(const typename PE<T>::V& v, int e) {
  if constexpr (sizeof(T) == 4) return v[e];
  else return (e & 1) ? bf_hi(v[e >> 1]) : bf_lo(v[e >> 1]);
}

struct PanelGeom {
  int64_t panels, splits, kc;
};

// Splits of K.  A split takes the R-row batches (R = rows_per_batch, one
// batch of the whole workgroup) split, split + S, split + 2S, ... of K, so
// the workgroups in flight read one window of S neighbouring batches of x2
// rows.  The split count is the request raised so that no split has more
// than kc_max / R batches (the kernel's unrolled bound) and capped at the
// number of batches (none is empty); kc = rows of the largest split.
PanelGeom panel_geom(int64_t N, int64_t K, int split_k, int pw, int kc_max, int rows_per_batch) {
  PanelGeom g;
  g.panels = cdiv(N, pw);
  if (K <= 0) {
    g.splits = 1;
    g.kc = 0;
    return g;
  }
  const int64_t kblk = cdiv(K, rows_per_batch), per = kc_max / rows_per_batch;
  int64_t s = split_k < 1 ? 1 : split_k;
  s = std::max(s, cdiv(kblk, per));
  s = std::min(s, kblk);
  g.splits = s;
  g.kc = cdiv(kblk, s) * rows_per_batch;
  return g;
}

template <typename T, int WAVES, int MV, bool CA, int KC, int BT>
__global__ __launch_bounds__(WAVES * 64) void panel_kernel(const T* __restrict__ x1, const T* __restrict__ x2,
                                                           float* __restrict__ out, int M, int N, int K,
                                                           int64_t ldx1, int64_t ldx2, int64_t ldo,
                                                           unsigned* __restrict__ counters,
                                                           float* __restrict__ part) {
  static_assert(MV >= 1 && MV <= 4, "M <= 4");
  static_assert(KC % (2 * WAVES * BT) == 0 && KC <= kKcMax, "whole batches of row pairs");
  using E = PE<T>;
  typedef typename E::V V;
  constexpr int CPL = E::CPL, PW = kPanelOf<T>;
  constexpr int VPL = PW / 64;         // columns per lane of wave 0 after the reduction
  constexpr int R = 2 * WAVES * BT;    // rows of one workgroup batch
  constexpr int PPW = KC / (2 * WAVES);  // row pairs per wave at most
  constexpr uint32_t EB = E::BYTES;
  __shared__ float red[WAVES][MV][PW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rr = lane >> 5, cq = lane & 31;
  const int panel = blockIdx.x, split = blockIdx.y;
  const int panels = gridDim.x, S = gridDim.y;
  const int n0 = panel * PW;
  const bool gok = n0 + CPL * cq < N;  // N % CPL == 0: the lane's group is all in or all out
  // Batches of this split: global batches split, split + S, ... of R rows
  // each (at most KC / R of them: the launcher's split count sees to it).
  const int kblk = (K + R - 1) / R;
  const int nbat = split < kblk ? (kblk - split + S - 1) / S : 0;

  // In a batch, row pair p (rows 2p, 2p + 1 of the batch) belongs to wave
  // p % W; pair q of this wave is p = q * W + wave.  Resources are based at
  // the batch: 32-bit offsets (the launcher checks KC * ldx2 and KC * ldx1
  // fit, and R <= KC).
  auto x1_off = [&](int m, int row) -> uint32_t {
    return EB * (CA ? (uint32_t)row * (uint32_t)ldx1 + (uint32_t)m : (uint32_t)m * (uint32_t)ldx1 + (uint32_t)row);
  };
  auto ld_x1 = [&](const BufRsrc& rx1, uint32_t o) -> float {
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx1, (int)o, 0, 0));
    else return __int_as_float((int)__builtin_amdgcn_raw_buffer_load_b16(rx1, (int)o, 0, 0) << 16);
  };

  // Rows past K are masked by the resources' extents: a batch's x2
  // resource ends at its last row before K, and so does its x1 resource
  // when M <= 1 and x1 is row-major (offsets stay below R rows: the launcher
  // checks KC * ldx2 and KC * ldx1 fit in 31 bits).  Columns past N: the
  // lane's base offset is kOob, and kOob plus an offset below 2^31 stays out
  // of range.  No select or compare per load: around the offset arithmetic
  // one became a branch per load.
  constexpr bool kX1Extent = MV == 1 && !CA;
  const uint32_t lane_off = gok ? EB * (uint32_t)(CPL * cq) : kOob;
  // (Every input is wave-uniform; make_rsrc_uniform keeps the resources in
  // scalar registers, which the min / max of the row count would otherwise
  // lose, wrapping each load in a waterfall loop.)
  auto x2_rsrc = [&](int64_t row0, int rows) {
    return make_rsrc_uniform(x2 + row0 * ldx2 + n0, (uint32_t)max(rows, 0) * (uint32_t)ldx2 * EB);
  };
  auto x1_rsrc = [&](int64_t row0, int rows) {
    return make_rsrc_uniform(CA ? x1 + row0 * ldx1 : x1 + row0, kX1Extent ? (uint32_t)max(rows, 0) * EB : 0x7FFFFFFFu);
  };

  float acc[MV][CPL];
#pragma unroll
  for (int m = 0; m < MV; ++m)
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[m][c] = 0.f;
  // Batches of BT row pairs per wave, fully unrolled up to KC / R.  x1:
  // every lane of a row needs the same MV values; for M == 1 each lane loads
  // its own (one address per row), for M <= 4 lane cq < MV of the row loads
  // x1[cq][row] and the row's lanes take them by shuffles once it has
  // arrived.  Rows past K load zeros from both operands.
  struct Batch {
    V v[BT];
    float x[BT];  // the lane's own x1 load
  };
  auto load_batch = [&](int bi, Batch& B) __attribute__((always_inline)) {
    const int kb = (bi * S + split) * R;  // the batch's first row
    const int left = K - kb;               // rows of K from it
    const BufRsrc rx2 = x2_rsrc(kb, min(left, R));
    const BufRsrc rx1 = x1_rsrc(kb, min(left, R));
#pragma unroll
    for (int q = 0; q < BT; ++q) {
      const int row = 2 * (q * WAVES + wave) + rr;
      B.v[q] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(
                                         rx2, (int)(lane_off + EB * (uint32_t)row * (uint32_t)ldx2), 0, kCpolX2));
      // Explicit masks (x1 column-major or M > 1) get bit 31 or-ed in: every
      // offset here is below 2^31 when the element is valid.
      if constexpr (kX1Extent) B.x[q] = ld_x1(rx1, x1_off(0, row));
      else if constexpr (MV == 1) B.x[q] = ld_x1(rx1, oob_unless((row < left) & (M > 0)) | x1_off(0, row));
      else B.x[q] = ld_x1(rx1, oob_unless((row < left) & (cq < MV) & (cq < M)) | x1_off(cq, row));
    }
  };
  auto fma_batch = [&](const Batch& B) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < BT; ++q) {
      float a[MV];
      if constexpr (MV == 1) a[0] = B.x[q];
      else {
#pragma unroll
        for (int m = 0; m < MV; ++m) a[m] = __shfl(B.x[q], (lane & 32) + m);
      }
#pragma unroll
      for (int m = 0; m < MV; ++m)
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[m][c] = __builtin_fmaf(a[m], elem<T>(B.v[q], c), acc[m][c]);
    }
  };
  // One batch at a time (the chip's workgroups then read one window of
  // rows); the workgroup stops after its last batch.
#pragma unroll
  for (int bi = 0; bi < PPW / BT; ++bi) {
    if (bi >= nbat) break;  // workgroup-uniform
    Batch B;
    load_batch(bi, B);
    fma_batch(B);
  }

  // The two rows of a pair meet in a shuffle, the waves in LDS (wave order).
#pragma unroll
  for (int m = 0; m < MV; ++m)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const float v = acc[m][c] + __shfl_xor(acc[m][c], 32);
      if (rr == 0) red[wave][m][CPL * cq + c] = v;
    }
  __syncthreads();
  if (wave != 0) return;
  // Wave 0, lane l: columns n0 + 64 v + l (v < VPL) of rows m < MV.
  float t[MV][VPL];
#pragma unroll
  for (int m = 0; m < MV; ++m)
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      float x = red[0][m][64 * v + lane];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) x += red[w][m][64 * v + lane];
      t[m][v] = x;
    }
  auto live = [&](int m, int v) { return (m < M) & (n0 + 64 * v + lane < N); };
  if (S == 1) {
#pragma unroll
    for (int m = 0; m < MV; ++m)
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        if (live(m, v)) out[(int64_t)m * ldo + n0 + 64 * v + lane] = t[m][v];
    return;
  }

  // Split K.  Partial of split s: kRows x PW floats at ((s * panels + panel) * kRows + m) * PW + col.
  const BufRsrc prs = make_rsrc(part);
  auto poff = [&](int s, int m, int v) {
    return 4u * ((((uint32_t)s * (uint32_t)panels + (uint32_t)panel) * kRows + (uint32_t)m) * PW +
                 (uint32_t)(64 * v + lane));
  };
#pragma unroll
  for (int m = 0; m < MV; ++m)
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, t[m][v]), prs,
                                            (int)(live(m, v) ? poff(split, m, v) : kOob), 0, kCpolSc1);
  __builtin_amdgcn_s_waitcnt(0);
  unsigned prev = 0;
  if (lane == 0)
    prev = __hip_atomic_fetch_add(&counters[panel * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = (unsigned)__builtin_amdgcn_readfirstlane((int)prev);
  if (prev != (unsigned)(S - 1)) return;
  if (lane == 0) __hip_atomic_store(&counters[panel * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float sum[MV][VPL];
#pragma unroll
  for (int m = 0; m < MV; ++m)
#pragma unroll
    for (int v = 0; v < VPL; ++v) sum[m][v] = 0.f;
  // Every load of a batch of 8 splits is issued before the first add; the
  // own split's values come from registers, at their place in split order.
  for (int s0 = 0; s0 < S; s0 += 8) {
    float p[8][MV][VPL];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int m = 0; m < MV; ++m)
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const int s = s0 + j;
          p[j][m][v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                     prs, (int)((s < S) & (s != split) & live(m, v) ? poff(s, m, v) : kOob),
                                                     0, kCpolSc1));
        }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int m = 0; m < MV; ++m)
#pragma unroll
        for (int v = 0; v < VPL; ++v) sum[m][v] += s0 + j == split ? t[m][v] : p[j][m][v];
  }
#pragma unroll
  for (int m = 0; m < MV; ++m)
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      if (live(m, v)) out[(int64_t)m * ldo + n0 + 64 * v + lane] = sum[m][v];
}

}  // namespace

// Streaming-kernel fallback (skinny.hip): variants of it for the layouts and
// alignments the panel kernel does not take.
template <typename T, int WAVES, int UB, int MV>
hipError_t launch_skinny_fallback(const MatmulArgs& a);

namespace {

// Row-major x2 with 16-byte groups that never straddle N (N and ldx2
// multiples of CPL, x2 16-byte aligned), M <= MV, x1 in either layout: the
// panel kernel.  Anything else runs the streaming kernel with the same split.
template <typename T, int WAVES, int MV, int KC, int BT>
hipError_t launch_panel(const MatmulArgs& a) {
  constexpr int CPL = PE<T>::CPL, PW = kPanelOf<T>;
  constexpr int64_t EB = sizeof(T), lim = (int64_t(1) << 31) - 64;
  auto aligned = [](const void* p, size_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  const bool ca = a.layout & TILEC_X1_COL_MAJOR;
  const bool fits = !(a.layout & TILEC_X2_COL_MAJOR) && a.M <= MV && a.N % CPL == 0 && a.ldx2 % CPL == 0 &&
                    aligned(a.x2, 16) && KC * a.ldx2 * EB < lim && (ca ? KC * a.ldx1 * EB : 4 * a.ldx1 * EB + KC * EB) < lim;
  if (!fits) return launch_skinny_fallback<T, 4, 2, MV>(a);
  const PanelGeom g = panel_geom(a.N, a.K, a.split_k, PW, KC, 2 * WAVES * BT);
  unsigned* counters = g.splits > 1 ? a.counters : nullptr;
  float* part = g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr;
  const dim3 grid((unsigned)g.panels, (unsigned)g.splits);
  if (ca)
    hipLaunchKernelGGL((panel_kernel<T, WAVES, MV, true, KC, BT>), grid, dim3(WAVES * 64), 0, a.stream,
                       static_cast<const T*>(a.x1), static_cast<const T*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K,
                       a.ldx1, a.ldx2, a.ldo, counters, part);
  else
    hipLaunchKernelGGL((panel_kernel<T, WAVES, MV, false, KC, BT>), grid, dim3(WAVES * 64), 0, a.stream,
                       static_cast<const T*>(a.x1), static_cast<const T*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K,
                       a.ldx1, a.ldx2, a.ldo, counters, part);
  return hipGetLastError();
}

}  // namespace

// Scratch of a panel variant: what the panel kernel needs, or what the
// streaming fallback needs at the same split, whichever is larger (the size
// queries do not see the pointers that decide between them).
size_t skinny_counter_bytes(int dtype, int64_t M, int64_t N, int64_t K, int split_k);
size_t skinny_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K, int split_k);

// Rows of one workgroup batch of a panel variant (unroll = row pairs per
// wave and batch).
static int panel_batch_rows(const VariantDesc& d) { return 2 * d.waves * d.unroll; }

static PanelGeom panel_geom_of(const VariantDesc& d, int64_t N, int64_t K, int split_k) {
  return panel_geom(N, K, split_k, d.bn, d.bk, panel_batch_rows(d));
}

int64_t panel_effective_splits(const VariantDesc& d, int64_t N, int64_t K, int split_k) {
  return panel_geom_of(d, N, K, split_k).splits;
}

size_t panel_workspace_bytes(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  const PanelGeom g = panel_geom_of(d, N, K, split_k);
  const size_t own = g.splits > 1 ? (size_t)g.splits * g.panels * kRows * d.bn * sizeof(float) : 0;
  return std::max(own, skinny_workspace_bytes(d.dtype, M, N, K, split_k));
}
size_t panel_counter_bytes(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  const PanelGeom g = panel_geom_of(d, N, K, split_k);
  const size_t own = g.splits > 1 ? (size_t)g.panels * kCounterStride * sizeof(unsigned) : 0;
  return std::max(own, skinny_counter_bytes(d.dtype, M, N, K, split_k));
}

// Variant table of this family (appended after the streaming and tile
// tables, so earlier variant ids are unchanged).  BM = 16 rows (partial
// slots), BN = panel width, BK = KC, the most rows of K one workgroup takes
// (512 fp32 / 256 bf16: one workgroup per CU at K = N = 4096), max_m = MV,
// unroll = BT, row pairs per wave and batch (batches of 2 W BT = 64 rows);
// an automatic split aims at one workgroup per CU.
static VariantDesc panel_desc(const char* name, int dtype, int waves, int max_m, int kc, int bt,
                              hipError_t (*launch)(const MatmulArgs&)) {
  VariantDesc d{name, TILEC_FAMILY_SKINNY, dtype, kRows, dtype == TILEC_BF16 ? kPanelOf<u16> : kPanelOf<float>,
                kc, waves, max_m, bt, launch};
  d.workspace_bytes = panel_workspace_bytes;
  d.counter_bytes = panel_counter_bytes;
  d.effective_splits = panel_effective_splits;
  d.wgs_per_cu = 1;
  return d;
}

const VariantDesc* panel_variants(int* count) {
  static const VariantDesc t[] = {
      panel_desc("skinny_f32_p_v1_w8", TILEC_F32, 8, 1, 512, 4, launch_panel<float, 8, 1, 512, 4>),
      panel_desc("skinny_f32_p_v4_w8", TILEC_F32, 8, 4, 512, 4, launch_panel<float, 8, 4, 512, 4>),
      panel_desc("skinny_bf16_p_v1_w8", TILEC_BF16, 8, 1, 256, 4, launch_panel<u16, 8, 1, 256, 4>),
      panel_desc("skinny_bf16_p_v4_w8", TILEC_BF16, 8, 4, 256, 4, launch_panel<u16, 8, 4, 256, 4>),
      panel_desc("skinny_f32_p_v1_w4", TILEC_F32, 4, 1, 512, 8, launch_panel<float, 4, 1, 512, 8>),
      panel_desc("skinny_bf16_p_v1_w4", TILEC_BF16, 4, 1, 256, 8, launch_panel<u16, 4, 1, 256, 8>),
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace tilec
