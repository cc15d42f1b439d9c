// Direct-operand MFMA kernel (fp32): out[M,N] = x1[M,K] · x2[K,N] for outputs
// too small to fill MI355X with LDS-staged tiles — the GEMV regime (M <= 16,
// x2 streamed from HBM once) and small-output GEMMs such as 513 x 3001 x 127
// or 512 x 4096 x 64, where a few dozen output tiles must share 256 CUs by
// splitting K.
//
// Replaces, for these shapes, the reference's 64x64 tile kernel
// (`_matmul_tiled`, tilec/ext.py:13-24: one program per output tile, a
// masked BK-step K loop, `acc += dot`) and its legacy split-K dot product
// (README.md:57,73; config space tilec/ext.py:29-51).  Same result up to
// fp32 summation order: masked loads read zeros past every edge.
//
// What runs, MI355X-first:
//   * No LDS staging.  With K split this finely nothing is reused across the
//     waves of a workgroup, so every wave loads its MFMA operands straight
//     from memory into registers: a workgroup of W waves owns one BM x BN
//     output tile (BM = 16 TI, BN = 64 TJ) and one K chunk, and wave w takes
//     the chunk's 16-row steps w, w + W, ...  The waves meet once, at the
//     end, in LDS.
//   * v_mfma_f32_16x16x4f32 with the operands as they lie in memory.  Lane
//     l (i = l % 16, h = l / 16) of a step starting at row kr:
//       - x1 row-major: one 16-byte load of x1[m0 + 16 ti + i][kr + 4h ..
//         + 3]; its element t is the A operand of k-step t (k = kr + 4h + t);
//       - x1 column-major: four 4-byte loads of the same elements;
//       - x2 row-major: per k-step t one 16-byte load of row kr + 4h + t,
//         columns n0 + 64 tj + 4i .. + 3; its element e is the B operand of
//         the MFMA for columns n0 + 64 tj + 4j + e (j = MFMA column);
//       - x2 column-major: per e one 16-byte load of column n0 + 64 tj + 4i
//         + e, rows kr + 4h .. + 3 (element t for k-step t).
//     A step is 16 TI TJ MFMAs on TI + 4 TJ (row-major x1) 16-byte loads.
//     Accumulator register r of MFMA (ti, tj, e) holds out[m0 + 16 ti + 4h
//     + r][n0 + 64 tj + 4i + e]: for fixed r the four e are four adjacent
//     columns, so results leave as 16-byte stores.
//   * A wave issues the loads of up to BT steps at once and starts its
//     MFMAs as they arrive (in issue order).  The host sizes K chunks so
//     that at the splits the tuner picks a wave's whole chunk is one such
//     batch: latency is paid once, with every load in flight.
//   * Edges by address: rows past the chunk or M and columns past N load
//     zeros through buffer resources that end at the matrix's last element;
//     a 16-byte group along K that straddles the chunk's end is cleared
//     element-wise.  Groups along M or N that straddle an edge need no
//     clearing: their extra elements only reach outputs that are never
//     stored.
//   * Split K: the workgroup's partial goes through the deterministic
//     count-and-combine protocol of the tile kernels (splitk_combine): the
//     last workgroup of a tile adds the partials in split order.
//   * Grid: tiles fastest, K chunks slowest, so the workgroups in flight read
//     the same rows of a streamed x2 side by side.
#include <algorithm>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

// The 64 x 64 fp32 tile GEMM, unsplit (gemm_f32.hip).
hipError_t launch_gemm_f32_unsplit(const MatmulArgs& a);

namespace {

constexpr int kStep = 16;  // rows of K per wave step: four 16x16x4 k-steps

// Four floats at a 4-byte aligned address (one dwordx4 access on CDNA).
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// Bytes from a resource's base to the end of a matrix whose last row is
// rows_left - 1 rows below it (row stride ld) and cols_left long from the
// base column; clamped to the resource's 31-bit range.
__device__ __forceinline__ uint32_t span_bytes(int64_t rows_left, int64_t ld, int64_t cols_left) {
  if (rows_left <= 0 || cols_left <= 0) return 0u;
  const int64_t b = 4 * ((rows_left - 1) * ld + cols_left);
  return b > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)b;
}

// One batch of BT steps of a wave's operands (one register set).
template <int TI, int TJ, int BT>
struct Frag {
  f32x4 a[BT][TI];     // element t: A operand of k-step t
  f32x4 b[BT][TJ][4];  // x2 row-major: [t] element e; column-major: [e] element t
};

// CA: x1 column-major (x1[m + k * ldx1]); CB: x2 column-major (x2[k + n *
// ldx2]); NT2: x2 is streamed once (non-temporal loads); BT: steps per
// batch of loads; PIPE: two register sets, the next batch's loads issued
// before the current batch's MFMAs.
template <int TI, int TJ, int W, int BT, bool CA, bool CB, bool NT2, bool PIPE>
__global__ __launch_bounds__(W * 64) void direct_kernel(const float* __restrict__ x1, const float* __restrict__ x2,
                                                        float* __restrict__ out, int M, int N, int K, int64_t ldx1,
                                                        int64_t ldx2, int64_t ldo, int kc, int tiles_n,
                                                        unsigned* __restrict__ counters, float* __restrict__ part) {
  constexpr int BM = 16 * TI, BN = 64 * TJ;
  constexpr int ITEMS = 4 * TI * TJ;       // 16-byte results per lane of a wave tile
  constexpr int NV = (ITEMS + W - 1) / W;  // per thread after the waves meet
  constexpr int NT = W * 64;
  constexpr int CP2 = NT2 ? 2 : 0;
  extern __shared__ __align__(16) f32x4 red[];  // [W][ITEMS][64], then the split-K flag

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, h = lane >> 4;
  const int tile = blockIdx.x, split = blockIdx.y, S = gridDim.y, tiles = gridDim.x;
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * kc;
  const int nrows = max(0, min(K - kbeg, kc));

  // One resource per operand, based at this tile and chunk (the host keeps
  // every offset below 2^31).
  const BufRsrc r1 = CA ? make_rsrc_uniform(x1 + (int64_t)kbeg * ldx1 + m0, span_bytes(K - kbeg, ldx1, M - m0))
                        : make_rsrc_uniform(x1 + (int64_t)m0 * ldx1 + kbeg, span_bytes(M - m0, ldx1, K - kbeg));
  const BufRsrc r2 = CB ? make_rsrc_uniform(x2 + (int64_t)n0 * ldx2 + kbeg, span_bytes(N - n0, ldx2, K - kbeg))
                        : make_rsrc_uniform(x2 + (int64_t)kbeg * ldx2 + n0, span_bytes(K - kbeg, ldx2, N - n0));
  bool mok[TI], nok[TJ][4];
#pragma unroll
  for (int ti = 0; ti < TI; ++ti) mok[ti] = m0 + 16 * ti + li < M;
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
    for (int e = 0; e < 4; ++e) nok[tj][e] = n0 + 64 * tj + 4 * li + (CB ? e : 0) < N;

  const int nsteps = (nrows + kStep - 1) / kStep;
  const int mine = nsteps > wave ? (nsteps - wave + W - 1) / W : 0;
  const int nb = (mine + BT - 1) / BT;

  auto load = [&](Frag<TI, TJ, BT>& f, int b) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < BT; ++q) {
      const int kr = ((b * BT + q) * W + wave) * kStep + 4 * h;  // this lane's first row of the step
      const int valid = nrows - kr;                                    // rows of its group in the chunk
#pragma unroll
      for (int ti = 0; ti < TI; ++ti) {
        const uint32_t m = 16 * ti + li;
        if constexpr (CA) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            f.a[q][ti][t] = load_f32(r1, (mok[ti] & (t < valid)) ? 4u * ((uint32_t)(kr + t) * (uint32_t)ldx1 + m) : kOob);
        } else {
          f.a[q][ti] = load_f32x4(r1, (mok[ti] & (valid > 0)) ? 4u * (m * (uint32_t)ldx1 + (uint32_t)kr) : kOob);
        }
      }
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          if constexpr (CB) {
            const uint32_t n = 64 * tj + 4 * li + x;
            f.b[q][tj][x] = load_f32x4(r2, (nok[tj][x] & (valid > 0)) ? 4u * (n * (uint32_t)ldx2 + (uint32_t)kr) : kOob);
          } else {
            const uint32_t n = 64 * tj + 4 * li;
            f.b[q][tj][x] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           r2, (int)((nok[tj][0] & (x < valid)) ? 4u * ((uint32_t)(kr + x) * (uint32_t)ldx2 + n) : kOob),
                           0, CP2));
          }
        }
    }
  };

  f32x4 acc[TI][TJ][4];
#pragma unroll
  for (int ti = 0; ti < TI; ++ti)
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[ti][tj][e] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A 16-byte group along K that straddles the chunk's end is cleared here,
  // at its use, so that the clearing does not make the next batch's loads
  // wait for this one.
  auto compute = [&](const Frag<TI, TJ, BT>& f, int b) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < BT; ++q) {
      const int valid = nrows - (((b * BT + q) * W + wave) * kStep + 4 * h);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int ti = 0; ti < TI; ++ti) {
          const float a = CA || t == 0 ? f.a[q][ti][t] : (t < valid ? f.a[q][ti][t] : 0.f);
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float bv = CB ? (t == 0 || t < valid ? f.b[q][tj][e][t] : 0.f) : f.b[q][tj][t][e];
              acc[ti][tj][e] = mfma16x16x4(a, bv, acc[ti][tj][e]);
            }
        }
    }
  };

  if constexpr (PIPE) {
    // Batch b + 1 is in flight while batch b is multiplied; a load past the
    // wave's last batch is masked (valid <= 0) and touches no memory.
    Frag<TI, TJ, BT> fa, fb;
    if (nb > 0) load(fa, 0);
    int b = 0;
    for (; b + 1 < nb; b += 2) {
      load(fb, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(fa, b);
      __builtin_amdgcn_sched_barrier(0);
      load(fa, b + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(fb, b + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (b < nb) compute(fa, b);
  } else {
    for (int b = 0; b < nb; ++b) {
      Frag<TI, TJ, BT> f;
      load(f, b);
      // Keep every load of the batch ahead of the first MFMA (the scheduler
      // would otherwise interleave them to save registers, and wait for each).
      __builtin_amdgcn_sched_barrier(0);
      compute(f, b);
    }
  }

  // The waves meet in LDS; thread (w, l) then owns results w, w + W, ... of
  // lane l, summed in wave order.
#pragma unroll
  for (int ti = 0; ti < TI; ++ti)
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[(wave * ITEMS + (ti * TJ + tj) * 4 + r) * 64 + lane] =
            f32x4{acc[ti][tj][0][r], acc[ti][tj][1][r], acc[ti][tj][2][r], acc[ti][tj][3][r]};
  __syncthreads();
  f32x4 v[NV];
  bool live[NV];
  int row[NV], col[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int it = wave + W * j;
    const int r = it & 3, tt = it >> 2;
    row[j] = m0 + 16 * (tt / TJ) + 4 * h + r;
    col[j] = n0 + 64 * (tt % TJ) + 4 * li;
    live[j] = (it < ITEMS) & (row[j] < M) & (col[j] < N);
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
    if (it < ITEMS) {
#pragma unroll
      for (int w = 0; w < W; ++w) s += red[(w * ITEMS + it) * 64 + lane];
    }
    v[j] = s;
  }
  if (S > 1 && !splitk_combine<NT, NV>(v, live, split, S, tile, tiles, part, counters,
                                       reinterpret_cast<int*>(red + W * ITEMS * 64)))
    return;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (!live[j]) continue;
    float* p = out + (int64_t)row[j] * ldo + col[j];
    if (col[j] + 4 <= N) {
      *reinterpret_cast<f32x4_a4*>(p) = v[j];
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (col[j] + c < N) p[c] = v[j][c];
    }
  }
}

struct DirectGeom {
  int64_t tiles_m, tiles_n, splits, kc;
};

// K chunk per split: a multiple of kStep rows, recomputed so no split is
// empty.
DirectGeom direct_geom(int64_t M, int64_t N, int64_t K, int split_k, int bm, int bn) {
  DirectGeom g;
  g.tiles_m = cdiv(M, bm);
  g.tiles_n = cdiv(N, bn);
  if (K <= 0) {
    g.splits = 1;
    g.kc = 0;
    return g;
  }
  const int64_t s = split_k < 1 ? 1 : split_k;
  g.kc = cdiv(cdiv(K, s), kStep) * kStep;
  g.splits = cdiv(K, g.kc);
  return g;
}

// Whether every operand offset from the tile's resources stays below 2^31:
// (rows spanned - 1) * stride + one row's span, in bytes.
bool direct_offsets_fit(const MatmulArgs& a, const DirectGeom& g, int bm, int bn) {
  constexpr int64_t lim = (int64_t(1) << 31) - 64;
  const int64_t kc = std::max<int64_t>(g.kc, 1);
  const int64_t o1 = (a.layout & TILEC_X1_COL_MAJOR) ? (kc - 1) * a.ldx1 + bm : (int64_t)(bm - 1) * a.ldx1 + kc;
  const int64_t o2 = (a.layout & TILEC_X2_COL_MAJOR) ? (int64_t)(bn - 1) * a.ldx2 + kc : (kc - 1) * a.ldx2 + bn;
  return 4 * o1 < lim && 4 * o2 < lim;
}

template <int TI, int TJ, int W>
constexpr size_t direct_lds_bytes() {
  return (size_t)W * 4 * TI * TJ * 64 * sizeof(f32x4) + 16;
}

template <int TI, int TJ, int W, int BT, bool NT2, bool PIPE, bool CA, bool CB>
hipError_t launch_direct_layout(const MatmulArgs& a, const DirectGeom& g) {
  auto k = direct_kernel<TI, TJ, W, BT, CA, CB, NT2, PIPE>;
  constexpr size_t lds = direct_lds_bytes<TI, TJ, W>();
  static std::atomic<uint64_t> lds_devices{0};
  const hipError_t e = raise_lds_limit((const void*)k, lds, lds_devices);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)(g.tiles_m * g.tiles_n), (unsigned)g.splits), dim3(W * 64), lds, a.stream,
                     static_cast<const float*>(a.x1), static_cast<const float*>(a.x2), a.out, (int)a.M, (int)a.N,
                     (int)a.K, a.ldx1, a.ldx2, a.ldo, (int)g.kc, (int)g.tiles_n,
                     g.splits > 1 ? a.counters : nullptr, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr);
  return hipGetLastError();
}

template <int TI, int TJ, int W, int BT, bool NT2, bool PIPE = false>
hipError_t launch_direct(const MatmulArgs& a) {
  const DirectGeom g = direct_geom(a.M, a.N, a.K, a.split_k, 16 * TI, 64 * TJ);
  if (g.tiles_m * g.tiles_n == 0) return hipSuccess;
  // Strides too large for 32-bit offsets over a chunk: the unsplit 64 x 64
  // tile GEMM, which addresses such operands itself and needs no scratch.
  if (!direct_offsets_fit(a, g, 16 * TI, 64 * TJ)) return launch_gemm_f32_unsplit(a);
  switch (a.layout & 3) {
    case 0: return launch_direct_layout<TI, TJ, W, BT, NT2, PIPE, false, false>(a, g);
    case TILEC_X1_COL_MAJOR: return launch_direct_layout<TI, TJ, W, BT, NT2, PIPE, true, false>(a, g);
    case TILEC_X2_COL_MAJOR: return launch_direct_layout<TI, TJ, W, BT, NT2, PIPE, false, true>(a, g);
    default: return launch_direct_layout<TI, TJ, W, BT, NT2, PIPE, true, true>(a, g);
  }
}

// Partials per split: NV 16-byte values per thread of each tile (the layout
// of splitk_combine).
size_t direct_workspace_bytes(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  const DirectGeom g = direct_geom(M, N, K, split_k, d.bm, d.bn);
  if (g.splits <= 1) return 0;
  const int64_t items = 4 * (d.bm / 16) * (d.bn / 64);
  const int64_t nv = cdiv(items, d.waves);
  return (size_t)(g.splits * g.tiles_m * g.tiles_n * nv * d.waves * 64 * 16);
}
size_t direct_counter_bytes(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  const DirectGeom g = direct_geom(M, N, K, split_k, d.bm, d.bn);
  if (g.splits <= 1) return 0;
  return (size_t)(g.tiles_m * g.tiles_n * kSplitCounterStride * sizeof(unsigned));
}

VariantDesc direct_desc(const char* name, int ti, int tj, int waves, int bt, bool pipe,
                        hipError_t (*launch)(const MatmulArgs&)) {
  VariantDesc d{name, TILEC_FAMILY_DIRECT, TILEC_F32, 16 * ti, 64 * tj, kStep, waves, 0, pipe ? 2 * bt : bt, launch};
  d.workspace_bytes = direct_workspace_bytes;
  d.counter_bytes = direct_counter_bytes;
  d.wgs_per_cu = waves >= 8 ? 1 : 2;
  return d;
}

}  // namespace

// Splits the kernel runs for a requested split_k.
int64_t direct_effective_splits(int64_t K, int split_k) { return direct_geom(1, 1, K, split_k, 16, 64).splits; }

// Variant table of this family (appended after the earlier tables, so their
// variant ids are unchanged).  BM x BN = the output tile, BK = the 16-row
// step, unroll = steps of loads a wave has in flight (BT, or 2 BT with two
// register sets).  The 16 x 128 tile with 8 waves streams x2 once
// (non-temporal loads, one workgroup per CU); the others are for
// small-output GEMMs.
const VariantDesc* direct_variants(int* count) {
  static const VariantDesc t[] = {
      direct_desc("direct_f32_16x128_w8", 1, 2, 8, 4, false, launch_direct<1, 2, 8, 4, true>),
      direct_desc("direct_f32_16x64_w4", 1, 1, 4, 8, false, launch_direct<1, 1, 4, 8, false>),
      direct_desc("direct_f32_32x64_w4", 2, 1, 4, 6, false, launch_direct<2, 1, 4, 6, false>),
      direct_desc("direct_f32_32x128_w4", 2, 2, 4, 4, false, launch_direct<2, 2, 4, 4, false>),
      direct_desc("direct_f32_64x64_w4", 4, 1, 4, 4, false, launch_direct<4, 1, 4, 4, false>),
      // 8 waves (two per SIMD) on the small tiles: one wave's loads wait
      // while the other's MFMAs run
      direct_desc("direct_f32_16x64_w8", 1, 1, 8, 4, false, launch_direct<1, 1, 8, 4, false>),
      direct_desc("direct_f32_32x64_w8", 2, 1, 8, 4, false, launch_direct<2, 1, 8, 4, false>),
      // Two register sets: a wave's next batch loads while its current one
      // is multiplied, so K chunks of several batches (fewer splits, a
      // shorter combine) do not pay the memory latency per batch
      direct_desc("direct_f32_16x64_w8_db", 1, 1, 8, 4, true, launch_direct<1, 1, 8, 4, false, true>),
      direct_desc("direct_f32_16x64_w4_db", 1, 1, 4, 3, true, launch_direct<1, 1, 4, 3, false, true>),
      direct_desc("direct_f32_32x64_w4_db", 2, 1, 4, 2, true, launch_direct<2, 1, 4, 2, false, true>),
      direct_desc("direct_f32_32x64_w8_db", 2, 1, 8, 3, true, launch_direct<2, 1, 8, 3, false, true>),
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace tilec
