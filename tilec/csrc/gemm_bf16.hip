// LDS-staged bf16 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x16_bf16):
//   C[M,N] (fp32) = A[M,K] (bf16) · B[K,N] (bf16), fp32 accumulate; A and B
//   each row- or column-major, read in place.
//
// Same tile semantics as the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24) — zero accumulator, masked K steps with `other=0.0`,
// masked store — on bf16 inputs, which the reference (fp32 only,
// src/lib.rs:19) does not take.  Layout in LDS:
//   As[m][k]  k-contiguous rows, padded by 16 bytes so the 16-byte operand
//             reads of 16 consecutive rows fall in distinct banks;
//   Bs[n][k]  B transposed while it is written to LDS, so the B operand of
//             every MFMA is also one 16-byte LDS read per lane.
// A and B tiles are double-buffered with one barrier per K step and the next
// tile's global loads issued before the current tile's MFMAs.
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;
typedef u16 u16x8 __attribute__((ext_vector_type(8)));

template <int BM, int BN, int BK, int WM, int WN>
struct GemmBf16 {
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int LDS_K = BK + 8;  // row length in elements (16-byte pad)
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BK % 16 == 0, "BK");
  static constexpr size_t kLds = sizeof(u16) * 2 * LDS_K * (BM + BN);
};

template <bool VEC>
__device__ __forceinline__ u16x8 ld8(const u16* __restrict__ p, bool ok_all, int valid) {
  if (VEC) {
    const u16x8 v = *reinterpret_cast<const u16x8*>(p);
    const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    return ok_all ? v : z;
  } else {
    u16x8 v;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u16 x = p[c < valid ? c : 0];
      v[c] = c < valid ? x : (u16)0;
    }
    return v;
  }
}

// One operand's tile per K step: R rows of its outer dimension (M for x1, N
// for x2) by BK of K, global -> registers -> LDS.  KC: element (r, k) at
// X[r * ld + k] (row-major x1, column-major x2), moved as 8 consecutive k;
// otherwise at X[k * ld + r], moved as 8 consecutive r.  In LDS the tile is
// S[r][k] with rows of BK + 8 elements: a KC group is one 16-byte store, the
// other kind is transposed by 8 element stores.
template <int R, int BK, int NT, bool KC, bool VEC>
struct OperandBf16 {
  static constexpr int Q = R * BK / 8 / NT;
  static constexpr int LDS_K = BK + 8;
  static_assert(R * BK % (8 * NT) == 0, "tile loads must divide evenly");
  typedef u16x8 Regs[Q];

  // Tile row and tile k of the first element of thread tid's group p.
  __device__ __forceinline__ static void coord(int tid, int p, int& r, int& k) {
    const int e = tid + p * NT;
    if constexpr (KC) {
      r = e / (BK / 8);
      k = 8 * (e % (BK / 8));
    } else {
      k = e / (R / 8);
      r = 8 * (e % (R / 8));
    }
  }

  // K step kt of the tile at outer row r0 (of Rtot).  MASK: clamp + select
  // at every edge; otherwise whole 16-byte groups.
  __device__ __forceinline__ static void load(Regs& v, const u16* __restrict__ X, int64_t ld, int r0, int Rtot, int K,
                                              int tid, int kt, bool mask) {
    const int k0 = kt * BK;
#pragma unroll
    for (int p = 0; p < Q; ++p) {
      int tr, tk;
      coord(tid, p, tr, tk);
      const int gr = r0 + tr, gk = k0 + tk;
      const int64_t at = KC ? (int64_t)gr * ld + gk : (int64_t)gk * ld + gr;
      if (!mask) {
        v[p] = ld8<VEC>(X + at, true, 8);
      } else {
        const int valid = KC ? (gr < Rtot ? max(0, min(8, K - gk)) : 0) : (gk < K ? max(0, min(8, Rtot - gr)) : 0);
        v[p] = ld8<VEC>(X + (valid > 0 ? at : 0), valid == 8, valid);
      }
    }
  }

  __device__ __forceinline__ static void store(const Regs& v, u16* __restrict__ S, int tid) {
#pragma unroll
    for (int p = 0; p < Q; ++p) {
      int tr, tk;
      coord(tid, p, tr, tk);
      if constexpr (KC) {
        *reinterpret_cast<u16x8*>(S + tr * LDS_K + tk) = v[p];
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) S[(tr + c) * LDS_K + tk] = v[p][c];
      }
    }
  }
};

// CA: x1 column-major (element (m, k) at A[m + k * lda]); CB: x2 column-major
// (element (k, n) at B[k + n * ldb]).
template <int BM, int BN, int BK, int WM, int WN, bool VEC, bool CA, bool CB>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_kernel(
    const u16* __restrict__ A, const u16* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int xcds, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = GemmBf16<BM, BN, BK, WM, WN>;
  using OpA = OperandBf16<BM, BK, P::NT, !CA, VEC>;
  using OpB = OperandBf16<BN, BK, P::NT, CB, VEC>;
  extern __shared__ __align__(16) u16 lds_u16[];
  __shared__ int last_flag;
  u16* As = lds_u16;                          // [2][BM][LDS_K]
  u16* Bs = lds_u16 + 2 * BM * P::LDS_K;      // [2][BN][LDS_K]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, xcds, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);
  // K steps [kt0, kt1) of this workgroup (grid y = K splits).
  const int split = blockIdx.y, S = gridDim.y;
  const int kt0 = split * split_steps;
  const int kt1 = min((K + BK - 1) / BK, kt0 + split_steps);
  const int nk_full = K / BK;

  typename OpA::Regs ra;
  typename OpB::Regs rb;
  auto gload = [&](int kt, bool mask) {
    OpA::load(ra, A, lda, m0, M, K, tid, kt, mask);
    OpB::load(rb, B, ldb, n0, N, K, tid, kt, mask);
  };
  auto sstore = [&](int buf) {
    OpA::store(ra, As + buf * BM * P::LDS_K, tid);
    OpB::store(rb, Bs + buf * BN * P::LDS_K, tid);
  };

  f32x16 acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (kt0 < kt1) {
    gload(kt0, !(interior && kt0 < nk_full));
    sstore(0);
    __syncthreads();
  }

  const int arow = wm * P::WTM + (lane & 31);
  const int bcol = wn * P::WTN + (lane & 31);
  const int khalf = lane >> 5;

  for (int kt = kt0; kt < kt1; ++kt) {
    const int buf = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) gload(kt + 1, !(interior && kt + 1 < nk_full));
    const u16* as = As + buf * BM * P::LDS_K;
    const u16* bs = Bs + buf * BN * P::LDS_K;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int k = 16 * ks + 8 * khalf;
      bf16x8 a[P::TM], b[P::TN];
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(as + (arow + 32 * i) * P::LDS_K + k);
#pragma unroll
      for (int j = 0; j < P::TN; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(bs + (bcol + 32 * j) * P::LDS_K + k);
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x16bf16(a[i], b[j], acc[i][j]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
  }

  const int row_base = m0 + wm * P::WTM + 4 * khalf;
  const int col_base = n0 + bcol;
  if (S > 1 && !splitk_tile<P::TM, P::TN, P::NT>(acc, split, S, blockIdx.x, gridDim.x, ws, counters, &last_flag,
                                                  row_base, col_base, M, N))
    return;
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j) {
      const int gn = col_base + 32 * j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = row_base + 32 * i + 8 * (r >> 2) + (r & 3);
        if (interior || (gm < M && gn < N)) C[(int64_t)gm * ldc + gn] = acc[i][j][r];
      }
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool VEC, bool CA, bool CB>
hipError_t launch_one(const MatmulArgs& a, dim3 grid) {
  using P = GemmBf16<BM, BN, BK, WM, WN>;
  auto k = gemm_bf16_kernel<BM, BN, BK, WM, WN, VEC, CA, CB>;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * 16 > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  grid.y = (unsigned)g.splits;
  const size_t lds = P::kLds;
  static std::atomic<uint64_t> lds_devices{0};
  const hipError_t e = raise_lds_limit((const void*)k, lds, lds_devices);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, grid, dim3(WM * WN * 64), lds, a.stream, static_cast<const u16*>(a.x1),
                     static_cast<const u16*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo,
                     8, device_xcds(), (int)g.steps, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr, g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

}  // namespace

template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB, int MF>
hipError_t launch_gemm_bf16_lds(const MatmulArgs& a);  // gemm_bf16_lds.hip

namespace {

// Aligned operands (16-byte base, K, N, lda, ldb multiples of 8) whose tile
// offsets fit 32 bits run the LDS-DMA kernel of gemm_bf16_lds.hip with a
// ring of NBUF stage buffers of BK; everything else runs the generic kernel
// above with the same output tile (NBUF == 0: generic kernel only).  Both
// use the variant's WM x WN waves, so a K split is possible in one exactly
// when it is in the other.
template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB, int MF>
hipError_t launch_layout(const MatmulArgs& a) {
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  // 16-byte groups of 8 elements never straddle an edge: each operand's
  // contiguous extent (K, or M / N for the r-contiguous layouts) and both
  // strides are multiples of 8, and the bases are 16-byte aligned.
  const int64_t a_run = CA ? a.M : a.K, b_run = CB ? a.K : a.N;
  const bool vec = (a_run % 8 == 0) && (b_run % 8 == 0) && (a.ldx1 % 8 == 0) && (a.ldx2 % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.x1) % 16 == 0) && (reinterpret_cast<uintptr_t>(a.x2) % 16 == 0);
  if constexpr (NBUF > 0) {
    // The LDS-DMA kernel's byte offsets within one K step: (strided rows of
    // the tile) * ld * 2 < 2^31 — BM or BN rows for a k-contiguous operand,
    // BK rows for an r-contiguous one.
    const int64_t a_rows = CA ? BK : BM, b_rows = CB ? BN : BK;
    if (vec && a_rows * a.ldx1 * 2 < (int64_t(1) << 31) - 4096 && b_rows * a.ldx2 * 2 < (int64_t(1) << 31) - 4096)
      return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, CA, CB, MF>(a);
  }
  dim3 grid((unsigned)tiles);
  return vec ? launch_one<BM, BN, 64, WM, WN, true, CA, CB>(a, grid)
             : launch_one<BM, BN, 64, WM, WN, false, CA, CB>(a, grid);
}

// Aligned operands (16-byte base, contiguous extents and strides multiples
// of 8) whose tile offsets fit 32 bits run the LDS-DMA kernel of
// gemm_bf16_lds.hip with a ring of NBUF stage buffers of BK; everything else
// runs the generic kernel above with the same output tile (NBUF == 0: generic
// kernel only).  Both use the variant's WM x WN waves, so a K split is
// possible in one exactly when it is in the other.
template <int BM, int BN, int BK, int NBUF, int WM = 2, int WN = 2, int MF = 32>
hipError_t launch_gemm_bf16(const MatmulArgs& a) {
  switch (a.layout & 3) {
    case 0: return launch_layout<BM, BN, BK, NBUF, WM, WN, false, false, MF>(a);
    case TILEC_X1_COL_MAJOR: return launch_layout<BM, BN, BK, NBUF, WM, WN, true, false, MF>(a);
    case TILEC_X2_COL_MAJOR: return launch_layout<BM, BN, BK, NBUF, WM, WN, false, true, MF>(a);
    default: return launch_layout<BM, BN, BK, NBUF, WM, WN, true, true, MF>(a);
  }
}

// out[c][r] = in[r][c] for r < R, c < C: `in` row-major with row stride ld,
// `out` row-major [C][R] (row stride R).  A 64 x 64 tile per workgroup goes
// through LDS: 16-byte loads of input rows, 16-byte stores of output rows.
// LDS rows are 128 bytes (8 chunks of 8 elements) with chunk c of row r
// stored at c ^ ((r >> 3) & 7): the 8 rows one column read touches sit 8
// apart, so the swizzle puts them in 8 different chunks and a wave's 2-byte
// column reads spread over 32 banks.  The caller guarantees C, R and ld are
// multiples of 8 and both pointers 16-byte aligned, so 16-byte groups never
// straddle an edge; the grid covers cdiv(C, 64) x cdiv(R, 64) tiles.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const u16* __restrict__ in, u16* __restrict__ out, int R,
                                                             int C, int64_t ld) {
  __shared__ __align__(16) u16 tile[64 * 64];
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  auto at = [](int row, int col) { return row * 64 + 8 * ((col >> 3) ^ ((row >> 3) & 7)) + (col & 7); };
  u16x8 v[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int id = tid + 256 * i, row = id >> 3, ch = id & 7;  // 64 rows x 8 chunks
    v[i] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (r0 + row < R && c0 + 8 * ch < C) v[i] = *reinterpret_cast<const u16x8*>(in + (int64_t)(r0 + row) * ld + c0 + 8 * ch);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int id = tid + 256 * i, row = id >> 3, ch = id & 7;
    *reinterpret_cast<u16x8*>(&tile[at(row, 8 * ch)]) = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int id = tid + 256 * i, ch = id & 7, orow = id >> 3;  // output row = input column c0 + orow
    u16x8 w;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = tile[at(8 * ch + e, orow)];
    if (c0 + orow < C && r0 + 8 * ch < R) *reinterpret_cast<u16x8*>(out + (int64_t)(c0 + orow) * R + r0 + 8 * ch) = w;
  }
}

hipError_t transpose_bf16(const void* in, void* out, int64_t R, int64_t C, int64_t ld, hipStream_t stream) {
  const dim3 grid((unsigned)cdiv(C, 64), (unsigned)cdiv(R, 64));
  hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, stream, static_cast<const u16*>(in),
                     static_cast<u16*>(out), (int)R, (int)C, ld);
  return hipGetLastError();
}

// A prep variant: make both operands k-contiguous (x1 row-major, x2
// column-major) by transposing whichever is not into the workspace, then run
// the LDS-DMA kernel on them.  That layout needs no transposing LDS reads and
// walks each operand along its rows; on 8192^3 it runs about 18% faster than
// row-major x2.  Shapes the aligned kernel cannot take, and operands already
// k-contiguous, run the plain variant.
template <int BM, int BN, int BK, int NBUF, int WM, int WN, int MF = 32>
hipError_t launch_gemm_bf16_kc(const MatmulArgs& a) {
  const bool ca = a.layout & TILEC_X1_COL_MAJOR, cb = a.layout & TILEC_X2_COL_MAJOR;
  auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool ok = a.M % 8 == 0 && a.N % 8 == 0 && a.K % 8 == 0 && a.ldx1 % 8 == 0 && a.ldx2 % 8 == 0 &&
                  aligned(a.x1) && aligned(a.x2) && aligned(a.workspace) && a.K > 0 &&
                  (int64_t)BM * a.K * 2 < (int64_t(1) << 31) - 4096 && (int64_t)BN * a.K * 2 < (int64_t(1) << 31) - 4096 &&
                  a.M * a.K < (int64_t(1) << 31) && a.K * a.N < (int64_t(1) << 31);
  if (!ok || (!ca && cb)) return launch_gemm_bf16<BM, BN, BK, NBUF, WM, WN, MF>(a);
  MatmulArgs b = a;
  char* ws = static_cast<char*>(a.workspace);
  if (ca) {  // x1 is [K][M] in memory: its transpose is x1 row-major [M][K]
    const hipError_t e = transpose_bf16(a.x1, ws, a.K, a.M, a.ldx1, a.stream);
    if (e != hipSuccess) return e;
    b.x1 = ws;
    b.ldx1 = a.K;
  }
  if (!cb) {  // x2 is [K][N] in memory: its transpose is x2 column-major ([N][K])
    char* wb = ws + prep_offset_b(a.M, a.K);
    const hipError_t e = transpose_bf16(a.x2, wb, a.K, a.N, a.ldx2, a.stream);
    if (e != hipSuccess) return e;
    b.x2 = wb;
    b.ldx2 = a.K;
  }
  b.layout = TILEC_X2_COL_MAJOR;
  b.split_k = 1;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  b.counters = nullptr;
  return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, false, true, MF>(b);
}

// ---------------------------------------------------------------------------
// Pad variants: an operand whose rows are not whole 16-byte groups (its
// contiguous extent or row stride not a multiple of 8 elements, e.g. an odd
// K) cannot take the LDS-DMA kernel's 16-byte copies, and the plain variants
// run the generic kernel for it (2-3x slower on MI355X).  These variants
// first copy the operands into the workspace in the caller's layout, the
// contiguous extent and row stride rounded up to 8 elements and K up to the
// K step, zero-filled (both operands when K is not a whole number of K
// steps, else only those whose rows are not whole 16-byte groups), then run
// the LDS-DMA kernel.  Zeros add
// nothing to the product; C is written as the caller's M x N (column chunks
// past N may read padding, never store it).  Workspace: [x1 padded][x2
// padded][split-K partials], each 256-byte aligned.  The copies are
// common.h's pad_copy.
// ---------------------------------------------------------------------------

// Padded extents: K up to the K step, the contiguous extent of a
// column-major x1 (M) or a row-major x2 (N) up to 8.  Sized for either
// layout, since the size queries do not see it.
struct PadGeomBf16 {
  int64_t kp, m8, n8;
  size_t x1_bytes, x2_bytes;  // 256-byte aligned
};
inline PadGeomBf16 pad_geom_bf16(int64_t M, int64_t N, int64_t K, int64_t bk) {
  PadGeomBf16 g;
  g.kp = cdiv(K, bk) * bk;
  g.m8 = cdiv(M, 8) * 8;
  g.n8 = cdiv(N, 8) * 8;
  g.x1_bytes = (size_t)cdiv(g.m8 * g.kp * 2, 256) * 256;
  g.x2_bytes = (size_t)cdiv(g.n8 * g.kp * 2, 256) * 256;
  return g;
}

size_t pad_workspace_bytes_bf16(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  if (M == 0 || N == 0 || K == 0) return 0;
  const PadGeomBf16 p = pad_geom_bf16(M, N, K, d.bk);
  const SplitGeom g = gemm_split_geom(p.kp, d.bk, split_k);
  const size_t partials = g.splits > 1 ? (size_t)g.splits * cdiv(M, d.bm) * cdiv(N, d.bn) * d.bm * d.bn * 4 : 0;
  return p.x1_bytes + p.x2_bytes + partials;
}
size_t pad_counter_bytes_bf16(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  if (M == 0 || N == 0 || K == 0 || gemm_split_geom(K, d.bk, split_k).splits <= 1) return 0;
  return (size_t)cdiv(M, d.bm) * cdiv(N, d.bn) * kSplitCounterStride * sizeof(unsigned);
}

template <int BM, int BN, int BK, int NBUF, int WM, int WN, int MF>
hipError_t launch_gemm_bf16_pad(const MatmulArgs& a) {
  if (a.M == 0 || a.N == 0 || a.K == 0) return launch_gemm_bf16<BM, BN, BK, NBUF, WM, WN, MF>(a);
  const bool ca = a.layout & TILEC_X1_COL_MAJOR, cb = a.layout & TILEC_X2_COL_MAJOR;
  const PadGeomBf16 p = pad_geom_bf16(a.M, a.N, a.K, BK);
  // Stored (rows x cols) of each operand, before and after padding.
  const int64_t r1 = ca ? a.K : a.M, c1 = ca ? a.M : a.K, r1p = ca ? p.kp : a.M, c1p = ca ? p.m8 : p.kp;
  const int64_t r2 = cb ? a.N : a.K, c2 = cb ? a.K : a.N, r2p = cb ? a.N : p.kp, c2p = cb ? p.kp : p.n8;
  // The LDS-DMA kernel's byte offsets within one K step (strided rows of a
  // tile times the row stride, as launch_layout checks them) and the copy
  // kernel's 32-bit extents; beyond them the plain variant on the operands
  // as they are (its workspace use is only the split partials).
  constexpr int64_t lim = (int64_t(1) << 31) - 4096;
  if ((ca ? BK : BM) * c1p * 2 >= lim || (cb ? BN : BK) * c2p * 2 >= lim || std::max(r1p, c1p) >= lim ||
      std::max(r2p, c2p) >= lim || reinterpret_cast<uintptr_t>(a.workspace) % 16 != 0)
    return launch_gemm_bf16<BM, BN, BK, NBUF, WM, WN, MF>(a);
  // With K a whole number of K steps, an operand whose rows are already whole
  // 16-byte groups (extent, stride and base) is read in place; only the
  // other is copied.
  auto in_place = [&](const void* x, int64_t c, int64_t ld, int64_t rows_per_step) {
    return a.K % BK == 0 && c % 8 == 0 && ld % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           rows_per_step * ld * 2 < lim;
  };
  const bool keep1 = in_place(a.x1, c1, a.ldx1, ca ? BK : BM), keep2 = in_place(a.x2, c2, a.ldx2, cb ? BN : BK);
  char* ws = static_cast<char*>(a.workspace);
  u16* x1p = reinterpret_cast<u16*>(ws);
  u16* x2p = reinterpret_cast<u16*>(ws + p.x1_bytes);
  const hipError_t e = pad_copy<2>(a.x1, x1p, r1, c1, a.ldx1, keep1 ? 0 : r1p, c1p, a.x2, x2p, r2, c2, a.ldx2,
                                   keep2 ? 0 : r2p, c2p, a.stream);
  if (e != hipSuccess) return e;
  MatmulArgs b = a;
  b.x1 = keep1 ? a.x1 : x1p;
  b.x2 = keep2 ? a.x2 : x2p;
  b.K = p.kp;
  b.ldx1 = keep1 ? a.ldx1 : c1p;
  b.ldx2 = keep2 ? a.ldx2 : c2p;
  b.workspace = ws + p.x1_bytes + p.x2_bytes;
  b.workspace_bytes = a.workspace_bytes - p.x1_bytes - p.x2_bytes;
  switch (a.layout & 3) {
    case 0: return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, false, false, MF>(b);
    case TILEC_X1_COL_MAJOR: return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, true, false, MF>(b);
    case TILEC_X2_COL_MAJOR: return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, false, true, MF>(b);
    default: return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, true, true, MF>(b);
  }
}

}  // namespace

// Variant table for this family (its order is part of the variant numbering).
// BK is the K step of the LDS-DMA kernel and `unroll` its ring depth.
const VariantDesc* gemm_bf16_variants(int* count) {
  static const VariantDesc t[] = {
      {"gemm_bf16_256x256x32_r4", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 32, 4, 0, 4,
       launch_gemm_bf16<256, 256, 32, 4>},
      {"gemm_bf16_256x256x64_r2", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 64, 8, 0, 2,
       launch_gemm_bf16<256, 256, 64, 2, 2, 4>},
      {"gemm_bf16_256x128x64_r3", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 64, 8, 0, 3,
       launch_gemm_bf16<256, 128, 64, 3, 4, 2>},
      {"gemm_bf16_256x128x32_r4", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 32, 4, 0, 4,
       launch_gemm_bf16<256, 128, 32, 4>},
      {"gemm_bf16_128x128x64_r4", TILEC_FAMILY_GEMM, TILEC_BF16, 128, 128, 64, 8, 0, 4,
       launch_gemm_bf16<128, 128, 64, 4, 2, 4>},
      {"gemm_bf16_64x64x64_w2x2", TILEC_FAMILY_GEMM, TILEC_BF16, 64, 64, 64, 4, 0, 1,
       launch_gemm_bf16<64, 64, 64, 0>},
      // k-contiguous operands through the workspace (launch_gemm_bf16_kc)
      {"gemm_bf16_256x256x64_r2_kc", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 64, 8, 0, 2,
       launch_gemm_bf16_kc<256, 256, 64, 2, 2, 4>, 1},
      {"gemm_bf16_256x128x64_r3_kc", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 64, 8, 0, 3,
       launch_gemm_bf16_kc<256, 128, 64, 3, 4, 2>, 1},
      {"gemm_bf16_128x128x64_r4_kc", TILEC_FAMILY_GEMM, TILEC_BF16, 128, 128, 64, 8, 0, 4,
       launch_gemm_bf16_kc<128, 128, 64, 4, 2, 4>, 1},
      {"gemm_bf16_256x256x32_r4w8", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 32, 8, 0, 4,
       launch_gemm_bf16<256, 256, 32, 4, 2, 4>},
      {"gemm_bf16_256x256x32_r4w8_kc", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 32, 8, 0, 4,
       launch_gemm_bf16_kc<256, 256, 32, 4, 2, 4>, 1},
      // 16x16x32 MFMAs (the same tiles; K % BK != 0 runs the 32x32 kernel)
      {"gemm_bf16_256x256x64_r2_m16", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 64, 8, 0, 2,
       launch_gemm_bf16<256, 256, 64, 2, 2, 4, 16>},
      {"gemm_bf16_256x256x32_r4w8_m16", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 32, 8, 0, 4,
       launch_gemm_bf16<256, 256, 32, 4, 2, 4, 16>},
      {"gemm_bf16_256x128x64_r3_m16", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 64, 8, 0, 3,
       launch_gemm_bf16<256, 128, 64, 3, 4, 2, 16>},
      {"gemm_bf16_128x128x64_r4_m16", TILEC_FAMILY_GEMM, TILEC_BF16, 128, 128, 64, 8, 0, 4,
       launch_gemm_bf16<128, 128, 64, 4, 2, 4, 16>},
      // operands padded into the workspace for the LDS-DMA kernel
      {"gemm_bf16_256x256x64_r2_m16_pad", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 64, 8, 0, 2,
       launch_gemm_bf16_pad<256, 256, 64, 2, 2, 4, 16>, 0, pad_workspace_bytes_bf16, pad_counter_bytes_bf16},
      {"gemm_bf16_256x128x64_r3_m16_pad", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 64, 8, 0, 3,
       launch_gemm_bf16_pad<256, 128, 64, 3, 4, 2, 16>, 0, pad_workspace_bytes_bf16, pad_counter_bytes_bf16},
      {"gemm_bf16_128x128x64_r4_m16_pad", TILEC_FAMILY_GEMM, TILEC_BF16, 128, 128, 64, 8, 0, 4,
       launch_gemm_bf16_pad<128, 128, 64, 4, 2, 4, 16>, 0, pad_workspace_bytes_bf16, pad_counter_bytes_bf16},
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace tilec
