// LDS-staged fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2f32):
//   C[M,N] = A[M,K] · B[K,N], fp32, fp32 accumulate; C row-major, A and B
//   each row- or column-major (a column-major operand is read in place:
//   the transposed view x.T of a contiguous matrix needs no copy).
//
// Semantics follow the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24): one workgroup per BM x BN output tile, an accumulator
// that starts at zero, a K loop in steps of BK over masked tiles of A and B
// (`other=0.0`), and a masked store.  What runs underneath is MI355X-native:
//   * 64-wide waves arranged WM x WN, each owning a (BM/WM) x (BN/WN) block of
//     32x32 MFMA accumulators held in registers for the whole K loop (8-wave
//     grids keep two waves per SIMD on one large tile: their MFMAs cover each
//     other's barrier and load waits);
//   * A and B tiles double-buffered in LDS with one barrier per K step; the
//     next tile's global loads are issued before the current tile's MFMAs;
//   * tiles kept in LDS as loaded (16-byte stores): a k-contiguous operand
//     gives each lane the 4 consecutive k of four MFMAs in one 16-byte read
//     (the MFMAs of an 8-deep k chunk take k = 8c + 4h + e in lane half h),
//     the other kind one 4-byte read per MFMA, both free of bank conflicts;
//   * branch-free edges, as the reference's if-converted masked loads
//     (README.md:50): with row strides that fit 32-bit offsets (BUF), every
//     tile loads through buffer resources that end at the matrix's last
//     element — rows past M (A) or K (B) get an out-of-range offset and load
//     zeros, and when K or N is not a multiple of 4 a per-element select
//     clears the columns past the edge of the quad that straddles it — so
//     edge tiles cost what interior ones do; otherwise clamped addresses plus
//     selects on edge tiles and the K tail;
//   * XCD-aware, grouped tile order (tile_of in common.h).
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB>
hipError_t launch_gemm_f32_lds(const MatmulArgs& a);  // gemm_f32_lds.hip

namespace {

template <int BM, int BN, int BK, int WM, int WN>
struct GemmF32 {
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BK % 8 == 0, "BK: whole 8-deep k chunks");
  // K chunk (8 deep: four MFMA k-pairs) before whose MFMAs the next tile goes
  // from registers to LDS; its loads were issued a step earlier.  Storing
  // early leaves the LDS writes the rest of the step to complete under the
  // matrix cores: waves with at least 96 MFMAs per step (the 256 x 256
  // tiles) store after their first chunk, other 8-wave tiles mid-step (at
  // 4096^3 and 2048^3 these beat every other
  // position: chunk 0 waits for loads still in flight, later positions
  // leave the writes less cover).  4-wave tiles run two workgroups per CU,
  // whose barriers interleave, and store at the end of the step.
  // Waves per SIMD the register budget is held to: 4-wave workgroups with
  // at most 128 accumulators per lane fit two workgroups per CU, whose
  // barriers are independent, so one's MFMAs cover the other's waits.
  static constexpr int kWavesPerSimd = (WM * WN == 4 && TM * TN * 16 <= 128) ? 2 : 1;
  static constexpr int KS = BK / 8;
  static constexpr int kStoreAt = TM * TN * BK / 2 >= 96 ? 1 : (WM * WN == 8 ? KS / 2 : KS);
};

// Four consecutive floats at a 4-byte aligned address: one dwordx4 load,
// which CDNA performs for any dword-aligned address.
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

template <bool VEC>
__device__ __forceinline__ f32x4 ld4(const float* __restrict__ p, bool ok_all, int valid) {
  // valid: number of leading elements in bounds (0..4); VEC => valid in {0,4}
  if (VEC) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
    return ok_all ? v : f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    f32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float x = p[c < valid ? c : 0];
      v[c] = c < valid ? x : 0.f;
    }
    return v;
  }
}

// Bytes from p to the end of a matrix of `rows` rows (row stride ld, last
// row `cols` long), clamped to a buffer's 31-bit range; 0 if none.
__device__ __forceinline__ uint32_t extent(int64_t rows_left, int64_t ld, int64_t cols_left) {
  if (rows_left <= 0 || cols_left <= 0) return 0u;
  const int64_t bytes = 4 * ((rows_left - 1) * ld + cols_left);
  return bytes > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)bytes;
}

// One operand's tile per K step: R rows of the operand's outer dimension (M
// for x1, N for x2) by BK of K, moved global -> registers -> LDS.  KC: the
// operand's element (r, k) is X[r * ld + k] (k contiguous: row-major x1,
// column-major x2); otherwise X[k * ld + r] (r contiguous: row-major x2,
// column-major x1).  Each thread moves Q quads of 4 elements contiguous in
// memory.
//
// LDS layout, as loaded (16-byte stores, no transposition):
//   KC: S[r][k], rows of LK = BK + 4 floats.  An MFMA operand fragment is one
//     16-byte read of 4 consecutive k; lanes 0-7 read rows r..r+7 of one
//     chunk, 9 (or 5) chunks apart mod 16: no bank conflicts.
//   RC: S[k][r], rows of LR = R + 8 floats.  An operand is one 4-byte read
//     per MFMA: 32 consecutive r per half wave at rows k and k + 4, whose
//     4 * LR = 32 mod 64 banks apart: the halves use disjoint banks.
template <int R, int BK, int NT, bool KC, bool VEC, bool BUF>
struct OperandF32 {
  static constexpr int Q = R * BK / 4 / NT;
  static constexpr int LK = BK + 4, LR = R + 8;
  static constexpr int STAGE = KC ? R * LK : BK * LR;  // floats per LDS stage
  static_assert(R % 32 == 0 && BK % 8 == 0, "tile shape");
  static_assert(R * BK % (4 * NT) == 0, "tile loads must divide evenly");
  const float* X;
  int64_t ld;
  int r0, Rtot, K;
  int tr[Q], tk[Q], rvalid[Q];
  uint32_t off[Q];
  f32x4 v[2][Q];  // two register sets: one tile waits for its LDS store while the next loads

  // Tile row and tile k of the first element of quad e.
  __device__ __forceinline__ static void coord(int e, int& r, int& k) {
    if constexpr (KC) {
      r = e / (BK / 4);
      k = 4 * (e % (BK / 4));
    } else {
      k = e / (R / 4);
      r = 4 * (e % (R / 4));
    }
  }

  __device__ __forceinline__ void init(const float* X_, int64_t ld_, int r0_, int Rtot_, int K_, int tid) {
    X = X_;
    ld = ld_;
    r0 = r0_;
    Rtot = Rtot_;
    K = K_;
#pragma unroll
    for (int p = 0; p < Q; ++p) {
      coord(tid + p * NT, tr[p], tk[p]);
      if constexpr (BUF) {
        // The outer dimension's edge is fixed per tile: quads past it get kOob
        // once; K's edge moves with the step.
        if constexpr (KC) {
          rvalid[p] = r0 + tr[p] < Rtot ? 4 : 0;
          off[p] = rvalid[p] ? 4u * ((uint32_t)tr[p] * (uint32_t)ld + (uint32_t)tk[p]) : kOob;
        } else {
          rvalid[p] = max(0, min(4, Rtot - (r0 + tr[p])));
          off[p] = rvalid[p] > 0 ? 4u * ((uint32_t)tk[p] * (uint32_t)ld + (uint32_t)tr[p]) : kOob;
        }
      }
    }
  }

  // Global -> registers for K step kt.  BUF: a resource that ends at the
  // matrix's last element, out-of-range offsets for masked quads, and (when
  // !VEC) a select that clears the columns past the edge inside the quad that
  // straddles it.  Otherwise MASK selects clamped, per-element loads at
  // every edge and unmasked 16-byte loads elsewhere.
  // `live` false (BUF only): the tile lies past this workgroup's K range;
  // its loads still issue, through an empty resource (zeros, no traffic), so
  // every step issues the same loads and the compiler's wait before the LDS
  // store counts only the loads that store needs.
  template <int SET>
  __device__ __forceinline__ void load(int kt, bool mask, bool live = true) {
    const int k0 = kt * BK;
    if constexpr (BUF) {
      const uint32_t n = KC ? extent(Rtot - r0, ld, K - k0) : extent(K - k0, ld, Rtot - r0);
      const BufRsrc rs = make_rsrc(X + (KC ? (int64_t)r0 * ld + k0 : (int64_t)k0 * ld + r0), live ? n : 0u);
#pragma unroll
      for (int p = 0; p < Q; ++p) {
        f32x4 x = load_f32x4(rs, k0 + tk[p] < K ? off[p] : kOob);
        if constexpr (!VEC) {
          const int valid = KC ? K - (k0 + tk[p]) : rvalid[p];
#pragma unroll
          for (int c = 1; c < 4; ++c) x[c] = c < valid ? x[c] : 0.f;
        }
        v[SET][p] = x;
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < Q; ++p) {
      const int gr = r0 + tr[p], gk = k0 + tk[p];
      const int64_t at = KC ? (int64_t)gr * ld + gk : (int64_t)gk * ld + gr;
      if (!mask) {  // whole quad in bounds: one (dword-aligned) 16-byte load
        v[SET][p] = *reinterpret_cast<const f32x4_a4*>(X + at);
      } else {
        const int valid = KC ? (gr < Rtot ? max(0, min(4, K - gk)) : 0) : (gk < K ? max(0, min(4, Rtot - gr)) : 0);
        v[SET][p] = ld4<VEC>(X + (valid > 0 ? at : 0), valid == 4, valid);
      }
    }
  }

  template <int SET>
  __device__ __forceinline__ void store(float* __restrict__ S) const {
#pragma unroll
    for (int p = 0; p < Q; ++p)
      *reinterpret_cast<f32x4*>(S + (KC ? tr[p] * LK + tk[p] : tk[p] * LR + tr[p])) = v[SET][p];
  }

  // Operand values of rows r0 + lane % 32 for the four MFMAs of k chunk c
  // (k = 8c .. 8c + 7): MFMA e takes k = 8c + 4h + e in lane half h, so a
  // KC fragment is the lane's 4 consecutive k in one read.
  __device__ __forceinline__ static f32x4 frag(const float* __restrict__ S, int r, int c, int h) {
    if constexpr (KC) {
      return *reinterpret_cast<const f32x4*>(S + r * LK + 8 * c + 4 * h);
    } else {
      const float* p = S + (8 * c + 4 * h) * LR + r;
      return f32x4{p[0], p[LR], p[2 * LR], p[3 * LR]};
    }
  }
};

// CA: x1 is column-major (element (m, k) at A[m + k * lda]); CB: x2 is
// column-major (element (k, n) at B[k + n * ldb]).
template <int BM, int BN, int BK, int WM, int WN, bool VEC, bool BUF, bool CA, bool CB>
__global__ __launch_bounds__(WM * WN * 64, (GemmF32<BM, BN, BK, WM, WN>::kWavesPerSimd)) void gemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int xcds, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = GemmF32<BM, BN, BK, WM, WN>;
  using OpA = OperandF32<BM, BK, P::NT, !CA, VEC, BUF>;
  using OpB = OperandF32<BN, BK, P::NT, CB, VEC, BUF>;
  extern __shared__ __align__(16) float lds[];
  __shared__ int last_flag;
  float* As = lds;                   // 2 stages of OpA::STAGE floats
  float* Bs = lds + 2 * OpA::STAGE;  // 2 stages of OpB::STAGE floats

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

  OpA opa;
  OpB opb;
  opa.init(A, lda, m0, M, K, tid);
  opb.init(B, ldb, n0, N, K, tid);
  // Tile t (counted from kt0) moves through register set t % 2 and LDS
  // buffer t % 2.
  auto gload = [&](auto set, int kt, bool mask, bool live = true) {
    opa.template load<decltype(set)::value>(kt, mask, live);
    opb.template load<decltype(set)::value>(kt, mask, live);
  };
  auto sstore = [&](auto set) {
    constexpr int T = decltype(set)::value;
    opa.template store<T>(As + T * OpA::STAGE);
    opb.template store<T>(Bs + T * OpB::STAGE);
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;

  f32x16 acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (kt0 < kt1) {
    gload(Set0{}, kt0, !(interior && kt0 < nk_full));
    if (kt0 + 1 < kt1) gload(Set1{}, kt0 + 1, !(interior && kt0 + 1 < nk_full));
    sstore(Set0{});
    __syncthreads();
  }

  const int arow = wm * P::WTM + (lane & 31);
  const int bcol = wn * P::WTN + (lane & 31);
  const int khalf = lane >> 5;

  // Step t computes from LDS buffer t % 2 and stores tile t + 1 (loaded one
  // step earlier into set (t + 1) % 2) into the other buffer, which was last
  // read in step t - 1, before that step's barrier; it issues the loads of
  // tile t + 2 into set t % 2, whose tile went to LDS in step t - 1.  A load
  // thus has one to two steps to arrive.  Past the last tile the store
  // rewrites stale registers into a buffer no one reads again; storing
  // unconditionally keeps the step one basic block.
  auto step = [&](int kt, auto par) __attribute__((always_inline)) {
    constexpr int T = decltype(par)::value;
    using Next = std::integral_constant<int, T ^ 1>;
    if (BUF)
      gload(par, kt + 2, false, kt + 2 < kt1);
    else if (kt + 2 < kt1)
      gload(par, kt + 2, !(interior && kt + 2 < nk_full));
    const float* as = As + T * OpA::STAGE;
    const float* bs = Bs + T * OpB::STAGE;
#pragma unroll
    for (int c = 0; c < P::KS; ++c) {
      if (c == P::kStoreAt) sstore(Next{});
      f32x4 a[P::TM], b[P::TN];
#pragma unroll
      for (int i = 0; i < P::TM; ++i) a[i] = OpA::frag(as, arow + 32 * i, c, khalf);
#pragma unroll
      for (int j = 0; j < P::TN; ++j) b[j] = OpB::frag(bs, bcol + 32 * j, c, khalf);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < P::TM; ++i)
#pragma unroll
          for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x2(a[i][e], b[j][e], acc[i][j]);
    }
    if (P::kStoreAt == P::KS) sstore(Next{});
    __syncthreads();
  };
  int kt = kt0;
  for (; kt + 1 < kt1; kt += 2) {
    step(kt, Set0{});
    step(kt + 1, Set1{});
  }
  if (kt < kt1) step(kt, Set0{});

  // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each block.
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

template <int BM, int BN, int BK, int WM, int WN, bool VEC, bool BUF, bool CA, bool CB>
hipError_t launch_one(const MatmulArgs& a, dim3 grid) {
  using P = GemmF32<BM, BN, BK, WM, WN>;
  auto k = gemm_f32_kernel<BM, BN, BK, WM, WN, VEC, BUF, CA, CB>;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * 16 > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  grid.y = (unsigned)g.splits;
  const size_t lds = sizeof(float) * 2 *
                     (OperandF32<BM, BK, P::NT, !CA, VEC, BUF>::STAGE + OperandF32<BN, BK, P::NT, CB, VEC, BUF>::STAGE);
  static std::atomic<uint64_t> lds_devices{0};
  const hipError_t e = raise_lds_limit((const void*)k, lds, lds_devices);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, grid, dim3(WM * WN * 64), lds, a.stream, static_cast<const float*>(a.x1),
                     static_cast<const float*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo,
                     8, device_xcds(), (int)g.steps, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr, g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, bool CA, bool CB>
hipError_t launch_layout(const MatmulArgs& a) {
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  // 16-byte quads never straddle an edge: the contiguous extent of each
  // operand (K, or M / N for the r-contiguous layouts) and both strides are
  // multiples of 4, and the bases are 16-byte aligned.
  const int64_t a_run = CA ? a.M : a.K, b_run = CB ? a.K : a.N;
  const bool vec = (a_run % 4 == 0) && (b_run % 4 == 0) && (a.ldx1 % 4 == 0) && (a.ldx2 % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.x1) % 16 == 0) && (reinterpret_cast<uintptr_t>(a.x2) % 16 == 0);
  // Buffer offsets inside one K step: (strided rows of the tile) * ld * 4 +
  // one row's span < 2^31.
  const int64_t a_rows = CA ? BK : BM, a_span = CA ? BM : BK;
  const int64_t b_rows = CB ? BN : BK, b_span = CB ? BK : BN;
  const bool buf = a_rows * a.ldx1 * 4 + 4 * a_span < (int64_t(1) << 31) &&
                   b_rows * a.ldx2 * 4 + 4 * b_span < (int64_t(1) << 31);
  dim3 grid((unsigned)tiles);
  if (buf)
    return vec ? launch_one<BM, BN, BK, WM, WN, true, true, CA, CB>(a, grid)
               : launch_one<BM, BN, BK, WM, WN, false, true, CA, CB>(a, grid);
  return vec ? launch_one<BM, BN, BK, WM, WN, true, false, CA, CB>(a, grid)
             : launch_one<BM, BN, BK, WM, WN, false, false, CA, CB>(a, grid);
}

// Aligned operands (16-byte bases, contiguous extents and strides multiples
// of 4) whose per-step offsets fit 32 bits run the LDS-DMA kernel of
// gemm_f32_lds.hip with a ring of NBUF stage buffers; everything else runs
// the register-staged kernel above with the same tile and waves.
template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB>
hipError_t launch_layout_lds(const MatmulArgs& a) {
  const int64_t a_run = CA ? a.M : a.K, b_run = CB ? a.K : a.N;
  const bool vec = (a_run % 4 == 0) && (b_run % 4 == 0) && (a.ldx1 % 4 == 0) && (a.ldx2 % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.x1) % 16 == 0) && (reinterpret_cast<uintptr_t>(a.x2) % 16 == 0);
  const int64_t a_rows = CA ? BK : BM, b_rows = CB ? BN : BK;
  constexpr int64_t lim = (int64_t(1) << 31) - 4096;
  if (vec && a_rows * a.ldx1 * 4 < lim && b_rows * a.ldx2 * 4 < lim)
    return launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, CA, CB>(a);
  return launch_layout<BM, BN, BK, WM, WN, CA, CB>(a);
}

template <int BM, int BN, int BK, int NBUF, int WM, int WN>
hipError_t launch_gemm_f32_dma(const MatmulArgs& a) {
  switch (a.layout & 3) {
    case 0: return launch_layout_lds<BM, BN, BK, NBUF, WM, WN, false, false>(a);
    case TILEC_X1_COL_MAJOR: return launch_layout_lds<BM, BN, BK, NBUF, WM, WN, true, false>(a);
    case TILEC_X2_COL_MAJOR: return launch_layout_lds<BM, BN, BK, NBUF, WM, WN, false, true>(a);
    default: return launch_layout_lds<BM, BN, BK, NBUF, WM, WN, true, true>(a);
  }
}

template <int BM, int BN, int BK, int WM, int WN>
hipError_t launch_gemm_f32(const MatmulArgs& a) {
  switch (a.layout & 3) {
    case 0: return launch_layout<BM, BN, BK, WM, WN, false, false>(a);
    case TILEC_X1_COL_MAJOR: return launch_layout<BM, BN, BK, WM, WN, true, false>(a);
    case TILEC_X2_COL_MAJOR: return launch_layout<BM, BN, BK, WM, WN, false, true>(a);
    default: return launch_layout<BM, BN, BK, WM, WN, true, true>(a);
  }
}

}  // namespace

// The 64 x 64 tile with K unsplit: the fallback of kernels whose own
// addressing does not cover an operand's strides.
hipError_t launch_gemm_f32_unsplit(const MatmulArgs& a) {
  MatmulArgs b = a;
  b.split_k = 1;
  return launch_gemm_f32<64, 64, 16, 2, 2>(b);
}

// ---------------------------------------------------------------------------
// Pad variants: each operand is first copied into the workspace with its
// contiguous extent and row stride rounded up to 4 floats and K rounded up to
// BK, zero-filled, so the direct-to-LDS kernel takes operands whose rows are
// not 16-byte aligned (an odd K or N: the ragged BASELINE shapes run the
// register-staged kernel otherwise).  The padding is zeros, so it adds
// nothing to the product; C is written as the caller's M x N (the kernel's
// column chunks past N may read padding, never store it).  Workspace:
// [x1 padded][x2 padded][split-K partials], each 256-byte aligned.  The
// copies are common.h's pad_copy.
// ---------------------------------------------------------------------------

// Padded extents: K up to the K step, the contiguous extent of a
// column-major x1 (M) or a row-major x2 (N) up to 4.  Sized for either
// layout, since the size queries do not see it.
struct PadGeom {
  int64_t kp, m4, n4;
  size_t x1_bytes, x2_bytes;  // 256-byte aligned
};
inline PadGeom pad_geom(int64_t M, int64_t N, int64_t K, int64_t bk) {
  PadGeom g;
  g.kp = cdiv(K, bk) * bk;
  g.m4 = cdiv(M, 4) * 4;
  g.n4 = cdiv(N, 4) * 4;
  g.x1_bytes = (size_t)cdiv(g.m4 * g.kp * 4, 256) * 256;
  g.x2_bytes = (size_t)cdiv(g.n4 * g.kp * 4, 256) * 256;
  return g;
}

size_t pad_workspace_bytes(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  if (M == 0 || N == 0 || K == 0) return 0;
  const PadGeom p = pad_geom(M, N, K, d.bk);
  const SplitGeom g = gemm_split_geom(p.kp, d.bk, split_k);
  const size_t partials = g.splits > 1 ? (size_t)g.splits * cdiv(M, d.bm) * cdiv(N, d.bn) * d.bm * d.bn * 4 : 0;
  return p.x1_bytes + p.x2_bytes + partials;
}
size_t pad_counter_bytes(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) {
  if (M == 0 || N == 0 || K == 0 || gemm_split_geom(K, d.bk, split_k).splits <= 1) return 0;
  return (size_t)cdiv(M, d.bm) * cdiv(N, d.bn) * kSplitCounterStride * sizeof(unsigned);
}

template <int BM, int BN, int BK, int NBUF, int WM, int WN>
hipError_t launch_gemm_f32_pad(const MatmulArgs& a) {
  if (a.M == 0 || a.N == 0 || a.K == 0) return launch_gemm_f32_dma<BM, BN, BK, NBUF, WM, WN>(a);
  const bool ca = a.layout & TILEC_X1_COL_MAJOR, cb = a.layout & TILEC_X2_COL_MAJOR;
  const PadGeom p = pad_geom(a.M, a.N, a.K, BK);
  // Stored (rows x cols) of each operand, before and after padding.
  const int64_t r1 = ca ? a.K : a.M, c1 = ca ? a.M : a.K, r1p = ca ? p.kp : a.M, c1p = ca ? p.m4 : p.kp;
  const int64_t r2 = cb ? a.N : a.K, c2 = cb ? a.K : a.N, r2p = cb ? a.N : p.kp, c2p = cb ? p.kp : p.n4;
  // The direct-to-LDS kernel's per-step offsets: (strided rows of a tile) *
  // ld * 4 < 2^31; beyond that the register-staged kernel on the operands
  // as they are (its workspace use is only the split partials).
  constexpr int64_t lim = (int64_t(1) << 31) - 4096;
  if ((ca ? BK : BM) * c1p * 4 >= lim || (cb ? BN : BK) * c2p * 4 >= lim || r1p * c1p >= (int64_t(1) << 31) ||
      r2p * c2p >= (int64_t(1) << 31) || reinterpret_cast<uintptr_t>(a.workspace) % 16 != 0)
    return launch_gemm_f32<BM, BN, BK, WM, WN>(a);
  // With K a whole number of K steps, an operand whose rows are already whole
  // 16-byte groups (extent, stride and base) is read in place; only the
  // other is copied.
  auto in_place = [&](const void* x, int64_t c, int64_t ld, int64_t rows_per_step) {
    return a.K % BK == 0 && c % 4 == 0 && ld % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           rows_per_step * ld * 4 < lim;
  };
  const bool keep1 = in_place(a.x1, c1, a.ldx1, ca ? BK : BM), keep2 = in_place(a.x2, c2, a.ldx2, cb ? BN : BK);
  char* ws = static_cast<char*>(a.workspace);
  float* x1p = reinterpret_cast<float*>(ws);
  float* x2p = reinterpret_cast<float*>(ws + p.x1_bytes);
  const hipError_t e = pad_copy<4>(a.x1, x1p, r1, c1, a.ldx1, keep1 ? 0 : r1p, c1p, a.x2, x2p, r2, c2, a.ldx2,
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
    case 0: return launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, false, false>(b);
    case TILEC_X1_COL_MAJOR: return launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, true, false>(b);
    case TILEC_X2_COL_MAJOR: return launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, false, true>(b);
    default: return launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, true, true>(b);
  }
}

// Variant table for this family (its order is part of the variant numbering).
const VariantDesc* gemm_f32_variants(int* count) {
  static const VariantDesc t[] = {
      {"gemm_f32_256x256x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 256, 256, 16, 4, 0, 1,
       launch_gemm_f32<256, 256, 16, 2, 2>},
      {"gemm_f32_256x128x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 256, 128, 16, 4, 0, 1,
       launch_gemm_f32<256, 128, 16, 2, 2>},
      {"gemm_f32_128x128x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 16, 4, 0, 1,
       launch_gemm_f32<128, 128, 16, 2, 2>},
      {"gemm_f32_128x64x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 128, 64, 16, 4, 0, 1,
       launch_gemm_f32<128, 64, 16, 2, 2>},
      {"gemm_f32_64x64x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 64, 64, 16, 4, 0, 1,
       launch_gemm_f32<64, 64, 16, 2, 2>},
      {"gemm_f32_256x256x16_w2x4", TILEC_FAMILY_GEMM, TILEC_F32, 256, 256, 16, 8, 0, 1,
       launch_gemm_f32<256, 256, 16, 2, 4>},
      {"gemm_f32_256x256x32_w2x4", TILEC_FAMILY_GEMM, TILEC_F32, 256, 256, 32, 8, 0, 1,
       launch_gemm_f32<256, 256, 32, 2, 4>},
      {"gemm_f32_128x128x16_w2x4", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 16, 8, 0, 1,
       launch_gemm_f32<128, 128, 16, 2, 4>},
      {"gemm_f32_128x128x32_w2x4", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 32, 8, 0, 1,
       launch_gemm_f32<128, 128, 32, 2, 4>},
      {"gemm_f32_128x128x32_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 32, 4, 0, 1,
       launch_gemm_f32<128, 128, 32, 2, 2>},
      {"gemm_f32_128x128x64_w2x4", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 64, 8, 0, 1,
       launch_gemm_f32<128, 128, 64, 2, 4>},
      // direct-to-LDS copies (gemm_f32_lds.hip); unroll = ring depth
      {"gemm_f32_256x256x32_w2x4_lds", TILEC_FAMILY_GEMM, TILEC_F32, 256, 256, 32, 8, 0, 2,
       launch_gemm_f32_dma<256, 256, 32, 2, 2, 4>},
      {"gemm_f32_128x128x32_w2x4_lds", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 32, 8, 0, 3,
       launch_gemm_f32_dma<128, 128, 32, 3, 2, 4>},
      {"gemm_f32_128x128x64_w2x4_lds", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 64, 8, 0, 2,
       launch_gemm_f32_dma<128, 128, 64, 2, 2, 4>},
      {"gemm_f32_64x64x32_w2x2_lds", TILEC_FAMILY_GEMM, TILEC_F32, 64, 64, 32, 4, 0, 3,
       launch_gemm_f32_dma<64, 64, 32, 3, 2, 2>},
      {"gemm_f32_64x64x64_w2x2_lds", TILEC_FAMILY_GEMM, TILEC_F32, 64, 64, 64, 4, 0, 3,
       launch_gemm_f32_dma<64, 64, 64, 3, 2, 2>},
      // operands padded into the workspace for the direct-to-LDS kernel
      {"gemm_f32_128x128x32_w2x4_pad", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 32, 8, 0, 3,
       launch_gemm_f32_pad<128, 128, 32, 3, 2, 4>, 0, pad_workspace_bytes, pad_counter_bytes},
      {"gemm_f32_64x64x32_w2x2_pad", TILEC_FAMILY_GEMM, TILEC_F32, 64, 64, 32, 4, 0, 3,
       launch_gemm_f32_pad<64, 64, 32, 3, 2, 2>, 0, pad_workspace_bytes, pad_counter_bytes},
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace tilec
