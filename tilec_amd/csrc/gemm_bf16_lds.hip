// bf16 GEMM for aligned operands, C[M,N] (fp32) = A[M,K] · B[K,N] (bf16,
// row-major), fp32 accumulate, on v_mfma_f32_32x32x16_bf16.
//
// Same tile semantics as the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24): zero accumulator, K steps over masked tiles with
// `other=0.0`, masked store.  Built for gfx950:
//   * Global -> LDS with buffer_load_dwordx4 ... lds: each lane moves 16 bytes
//     straight into LDS, no VGPR staging, asynchronously; the next K step's
//     tiles are in flight while the current one is multiplied (two LDS
//     buffers, one barrier per K step).
//   * A lives in LDS row-major (k contiguous, 128-byte rows) with the 16-byte
//     chunks of row i XOR-swizzled by (i >> 1) & 7, so the 16-byte operand
//     reads of 16 consecutive rows hit distinct banks.
//   * B lives in LDS as it is in memory (n contiguous) and the MFMA B operand
//     (8 consecutive k of one column per lane) comes from two
//     ds_read_b64_tr_b16 transposing reads; chunks of row k are swizzled by
//     4 * (k & 3) so the 8 rows one read touches spread over the banks.
//   * Masking is done on addresses: chunks past M, N or K get an out-of-range
//     buffer offset and land in LDS as zeros.  Operands must be 16-byte
//     aligned with K, N, lda, ldb multiples of 8 (the launcher checks; other
//     shapes go to the generic kernel in gemm_bf16.hip).
//   * XCD-aware grouped tile order (tile_of in common.h).
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;
typedef short i16x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kBK = 64;

template <int BM, int BN, int WM, int WN>
struct LdsGemm {
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int A_CHUNKS = BM * kBK / 8;  // 16-byte chunks per stage
  static constexpr int B_CHUNKS = kBK * BN / 8;
  static constexpr int A_INSTR = A_CHUNKS / 64 / NW;  // DMA instructions per wave per stage
  static constexpr int B_INSTR = B_CHUNKS / 64 / NW;
  static constexpr int B_ROW_CHUNKS = BN / 8;
  static constexpr int A_BYTES = BM * kBK * 2, B_BYTES = kBK * BN * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(A_CHUNKS % (64 * NW) == 0 && B_CHUNKS % (64 * NW) == 0, "DMA must divide evenly");
  static_assert(BN % 128 == 0, "B swizzle needs rows of >= 16 chunks");
};

__device__ __forceinline__ int swz_a(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int swz_b(int krow) { return 4 * (krow & 3); }

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_bf16_lds_kernel(
    const u16* __restrict__ A, const u16* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m) {
  using P = LdsGemm<BM, BN, WM, WN>;
  // Two stage buffers as distinct LDS objects: every access below names its
  // buffer statically, so the compiler can tell that reads of one buffer do
  // not depend on the DMA writes in flight to the other.
  __shared__ __align__(16) char lds0[P::STAGE_BYTES];
  __shared__ __align__(16) char lds1[P::STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = (K + kBK - 1) / kBK;

  // ---- global -> LDS for K step kt into buffer buf ---------------------------
  // Physical chunk p of the A stage holds row p / 8, logical chunk
  // (p % 8) ^ swz_a(row); of the B stage, k-row p / (BN/8), logical chunk
  // (p % (BN/8)) ^ swz_b(row).  Instruction i of this wave fills physical
  // chunks [64 * (wave * INSTR + i), +64), lane l the l-th of them.
  auto dma = [&](int kt, char* st) {
    const int k0 = kt * kBK;
    const BufRsrc ra = make_rsrc(A + (int64_t)m0 * lda + k0);
    const BufRsrc rb = make_rsrc(B + (int64_t)k0 * ldb + n0);
#pragma unroll
    for (int i = 0; i < P::A_INSTR; ++i) {
      const int pbase = 64 * (wave * P::A_INSTR + i);
      const int p = pbase + lane;
      const int row = p >> 3, c = (p & 7) ^ swz_a(row);
      const bool ok = (m0 + row < M) & (k0 + 8 * c < K);
      const uint32_t off = 2u * ((uint32_t)row * (uint32_t)lda + 8u * c);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + 16 * pbase), 16, ok ? off : kOob, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < P::B_INSTR; ++i) {
      const int pbase = 64 * (wave * P::B_INSTR + i);
      const int p = pbase + lane;
      const int row = p / P::B_ROW_CHUNKS, c = (p % P::B_ROW_CHUNKS) ^ swz_b(row);
      const bool ok = (k0 + row < K) & (n0 + 8 * c < N);
      const uint32_t off = 2u * ((uint32_t)row * (uint32_t)ldb + 8u * c);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(st + P::A_BYTES + 16 * pbase), 16, ok ? off : kOob,
                                               0, 0, 0);
    }
  };

  f32x16 acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Per-lane fragment addressing (bytes within a stage).
  const int h = lane >> 5;               // which 8 of a k16 step (A) / B lane half
  const int g = lane >> 4, jj = lane & 15;
  int a_row[P::TM];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) a_row[i] = wm * P::WTM + 32 * i + (lane & 31);
  int b_n[P::TN];
#pragma unroll
  for (int j = 0; j < P::TN; ++j) b_n[j] = wn * P::WTN + 32 * j + 16 * (g & 1) + 4 * (jj & 3);
  const int b_krow = 8 * (g >> 1) + (jj >> 2);  // + 16 * ks (+ 4 for the second read)

  auto a_addr = [&](int i, int ks) {
    const int row = a_row[i], c = 2 * ks + h;
    return 16 * (row * 8 + (c ^ swz_a(row)));
  };
  auto b_addr = [&](int j, int krow) {
    const int n = b_n[j];
    return P::A_BYTES + 16 * (krow * P::B_ROW_CHUNKS + ((n >> 3) ^ swz_b(krow))) + 8 * ((n >> 2) & 1);
  };

  auto compute = [&](const char* st) {
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 a[P::TM], b[P::TN];
#pragma unroll
      for (int i = 0; i < P::TM; ++i) a[i] = *reinterpret_cast<const bf16x8*>(st + a_addr(i, ks));
#pragma unroll
      for (int j = 0; j < P::TN; ++j) {
        const int kr = 16 * ks + b_krow;
        const i16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4v*)(st + b_addr(j, kr)));
        const i16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4v*)(st + b_addr(j, kr + 4)));
        typedef short i16x8v __attribute__((ext_vector_type(8)));
        const i16x8v both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        b[j] = __builtin_bit_cast(bf16x8, both);
      }
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x16bf16(a[i], b[j], acc[i][j]);
    }
  };

  // K loop unrolled by two so each half uses a fixed buffer.  The DMA of the
  // step after next is issued unconditionally: past K its chunks are out of
  // range and write zeros nobody reads, which keeps the body straight-line.
  if (nk > 0) {
    dma(0, lds0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  int kt = 0;
  // sched_barrier keeps each DMA issue ahead of the MFMAs it overlaps.
  for (; kt + 2 <= nk; kt += 2) {
    dma(kt + 1, lds1);
    __builtin_amdgcn_sched_barrier(0);
    compute(lds0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    dma(kt + 2, lds0);
    __builtin_amdgcn_sched_barrier(0);
    compute(lds1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (kt < nk) compute(lds0);

  // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each block.
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);
  const int row_base = m0 + wm * P::WTM + 4 * h;
  const int col_base = n0 + wn * P::WTN + (lane & 31);
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

}  // namespace

// Launch the LDS-DMA kernel; the caller has checked alignment (16-byte
// operands, K, N, lda, ldb multiples of 8) and the 32-bit offset limits.
template <int BM, int BN, int WM, int WN>
hipError_t launch_gemm_bf16_lds(const MatmulArgs& a) {
  using P = LdsGemm<BM, BN, WM, WN>;
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_bf16_lds_kernel<BM, BN, WM, WN>), dim3((unsigned)tiles), dim3(P::NT), 0, a.stream,
                     static_cast<const u16*>(a.x1), static_cast<const u16*>(a.x2), a.out, (int)a.M, (int)a.N,
                     (int)a.K, a.ldx1, a.ldx2, a.ldo, 4);
  return hipGetLastError();
}

template hipError_t launch_gemm_bf16_lds<256, 256, 2, 2>(const MatmulArgs&);
template hipError_t launch_gemm_bf16_lds<256, 128, 2, 2>(const MatmulArgs&);
template hipError_t launch_gemm_bf16_lds<128, 128, 2, 2>(const MatmulArgs&);

}  // namespace tilec
