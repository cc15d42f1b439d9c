// bf16 GEMM for aligned operands, C[M,N] (fp32) = A[M,K] · B[K,N] (bf16,
// row-major), fp32 accumulate, on v_mfma_f32_32x32x16_bf16.
//
// Same tile semantics as the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24): zero accumulator, K steps over masked tiles with
// `other=0.0`, masked store.  Built for gfx950:
//   * Global -> LDS with buffer_load_dwordx4 ... lds: each lane moves 16 bytes
//     straight into LDS, asynchronously, with no VGPR staging.  K steps of BK
//     cycle through a ring of NBUF stage buffers: the loads of step k+NBUF-1
//     are issued while step k is multiplied, so NBUF-1 steps (up to 96 KiB
//     per CU) are in flight — the global->LDS stream, not the matrix cores,
//     is what a shallower pipeline is limited by.
//   * The stage buffers are distinct LDS objects and the K loop is unrolled
//     over the ring, so every access names its buffer statically and the
//     compiler knows reads of one buffer do not wait on loads into another.
//   * A lives in LDS row-major (k contiguous) with its 16-byte chunks
//     XOR-swizzled per row, so the 16-byte operand reads of 16 consecutive
//     rows hit distinct banks.
//   * B lives in LDS as it is in memory (n contiguous) and the MFMA B operand
//     (8 consecutive k of one column per lane) comes from two
//     ds_read_b64_tr_b16 transposing reads; chunks of row k are swizzled by
//     4 * (k & 3) so the 8 rows one read touches spread over the banks.
//   * Masking is done on addresses: chunks past M, N or K get an out-of-range
//     buffer offset and land in LDS as zeros.  Operands must be 16-byte
//     aligned with K, N, lda, ldb multiples of 8 (the launcher checks; other
//     shapes go to the generic kernel in gemm_bf16.hip).
//   * Per K step, the MFMAs of the previous step's last k-slice (read into
//     registers before the barrier) run right after it, threaded one-for-one
//     with the next step's loads, so neither the barrier nor the load issue
//     leaves the matrix cores idle.  With 8 waves (2 per SIMD) one wave's
//     MFMAs also cover the other's LDS waits.
//   * XCD-aware grouped tile order (tile_of in common.h).
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;
typedef short i16x4v __attribute__((ext_vector_type(4)));
typedef short i16x8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int BM, int BN, int BK, int NBUF, int WM, int WN>
struct LdsGemm {
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int A_ROW_CHUNKS = BK / 8;  // 16-byte chunks per A row
  static constexpr int B_ROW_CHUNKS = BN / 8;  // 16-byte chunks per B row
  static constexpr int A_CHUNKS = BM * A_ROW_CHUNKS;
  static constexpr int B_CHUNKS = BK * B_ROW_CHUNKS;
  static constexpr int A_INSTR = A_CHUNKS / 64 / NW;  // DMA instructions per wave per step
  static constexpr int B_INSTR = B_CHUNKS / 64 / NW;
  static constexpr int IPS = A_INSTR + B_INSTR;
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(A_CHUNKS % (64 * NW) == 0 && B_CHUNKS % (64 * NW) == 0, "DMA must divide evenly");
  static_assert(BN % 128 == 0, "B swizzle needs rows of >= 16 chunks");
  static_assert(BK == 32 || BK == 64, "A swizzle covers 4 or 8 chunks per row");
  static_assert(NBUF >= 2 && NBUF <= 4, "ring of 2..4 stage buffers");
  static_assert((size_t)NBUF * STAGE_BYTES <= 160 * 1024, "LDS is 160 KiB");
  static_assert((NBUF - 2) * IPS <= 63, "vmcnt is 6 bits");
};

// A: chunk c of row i is stored at (c ^ swz) within the row; BK=64 rows are
// 128 B (8 chunks, 2 rows per 256-byte bank line), BK=32 rows 64 B (4 chunks).
template <int BK>
__device__ __forceinline__ int swz_a(int row) {
  return BK == 64 ? (row >> 1) & 7 : (row >> 2) & 3;
}
__device__ __forceinline__ int swz_b(int krow) { return 4 * (krow & 3); }

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left unconstrained (gfx9
// encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Scheduling groups "1 MFMA, then its share of the IPS loads", NM times.
template <int NM, int IPS, int X = 0>
__device__ __forceinline__ void sched_mfma_vmem() {
  if constexpr (X < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int n = (X + 1) * IPS / NM - X * IPS / NM;
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x020, n, 0);
    sched_mfma_vmem<NM, IPS, X + 1>();
  }
}

template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool KFULL>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_bf16_lds_kernel(
    const u16* __restrict__ A, const u16* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = LdsGemm<BM, BN, BK, NBUF, WM, WN>;
  constexpr int KS = BK / 16;  // MFMA k-slices per step
  __shared__ int last_flag;
  // The ring: distinct LDS objects (those past NBUF are never referenced).
  __shared__ __align__(16) char lds0[P::STAGE_BYTES];
  __shared__ __align__(16) char lds1[P::STAGE_BYTES];
  __shared__ __align__(16) char lds2[NBUF > 2 ? P::STAGE_BYTES : 16];
  __shared__ __align__(16) char lds3[NBUF > 3 ? P::STAGE_BYTES : 16];
  auto buf = [&](auto I) -> char* {
    constexpr int i = decltype(I)::value;
    if constexpr (i == 0) return lds0;
    else if constexpr (i == 1) return lds1;
    else if constexpr (i == 2) return lds2;
    else return lds3;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // This workgroup's K steps: [kt0, kt0 + nk) of the cdiv(K, BK) steps
  // (grid y = K splits of split_steps steps each; one split = all of K).
  const int split = blockIdx.y, S = gridDim.y;
  const int kt0 = split * split_steps;
  const int nk = max(0, min((K + BK - 1) / BK, kt0 + split_steps) - kt0);

  // ---- global -> LDS for K step kt (local: absolute step kt0 + kt) ----------
  // Physical chunk p of the A stage holds row p / A_ROW_CHUNKS, logical chunk
  // (p % A_ROW_CHUNKS) ^ swz_a(row); of the B stage, k-row p / B_ROW_CHUNKS,
  // logical chunk (p % B_ROW_CHUNKS) ^ swz_b(row).  Instruction i of this
  // wave fills physical chunks [64 * (wave * INSTR + i), +64), lane l the
  // l-th of them.  A lane's byte offset from the step's base is the same in
  // every step; rows past M and columns past N get kOob once, here.  A step
  // past this workgroup's range gets a resource of zero records, so its
  // loads touch nothing.  When K % BK != 0 (!KFULL) the last step also masks
  // A's chunks past K per lane and B's rows past K by the resource's size.
  uint32_t off_a[P::A_INSTR], off_b[P::B_INSTR];
  // Column within the A stage of this lane's chunk of instruction i;
  // recomputed where needed rather than held in registers.
  auto dma_a_kcol = [&](int i) {
    const int p = 64 * (wave * P::A_INSTR + i) + lane;
    const int row = p / P::A_ROW_CHUNKS;
    return 8 * ((p % P::A_ROW_CHUNKS) ^ swz_a<BK>(row));
  };
#pragma unroll
  for (int i = 0; i < P::A_INSTR; ++i) {
    const int p = 64 * (wave * P::A_INSTR + i) + lane;
    const int row = p / P::A_ROW_CHUNKS;
    off_a[i] = m0 + row < M ? 2u * ((uint32_t)row * (uint32_t)lda + (uint32_t)dma_a_kcol(i)) : kOob;
  }
#pragma unroll
  for (int i = 0; i < P::B_INSTR; ++i) {
    const int p = 64 * (wave * P::B_INSTR + i) + lane;
    const int row = p / P::B_ROW_CHUNKS, c = (p % P::B_ROW_CHUNKS) ^ swz_b(row);
    off_b[i] = n0 + 8 * c < N ? 2u * ((uint32_t)row * (uint32_t)ldb + 8u * c) : kOob;
  }
  // Instruction q (0 <= q < IPS) of step kt: A instructions first, then B.
  auto dma_one = [&](int q, int kt, char* st) __attribute__((always_inline)) {
    const int k0 = (kt0 + kt) * BK;
    const uint32_t recs = kt < nk ? 0x7FFFFFFFu : 0u;
    if (q < P::A_INSTR) {
      const BufRsrc ra = make_rsrc(A + (int64_t)m0 * lda + k0, recs);
      uint32_t off = off_a[q];
      if constexpr (!KFULL) off = k0 + dma_a_kcol(q) < K ? off : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + 16 * 64 * (wave * P::A_INSTR + q)), 16, off, 0,
                                               0, 0);
    } else {
      const int i = q - P::A_INSTR;
      // B's K edge is the end of whole rows: a resource of (K - k0) rows
      // masks the rows past it without a per-lane test.
      uint32_t recs_b = recs;
      if constexpr (!KFULL) recs_b = kt < nk ? (uint32_t)min<int64_t>((int64_t)(K - k0) * ldb * 2, 0x7FFFFFFF) : 0u;
      const BufRsrc rb = make_rsrc(B + (int64_t)k0 * ldb + n0, recs_b);
      // (a copy, not the array element itself: passed straight to the
      // builtin, the element makes the host pass drop the kernel's stub)
      const uint32_t off = off_b[i];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(st + P::A_BYTES + 16 * 64 * (wave * P::B_INSTR + i)),
                                               16, off, 0, 0, 0);
    }
  };
  auto dma = [&](int kt, char* st) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < P::IPS; ++q) dma_one(q, kt, st);
  };

  f32x16 acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Per-lane fragment addressing (bytes within a stage).
  const int h = lane >> 5;
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
    return 16 * (row * P::A_ROW_CHUNKS + (c ^ swz_a<BK>(row)));
  };
  auto b_addr = [&](int j, int krow) {
    const int n = b_n[j];
    return P::A_BYTES + 16 * (krow * P::B_ROW_CHUNKS + ((n >> 3) ^ swz_b(krow))) + 8 * ((n >> 2) & 1);
  };

  // The operands of one k-slice: A rows of the wave's 32-row blocks, B
  // columns of its 32-column blocks (8 consecutive k each).
  struct Frag {
    bf16x8 a[P::TM], b[P::TN];
  };
  auto read = [&](const char* st, int ks, Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::TM; ++i) f.a[i] = *reinterpret_cast<const bf16x8*>(st + a_addr(i, ks));
#pragma unroll
    for (int j = 0; j < P::TN; ++j) {
      const int kr = 16 * ks + b_krow;
      const i16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4v*)(st + b_addr(j, kr)));
      const i16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4v*)(st + b_addr(j, kr + 4)));
      f.b[j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::TM; ++i)
#pragma unroll
      for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x16bf16(f.a[i], f.b[j], acc[i][j]);
  };
  // The MFMAs of f with the loads of step kt threaded between them, so the
  // loads issue while the matrix cores are busy.
  auto mma_dma = [&](const Frag& f, int kt, char* st) __attribute__((always_inline)) {
    constexpr int NM = P::TM * P::TN;
#pragma unroll
    for (int x = 0; x < NM; ++x) {
      const int i = x / P::TN, j = x % P::TN;
      acc[i][j] = mfma32x32x16bf16(f.a[i], f.b[j], acc[i][j]);
#pragma unroll
      for (int q = x * P::IPS / NM; q < (x + 1) * P::IPS / NM; ++q) dma_one(q, kt, st);
    }
    sched_mfma_vmem<NM, P::IPS>();
  };

  // Software pipeline over K steps.  Entering step kt (ring slot I): f[0]
  // holds (or is loading) k-slice 0 of step kt; f[1] holds the last k-slice
  // of step kt-1, whose MFMAs have not been issued (zeros before step 0).
  // Step kt:
  //   1. MFMAs of f[1], threaded with the loads of step kt+NBUF-1 into the
  //      slot step kt-1 used — every wave finished reading that slot before
  //      the last barrier — so the matrix cores stay busy across it;
  //   2. k-slices 0 .. KS-2 of step kt, each one's MFMAs overlapping the LDS
  //      reads of the next; the last k-slice is read into f[1];
  //   3. wait for those reads and for this wave's loads of step kt+1 (at most
  //      NBUF-2 later steps in flight; loads complete in issue order), then
  //      the barrier: step kt+1 is in LDS for every wave and no wave reads
  //      step kt's slot again;
  //   4. read k-slice 0 of step kt+1 into f[0].
  Frag f[2];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) f[1].a[i] = bf16x8{};
#pragma unroll
  for (int j = 0; j < P::TN; ++j) f[1].b[j] = bf16x8{};

  constexpr int WAIT = (NBUF - 2) * P::IPS;
  auto step = [&](auto I, int kt) __attribute__((always_inline)) {
    constexpr int i = decltype(I)::value;
    char* const cur = buf(I);
    mma_dma(f[1], kt + NBUF - 1, buf(std::integral_constant<int, (i + NBUF - 1) % NBUF>{}));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      read(cur, ks + 1, f[(ks + 1) & 1]);
      mma(f[ks & 1]);
    }
    // The step's MFMAs stay ahead of the wait: nothing crosses this point.
    __builtin_amdgcn_sched_barrier(0);
    // vmcnt(WAIT) lgkmcnt(0) (gfx9 encoding, expcnt unconstrained)
    __builtin_amdgcn_s_waitcnt((WAIT & 15) | ((WAIT >> 4) << 14) | (7 << 4));
    __syncthreads();
    read(buf(std::integral_constant<int, (i + 1) % NBUF>{}), 0, f[0]);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: steps 0 .. NBUF-2 in flight, step 0 landed everywhere, its
  // first k-slice being read.
  if (nk > 0) {
    dma(0, lds0);
    if constexpr (NBUF > 2) dma(1, lds1);
    if constexpr (NBUF > 3) dma(2, lds2);
    wait_vmcnt<WAIT>();
    __syncthreads();
    read(lds0, 0, f[0]);
  }
  int kt = 0;
  for (; kt + NBUF <= nk; kt += NBUF) {
    step(std::integral_constant<int, 0>{}, kt);
    step(std::integral_constant<int, 1>{}, kt + 1);
    if constexpr (NBUF > 2) step(std::integral_constant<int, 2>{}, kt + 2);
    if constexpr (NBUF > 3) step(std::integral_constant<int, 3>{}, kt + 3);
  }
  // Remaining steps (fewer than NBUF): same slots in order.
  if (kt < nk) step(std::integral_constant<int, 0>{}, kt);
  if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
  if constexpr (NBUF > 2) {
    if (kt + 2 < nk) step(std::integral_constant<int, 2>{}, kt + 2);
  }
  mma(f[1]);  // last k-slice of the last step (zeros if K == 0)
  // Loads issued for steps past K still write (zeros) into LDS: let them
  // land before this workgroup can finish and release its LDS.
  __builtin_amdgcn_s_waitcnt(0);

  // Split K: publish this workgroup's partial tile; the last of the tile's
  // splits adds them in split order and writes C.
  // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each block.
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);
  const int row_base = m0 + wm * P::WTM + 4 * h;
  const int col_base = n0 + wn * P::WTN + (lane & 31);
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

}  // namespace

// Launch the LDS-DMA kernel; the caller has checked alignment (16-byte
// operands, K, N, lda, ldb multiples of 8) and the 32-bit offset limits.
template <int BM, int BN, int BK, int NBUF, int WM, int WN>
hipError_t launch_gemm_bf16_lds(const MatmulArgs& a) {
  using P = LdsGemm<BM, BN, BK, NBUF, WM, WN>;
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * 16 > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  auto kern = a.K % BK == 0 ? gemm_bf16_lds_kernel<BM, BN, BK, NBUF, WM, WN, true>
                            : gemm_bf16_lds_kernel<BM, BN, BK, NBUF, WM, WN, false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)g.splits), dim3(P::NT), 0, a.stream,
                     static_cast<const u16*>(a.x1), static_cast<const u16*>(a.x2), a.out, (int)a.M, (int)a.N,
                     (int)a.K, a.ldx1, a.ldx2, a.ldo, 4, (int)g.steps, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr,
                     g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

template hipError_t launch_gemm_bf16_lds<256, 256, 32, 4, 2, 2>(const MatmulArgs&);
template hipError_t launch_gemm_bf16_lds<256, 256, 64, 2, 2, 4>(const MatmulArgs&);
template hipError_t launch_gemm_bf16_lds<256, 128, 64, 3, 4, 2>(const MatmulArgs&);
template hipError_t launch_gemm_bf16_lds<256, 128, 32, 4, 2, 2>(const MatmulArgs&);
template hipError_t launch_gemm_bf16_lds<128, 128, 64, 4, 2, 4>(const MatmulArgs&);

}  // namespace tilec
