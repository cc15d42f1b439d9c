// fp32 GEMM for aligned operands with direct-to-LDS copies, C[M,N] =
// A[M,K] · B[K,N] (each operand row- or column-major, read in place), fp32
// accumulate on v_mfma_f32_32x32x2f32.
//
// Same tile semantics as the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24): zero accumulator, K steps over masked tiles with
// `other=0.0`, masked store.  It is the register-staged fp32 kernel of
// gemm_f32.hip with its data movement replaced:
//   * Global -> LDS with buffer_load_dwordx4 ... lds: each lane moves 16 bytes
//     (four floats) straight into LDS, so the tile copies hold no VGPRs.  The
//     8-wave 256 x 256 tile of the register-staged kernel spends 64 of its
//     256 registers per lane on two in-flight copies; here they hold a second
//     set of MFMA operands, so every k-chunk's LDS reads are issued a whole
//     chunk (32 MFMAs) before their first use.
//   * K steps of BK cycle through NBUF stage buffers (distinct LDS objects,
//     the K loop unrolled over them); the copies of step k+NBUF-1 are issued
//     among the MFMAs that open step k.
//   * Each operand lives in LDS as in memory, in 16-byte chunks.  One whose
//     memory runs along K (row-major A, column-major B) is stored in rows of
//     BK with chunk c of row r at c ^ swz(r), so the 16-byte reads of 16
//     consecutive rows (4 consecutive k of each) hit distinct banks.  One
//     whose memory runs along M or N is stored in rows of k with chunk c of
//     k-row k at c ^ (8 ((k >> 2) & 1)): the two lane halves of a 4-byte read
//     take k-rows 4 apart, which the swizzle moves to opposite bank halves.
//   * The MFMAs of an 8-deep k chunk take k = 8c + 4h + e in lane half h
//     (e < 4), in the register-staged kernel's order, so both kernels give
//     bit-identical results.
//   * Masking is done on addresses: chunks past M, N or K get an out-of-range
//     buffer offset and land in LDS as zeros.  Operands must be 16-byte
//     aligned with contiguous extents and strides multiples of 4 (the
//     launcher checks; other shapes run the register-staged kernel).
//   * XCD-aware grouped tile order (tile_of in common.h).
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// How one operand's tile (R rows of its outer dimension — M for A, N for B —
// by BK of K) sits in a stage buffer, in 16-byte chunks of four floats.
//   KC (k contiguous in memory): R rows of BK floats, chunk c of row r at
//     c ^ swz(r); a lane's four consecutive k of one row are one 16-byte read.
//   otherwise: BK rows of R floats, chunk c of k-row k at c ^ swz(k); an MFMA
//     operand is one 4-byte read.
template <int R, int BK, int NW, bool KC>
struct StageF {
  static constexpr bool kKC = KC;
  static constexpr int ROW_CHUNKS = KC ? BK / 4 : R / 4;  // 16-byte chunks per stored row
  static constexpr int ROW_BYTES = 16 * ROW_CHUNKS;
  static constexpr int CHUNKS = R * BK / 4;
  static constexpr int INSTR = CHUNKS / 64 / NW;  // DMA instructions per wave per step
  static constexpr int BYTES = R * BK * 4;
  static_assert(CHUNKS % (64 * NW) == 0, "DMA must divide evenly");
  static_assert(KC ? (BK == 64 || BK == 32 || BK == 16) : (R % 64 == 0), "swizzles cover these row widths");
  // 256-byte rows (BK = 64) each span all 64 banks, so r & 15 gives 16
  // consecutive rows 16 different chunks; 128-byte rows (BK = 32): rows r and
  // r + 2 share a bank line position, so (r >> 1) & 7 spreads 16 rows over 8
  // chunks of each bank half; 64-byte rows (BK = 16): (r >> 2) & 3.  Rows of
  // k: bit 3 of the chunk index.
  __device__ __forceinline__ static int swz(int row) {
    if constexpr (KC) return BK == 64 ? row & 15 : BK == 32 ? (row >> 1) & 7 : (row >> 2) & 3;
    else return ((row >> 2) & 1) << 3;
  }
  // Stored row and logical chunk of physical chunk p.
  __device__ __forceinline__ static void chunk(int p, int& row, int& lc) {
    row = p / ROW_CHUNKS;
    lc = (p % ROW_CHUNKS) ^ swz(row);
  }
};

template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB>
struct LdsGemmF32 {
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  using SA = StageF<BM, BK, NW, !CA>;
  using SB = StageF<BN, BK, NW, CB>;
  static constexpr int A_INSTR = SA::INSTR, B_INSTR = SB::INSTR;
  static constexpr int IPS = A_INSTR + B_INSTR;
  static constexpr int A_BYTES = SA::BYTES;
  static constexpr int STAGE_BYTES = SA::BYTES + SB::BYTES;
  static constexpr int KS = BK / 8;  // 8-deep k chunks per step
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(KS % 2 == 0, "chunks alternate between two operand sets");
  static_assert(NBUF >= 2 && NBUF <= 3, "ring of 2..3 stage buffers");
  static_assert((size_t)NBUF * STAGE_BYTES <= 160 * 1024, "LDS is 160 KiB");
  static_assert((NBUF - 2) * IPS <= 63, "vmcnt is 6 bits");
};

// Barrier between K steps without the memory fence of __syncthreads: the
// wait before it (vmcnt(WAIT) lgkmcnt(0)) already completes this wave's
// copies of the next step and its reads of the slot the next copies reuse;
// a workgroup fence would in addition wait for every copy in flight.  The
// empty asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void step_barrier_f32() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Scheduling groups "1 MFMA, then its share of the IPS copies", NM times.
template <int NM, int IPS, int X = 0>
__device__ __forceinline__ void sched_mfma_copies() {
  if constexpr (X < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int n = (X + 1) * IPS / NM - X * IPS / NM;
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x020, n, 0);
    sched_mfma_copies<NM, IPS, X + 1>();
  }
}

template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool KFULL, bool CA, bool CB>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_f32_lds_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int xcds, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = LdsGemmF32<BM, BN, BK, NBUF, WM, WN, CA, CB>;
  using SA = typename P::SA;
  using SB = typename P::SB;
  constexpr int KS = P::KS;
  __shared__ int last_flag;
  __shared__ __align__(16) char lds0[P::STAGE_BYTES];
  __shared__ __align__(16) char lds1[P::STAGE_BYTES];
  __shared__ __align__(16) char lds2[NBUF > 2 ? P::STAGE_BYTES : 16];
  auto buf = [&](auto I) -> char* {
    constexpr int i = decltype(I)::value;
    if constexpr (i == 0) return lds0;
    else if constexpr (i == 1) return lds1;
    else return lds2;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, xcds, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int split = blockIdx.y, S = gridDim.y;
  const int kt0 = split * split_steps;
  const int nk = max(0, min((K + BK - 1) / BK, kt0 + split_steps) - kt0);

  // ---- global -> LDS for K step kt (local: absolute step kt0 + kt) ----------
  // Instruction i of this wave fills physical chunks [64 * (wave * INSTR + i),
  // +64), lane l the l-th of them.  A lane's byte offset from the step's base
  // is the same in every step; chunks past M or N get kOob once, here.  A
  // step past this workgroup's range gets a resource of zero records.  When
  // K % BK != 0 (!KFULL) the last step also masks K: per lane for a
  // k-contiguous operand (its chunk's k column), by the resource's size for
  // the other kind (whole stored rows of K).
  uint32_t off_a[P::A_INSTR], off_b[P::B_INSTR];
  auto kcol = [&](auto st, int i) {
    using T = decltype(st);
    int row, lc;
    T::chunk(64 * (wave * T::INSTR + i) + lane, row, lc);
    return 4 * lc;
  };
#pragma unroll
  for (int i = 0; i < P::A_INSTR; ++i) {
    int row, lc;
    SA::chunk(64 * (wave * P::A_INSTR + i) + lane, row, lc);
    const bool in = CA ? m0 + 4 * lc < M : m0 + row < M;  // stored row = k (CA) or m
    off_a[i] = in ? 4u * ((uint32_t)row * (uint32_t)lda + 4u * lc) : kOob;
  }
#pragma unroll
  for (int i = 0; i < P::B_INSTR; ++i) {
    int row, lc;
    SB::chunk(64 * (wave * P::B_INSTR + i) + lane, row, lc);
    const bool in = CB ? n0 + row < N : n0 + 4 * lc < N;  // stored row = n (CB) or k
    off_b[i] = in ? 4u * ((uint32_t)row * (uint32_t)ldb + 4u * lc) : kOob;
  }
  auto op_rsrc = [&](const float* X, int64_t ld, int r0, bool kcontig, int k0, bool live) {
    const float* base = kcontig ? X + (int64_t)r0 * ld + k0 : X + (int64_t)k0 * ld + r0;
    uint32_t recs = live ? 0x7FFFFFFFu : 0u;
    if (!KFULL && !kcontig && live) recs = (uint32_t)min<int64_t>((int64_t)(K - k0) * ld * 4, 0x7FFFFFFF);
    return make_rsrc_uniform(base, recs);
  };
  auto dma_one = [&](int q, int kt, char* st) __attribute__((always_inline)) {
    const int k0 = (kt0 + kt) * BK;
    const bool live = kt < nk;
    if (q < P::A_INSTR) {
      const BufRsrc ra = op_rsrc(A, lda, m0, !CA, k0, live);
      uint32_t off = off_a[q];
      if constexpr (!KFULL && !CA) off = k0 + kcol(SA{}, q) < K ? off : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + 16 * 64 * (wave * P::A_INSTR + q)), 16, off, 0,
                                               0, 0);
    } else {
      const int i = q - P::A_INSTR;
      const BufRsrc rb = op_rsrc(B, ldb, n0, CB, k0, live);
      uint32_t off = off_b[i];
      if constexpr (!KFULL && CB) off = k0 + kcol(SB{}, i) < K ? off : kOob;
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

  // Operands of one 8-deep k chunk c: lane (row / column l % 32 of each
  // 32-block, half h = l / 32) holds k = 8c + 4h + e in element e.
  //   k-contiguous stage: logical chunk 2c + h of its row, one 16-byte read;
  //   other kind: four 4-byte reads of k-rows 8c + 4h + e, whose swizzle is
  //   8h for every c and e, so each read is the lane's offset (computed
  //   once, kept opaque so the compiler's per-object LDS alias scopes reach
  //   every read) plus a constant.
  const int h = lane >> 5;
  int a_r[P::TM], b_r[P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) a_r[i] = wm * P::WTM + 32 * i + (lane & 31);
#pragma unroll
  for (int j = 0; j < P::TN; ++j) b_r[j] = wn * P::WTN + 32 * j + (lane & 31);
  auto rc_off = [&](auto st_t, int r) -> uint32_t {
    using T = decltype(st_t);
    return (uint32_t)(4 * h * T::ROW_BYTES + 16 * ((r >> 2) ^ (h << 3)) + 4 * (r & 3));
  };
  uint32_t ro_a[P::TM], ro_b[P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) {
    ro_a[i] = SA::kKC ? 0u : rc_off(SA{}, a_r[i]);
    asm volatile("" : "+v"(ro_a[i]));
  }
#pragma unroll
  for (int j = 0; j < P::TN; ++j) {
    ro_b[j] = SB::kKC ? 0u : (uint32_t)P::A_BYTES + rc_off(SB{}, b_r[j]);
    asm volatile("" : "+v"(ro_b[j]));
  }
  // kc stage: `area` is the operand's area, r its row.  Other kind: `area` is
  // the stage base, `off` the lane's offset from ro_a / ro_b.
  auto frag = [&](auto st_t, const char* area, int r, uint32_t off, int c) __attribute__((always_inline)) -> f32x4 {
    using T = decltype(st_t);
    if constexpr (T::kKC) {
      const int ch = 2 * c + h;
      return *reinterpret_cast<const f32x4*>(area + 16 * (r * T::ROW_CHUNKS + (ch ^ T::swz(r))));
    } else {
      const char* p = area + off;
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = *reinterpret_cast<const float*>(p + T::ROW_BYTES * (8 * c + e));
      return v;
    }
  };
  struct Frag {
    f32x4 a[P::TM], b[P::TN];
  };
  auto read = [&](const char* st, int c, Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::TM; ++i) f.a[i] = frag(SA{}, st, a_r[i], ro_a[i], c);
#pragma unroll
    for (int j = 0; j < P::TN; ++j) f.b[j] = frag(SB{}, SB::kKC ? st + P::A_BYTES : st, b_r[j], ro_b[j], c);
  };
  auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x2(f.a[i][e], f.b[j][e], acc[i][j]);
  };
  // The MFMAs of f with the copies of step kt threaded between them.
  auto mma_dma = [&](const Frag& f, int kt, char* st) __attribute__((always_inline)) {
    constexpr int NM = 4 * P::TM * P::TN;
#pragma unroll
    for (int x = 0; x < NM; ++x) {
      const int e = x / (P::TM * P::TN), i = (x / P::TN) % P::TM, j = x % P::TN;
      acc[i][j] = mfma32x32x2(f.a[i][e], f.b[j][e], acc[i][j]);
#pragma unroll
      for (int q = x * P::IPS / NM; q < (x + 1) * P::IPS / NM; ++q) dma_one(q, kt, st);
    }
    sched_mfma_copies<NM, P::IPS>();
  };

  // Software pipeline over K steps (as in the bf16 LDS kernel).  Entering
  // step kt (ring slot I): f[0] holds (or is loading) chunk 0 of step kt;
  // f[1] holds the last chunk of step kt-1, whose MFMAs have not been issued
  // (zeros before step 0).  Step kt:
  //   1. MFMAs of f[1], threaded with the copies of step kt+NBUF-1 into the
  //      slot step kt-1 used (every wave finished reading it before the last
  //      barrier);
  //   2. chunks 0 .. KS-2 of step kt, each one's MFMAs overlapping the LDS
  //      reads of the next; the last chunk is read into f[1];
  //   3. wait for those reads and for this wave's copies of step kt+1, then
  //      the barrier: step kt+1 is in LDS for every wave;
  //   4. read chunk 0 of step kt+1 into f[0].
  Frag f[2];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) f[1].a[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < P::TN; ++j) f[1].b[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int WAIT = (NBUF - 2) * P::IPS;
  auto step = [&](auto I, int kt) __attribute__((always_inline)) {
    constexpr int i = decltype(I)::value;
    char* const cur = buf(I);
    mma_dma(f[1], kt + NBUF - 1, buf(std::integral_constant<int, (i + NBUF - 1) % NBUF>{}));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c + 1 < KS; ++c) {
      read(cur, c + 1, f[(c + 1) & 1]);
      mma(f[c & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((WAIT & 15) | ((WAIT >> 4) << 14) | (7 << 4));
    step_barrier_f32();
    read(buf(std::integral_constant<int, (i + 1) % NBUF>{}), 0, f[0]);
    __builtin_amdgcn_sched_barrier(0);
  };

  if (nk > 0) {
    dma(0, lds0);
    if constexpr (NBUF > 2) dma(1, lds1);
    __builtin_amdgcn_s_waitcnt((WAIT & 15) | ((WAIT >> 4) << 14) | (7 << 4) | (15 << 8));
    step_barrier_f32();
    read(lds0, 0, f[0]);
  }
  int kt = 0;
  for (; kt + NBUF <= nk; kt += NBUF) {
    step(std::integral_constant<int, 0>{}, kt);
    step(std::integral_constant<int, 1>{}, kt + 1);
    if constexpr (NBUF > 2) step(std::integral_constant<int, 2>{}, kt + 2);
  }
  if (kt < nk) step(std::integral_constant<int, 0>{}, kt);
  if constexpr (NBUF > 2) {
    if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
  }
  mma(f[1]);  // last chunk of the last step (zeros if K == 0)
  // Copies issued for steps past K still write (zeros) into LDS: let them
  // land before this workgroup can finish and release its LDS.
  __builtin_amdgcn_s_waitcnt(0);

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

// Launch the LDS-DMA fp32 kernel; the caller has checked alignment (16-byte
// operands, contiguous extents and strides multiples of 4) and the 32-bit
// offset limits.
template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB>
hipError_t launch_gemm_f32_lds(const MatmulArgs& a) {
  using P = LdsGemmF32<BM, BN, BK, NBUF, WM, WN, CA, CB>;
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * 16 > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  auto kern = a.K % BK == 0 ? gemm_f32_lds_kernel<BM, BN, BK, NBUF, WM, WN, true, CA, CB>
                            : gemm_f32_lds_kernel<BM, BN, BK, NBUF, WM, WN, false, CA, CB>;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)g.splits), dim3(P::NT), 0, a.stream,
                     static_cast<const float*>(a.x1), static_cast<const float*>(a.x2), a.out, (int)a.M, (int)a.N,
                     (int)a.K, a.ldx1, a.ldx2, a.ldo, 8, device_xcds(), (int)g.steps,
                     g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr, g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

#define TILEC_F32_LDS_VARIANT(BM, BN, BK, NBUF, WM, WN)                                           \
  template hipError_t launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, false, false>(const MatmulArgs&); \
  template hipError_t launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, true, false>(const MatmulArgs&);  \
  template hipError_t launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, false, true>(const MatmulArgs&);  \
  template hipError_t launch_gemm_f32_lds<BM, BN, BK, NBUF, WM, WN, true, true>(const MatmulArgs&);
TILEC_F32_LDS_VARIANT(256, 256, 32, 2, 2, 4)
TILEC_F32_LDS_VARIANT(128, 128, 32, 3, 2, 4)
TILEC_F32_LDS_VARIANT(128, 128, 64, 2, 2, 4)
TILEC_F32_LDS_VARIANT(64, 64, 32, 3, 2, 2)
TILEC_F32_LDS_VARIANT(64, 64, 64, 3, 2, 2)
#undef TILEC_F32_LDS_VARIANT

}  // namespace tilec
