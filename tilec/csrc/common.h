// Shared definitions for the gfx950 matmul kernels: vector types, MFMA
// wrappers, launch arguments, the variant table entry and the XCD-aware
// workgroup → output-tile mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>

namespace tilec {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Everything a launcher needs; filled by the C ABI after validation.
struct MatmulArgs {
  const void* x1;
  const void* x2;
  float* out;
  int64_t M, N, K;
  int64_t ldx1, ldx2, ldo;
  int layout;            // TILEC_X1_COL_MAJOR | TILEC_X2_COL_MAJOR bits
  int split_k;           // resolved (>= 1)
  void* workspace;       // split-K partial sums (scratch)
  size_t workspace_bytes;
  unsigned* counters;    // zero-initialised completion counters, left zero
  size_t counter_bytes;
  hipStream_t stream;
};

struct VariantDesc {
  const char* name;
  int family;  // TILEC_FAMILY_*
  int dtype;   // TILEC_F32 / TILEC_BF16
  int bm, bn, bk;
  int waves;
  int max_m;   // 0 = unbounded
  int unroll;
  // Launch on args.stream; returns hipError_t.
  hipError_t (*launch)(const MatmulArgs&);
  // 1: the launch first copies each operand that is not k-contiguous into
  // the workspace transposed (prep_workspace_bytes), then runs the tile GEMM
  // on k-contiguous operands; such variants never split K.
  int prep = 0;
  // Scratch sizes of a split K (nullptr: the family's own rule).
  size_t (*workspace_bytes)(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) = nullptr;
  size_t (*counter_bytes)(const VariantDesc& d, int64_t M, int64_t N, int64_t K, int split_k) = nullptr;
  // Workgroups per CU an automatic split aims for (streaming family).
  int wgs_per_cu = 2;
  // Set for variants whose own kernel needs no split-K scratch but which run
  // a splitting fallback for operands it does not take (the row-dot and
  // row-tile kernels): true when a call runs the variant's own kernel.  The
  // size queries cannot see pointers, so they stay conservative.
  bool (*own_kernel_runs)(const MatmulArgs&) = nullptr;
  // Split count a variant's own kernel runs for a requested split (nullptr:
  // the family's own rule); checked against the grid's 65535 limit.
  int64_t (*effective_splits)(const VariantDesc& d, int64_t N, int64_t K, int split_k) = nullptr;
};

// Workspace of a prep variant: a transposed copy of x1 (M x K) and of x2
// (K x N), bf16, each at a 256-byte aligned offset (whichever the layout
// needs; sized for both).
inline size_t prep_offset_b(int64_t M, int64_t K) { return (size_t)((M * K * 2 + 255) / 256 * 256); }
inline size_t prep_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return prep_offset_b(M, K) + (size_t)((K * N * 2 + 255) / 256 * 256);
}

// ---------------------------------------------------------------------------
// MFMA wrappers.  Lane layouts (lane l of 64):
//   16x16x4 f32 : A[i=l%16][k=l/16], B[k=l/16][j=l%16],
//                 D reg r -> D[i=4*(l/16)+r][j=l%16]
//   32x32x2 f32 : A[i=l%32][k=l/32], B[k=l/32][j=l%32],
//                 D reg r -> D[i=8*(r/4)+4*(l/32)+r%4][j=l%32]
//   32x32x16 bf16: A[i=l%32][k=8*(l/32)+0..7], B[k=8*(l/32)+0..7][j=l%32],
//                 D as 32x32x2
//   16x16x32 bf16: A[i=l%16][k=8*(l/16)+0..7], B[k=8*(l/16)+0..7][j=l%16],
//                 D as 16x16x4
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// 16x16x16 bf16: lane l holds A[l % 16][4 (l / 16) + j] and B[4 (l / 16) + j][l % 16]
// for j < 4 (element j in half j % 2 of dword j / 2).
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma16x16x16bf16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Raw buffer loads.  A load whose byte offset is >= the resource's
// num_records returns zeros without touching memory; kernels pass kOob as the
// offset of a masked element instead of selecting on the loaded value.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr uint32_t kOob = 0x80000000u;
// kOob when !ok, else 0: or-ed into an offset below 2^31 it masks the access
// with no select (a select around the offset's arithmetic can become a
// branch).
__device__ __forceinline__ uint32_t oob_unless(bool ok) { return (uint32_t)!ok << 31; }
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format

__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t num_records = 0x7FFFFFFFu) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_records, kRsrcWord3);
}
// make_rsrc for a base and extent the caller knows to be wave-uniform: both
// pass through readfirstlane, so the resource is built in scalar registers
// even where the compiler cannot prove uniformity itself (a divergent-looking
// resource makes it wrap each buffer instruction in a waterfall loop).
__device__ __forceinline__ BufRsrc make_rsrc_uniform(const void* base, uint32_t num_records) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  const uint32_t n = (uint32_t)__builtin_amdgcn_readfirstlane((int)num_records);
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), n);
}
__device__ __forceinline__ float load_f32(BufRsrc r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ f32x4 load_f32x4(BufRsrc r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// Agent-coherent (sc1) accesses: the cache policy of agent-scope atomic loads
// and stores, for data that workgroups on different XCDs exchange.
constexpr int kCpolSc1 = 16;
__device__ __forceinline__ f32x4 load_f32x4_coherent(BufRsrc r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCpolSc1));
}
__device__ __forceinline__ void store_f32x4_coherent(BufRsrc r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, (int)off, 0, kCpolSc1);
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// XCDs of the current device (MI355X: 8; fewer in a partitioned mode), read
// once per device; 8 if the query fails.
inline int device_xcds() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 8;
  if (dev >= 0 && dev < kMaxDev) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int x = 0;
  if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x <= 0) x = 8;
  if (dev >= 0 && dev < kMaxDev) cache[dev].store(x, std::memory_order_relaxed);
  return x;
}

// Kernels with more than 64 KiB of dynamic LDS need their limit raised once
// per device (the attribute belongs to the kernel on the current device).
// `done` is the caller's per-kernel record of devices already set up
// (devices 0..63; others are set on every launch).
inline hipError_t raise_lds_limit(const void* kernel, size_t lds, std::atomic<uint64_t>& done) {
  if (lds <= 65536) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? uint64_t(1) << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// ---------------------------------------------------------------------------
// Split-K combine for tile kernels (grid y = K splits).  Every workgroup of
// a tile holds its partial sums as NV f32x4 per thread.  It publishes them to
// `ws` in a per-thread layout — value v of thread t of split s of tile `tile`
// at float4 index ((s * tiles + tile) * NV + v) * NT + t, so each store and
// load instruction is contiguous across the workgroup — waits for the stores
// to complete, and counts itself in on the tile's counter (its own 256-byte
// line).  The workgroup that brings the count to S resets the counter, adds
// the S partials in split order (its own from registers), leaves the sums in
// `v` and returns true; the others return false.  The order of additions
// depends only on S, so results are deterministic.  Values whose `live` flag
// is false (outside the output: never stored) are neither published nor read
// back, so partial traffic scales with the valid part of a tile.  Coherence
// across XCDs without cache-wide fences: agent-coherent (sc1) data accesses,
// waits before the barrier, a relaxed agent-scope atomic for the count.  The
// host keeps S * tiles * NV * NT * 16 bytes below 2^31.
// ---------------------------------------------------------------------------
constexpr int kSplitCounterStride = 64;  // uint32s between tile counters
// Tile kernels split K only when a thread holds at most this many fp32
// accumulators: the combine keeps them, their sum and a batch of loads in
// registers (larger tiles would spill, and have enough tiles not to need it).
constexpr int kSplitMaxAccPerThread = 64;
__host__ __device__ constexpr bool tile_can_split(int bm, int bn, int waves) {
  return bm * bn <= kSplitMaxAccPerThread * 64 * waves;
}

template <int NT, int NV>
__device__ __forceinline__ bool splitk_combine(f32x4 (&v)[NV], const bool (&live)[NV], int split, int S, int tile,
                                               int tiles, float* __restrict__ ws, unsigned* __restrict__ counters,
                                               int* last_flag) {
  const uint32_t tid = threadIdx.x;
  const BufRsrc rw = make_rsrc(ws);
  auto off = [&](int s, int q) {
    return live[q] ? 16u * ((uint32_t)((s * tiles + tile) * NV + q) * NT + tid) : kOob;
  };
#pragma unroll
  for (int q = 0; q < NV; ++q) store_f32x4_coherent(rw, off(split, q), v[q]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid < 64) {
    unsigned prev = 0;
    if (tid == 0)
      prev = __hip_atomic_fetch_add(&counters[tile * kSplitCounterStride], 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    prev = (unsigned)__shfl((int)prev, 0);
    if (tid == 0) *last_flag = prev == (unsigned)(S - 1);
  }
  __syncthreads();
  if (!*last_flag) return false;
  if (tid == 0)
    __hip_atomic_store(&counters[tile * kSplitCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // CH splits per round of loads (at most 16 float4 in flight per thread).
  constexpr int CH = NV >= 16 ? 1 : 16 / NV;
  f32x4 t[NV];
#pragma unroll
  for (int q = 0; q < NV; ++q) t[q] = v[q];  // placeholder; overwritten by split 0 below
  for (int s0 = 0; s0 < S; s0 += CH) {
    f32x4 p[CH][NV];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int s = s0 + j;
      const bool load = s < S && s != split;
#pragma unroll
      for (int q = 0; q < NV; ++q) p[j][q] = load_f32x4_coherent(rw, load ? off(s, q) : kOob);
    }
    // Branch-free: an exit here would let the compiler sink each load
    // into its own guarded block and wait for them one at a time.
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int s = s0 + j;
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const f32x4 x = s == split ? v[q] : p[j][q];
        t[q] = s < S ? (s == 0 ? x : t[q] + x) : t[q];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NV; ++q) v[q] = t[q];
  return true;
}

// splitk_combine for the TM x TN blocks of 32x32 MFMA accumulators of the
// tile kernels: true (with the summed tile in acc) in the last split only.
// Block (i, j) register r of this lane is output row row_base + 32 i +
// 8 (r / 4) + r % 4, column col_base + 32 j (the 32x32 MFMA layout), so
// float4 q of a block is 4 consecutive rows of one column: live when its
// first row is below M and its column below N.
template <int TM, int TN, int NT>
__device__ __forceinline__ bool splitk_tile(f32x16 (&acc)[TM][TN], int split, int S, int tile, int tiles,
                                            float* __restrict__ ws, unsigned* __restrict__ counters,
                                            int* last_flag, int row_base, int col_base, int M, int N) {
  constexpr int NV = TM * TN * 4;
  if constexpr (TM * TN * 16 > kSplitMaxAccPerThread) {
    return true;  // never split (the host passes S == 1 for these tiles)
  } else {
  f32x4 v[NV];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[(i * TN + j) * 4 + q] =
            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
  bool live[NV];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        live[(i * TN + j) * 4 + q] = (row_base + 32 * i + 8 * q < M) & (col_base + 32 * j < N);
  if (!splitk_combine<NT, NV>(v, live, split, S, tile, tiles, ws, counters, last_flag)) return false;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][j][4 * q + c] = v[(i * TN + j) * 4 + q][c];
  return true;
  }
}

// splitk_tile for 16x16 MFMA blocks: lane l holds rows 4 (l / 16) .. +3 of
// column l % 16 of each block as one float4 (row_base and col_base are the
// lane's first row and column in block (0, 0)); live when the first of its
// rows is below M and its column below N.
template <int TM, int TN, int NT>
__device__ __forceinline__ bool splitk_tile16(f32x4 (&acc)[TM][TN], int split, int S, int tile, int tiles,
                                              float* __restrict__ ws, unsigned* __restrict__ counters,
                                              int* last_flag, int row_base, int col_base, int M, int N) {
  constexpr int NV = TM * TN;
  if constexpr (NV * 4 > kSplitMaxAccPerThread) {
    return true;  // never split (the host passes S == 1 for these tiles)
  } else {
  f32x4 v[NV];
  bool live[NV];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      v[i * TN + j] = acc[i][j];
      live[i * TN + j] = (row_base + 16 * i < M) & (col_base + 16 * j < N);
    }
  if (!splitk_combine<NT, NV>(v, live, split, S, tile, tiles, ws, counters, last_flag)) return false;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v[i * TN + j];
  return true;
  }
}

// K splits of a tile kernel: `steps` K steps of BK per split (the last may
// be shorter), `splits` = how many are non-empty.  K == 0: one empty split.
struct SplitGeom {
  int64_t splits, steps;
};
inline SplitGeom gemm_split_geom(int64_t K, int64_t BK, int split_k) {
  const int64_t total = cdiv(K, BK);
  if (total <= 0) return {1, 0};
  int64_t s = split_k < 1 ? 1 : split_k;
  if (s > total) s = total;
  const int64_t steps = cdiv(total, s);
  return {cdiv(total, steps), steps};
}

// ---------------------------------------------------------------------------
// Workgroup id -> output tile.
// The dispatcher hands workgroups to the device's XCDs round-robin (id i
// runs on XCD i % xcds; MI355X has 8, a partitioned device fewer) and every
// XCD has its own L2.  First renumber ids so that each XCD owns one
// contiguous range of "logical" ids (a bijection on [0, T) for any T), then
// walk tiles in groups of `group_m` tile-rows so the tiles an XCD runs at
// the same time share A row-panels and B column-panels in its L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tile_of(int bid, int xcds, int tiles_m, int tiles_n, int group_m,
                                        int& tm, int& tn) {
  const int T = tiles_m * tiles_n;
  const int xcd = bid % xcds;
  const int pos = bid / xcds;
  const int q = T / xcds, rem = T % xcds;
  const int lid = xcd * q + (xcd < rem ? xcd : rem) + pos;
  const int per_group = group_m * tiles_n;
  const int g = lid / per_group;
  const int first_m = g * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in_g = lid - g * per_group;
  tm = first_m + in_g % gsize;
  tn = in_g / gsize;
}

// ---------------------------------------------------------------------------
// Padding copy of the pad variants (gemm_f32.hip, gemm_bf16.hip): out (Rp x
// Cp, row stride Cp) = in (R x C, row stride ld) with zeros past R and C, for
// ESZ-byte elements at any element alignment of `in` and ld.  A thread
// writes one 16-byte chunk of an output row.  It reads the 16-byte aligned
// chunk of the input row holding the chunk's first element and, where the
// chunk's bytes run into it, the next aligned chunk, then shifts the bytes
// into place (v_alignbyte on a dword window chosen by the row's byte
// misalignment).  Every load holds at least one byte of the row it serves,
// so no access leaves that row's own 16-byte chunks: nothing past the
// matrix, no page the matrix does not touch.  Rows of 2^LG threads: narrow
// outputs pack 256 >> LG rows per workgroup.  Cp * ESZ % 16 == 0 and `out`
// is 16-byte aligned.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Bytes [b, b + 16) of the 32 bytes lo:hi (b < 16): v_alignbyte over the
// window of dwords that starts at dword b / 4.
__device__ __forceinline__ u32x4 funnel16(u32x4 lo, u32x4 hi, uint32_t b) {
  const uint32_t d[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  const uint32_t w = b >> 2, rb = b & 3;
  uint32_t e[5];
#pragma unroll
  for (int j = 0; j < 5; ++j) e[j] = w == 0 ? d[j] : w == 1 ? d[j + 1] : w == 2 ? d[j + 2] : d[j + 3];
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = __builtin_amdgcn_alignbyte(e[j + 1], e[j], rb);
  return v;
}

// v with its bytes from `keep` on cleared (keep <= 0: all of them).
__device__ __forceinline__ u32x4 keep_bytes(u32x4 v, int keep) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kb = keep - 4 * j;
    v[j] = kb >= 4 ? v[j] : kb <= 0 ? 0u : (v[j] & ((1u << (8 * kb)) - 1u));
  }
  return v;
}

// One operand of a padding copy: in (R x C, row stride ld) -> out (Rp x Cp,
// row stride Cp); rows of 2^lg threads, a gx x gy grid of workgroups.
struct PadCopyOp {
  const unsigned char* in;
  unsigned char* out;
  int64_t R, C, ld, Rp, Cp;
  int lg, gx, gy;
};

// Both operands in one launch: workgroups 0 .. gx0 gy0 - 1 copy the first,
// the rest the second (each operand its own grid, so one with few rows or
// narrow rows launches no empty workgroups for the other's shape).  At the
// sizes where the pad variants win, a second launch's fixed cost is a few
// per cent.
template <int ESZ>
__global__ __launch_bounds__(256) void pad_copy_kernel(PadCopyOp o0, PadCopyOp o1) {
  constexpr int EPC = 16 / ESZ;  // elements per 16-byte chunk
  const int n0 = o0.gx * o0.gy;
  const bool second = (int)blockIdx.x >= n0;
  const PadCopyOp& o = second ? o1 : o0;
  const int blk = (int)blockIdx.x - (second ? n0 : 0);
  const int bx = blk % o.gx, by = blk / o.gx;
  const int64_t nch = o.Cp / EPC;
  const int64_t ch = (int64_t)bx * (1 << o.lg) + (threadIdx.x & ((1 << o.lg) - 1));
  const int64_t rpb = 256 >> o.lg;  // rows per workgroup
  const int64_t c0 = ch * EPC;
  if (ch >= nch) return;
  for (int64_t r = (int64_t)by * rpb + (threadIdx.x >> o.lg); r < o.Rp; r += (int64_t)o.gy * rpb) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < o.R && c0 < o.C) {
      const uintptr_t start = reinterpret_cast<uintptr_t>(o.in) + (uintptr_t)(r * o.ld * ESZ);
      const uint32_t b = (uint32_t)(start & 15);  // the row's byte misalignment
      const uintptr_t lo = start - b + (uintptr_t)(c0 * ESZ);
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(lo);
      u32x4 a1 = {0u, 0u, 0u, 0u};
      if (b != 0 && c0 * ESZ + 16 < (int64_t)b + o.C * ESZ) a1 = *reinterpret_cast<const u32x4*>(lo + 16);
      v = funnel16(a0, a1, b);
      if (c0 + EPC > o.C) v = keep_bytes(v, (int)(o.C - c0) * ESZ);  // the row's last chunk: zero past C
    }
    *reinterpret_cast<u32x4*>(o.out + (r * o.Cp + c0) * ESZ) = v;
  }
}

// Padding copies of two operands (each: in, out, R, C, ld, Rp, Cp).
template <int ESZ>
inline hipError_t pad_copy(const void* in0, void* out0, int64_t R0, int64_t C0, int64_t ld0, int64_t Rp0, int64_t Cp0,
                           const void* in1, void* out1, int64_t R1, int64_t C1, int64_t ld1, int64_t Rp1, int64_t Cp1,
                           hipStream_t stream) {
  auto op = [](const void* in, void* out, int64_t R, int64_t C, int64_t ld, int64_t Rp, int64_t Cp) {
    PadCopyOp o{static_cast<const unsigned char*>(in), static_cast<unsigned char*>(out), R, C, ld, Rp, Cp, 0, 0, 0};
    const int64_t nch = Cp / (16 / ESZ);
    while (o.lg < 8 && (int64_t(1) << o.lg) < nch) ++o.lg;
    const int64_t rpb = 256 >> o.lg;
    const int64_t gx = (nch + (1 << o.lg) - 1) >> o.lg;
    int64_t gy = Rp > 0 && gx > 0 ? (Rp + rpb - 1) / rpb : 0;
    while (gy > 1 && gx * gy > (int64_t(1) << 29)) gy = (gy + 1) / 2;  // the row loop strides over the rest
    o.gx = (int)gx;
    o.gy = (int)gy;
    return o;
  };
  const PadCopyOp o0 = op(in0, out0, R0, C0, ld0, Rp0, Cp0), o1 = op(in1, out1, R1, C1, ld1, Rp1, Cp1);
  const int64_t blocks = (int64_t)o0.gx * o0.gy + (int64_t)o1.gx * o1.gy;
  if (blocks == 0) return hipSuccess;
  if ((int64_t)o0.gx * o0.gy >= (int64_t(1) << 30) || blocks >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pad_copy_kernel<ESZ>, dim3((unsigned)blocks), dim3(256), 0, stream, o0, o1);
  return hipGetLastError();
}

}  // namespace tilec
