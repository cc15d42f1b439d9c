// Row and column sums of a matrix, fp32 or bf16 in, fp32 out and accumulate:
//   axis 1:  out[r] = sum_c x[r][c]        (R outputs)
//   axis 0:  out[c] = sum_r x[r][c]        (C outputs)
// x is row-major with row stride ld; a column-major x is the row-major view
// of its transpose, so the host swaps the axis for it.
//
// This is the reduction the reference plans as `tl.sum` (README.md:88: a
// per-thread sum over register slots, a SIMD-group reduction, then a
// combine of SIMD-groups through threadgroup memory) and shows as `row_sum`
// (kernel1.py:8-15: out[r] = tl.sum(x[r, :]); `tl.ext.sum(x, axis=1)` is
// its op-level spelling).  On MI355X it is a pure HBM stream: 16-byte loads
// and VALU adds, no matrix cores.
//
// Row sums.  A row is handled by LPR lanes (a power of two the host picks
// so that each lane makes a few 16-byte loads: 1 lane for rows of up to
// 4 E elements, 64 for long rows), 64 / LPR rows per wave.  Lanes add their
// 16-byte groups into four fp32 accumulators, then the LPR lanes of a row
// meet in a butterfly of shuffles.  When there are too few rows to fill the
// chip, long rows are split across workgroups (grid y).
// Column sums.  The layout of the streaming GEMV: a workgroup owns a slab of
// 16 E columns (E = elements per 16 bytes); in each 16-row block, lane l
// (r = l / 16, q = l % 16) adds columns E q .. E q + E-1 of rows 4 r + u,
// u < 4, and waves take interleaved blocks.  The 4 row slots of a wave meet
// in shuffles, the waves in LDS.  Rows split across workgroups (grid y).
// Split reductions combine deterministically: every workgroup publishes its
// V partial sums, and the last to finish (completion counter) adds the S
// partials in split order, spread over all its threads when V is small
// (consecutive splits per group, then the groups in order), so any S costs
// about one memory round trip; it resets the counter to zero.
#include <algorithm>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;

constexpr int kWaves = 4;
constexpr int kNT = 64 * kWaves;
constexpr int kCounterStride = 64;  // uint32s between completion counters (own 256-byte line each)

__device__ __forceinline__ float load_f32_coherent(BufRsrc r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kCpolSc1));
}
__device__ __forceinline__ void store_f32_coherent(BufRsrc r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, (int)off, 0, kCpolSc1);
}
__device__ __forceinline__ float bf16_lo(int w) { return __int_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(int w) { return __int_as_float(w & (int)0xffff0000u); }

// Cross-workgroup sum of the V (<= kNT) values that threads t < V hold in
// `val`, over the S workgroups (splits) of `cell`.  Partial of split s:
// ws[(s * cells + cell) * kNT + t].  Returns true in the last workgroup to
// arrive, with the totals in `val`; false elsewhere.  `red` is kNT floats
// of LDS that the caller no longer needs.  Coherence across XCDs as in the
// GEMM combine: agent-coherent (sc1) stores and loads, a wait for the stores
// before the barrier, a relaxed agent-scope atomic for the count.
__device__ bool split_tail(float& val, int V, int split, int S, int cell, int cells, float* __restrict__ ws,
                           unsigned* __restrict__ counters, float* red, int* last_flag) {
  const int tid = threadIdx.x;
  const BufRsrc rw = make_rsrc(ws);
  const uint32_t split_stride = (uint32_t)cells * kNT;  // floats between splits
  store_f32_coherent(rw, tid < V ? 4u * ((uint32_t)split * split_stride + (uint32_t)cell * kNT + tid) : kOob, val);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid < 64) {
    unsigned prev = 0;
    if (tid == 0)
      prev = __hip_atomic_fetch_add(&counters[cell * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = (unsigned)__shfl((int)prev, 0);
    if (tid == 0) *last_flag = prev == (unsigned)(S - 1);
  }
  __syncthreads();
  if (!*last_flag) return false;
  if (tid == 0) __hip_atomic_store(&counters[cell * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int G = max(1, min(S, kNT / V));
  if (tid < V * G) {
    const int i = tid % V, g = tid / V;
    const int s_beg = (int)((int64_t)g * S / G), s_end = (int)((int64_t)(g + 1) * S / G);
    const uint32_t at = (uint32_t)cell * kNT + i;
    float t = 0.f;
    for (int s0 = s_beg; s0 < s_end; s0 += 8) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        p[j] = load_f32_coherent(rw, s0 + j < s_end ? 4u * ((uint32_t)(s0 + j) * split_stride + at) : kOob);
#pragma unroll
      for (int j = 0; j < 8; ++j) t += p[j];
    }
    red[tid] = t;
  }
  __syncthreads();
  if (tid < V) {
    float t = red[tid];
    for (int g = 1; g < G; ++g) t += red[g * V + tid];
    val = t;
  }
  return true;
}

// The 16-byte group of E elements at element c of the row `rs` is based at,
// raw (bf16 as pairs, low half first): elements at or past n load zeros.
// VEC: n and c are multiples of E, one 16-byte load; otherwise element by
// element.
// The matrix is read once: loads carry the non-temporal cache policy.
constexpr int kCpolNt = 2;
template <typename T, bool VEC>
__device__ __forceinline__ i32x4 load_group(const BufRsrc& rs, uint32_t row_off, int c, int n) {
  constexpr int E = 16 / (int)sizeof(T);
  constexpr uint32_t EB = sizeof(T);
  if constexpr (VEC) {
    const uint32_t off = c < n ? row_off + (uint32_t)c * EB : kOob;
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, kCpolNt));
  } else {
    int h[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t off = c + e < n ? row_off + (uint32_t)(c + e) * EB : kOob;
      if constexpr (E == 4) h[e] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, kCpolNt);
      else h[e] = (int)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, kCpolNt);
    }
    i32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = E == 4 ? h[i] : (h[2 * i] | (h[2 * i + 1] << 16));
    return w;
  }
}

// Element e of a raw group as fp32.  (The vector element goes through a
// value: __builtin_bit_cast of a vector-element lvalue reads element 0.)
template <typename T>
__device__ __forceinline__ float elem(const i32x4& w, int e) {
  if constexpr (sizeof(T) == 4) return __int_as_float(w[e]);
  else return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
}

// Grid: x = groups of kWaves * 64 / lpr rows, y = column splits of `chunk`
// columns (a multiple of 64 E).  U: 16-byte groups in flight per lane (16
// for long rows, whose workgroup then reads 64 KiB of x at once).
template <typename T, bool VEC, int U>
__global__ __launch_bounds__(kNT) void row_sum_kernel(const T* __restrict__ x, float* __restrict__ out, int R, int C,
                                                      int64_t ld, int lpr, int chunk, float* __restrict__ ws,
                                                      unsigned* __restrict__ counters) {
  constexpr int E = 16 / (int)sizeof(T);
  __shared__ float red[kNT];
  __shared__ int last_flag;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int rpw = 64 / lpr, rpg = kWaves * rpw;
  const int slot = wave * rpw + lane / lpr;  // row within the workgroup
  const int sub = lane & (lpr - 1);
  const int r = blockIdx.x * rpg + slot;
  const int split = blockIdx.y, S = gridDim.y;
  const int cbeg = split * chunk;
  const int n = r < R ? max(0, min(C, cbeg + chunk) - cbeg) : 0;  // this split's columns of the row
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // One resource per wave, at its first row (buffer resources are
  // wave-uniform); a lane's row is a byte offset from it.
  const BufRsrc rs = make_rsrc(x + (int64_t)(blockIdx.x * rpg + wave * rpw) * ld + cbeg);
  const uint32_t row_off = (uint32_t)(lane / lpr) * (uint32_t)ld * (uint32_t)sizeof(T);
  const int step = E * lpr;
  for (int c0 = E * sub; c0 < n; c0 += U * step) {
    i32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = load_group<T, VEC>(rs, row_off, c0 + u * step, n);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e & 3] += elem<T>(w[u], e);
  }
  float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  for (int o = lpr >> 1; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (S == 1) {
    if (sub == 0 && r < R) out[r] = s;
    return;
  }
  // Split columns: this workgroup's rpg row partials go through the tail.
  if (sub == 0) red[slot] = s;
  __syncthreads();
  float v = tid < rpg ? red[tid] : 0.f;
  __syncthreads();  // red is the tail's scratch from here on
  if (split_tail(v, rpg, split, S, blockIdx.x, gridDim.x, ws, counters, red, &last_flag)) {
    const int rr = blockIdx.x * rpg + tid;
    if (tid < rpg && rr < R) out[rr] = v;
  }
}

// Grid: x = slabs of 16 E columns, y = row splits of kc rows (a multiple of 16).
template <typename T, bool VEC>
__global__ __launch_bounds__(kNT) void col_sum_kernel(const T* __restrict__ x, float* __restrict__ out, int R, int C,
                                                      int64_t ld, int kc, float* __restrict__ ws,
                                                      unsigned* __restrict__ counters) {
  constexpr int E = 16 / (int)sizeof(T);
  constexpr int SLAB = 16 * E;
  constexpr int UB = 2;  // 16-row blocks in flight per wave: 4 UB groups per lane
  __shared__ float red[kWaves * SLAB > kNT ? kWaves * SLAB : kNT];
  __shared__ int last_flag;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int r4 = lane >> 4, q = lane & 15;
  const int slab = blockIdx.x, split = blockIdx.y, S = gridDim.y;
  const int n0 = slab * SLAB;
  const int rbeg = split * kc;
  const int nrows = max(0, min(R, rbeg + kc) - rbeg);
  const int nblocks = (nrows + 15) / 16;
  // This lane's group: columns n0 + E q .. + E-1 of each row it adds; the
  // loader sees the row from n0 + E q, so `cn` columns of it are in x.
  const int cn = C - (n0 + E * q);
  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  for (int b0 = wave; b0 < nblocks; b0 += kWaves * UB) {
    i32x4 w[UB][4];
#pragma unroll
    for (int j = 0; j < UB; ++j) {
      const int b = b0 + j * kWaves;  // may be past the split: its rows load nothing
      // One resource per wave and block, at the block's first row and the
      // slab's first column (wave-uniform); a lane's row and columns are a
      // byte offset from it.  Rows past the split get n = 0.
      const BufRsrc rs = make_rsrc(x + (int64_t)(rbeg + min(16 * b, nrows)) * ld + n0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int row = 4 * r4 + u;  // within the block
        const bool ok = 16 * b + row < nrows;
        const uint32_t off = ((uint32_t)row * (uint32_t)ld + (uint32_t)(E * q)) * (uint32_t)sizeof(T);
        w[j][u] = load_group<T, VEC>(rs, off, 0, ok ? cn : 0);
      }
    }
#pragma unroll
    for (int j = 0; j < UB; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] += elem<T>(w[j][u], e);
  }
  // The 4 row slots of the wave (lanes q, q + 16, q + 32, q + 48), then the waves.
#pragma unroll
  for (int e = 0; e < E; ++e) {
    acc[e] += __shfl_xor(acc[e], 16);
    acc[e] += __shfl_xor(acc[e], 32);
  }
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < E; ++e) red[wave * SLAB + E * q + e] = acc[e];
  }
  __syncthreads();
  float v = 0.f;
  if (tid < SLAB) {
    v = red[tid];
#pragma unroll
    for (int w2 = 1; w2 < kWaves; ++w2) v += red[w2 * SLAB + tid];
  }
  __syncthreads();  // red is the tail's scratch from here on
  if (S == 1) {
    if (tid < SLAB && n0 + tid < C) out[n0 + tid] = v;
    return;
  }
  if (split_tail(v, SLAB, split, S, slab, gridDim.x, ws, counters, red, &last_flag)) {
    if (tid < SLAB && n0 + tid < C) out[n0 + tid] = v;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side: geometry, buffers, launch.
// ---------------------------------------------------------------------------

namespace {

constexpr int kFillWgs = 512;  // about two workgroups per CU

int64_t next_pow2(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

}  // namespace

// Reduction over the rows (axis 1) or columns (axis 0) of an R x C row-major
// matrix of element size `esz`.
struct ReduceGeom {
  int64_t cells, splits, span;  // grid x, grid y, columns (axis 1) or rows (axis 0) per split
  int lpr;                      // axis 1: lanes per row
};

ReduceGeom reduce_geom(int64_t R, int64_t C, int esz, int axis) {
  const int64_t E = 16 / esz;
  ReduceGeom g{};
  if (axis == 1) {
    g.lpr = (int)std::min<int64_t>(64, next_pow2(std::max<int64_t>(1, cdiv(C, 4 * E))));
    const int64_t rpg = kWaves * (64 / g.lpr);
    g.cells = cdiv(std::max<int64_t>(R, 1), rpg);
    int64_t s = 1;
    // Too few rows to fill the chip: split long rows, each split giving every
    // lane of a row at least 8 groups.
    if (g.lpr == 64 && g.cells < kFillWgs) s = std::max<int64_t>(1, std::min(cdiv(kFillWgs, g.cells), C / (64 * E * 8)));
    const int64_t step = 64 * E;
    g.span = std::max<int64_t>(step, cdiv(cdiv(C, s), step) * step);
    g.splits = std::max<int64_t>(1, cdiv(C, g.span));
  } else {
    g.lpr = 0;
    g.cells = cdiv(std::max<int64_t>(C, 1), 16 * E);
    int64_t s = 1;
    // Too few slabs: split rows, each split giving every wave at least 4 blocks.
    if (g.cells < kFillWgs) s = std::max<int64_t>(1, std::min(cdiv(kFillWgs, g.cells), R / (16 * kWaves * 4)));
    g.span = std::max<int64_t>(16, cdiv(cdiv(R, s), 16) * 16);
    g.splits = std::max<int64_t>(1, cdiv(R, g.span));
  }
  return g;
}

size_t reduce_workspace_bytes(const ReduceGeom& g) {
  return g.splits > 1 ? (size_t)g.splits * g.cells * kNT * sizeof(float) : 0;
}
size_t reduce_counter_bytes(const ReduceGeom& g) {
  return g.splits > 1 ? (size_t)g.cells * kCounterStride * sizeof(unsigned) : 0;
}

namespace {

template <typename T, bool VEC>
hipError_t launch_reduce_t(const void* x, float* out, int64_t R, int64_t C, int64_t ld, int axis, const ReduceGeom& g,
                           float* ws, unsigned* counters, hipStream_t stream) {
  const dim3 grid((unsigned)g.cells, (unsigned)g.splits);
  if (axis == 1 && g.lpr == 64)
    hipLaunchKernelGGL((row_sum_kernel<T, VEC, 16>), grid, dim3(kNT), 0, stream, static_cast<const T*>(x), out,
                       (int)R, (int)C, ld, g.lpr, (int)g.span, ws, counters);
  else if (axis == 1)
    hipLaunchKernelGGL((row_sum_kernel<T, VEC, 4>), grid, dim3(kNT), 0, stream, static_cast<const T*>(x), out,
                       (int)R, (int)C, ld, g.lpr, (int)g.span, ws, counters);
  else
    hipLaunchKernelGGL((col_sum_kernel<T, VEC>), grid, dim3(kNT), 0, stream, static_cast<const T*>(x), out, (int)R,
                       (int)C, ld, (int)g.span, ws, counters);
  return hipGetLastError();
}

// The HBM read floor (a measurement aid): workgroup g of G reads the 16 KiB
// pieces g, g + G, g + 2G, ... of x, each lane four 16-byte non-temporal
// loads per piece, so the workgroups in flight read one moving window of
// G pieces; wave w of workgroup g writes the sum of what it read to
// sink[4 g + w] (no barrier, so no wave waits for another).  Nothing is
// combined across workgroups: the time is that of one pass over x plus the
// end of a kernel that stores something.
__global__ __launch_bounds__(kNT) void read_floor_kernel(const unsigned char* __restrict__ x, int64_t pieces,
                                                          float* __restrict__ sink) {
  constexpr uint32_t kPiece = 16384;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t p = blockIdx.x; p < pieces; p += gridDim.x) {
    const BufRsrc r = make_rsrc(x + p * kPiece, kPiece);
    f32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      v[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(16u * (threadIdx.x + kNT * u)), 0,
                                                                             kCpolNt));
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += v[u];
  }
  float t = (acc.x + acc.y) + (acc.z + acc.w);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
  if ((threadIdx.x & 63) == 0) sink[kWaves * blockIdx.x + (threadIdx.x >> 6)] = t;
}

}  // namespace

hipError_t launch_read_floor(const void* x, int64_t bytes, float* sink, int workgroups, hipStream_t stream) {
  hipLaunchKernelGGL(read_floor_kernel, dim3((unsigned)workgroups), dim3(kNT), 0, stream,
                     static_cast<const unsigned char*>(x), bytes / 16384, sink);
  return hipGetLastError();
}

// x row-major R x C with row stride ld; the caller has checked the limits.
hipError_t launch_reduce(const void* x, float* out, int64_t R, int64_t C, int64_t ld, int dtype, int axis,
                         float* ws, unsigned* counters, hipStream_t stream) {
  const int esz = dtype == TILEC_BF16 ? 2 : 4;
  const ReduceGeom g = reduce_geom(R, C, esz, axis);
  const int64_t E = 16 / esz;
  // 16-byte groups never straddle the edge of a row or of x.
  const bool vec = C % E == 0 && ld % E == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  if (g.splits <= 1) {
    ws = nullptr;
    counters = nullptr;
  }
  if (dtype == TILEC_BF16)
    return vec ? launch_reduce_t<u16, true>(x, out, R, C, ld, axis, g, ws, counters, stream)
               : launch_reduce_t<u16, false>(x, out, R, C, ld, axis, g, ws, counters, stream);
  return vec ? launch_reduce_t<float, true>(x, out, R, C, ld, axis, g, ws, counters, stream)
             : launch_reduce_t<float, false>(x, out, R, C, ld, axis, g, ws, counters, stream);
}

}  // namespace tilec
