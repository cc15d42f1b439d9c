// Shared definitions for the gfx950 matmul kernels: vector types, MFMA
// wrappers, launch arguments, the variant table entry and the XCD-aware
// workgroup → output-tile mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

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
};

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
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format

__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t num_records = 0x7FFFFFFFu) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_records, kRsrcWord3);
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

// ---------------------------------------------------------------------------
// Workgroup id -> output tile.
// The dispatcher hands workgroups to the 8 XCDs round-robin (id i runs on
// XCD i % 8) and every XCD has its own L2.  First renumber ids so that each
// XCD owns one contiguous range of "logical" ids (a bijection on [0, T) for
// any T), then walk tiles in groups of `group_m` tile-rows so the tiles an
// XCD runs at the same time share A row-panels and B column-panels in its L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int group_m,
                                        int& tm, int& tn) {
  const int T = tiles_m * tiles_n;
  const int xcd = bid & 7;
  const int pos = bid >> 3;
  const int q = T >> 3, rem = T & 7;
  const int lid = xcd * q + (xcd < rem ? xcd : rem) + pos;
  const int per_group = group_m * tiles_n;
  const int g = lid / per_group;
  const int first_m = g * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in_g = lid - g * per_group;
  tm = first_m + in_g % gsize;
  tn = in_g / gsize;
}

}  // namespace tilec
