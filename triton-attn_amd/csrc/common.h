// Shared device helpers for the tattn gfx950 kernels.
//
// MFMA shapes (lane layouts checked on an MI355X):
//   v_mfma_f32_32x32x16_f16  A[32][16] B[16][32] C[32][32]: 8 halves per lane per operand
//   v_mfma_f32_32x32x2f32    A[32][2]  B[2][32]  C[32][32]: 1 float per lane per operand
// With KPL = k values per lane (8 or 1) and h = lane / 32:
//   A operand : lane holds A[m = lane % 32][k = KPL*h + i], i < KPL
//   B operand : lane holds B[k = KPL*h + i][n = lane % 32]
//   C / D     : lane holds C[m = 8*(r/4) + 4*h + r%4][n = lane % 32], r < 16
// Every kernel keeps "the lane owns one row of the softmax" by putting the query (or key)
// index on n, so row reductions stay inside a lane plus one swap with lane ^ 32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tattn {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define TATTN_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;

// Element-type traits: MFMA operand type and instruction.
template <typename T> struct Elt;

template <> struct Elt<f16> {
  static constexpr int KPL = 8;  // k values per lane in one MFMA operand
  typedef f16x8 Op;
  static __device__ __forceinline__ f32x16 mfma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ Op zero() { return Op{}; }
};

template <> struct Elt<float> {
  static constexpr int KPL = 1;
  typedef float Op;
  static __device__ __forceinline__ f32x16 mfma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ Op zero() { return 0.0f; }
};

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_workitem_id_x() & 63; }

// v_permlane32_swap(x, x) returns, in its two results, {x[lane % 32], x[lane % 32 + 32]} (in
// some order) on every lane; a symmetric combine of the two gives the row value of both
// lane-halves without going through LDS.
__device__ __forceinline__ f32x2 both_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                            __builtin_bit_cast(uint32_t, x), false, false);
  return f32x2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ float max_halves(float x) {
  const f32x2 p = both_halves(x);
  return __builtin_fmaxf(p[0], p[1]);
}
__device__ __forceinline__ float sum_halves(float x) {
  const f32x2 p = both_halves(x);
  return p[0] + p[1];
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Round-to-nearest-even pack of two floats to halves (v_cvt_pk_f16_f32).
__device__ __forceinline__ f16x2 pack_f16(float a, float b) {
  return f16x2{(f16)a, (f16)b};
}

// Key permutation inside a 32-row tile: swaps bits 2 and 3 of the row index. Storing key r of
// a tile at LDS row perm32(r) makes the MFMA C layout hand every lane-half 8 consecutive keys
// per 16-key slice: C register r of lane-half h then holds key kappa(r, h).
__device__ __host__ __forceinline__ constexpr int perm32(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}
__device__ __host__ __forceinline__ constexpr int kappa(int r, int h) {
  return (r >> 3) * 16 + 8 * h + (r & 7);
}

// 16-byte global load / store helpers (addresses are 16-byte aligned by construction).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element (i % 4) of the
// 8-byte rows addressed by lanes (i / 4) + 4t of its group, t = 0..3. Addressing lane s of a
// group at row (k0 + s/4), column (n0 + 4*(s%4)) of a row-major [k][n] half matrix hands lane i
// the column n0 + i at rows k0..k0+3: a transposed read.
__device__ __forceinline__ f16x4 lds_read_tr(const TATTN_LDS char* p) {
  i16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TATTN_LDS i16x4*)(p));
  return __builtin_bit_cast(f16x4, t);
}

struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* m;
  int64_t sq[3], sk[3], sv[3], so[3];  // (z, h, n) strides in elements; d stride is 1
  int32_t Z, H, N;
  int32_t n_qblocks;
  float c;  // sm_scale * log2(e)
};

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  const float* m;
  float* delta;
  int64_t s[3];  // shared (z, h, n) strides in elements; d stride is 1
  int32_t Z, H, N;
  int32_t n_blocks;
  float c;      // sm_scale * log2(e)
  float scale;  // sm_scale
};

}  // namespace tattn
