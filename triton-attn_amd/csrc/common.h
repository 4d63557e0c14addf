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

#include <type_traits>

namespace tattn {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define TATTN_LDS __attribute__((address_space(3)))

template <int N> using IC = std::integral_constant<int, N>;

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

template <> struct Elt<bf16> {
  static constexpr int KPL = 8;
  typedef bf16x8 Op;
  static __device__ __forceinline__ f32x16 mfma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
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

// 16-bit element types (fp16, bf16): operand vectors, the round-to-nearest-even pack of two
// floats (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32) and the sum of a packed pair into a float
// accumulator (v_dot2 with (1, 1): exact products, one fp32 rounding).
template <typename T> struct H16;
template <> struct H16<f16> {
  typedef f16x2 V2;
  typedef f16x4 V4;
  typedef f16x8 V8;
  static __device__ __forceinline__ V2 pack(float a, float b) { return V2{(f16)a, (f16)b}; }
  static __device__ __forceinline__ float sum2(V2 x, float acc) {
    return __builtin_amdgcn_fdot2(x, V2{(f16)1.0f, (f16)1.0f}, acc, false);
  }
};
template <> struct H16<bf16> {
  typedef bf16x2 V2;
  typedef bf16x4 V4;
  typedef bf16x8 V8;
  static __device__ __forceinline__ V2 pack(float a, float b) { return V2{(bf16)a, (bf16)b}; }
  static __device__ __forceinline__ float sum2(V2 x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(x, V2{(bf16)1.0f, (bf16)1.0f}, acc, false);
  }
};

// Dot product of one 16-byte chunk of O and dO in float32: one FMA chain in element order. The
// delta preprocess and the dQ kernels that compute delta themselves both use it, and both then
// add chunk sums in the same butterfly order, so every path gives delta the same bits.
template <typename V8>
__device__ __forceinline__ float chunk_dot(V8 x, V8 y) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc = __builtin_fmaf((float)x[i], (float)y[i], acc);
  return acc;
}

// delta of a row from the chunk sums a lane holds when lane-half h2 owns chunks 2k + h2
// (k < NS) of it, in the preprocess's order: chunk sums paired CPR/2, CPR/4, ..., 1 chunks
// apart (CPR = 2 NS chunks per row), the last pair being the two lane-halves.
template <int NS>
__device__ __forceinline__ float row_delta(float (&s)[NS]) {
#pragma unroll
  for (int off = NS / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int k = 0; k < NS; ++k)
      if ((k & off) == 0 && k + off < NS) s[k] = s[k] + s[k + off];
  return sum_halves(s[0]);
}

// Forward softmax: the max used in the exponent moves only when a row's true max exceeds it by
// more than 2^kRescaleLog2 (lazy rescaling, exact in real arithmetic).
constexpr float kRescaleLog2 = 8.0f;

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
// A 16-byte store with the non-temporal cache policy, for outputs written once as whole 128-byte
// rows by the last kernel that touches them (dK, dV).
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element (i % 4) of the
// 8-byte rows addressed by lanes (i / 4) + 4t of its group, t = 0..3. Addressing lane s of a
// group at row (k0 + s/4), column (n0 + 4*(s%4)) of a row-major [k][n] half matrix hands lane i
// the column n0 + i at rows k0..k0+3: a transposed read.
__device__ __forceinline__ f16x4 lds_read_tr(const TATTN_LDS char* p) {
  i16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TATTN_LDS i16x4*)(p));
  return __builtin_bit_cast(f16x4, t);
}
template <typename T>
__device__ __forceinline__ typename H16<T>::V4 lds_tr(const TATTN_LDS char* p) {
  i16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TATTN_LDS i16x4*)(p));
  return __builtin_bit_cast(typename H16<T>::V4, t);
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
  int32_t items_x, gx;  // persistent kernel: work items per XCD, workgroups per XCD
  int32_t cus;          // persistent kernel: compute units of the device
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
  int32_t items_x, gx, cus;  // persistent kernels: items per XCD, workgroups per XCD, CUs
  int32_t fuse_delta;        // dQ computes delta from O and dO itself and stores it (no preprocess)
};

// Bytes spanned by rows [0, N) of a row-strided slice: every offset of a valid element is below
// it and every offset of row N or later is at or above it.
__host__ __device__ inline uint64_t slice_bytes(int64_t N, int64_t row_stride, int64_t D) {
  return (uint64_t)((N - 1) * row_stride + D) * 2;
}

// Value of lane 0 (for values the caller knows are wave-uniform: keeps them in scalar registers).
__device__ __forceinline__ uint32_t uniform32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}

// Range-checked buffer descriptor over rows [0, N) of one (z, h) slice: 16-byte loads at byte
// offsets at or past the slice size read as zero, so rows past the sequence end need no
// masking. Built once per workgroup from wave-uniform values (the descriptor must live in
// scalar registers; offsets vary per lane and per step).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const void* base, uint64_t bytes) {
  const uint64_t a = (uint64_t)base;
  const uint64_t ua = ((uint64_t)uniform32((uint32_t)(a >> 32)) << 32) | uniform32((uint32_t)a);
  return __builtin_amdgcn_make_buffer_rsrc((void*)ua, (short)0, (int)uniform32((uint32_t)bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 rsrc_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}


// Workgroup -> (z*H + h slice, block within the slice). Workgroups are dispatched round-robin over
// the 8 XCDs, so workgroup b runs on XCD b % 8, and each XCD has its own L2. Both orders keep a
// slice on one XCD when Z*H is a multiple of 8. grouped: the workgroups of an XCD take every block
// of one slice before the next slice, so the blocks that stream the same K/V (or Q/dO) rows run
// together and share them through that L2. Otherwise consecutive workgroups take consecutive
// slices and the blocks of a slice come one dispatch round apart, which keeps an order over block
// indices (the causal kernels' longest-first) global across the launch.
struct BlockCoord {
  int zh, blk;
};
__device__ __forceinline__ BlockCoord block_coord(int zhs, int nblk, bool grouped) {
  const int b = blockIdx.x;
  if (grouped && (zhs & 7) == 0) {
    const int l = b >> 3;
    return {(l / nblk) * 8 + (b & 7), l % nblk};
  }
  return {b % zhs, b / zhs};
}

// fp16 tiles are stored without padding, with the 16-byte chunks of row r XOR-permuted by
// swz(r). The permutation is chosen so that both access patterns of these tiles hit 64
// distinct banks per 256 bytes: 16 consecutive rows read at one chunk (natural MFMA operands,
// ds_read_b128), and 4 consecutive rows read across 4 aligned chunks (transposed operands,
// ds_read_b64_tr_b16). D=16 rows use the D=32 geometry (64 bytes, upper half unused).
template <int D>
struct Swz {
  static constexpr int RB = D < 32 ? 64 : D * 2;  // bytes per row
  static __device__ __forceinline__ int f(int r) {
    if constexpr (RB == 256) return ((r & 3) << 2) | ((r >> 2) & 3);
    else if constexpr (RB == 128) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else return (r >> 2) & 3;
  }
  // Byte address of byte `b` of row r (b < RB).
  static __device__ __forceinline__ int addr(int r, int b) { return r * RB + ((((b >> 4) ^ f(r)) << 4) | (b & 15)); }
};

}  // namespace tattn
