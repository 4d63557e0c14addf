// Backward attention kernels for gfx950: delta preprocess, dK/dV, dQ.
// Replaces src/tattn/kernels.py:151-337 (launched from src/tattn/api.py:102-146).
//
// Both GEMM kernels rebuild P = exp2(S * sm_scale * log2e - M) from the saved base-2
// log-sum-exp M (kernels.py:224, 312) and never materialise an N x N matrix. No atomics: the
// dK/dV kernel owns a block of keys and loops over queries, the dQ kernel owns a block of
// queries and loops over keys (the reference's split, kernels.py:180, 270).
//
// dK/dV, per wave (32*KTW keys, K and V resident as MFMA B operands):
//   S  = Q K^T, dP = dO V^T   (A = Q / dO rows from LDS)    C layout: lane = key
//   P  = exp2(S c - M[q]), dS = P (dP - delta[q])           M, delta per register
//   dV += P^T dO, dK += dS^T Q (A = P / dS straight from registers, B = dO / Q through
//                               transposed LDS reads)
// dQ, per wave (32*QTW queries, Q and dO resident as MFMA B operands):
//   S^T = K Q^T, dP^T = V dO^T (A = K / V rows from LDS)     C layout: lane = query
//   P^T, dS^T elementwise with per-lane M, delta
//   dQ^T += K^T dS^T          (A = K^T through transposed LDS reads, B = dS^T registers)
// P and dS are rounded to the element type only as MFMA operands (kernels.py:225, 228, 315);
// dK and dQ are scaled by sm_scale at the store (kernels.py:232, 319).
#include <type_traits>

#include <algorithm>

#include "bwd_pipe.h"
#include "common.h"
#include "launch.h"
#include "tiles.h"

namespace tattn {

// Base of row (z, h) for a flat workgroup index laid out as (block, zh) with zh fastest.
struct Head {
  int64_t off;  // element offset of (z, h)
  int64_t zh;
};
__device__ __forceinline__ Head head_of(const BwdParams& p, int zh) {
  const int64_t z = zh / p.H, h = zh % p.H;
  return Head{z * p.s[0] + h * p.s[1], zh};
}

// ---- delta = rowsum(dO * O) (kernels.py:324-337) -----------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(const BwdParams p) {
  constexpr int EPC = 16 / (int)sizeof(T), CPR = D / EPC, RPB = 256 / CPR;
  const int tid = threadIdx.x, ch = tid % CPR;
  const int nb = (p.N + RPB - 1) / RPB;
  const int zh = blockIdx.x / nb, blk = blockIdx.x % nb;
  const int row = blk * RPB + tid / CPR;
  const Head hd = head_of(p, zh);
  float acc = 0.0f;
  if (row < p.N) {
    const int64_t off = hd.off + (int64_t)row * p.s[2] + ch * EPC;
    const u32x4 a = ld16((const T*)p.o + off), b = ld16((const T*)p.dout + off);
    if constexpr (EPC == 8) {
      using V8 = typename H16<T>::V8;
      acc = chunk_dot(__builtin_bit_cast(V8, a), __builtin_bit_cast(V8, b));
    } else {
      const f32x4 x = __builtin_bit_cast(f32x4, a), y = __builtin_bit_cast(f32x4, b);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc += x[i] * y[i];
    }
  }
#pragma unroll
  for (int off = CPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (ch == 0 && row < p.N) p.delta[(int64_t)zh * p.N + row] = acc;
}

// ---- shared tile staging ----------------------------------------------------------------
// One step stages two [ROWS][D] tiles (rows in perm32 order inside each 32-row tile) and,
// through registers, the step's M and delta entries.
template <typename T, int D, int ROWS, int NT>
struct Stage2 {
  static constexpr int SZ = (int)sizeof(T);
  static constexpr int EPC = 16 / SZ;
  static constexpr int CPR = D / EPC;
  static constexpr int CHUNKS = ROWS * CPR;
  static constexpr int CPT = (CHUNKS + NT - 1) / NT;
  static constexpr int R = SZ == 2 ? Swz<D>::RB : D * SZ + 16;
  static constexpr int TILE = ROWS * R;
  u32x4 a[CPT], b[CPT];

  __device__ __forceinline__ void load(const T* A, const T* B, int64_t rs, int r0, int n, int tid) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + i * NT;
      const int row = ch / CPR, col = (ch % CPR) * EPC;
      const bool ok = (CHUNKS % NT == 0 || ch < CHUNKS) && r0 + row < n;
      const int64_t off = (int64_t)(ok ? r0 + row : 0) * rs + col;
      const u32x4 x = ld16(A + off), y = ld16(B + off);
      a[i] = ok ? x : u32x4{0, 0, 0, 0};
      b[i] = ok ? y : u32x4{0, 0, 0, 0};
    }
  }
  __device__ __forceinline__ void store(char* sa, char* sb, int tid) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + i * NT;
      if (CHUNKS % NT == 0 || ch < CHUNKS) {
        const int row = ch / CPR, cb = (ch % CPR) * 16;
        const int prow = (row & ~31) | perm32(row & 31);
        const int off = SZ == 2 ? Swz<D>::addr(prow, cb) : prow * R + cb;
        st16(sa + off, a[i]);
        st16(sb + off, b[i]);
      }
    }
  }
};

// Natural MFMA operand (16-bit types): 8 elements of LDS row `row` starting at element `col`
// (multiple of 8).
template <typename T, int D>
__device__ __forceinline__ typename H16<T>::V8 nat_operand(const char* tile, int row, int col) {
  return *reinterpret_cast<const TATTN_LDS typename H16<T>::V8*>((const TATTN_LDS char*)tile + Swz<D>::addr(row, col * 2));
}

// Transposed MFMA operand (16-bit types) from a perm32-ordered tile: k runs over the 16 rows of
// slice `sl` (row 16*sl + 8*h + i for lane-half h), m/n over columns 32*u + lane%32.
template <typename T, int D>
__device__ __forceinline__ typename H16<T>::V8 tr_operand(const char* tile, int sl, int u, int lane) {
  const int g = lane >> 4, src = lane & 15;
  const int colb = (32 * u + 16 * (g & 1) + 4 * (src & 3)) * 2;
  const int row = 16 * sl + 4 * (g >> 1) + (src >> 2);  // perm32 maps row 16sl+8h+4j+t to 16sl+8j+4h+t
  const TATTN_LDS char* base = (const TATTN_LDS char*)tile;
  const auto lo = lds_tr<T>(base + Swz<D>::addr(row, colb));
  const auto hi = lds_tr<T>(base + Swz<D>::addr(row + 8, colb));
  return typename H16<T>::V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// fp32 operand for the same role: one element per lane, row = key/query of C register r of
// the slice's tile for lane-half h, column 32*u + lane%32.
__device__ __forceinline__ float f32_operand(const char* tile, int R, int sl, int u, int lane, int D) {
  const int h = lane >> 5, d = 32 * u + (lane & 31), r = sl & 15;
  const int row = 32 * (sl >> 4) + 8 * (r >> 2) + 4 * h + (r & 3);  // perm32(kappa(r, h))
  return d < D ? *reinterpret_cast<const TATTN_LDS float*>((const TATTN_LDS char*)tile + row * R + d * 4)
               : 0.0f;
}

// ---- dK / dV (kernels.py:151-239) ----------------------------------------------------------
template <typename T, int D, int NW, int KTW, int BMQ>
struct DkdvCfg {
  static constexpr int NT = NW * 64;
  static constexpr int BNK = NW * KTW * 32;
  static constexpr int SZ = (int)sizeof(T);
  static constexpr int KPL = Elt<T>::KPL;
  static constexpr int SK = 2 * KPL;
  static constexpr int NSD = D / SK;
  static constexpr int QT = BMQ / 32;
  static constexpr int DT = (D + 31) / 32;
  static constexpr int NSQ = BMQ / SK;  // slices over the step's queries
  using St = Stage2<T, D, BMQ, NT>;
  static constexpr int STAGE = 2 * St::TILE + 2 * BMQ * 4;
  static constexpr int LDS = 2 * STAGE;
};

// OCC: waves per SIMD the register budget is sized for (1 gives 512 registers: D=128).
template <typename T, int D, int NW, int KTW, int BMQ, bool CAUSAL, int OCC>
__global__ __launch_bounds__(NW * 64, OCC) void dkdv_kernel(const BwdParams p) {
  using C = DkdvCfg<T, D, NW, KTW, BMQ>;
  using E = Elt<T>;
  using Op = typename E::Op;
  using St = typename C::St;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_blocks, !CAUSAL);
  const int zh = bc.zh, kblk_i = bc.blk;  // causal: small key blocks (most work) first
  const Head hd = head_of(p, zh);
  const T* Qg = (const T*)p.q + hd.off;
  const T* Kg = (const T*)p.k + hd.off;
  const T* Vg = (const T*)p.v + hd.off;
  const T* DOg = (const T*)p.dout + hd.off;
  const float* Mg = p.m + (int64_t)zh * N;
  const float* Dg = p.delta + (int64_t)zh * N;
  const int64_t rs = p.s[2];
  const float c = p.c;

  const int kblk = kblk_i * C::BNK;
  const int kw0 = kblk + w * KTW * 32;

  // Resident K, V as B operands: lane holds row kw0 + 32t + l32, columns KPL*h2 + SK*s + i.
  Op kop[KTW][C::NSD], vop[KTW][C::NSD];
#pragma unroll
  for (int t = 0; t < KTW; ++t) {
    const int key = kw0 + 32 * t + l32;
    const int64_t off = (int64_t)(key < N ? key : 0) * rs + C::KPL * h2;
#pragma unroll
    for (int s = 0; s < C::NSD; ++s) {
      const Op a = *reinterpret_cast<const Op*>(Kg + off + s * C::SK);
      const Op b = *reinterpret_cast<const Op*>(Vg + off + s * C::SK);
      kop[t][s] = key < N ? a : E::zero();
      vop[t][s] = key < N ? b : E::zero();
    }
  }
  f32x16 dk[KTW][C::DT], dv[KTW][C::DT];
#pragma unroll
  for (int t = 0; t < KTW; ++t)
#pragma unroll
    for (int u = 0; u < C::DT; ++u) dk[t][u] = dv[t][u] = f32x16{};

  const int lo = CAUSAL ? (kblk / BMQ) * BMQ : 0;  // kernels.py:206-208
  const int nsteps = (N - lo + BMQ - 1) / BMQ;

  St st;
  float mv = 0.0f, dlv = 0.0f;  // this thread's M / delta entry of the staged step
  auto gload = [&](int q0) {
    st.load(Qg, DOg, rs, q0, N, tid);
    if (tid < BMQ) {
      const int q = q0 + tid;
      mv = q < N ? Mg[q] : 0.0f;
      dlv = q < N ? Dg[q] : 0.0f;
    }
  };
  auto lstore = [&](int buf) {
    char* base = smem + buf * C::STAGE;
    st.store(base, base + St::TILE, tid);
    if (tid < BMQ) {
      float* mvec = reinterpret_cast<float*>(base + 2 * St::TILE);
      mvec[tid] = mv;
      mvec[BMQ + tid] = dlv;
    }
  };

  auto step = [&](const char* base, int q0, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const char* qs = base;
    const char* dos = base + St::TILE;
    const TATTN_LDS float* mvec = (const TATTN_LDS float*)(base + 2 * St::TILE);
    f32x16 s[KTW][C::QT], dp[KTW][C::QT];
#pragma unroll
    for (int t = 0; t < KTW; ++t)
#pragma unroll
      for (int j = 0; j < C::QT; ++j) s[t][j] = dp[t][j] = f32x16{};
#pragma unroll
    for (int j = 0; j < C::QT; ++j)
#pragma unroll
      for (int sd = 0; sd < C::NSD; ++sd) {
        Op qa, da;
        if constexpr (C::KPL == 8) {
          qa = nat_operand<T, D>(qs, 32 * j + l32, sd * C::SK + C::KPL * h2);
          da = nat_operand<T, D>(dos, 32 * j + l32, sd * C::SK + C::KPL * h2);
        } else {
          const int off = (32 * j + l32) * St::R + (sd * C::SK + C::KPL * h2) * C::SZ;
          qa = *reinterpret_cast<const TATTN_LDS Op*>((const TATTN_LDS char*)qs + off);
          da = *reinterpret_cast<const TATTN_LDS Op*>((const TATTN_LDS char*)dos + off);
        }
#pragma unroll
        for (int t = 0; t < KTW; ++t) {
          s[t][j] = E::mfma(qa, kop[t][sd], s[t][j]);
          dp[t][j] = E::mfma(da, vop[t][sd], dp[t][j]);
        }
      }
    // P and dS; register r of tile j holds query q0 + 32j + kappa(r, h2).
#pragma unroll
    for (int j = 0; j < C::QT; ++j) {
      float mr[16], dr[16];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          mr[8 * a + i] = mvec[32 * j + 16 * a + 8 * h2 + i];
          dr[8 * a + i] = mvec[BMQ + 32 * j + 16 * a + 8 * h2 + i];
        }
#pragma unroll
      for (int t = 0; t < KTW; ++t) {
        const int key = kw0 + 32 * t + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float pr = fast_exp2(__builtin_fmaf(s[t][j][r], c, -mr[r]));
          if constexpr (MASK) {
            const int q = q0 + 32 * j + kappa(r, h2);
            pr = key > q ? 0.0f : pr;
          }
          s[t][j][r] = pr;
          dp[t][j][r] = pr * (dp[t][j][r] - dr[r]);
        }
      }
    }
    // dV += P^T dO, dK += dS^T Q over the step's query slices.
#pragma unroll
    for (int sl = 0; sl < C::NSQ; ++sl) {
      Op pa[KTW], sa[KTW];
#pragma unroll
      for (int t = 0; t < KTW; ++t) {
        if constexpr (C::KPL == 8) {
          const int j = sl >> 1, b = (sl & 1) * 8;
          Op x, y;
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            const auto u = H16<T>::pack(s[t][j][b + i], s[t][j][b + i + 1]);
            const auto v = H16<T>::pack(dp[t][j][b + i], dp[t][j][b + i + 1]);
            x[i] = u[0]; x[i + 1] = u[1];
            y[i] = v[0]; y[i + 1] = v[1];
          }
          pa[t] = x;
          sa[t] = y;
        } else {
          pa[t] = s[t][sl >> 4][sl & 15];
          sa[t] = dp[t][sl >> 4][sl & 15];
        }
      }
#pragma unroll
      for (int u = 0; u < C::DT; ++u) {
        Op dob, qb;
        if constexpr (C::KPL == 8) {
          dob = tr_operand<T, D>(dos, sl, u, lane);
          qb = tr_operand<T, D>(qs, sl, u, lane);
          if (D < 32 && 32 * u + 16 * ((lane >> 4) & 1) >= D) dob = qb = E::zero();
        } else {
          dob = f32_operand(dos, St::R, sl, u, lane, D);
          qb = f32_operand(qs, St::R, sl, u, lane, D);
        }
#pragma unroll
        for (int t = 0; t < KTW; ++t) {
          dv[t][u] = E::mfma(pa[t], dob, dv[t][u]);
          dk[t][u] = E::mfma(sa[t], qb, dk[t][u]);
        }
      }
    }
  };

  if (nsteps > 0) {
    gload(lo);
    lstore(0);
  }
  __syncthreads();
  const int wave_last_key = kw0 + 32 * KTW - 1;
  for (int it = 0; it < nsteps; ++it) {
    const int q0 = lo + it * BMQ;
    if (it + 1 < nsteps) gload(q0 + BMQ);
    const char* base = smem + (it & 1) * C::STAGE;
    const bool idle = kw0 >= N || (CAUSAL && q0 + BMQ - 1 < kw0);
    if (!idle) {
      if (CAUSAL && q0 < wave_last_key)
        step(base, q0, std::true_type{});
      else
        step(base, q0, std::false_type{});
    }
    if (it + 1 < nsteps) lstore((it + 1) & 1);
    __syncthreads();
  }

  // Store: C register r of lane holds key 8*(r/4) + 4*h2 + r%4 of tile t, column 32u + l32.
  T* DKg = (T*)p.dk + hd.off;
  T* DVg = (T*)p.dv + hd.off;
#pragma unroll
  for (int t = 0; t < KTW; ++t)
#pragma unroll
    for (int u = 0; u < C::DT; ++u) {
      const int d = 32 * u + l32;
      if (d < D) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kw0 + 32 * t + 8 * (r >> 2) + 4 * h2 + (r & 3);
          if (key < N) {
            DKg[(int64_t)key * rs + d] = (T)(dk[t][u][r] * p.scale);
            DVg[(int64_t)key * rs + d] = (T)dv[t][u][r];
          }
        }
      }
    }
}

// ---- dQ (kernels.py:242-321) ---------------------------------------------------------------
template <typename T, int D, int NW, int QTW, int BNK>
struct DqCfg {
  static constexpr int NT = NW * 64;
  static constexpr int BMQ = NW * QTW * 32;
  static constexpr int SZ = (int)sizeof(T);
  static constexpr int KPL = Elt<T>::KPL;
  static constexpr int SK = 2 * KPL;
  static constexpr int NSD = D / SK;
  static constexpr int KT = BNK / 32;
  static constexpr int DT = (D + 31) / 32;
  static constexpr int NSK = BNK / SK;
  using St = Stage2<T, D, BNK, NT>;
  static constexpr int STAGE = 2 * St::TILE;
  static constexpr int LDS = 2 * STAGE;
};

// OCC: waves per SIMD the register budget is sized for (1 gives 512 registers: D=128).
template <typename T, int D, int NW, int QTW, int BNK, bool CAUSAL, int OCC>
__global__ __launch_bounds__(NW * 64, OCC) void dq_kernel(const BwdParams p) {
  using C = DqCfg<T, D, NW, QTW, BNK>;
  using E = Elt<T>;
  using Op = typename E::Op;
  using St = typename C::St;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_blocks, !CAUSAL);
  const int zh = bc.zh;
  int qb = bc.blk;
  if (CAUSAL) qb = p.n_blocks - 1 - qb;  // longest rows first
  const Head hd = head_of(p, zh);
  const T* Qg = (const T*)p.q + hd.off;
  const T* Kg = (const T*)p.k + hd.off;
  const T* Vg = (const T*)p.v + hd.off;
  const T* DOg = (const T*)p.dout + hd.off;
  const int64_t rs = p.s[2];
  const float c = p.c;

  const int qblk = qb * C::BMQ;
  const int qw0 = qblk + w * QTW * 32;

  Op qop[QTW][C::NSD], dop[QTW][C::NSD];
  float mrow[QTW], drow[QTW];
#pragma unroll
  for (int j = 0; j < QTW; ++j) {
    const int q = qw0 + 32 * j + l32;
    const int64_t off = (int64_t)(q < N ? q : 0) * rs + C::KPL * h2;
#pragma unroll
    for (int s = 0; s < C::NSD; ++s) {
      const Op a = *reinterpret_cast<const Op*>(Qg + off + s * C::SK);
      const Op b = *reinterpret_cast<const Op*>(DOg + off + s * C::SK);
      qop[j][s] = q < N ? a : E::zero();
      dop[j][s] = q < N ? b : E::zero();
    }
    mrow[j] = q < N ? p.m[(int64_t)zh * N + q] : 0.0f;
    drow[j] = q < N ? p.delta[(int64_t)zh * N + q] : 0.0f;
  }
  f32x16 dq[C::DT][QTW];
#pragma unroll
  for (int u = 0; u < C::DT; ++u)
#pragma unroll
    for (int j = 0; j < QTW; ++j) dq[u][j] = f32x16{};

  const int hi = CAUSAL ? min(qblk + C::BMQ, N) : N;
  const int nsteps = (hi + BNK - 1) / BNK;

  St st;
  auto step = [&](const char* ks, const char* vs, int kb, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x16 s[C::KT][QTW], dp[C::KT][QTW];
#pragma unroll
    for (int t = 0; t < C::KT; ++t) {
#pragma unroll
      for (int j = 0; j < QTW; ++j) s[t][j] = dp[t][j] = f32x16{};
#pragma unroll
      for (int sd = 0; sd < C::NSD; ++sd) {
        Op ka, va;
        if constexpr (C::KPL == 8) {
          ka = nat_operand<T, D>(ks, 32 * t + l32, sd * C::SK + C::KPL * h2);
          va = nat_operand<T, D>(vs, 32 * t + l32, sd * C::SK + C::KPL * h2);
        } else {
          const int off = (32 * t + l32) * St::R + (sd * C::SK + C::KPL * h2) * C::SZ;
          ka = *reinterpret_cast<const TATTN_LDS Op*>((const TATTN_LDS char*)ks + off);
          va = *reinterpret_cast<const TATTN_LDS Op*>((const TATTN_LDS char*)vs + off);
        }
#pragma unroll
        for (int j = 0; j < QTW; ++j) {
          s[t][j] = E::mfma(ka, qop[j][sd], s[t][j]);
          dp[t][j] = E::mfma(va, dop[j][sd], dp[t][j]);
        }
      }
    }
    // dS^T; register r of tile t holds key kb + 32t + kappa(r, h2); the lane's query is fixed.
#pragma unroll
    for (int j = 0; j < QTW; ++j) {
      const int q = qw0 + 32 * j + l32;
      const float nm = -mrow[j];
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float pr = fast_exp2(__builtin_fmaf(s[t][j][r], c, nm));
          if constexpr (MASK) {
            const int key = kb + 32 * t + kappa(r, h2);
            pr = (key >= N || (CAUSAL && key > q)) ? 0.0f : pr;
          }
          s[t][j][r] = pr * (dp[t][j][r] - drow[j]);
        }
    }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int sl = 0; sl < C::NSK; ++sl) {
      Op b[QTW];
#pragma unroll
      for (int j = 0; j < QTW; ++j) {
        if constexpr (C::KPL == 8) {
          const int t = sl >> 1, o = (sl & 1) * 8;
          Op x;
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            const auto u = H16<T>::pack(s[t][j][o + i], s[t][j][o + i + 1]);
            x[i] = u[0];
            x[i + 1] = u[1];
          }
          b[j] = x;
        } else {
          b[j] = s[sl >> 4][j][sl & 15];
        }
      }
#pragma unroll
      for (int u = 0; u < C::DT; ++u) {
        Op a;
        if constexpr (C::KPL == 8) {
          a = tr_operand<T, D>(ks, sl, u, lane);
          if (D < 32 && 32 * u + 16 * ((lane >> 4) & 1) >= D) a = E::zero();
        } else {
          a = f32_operand(ks, St::R, sl, u, lane, D);
        }
#pragma unroll
        for (int j = 0; j < QTW; ++j) dq[u][j] = E::mfma(a, b[j], dq[u][j]);
      }
    }
  };

  if (nsteps > 0) {
    st.load(Kg, Vg, rs, 0, N, tid);
    st.store(smem, smem + St::TILE, tid);
  }
  __syncthreads();
  const int wave_last = qw0 + QTW * 32 - 1;
  for (int it = 0; it < nsteps; ++it) {
    const int kb = it * BNK;
    if (it + 1 < nsteps) st.load(Kg, Vg, rs, kb + BNK, N, tid);
    const char* ks = smem + (it & 1) * C::STAGE;
    const char* vs = ks + St::TILE;
    const bool idle = qw0 >= N || (CAUSAL && kb > wave_last);
    if (!idle) {
      const bool need_mask = kb + BNK > N || (CAUSAL && kb + BNK - 1 > qw0);
      if (need_mask)
        step(ks, vs, kb, std::true_type{});
      else
        step(ks, vs, kb, std::false_type{});
    }
    if (it + 1 < nsteps) {
      char* nb = smem + ((it + 1) & 1) * C::STAGE;
      st.store(nb, nb + St::TILE, tid);
    }
    __syncthreads();
  }

  // dQ^T C layout: lane = query, register r = column 32u + 8*(r/4) + 4*h2 + r%4.
  T* DQg = (T*)p.dq + hd.off;
#pragma unroll
  for (int j = 0; j < QTW; ++j) {
    const int q = qw0 + 32 * j + l32;
    if (q < N) {
      T* row = DQg + (int64_t)q * rs;
#pragma unroll
      for (int u = 0; u < C::DT; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * u + 8 * g + 4 * h2;
          if (d0 < D) {
            if constexpr (C::KPL == 8) {
              typename H16<T>::V4 x;
#pragma unroll
              for (int i = 0; i < 4; ++i) x[i] = (T)(dq[u][j][4 * g + i] * p.scale);
              *reinterpret_cast<typename H16<T>::V4*>(row + d0) = x;
            } else {
              f32x4 x;
#pragma unroll
              for (int i = 0; i < 4; ++i) x[i] = dq[u][j][4 * g + i] * p.scale;
              *reinterpret_cast<f32x4*>(row + d0) = x;
            }
          }
        }
    }
  }
}

// ---- launch ------------------------------------------------------------------------------

template <typename T, int D>
static int run_preprocess(const BwdParams& p, hipStream_t st) {
  constexpr int CPR = D / (16 / (int)sizeof(T)), RPB = 256 / CPR;
  const int64_t nb = (p.N + RPB - 1) / RPB;
  const int64_t blocks = nb * p.Z * p.H;
  if (blocks > 0x7fffffff) return set_error(TATTN_E_ARG, "grid too large: %lld workgroups", (long long)blocks);
  bwd_preprocess_kernel<T, D><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(p);
  return check_launch("tattn_bwd_preprocess");
}

int launch_bwd_preprocess(const BwdParams& p, int D, int dtype, hipStream_t st) {
  if (dtype == 0) {
    switch (D) {
      case 16: return run_preprocess<f16, 16>(p, st);
      case 32: return run_preprocess<f16, 32>(p, st);
      case 64: return run_preprocess<f16, 64>(p, st);
      case 128: return run_preprocess<f16, 128>(p, st);
    }
  } else if (dtype == 2) {
    switch (D) {
      case 16: return run_preprocess<bf16, 16>(p, st);
      case 32: return run_preprocess<bf16, 32>(p, st);
      case 64: return run_preprocess<bf16, 64>(p, st);
      case 128: return run_preprocess<bf16, 128>(p, st);
    }
  } else {
    switch (D) {
      case 16: return run_preprocess<float, 16>(p, st);
      case 32: return run_preprocess<float, 32>(p, st);
      case 64: return run_preprocess<float, 64>(p, st);
      case 128: return run_preprocess<float, 128>(p, st);
    }
  }
  return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %d", D);
}

template <template <typename, int> class Table, typename T, int D, int I>
struct Entry {
  static constexpr TileEntry e = Table<T, D>::e[I];
};

// Buffer descriptors address a (z, h) slice with 32-bit offsets (plus two steps of look-ahead).
static bool slice_fits32(const BwdParams& p, int D) { return bwd_fits32(p, D); }

template <typename T, int D, int I>
static int launch_dkdv_entry(const BwdParams& p0, bool causal, hipStream_t st) {
  constexpr TileEntry e = DkdvTable<T, D>::e[I];
  constexpr int BNK = tile_rows(e);
  BwdParams p = p0;
  p.n_blocks = (p.N + BNK - 1) / BNK;
  const int64_t blocks = (int64_t)p.n_blocks * p.Z * p.H;
  if (blocks > 0x7fffffff) return set_error(TATTN_E_ARG, "grid too large: %lld workgroups", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(e.nw * 64);
  if constexpr (e.pipe == 3) {  // paired waves, 128 keys per workgroup (own translation unit)
    static_assert(sizeof(T) == 2 && e.nw == 8 && e.tiles == 1 && e.other == 32, "paired-wave dK/dV shape");
    if (slice_fits32(p, D)) return launch_split(p, D, std::is_same_v<T, bf16> ? 2 : 0, true, causal, st);
    p.n_blocks = (p.N + 127) / 128;  // slices beyond 2 GiB: 64-bit addressing
    const dim3 g2((unsigned)((int64_t)p.n_blocks * p.Z * p.H));
    if (causal)
      dkdv_kernel<T, D, 4, 1, 32, true, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
    else
      dkdv_kernel<T, D, 4, 1, 32, false, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
  } else if constexpr (e.pipe >= 1) {
    static_assert(sizeof(T) == 2 && D <= 128 && (e.tiles == 1 || D <= 64) && e.other == 32, "pipelined dK/dV shape");
    if constexpr (e.pipe == 2) {
      static_assert(e.tiles == 1 && D <= 64, "persistent dK/dV shape");
      if (slice_fits32(p, D) && bwd_persist_fits(e, (int64_t)p.Z * p.H, p.N, causal))  // own translation unit
        return launch_dkdv_persist(p0, D, std::is_same_v<T, bf16> ? 2 : 0, I, causal, st);
    }
    if (slice_fits32(p, D)) {
      if (causal)
        dkdv_pipe_kernel<T, D, e.nw, e.tiles, e.occ, true><<<grid, block, 0, st>>>(p);
      else
        dkdv_pipe_kernel<T, D, e.nw, e.tiles, e.occ, false><<<grid, block, 0, st>>>(p);
      return check_launch("tattn_bwd_dkdv");
    }
    p.n_blocks = (p.N + 127) / 128;  // slices beyond 2 GiB: 64-bit addressing
    const dim3 g2((unsigned)((int64_t)p.n_blocks * p.Z * p.H));
    if (causal)
      dkdv_kernel<T, D, 4, 1, 32, true, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
    else
      dkdv_kernel<T, D, 4, 1, 32, false, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
  } else {
    if (causal)
      dkdv_kernel<T, D, e.nw, e.tiles, e.other, true, e.occ><<<grid, block, 0, st>>>(p);
    else
      dkdv_kernel<T, D, e.nw, e.tiles, e.other, false, e.occ><<<grid, block, 0, st>>>(p);
  }
  return check_launch("tattn_bwd_dkdv");
}

template <typename T, int D, int I>
static int launch_dq_entry(const BwdParams& p0, bool causal, hipStream_t st) {
  constexpr TileEntry e = DqTable<T, D>::e[I];
  constexpr int BMQ = tile_rows(e);
  BwdParams p = p0;
  p.n_blocks = (p.N + BMQ - 1) / BMQ;
  const int64_t blocks = (int64_t)p.n_blocks * p.Z * p.H;
  if (blocks > 0x7fffffff) return set_error(TATTN_E_ARG, "grid too large: %lld workgroups", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(e.nw * 64);
  if constexpr (e.pipe == 3) {  // paired waves, 128 queries per workgroup (own translation unit)
    static_assert(sizeof(T) == 2 && e.nw == 8 && e.tiles == 1 && e.other == 32, "paired-wave dQ shape");
    if (slice_fits32(p, D)) return launch_split(p, D, std::is_same_v<T, bf16> ? 2 : 0, false, causal, st);
    p.n_blocks = (p.N + 127) / 128;  // slices beyond 2 GiB: 64-bit addressing
    const dim3 g2((unsigned)((int64_t)p.n_blocks * p.Z * p.H));
    if (causal)
      dq_kernel<T, D, 4, 1, 32, true, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
    else
      dq_kernel<T, D, 4, 1, 32, false, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
  } else if constexpr (e.pipe >= 1) {
    static_assert(sizeof(T) == 2 && D <= 128 && e.tiles == 1 && e.other == 32, "pipelined dQ shape");
    if constexpr (e.pipe == 2) {
      if (slice_fits32(p, D) && bwd_persist_fits(e, (int64_t)p.Z * p.H, p.N, causal))  // own translation unit
        return launch_dq_persist(p0, D, std::is_same_v<T, bf16> ? 2 : 0, I, causal, st);
    }
    if (slice_fits32(p, D)) {
      if (causal)
        dq_pipe_kernel<T, D, e.nw, e.occ, true><<<grid, block, 0, st>>>(p);
      else
        dq_pipe_kernel<T, D, e.nw, e.occ, false><<<grid, block, 0, st>>>(p);
      return check_launch("tattn_bwd_dq");
    }
    p.n_blocks = (p.N + 127) / 128;  // slices beyond 2 GiB: 64-bit addressing
    const dim3 g2((unsigned)((int64_t)p.n_blocks * p.Z * p.H));
    if (causal)
      dq_kernel<T, D, 4, 1, 32, true, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
    else
      dq_kernel<T, D, 4, 1, 32, false, D == 128 ? 1 : 2><<<g2, dim3(256), 0, st>>>(p);
  } else {
    if (causal)
      dq_kernel<T, D, e.nw, e.tiles, e.other, true, e.occ><<<grid, block, 0, st>>>(p);
    else
      dq_kernel<T, D, e.nw, e.tiles, e.other, false, e.occ><<<grid, block, 0, st>>>(p);
  }
  return check_launch("tattn_bwd_dq");
}

template <typename T, int D, size_t... I>
static int dispatch_dkdv(int id, const BwdParams& p, bool causal, hipStream_t st, std::index_sequence<I...>) {
  int rc = set_error(TATTN_E_CONFIG, "dK/dV config id %d out of range [0, %d) for D=%d", id,
                     (int)sizeof...(I), D);
  ((id == (int)I ? (rc = launch_dkdv_entry<T, D, I>(p, causal, st), 0) : 0), ...);
  return rc;
}

template <typename T, int D, size_t... I>
static int dispatch_dq(int id, const BwdParams& p, bool causal, hipStream_t st, std::index_sequence<I...>) {
  int rc = set_error(TATTN_E_CONFIG, "dQ config id %d out of range [0, %d) for D=%d", id,
                     (int)sizeof...(I), D);
  ((id == (int)I ? (rc = launch_dq_entry<T, D, I>(p, causal, st), 0) : 0), ...);
  return rc;
}

#define TATTN_BWD_SWITCH(FN, TABLE)                                                              \
  if (dtype == 0) {                                                                              \
    switch (D) {                                                                                 \
      case 16: return FN<f16, 16>(id, p, causal, st, std::make_index_sequence<TABLE<f16, 16>::n>{}); \
      case 32: return FN<f16, 32>(id, p, causal, st, std::make_index_sequence<TABLE<f16, 32>::n>{}); \
      case 64: return FN<f16, 64>(id, p, causal, st, std::make_index_sequence<TABLE<f16, 64>::n>{}); \
      case 128: return FN<f16, 128>(id, p, causal, st, std::make_index_sequence<TABLE<f16, 128>::n>{}); \
    }                                                                                            \
  } else if (dtype == 2) {                                                                       \
    switch (D) {                                                                                 \
      case 16: return FN<bf16, 16>(id, p, causal, st, std::make_index_sequence<TABLE<bf16, 16>::n>{}); \
      case 32: return FN<bf16, 32>(id, p, causal, st, std::make_index_sequence<TABLE<bf16, 32>::n>{}); \
      case 64: return FN<bf16, 64>(id, p, causal, st, std::make_index_sequence<TABLE<bf16, 64>::n>{}); \
      case 128: return FN<bf16, 128>(id, p, causal, st, std::make_index_sequence<TABLE<bf16, 128>::n>{}); \
    }                                                                                            \
  } else {                                                                                       \
    switch (D) {                                                                                 \
      case 16: return FN<float, 16>(id, p, causal, st, std::make_index_sequence<TABLE<float, 16>::n>{}); \
      case 32: return FN<float, 32>(id, p, causal, st, std::make_index_sequence<TABLE<float, 32>::n>{}); \
      case 64: return FN<float, 64>(id, p, causal, st, std::make_index_sequence<TABLE<float, 64>::n>{}); \
      case 128: return FN<float, 128>(id, p, causal, st, std::make_index_sequence<TABLE<float, 128>::n>{}); \
    }                                                                                            \
  }                                                                                              \
  return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %d", D);

int launch_bwd_dkdv(const BwdParams& p, int D, int dtype, bool causal, int id, hipStream_t st) {
  TATTN_BWD_SWITCH(dispatch_dkdv, DkdvTable)
}

int launch_bwd_dq(const BwdParams& p, int D, int dtype, bool causal, int id, hipStream_t st) {
  TATTN_BWD_SWITCH(dispatch_dq, DqTable)
}

int dkdv_lds_bytes(int D, int dtype, const TileEntry& e) {
  const int r = dtype != 1 ? (D < 32 ? 64 : 2 * D) : 4 * D + 16;
  if (e.pipe == 3) return 4 * (2 * 32 * r + 256) + 2 * 4 * 32 * 32 * 4;  // ring + P exchange buffers
  if (e.pipe == 2) return 4 * (2 * 32 * r + 256) + e.nw * 2 * 32 * r;     // ring + K/V staging tiles
  if (e.pipe) return 4 * (2 * 32 * r + 256);
  return 2 * (2 * e.other * r + 2 * e.other * 4);
}

int dq_lds_bytes(int D, int dtype, const TileEntry& e) {
  const int r = dtype != 1 ? (D < 32 ? 64 : 2 * D) : 4 * D + 16;
  if (e.pipe == 3) return 4 * (2 * 32 * r) + 2 * 4 * 32 * 32 * 4;  // ring + P exchange buffers
  if (e.pipe == 2) return 4 * (2 * 32 * r) + e.nw * 32 * r;  // ring + per-wave dQ rows
  if (e.pipe) return 4 * (2 * 32 * r);
  return 2 * (2 * e.other * r);
}

}  // namespace tattn
