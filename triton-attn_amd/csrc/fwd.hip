// Forward attention kernel for gfx950 (replaces src/tattn/kernels.py:57-148).
//
// One workgroup = NW waves = block_m = NW * QT * 32 query rows of one (z, h). Each wave owns
// QT 32-query MFMA tiles and keeps its Q operands in registers. Keys stream in steps of BN
// rows through a double-buffered LDS stage (K with the perm32 row order, V row-major), with
// the next step's global loads in flight during the current step's math.
//
// Per step and wave:
//   S^T = K Q^T        (A = K rows from LDS, B = Q^T from registers), C layout: lane = query
//   online softmax     row max over the lane's 16*KT scores + one lane^32 swap; base-2
//                      exponent with the scale folded into one FMA; float32 state
//   O^T += V^T P^T     (A = V^T via transposed LDS reads, B = P^T straight from registers:
//                      P is rounded to the element type first, as the reference does at
//                      kernels.py:139)
// Rescaling is lazy: the max used in the exponent only moves when a row's true max exceeds
// it by more than 2^kRescaleLog2 (bounded growth of P, exact in real arithmetic because the
// same max enters the running sum and the accumulator); M = max + log2(sum) is the base-2
// log-sum-exp either way (kernels.py:143).
//
// Causal: key steps entirely above the workgroup's last row are never loaded; steps entirely
// above a wave's last row are skipped by that wave; only steps that cross the diagonal or the
// sequence end pay for per-element masks (kernels.py:117-131).
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "tiles.h"

namespace tattn {

template <typename T, int D, int NW, int QT, int BN>
struct FwdCfg {
  static constexpr int NT = NW * 64;
  static constexpr int BM = NW * QT * 32;
  static constexpr int SZ = (int)sizeof(T);
  static constexpr int KPL = Elt<T>::KPL;
  static constexpr int SK = 2 * KPL;        // k extent of one MFMA
  static constexpr int NSD = D / SK;        // MFMA slices over d (S^T)
  static constexpr int KT = BN / 32;        // 32-key tiles per step
  static constexpr int DT = (D + 31) / 32;  // 32-row tiles over d (O^T)
  static constexpr int NSK = BN / SK;       // MFMA slices over keys (O^T)
  static constexpr int RK = D * SZ + 16;    // LDS row stride of K, bytes
  static constexpr int RV = D * SZ + (SZ == 2 ? 32 : 16);
  static constexpr int KBYTES = BN * RK;
  static constexpr int STAGE = KBYTES + BN * RV;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int EPC = 16 / SZ;       // elements per 16-byte chunk
  static constexpr int CPR = D / EPC;       // chunks per row
  static constexpr int CHUNKS = BN * CPR;
  static constexpr int CPT = (CHUNKS + NT - 1) / NT;  // chunks per thread per tensor
  static_assert(D % SK == 0 && BN % 32 == 0, "tile shape");
};

// OCC: waves per SIMD the register budget is sized for (1 gives 512 registers: D=128 in fp32).
template <typename T, int D, int NW, int QT, int BN, bool CAUSAL, int OCC>
__global__ __launch_bounds__(NW * 64, OCC) void fwd_generic_kernel(const FwdParams p) {
  using C = FwdCfg<T, D, NW, QT, BN>;
  using E = Elt<T>;
  using Op = typename E::Op;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_qblocks, !CAUSAL);
  const int zh = bc.zh;
  int qb = bc.blk;
  if (CAUSAL) qb = p.n_qblocks - 1 - qb;  // longest rows first
  const int64_t z = zh / p.H, hh = zh % p.H;
  const T* Q = (const T*)p.q + z * p.sq[0] + hh * p.sq[1];
  const T* K = (const T*)p.k + z * p.sk[0] + hh * p.sk[1];
  const T* V = (const T*)p.v + z * p.sv[0] + hh * p.sv[1];
  T* O = (T*)p.o + z * p.so[0] + hh * p.so[1];
  float* M = p.m ? p.m + (int64_t)zh * N : nullptr;  // null: M not stored
  const int64_t sqn = p.sq[2], skn = p.sk[2], svn = p.sv[2], son = p.so[2];
  const float c = p.c;

  const int qblk = qb * C::BM;
  const int qw0 = qblk + w * QT * 32;  // first query row of this wave

  // Q^T operands: lane holds Q[q = qw0 + 32j + l32][KPL*h2 + SK*s + i].
  Op qop[QT][C::NSD];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int row = qw0 + 32 * j + l32;
    const T* src = Q + (int64_t)(row < N ? row : 0) * sqn + C::KPL * h2;
#pragma unroll
    for (int s = 0; s < C::NSD; ++s) {
      Op x = *reinterpret_cast<const Op*>(src + s * C::SK);
      qop[j][s] = row < N ? x : E::zero();
    }
  }

  const int hi = CAUSAL ? min(qblk + C::BM, N) : N;
  const int nsteps = (hi + BN - 1) / BN;

  // Global -> register prefetch of one K and one V step.
  u32x4 pk[C::CPT], pv[C::CPT];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < C::CPT; ++i) {
      const int ch = tid + i * C::NT;
      const int row = ch / C::CPR, col = (ch % C::CPR) * C::EPC;
      const int key = kb + row;
      const bool ok = (C::CHUNKS % C::NT == 0 || ch < C::CHUNKS) && key < N;
      const int64_t kr = ok ? key : 0;
      u32x4 a = ld16(K + kr * skn + col), b = ld16(V + kr * svn + col);
      pk[i] = ok ? a : u32x4{0, 0, 0, 0};
      pv[i] = ok ? b : u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf) {
    char* ks = smem + buf * C::STAGE;
    char* vs = ks + C::KBYTES;
#pragma unroll
    for (int i = 0; i < C::CPT; ++i) {
      const int ch = tid + i * C::NT;
      if (C::CHUNKS % C::NT == 0 || ch < C::CHUNKS) {
        const int row = ch / C::CPR, cb = (ch % C::CPR) * 16;
        const int krow = (row & ~31) | perm32(row & 31);
        st16(ks + krow * C::RK + cb, pk[i]);
        st16(vs + row * C::RV + cb, pv[i]);
      }
    }
  };

  float mrow[QT], lrow[QT];
  f32x16 acc[C::DT][QT];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    mrow[j] = -__builtin_inff();
    lrow[j] = 0.0f;
#pragma unroll
    for (int u = 0; u < C::DT; ++u) acc[u][j] = f32x16{};
  }

  auto step = [&](const char* ks, const char* vs, int kb, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x16 s[C::KT][QT];
#pragma unroll
    for (int t = 0; t < C::KT; ++t) {
#pragma unroll
      for (int j = 0; j < QT; ++j) s[t][j] = f32x16{};
#pragma unroll
      for (int sd = 0; sd < C::NSD; ++sd) {
        const char* a = ks + (32 * t + l32) * C::RK + (sd * C::SK + C::KPL * h2) * C::SZ;
        const Op kop = *reinterpret_cast<const TATTN_LDS Op*>((const TATTN_LDS char*)a);
#pragma unroll
        for (int j = 0; j < QT; ++j) s[t][j] = E::mfma(kop, qop[j][sd], s[t][j]);
      }
    }
    // Hidden keys: excluded from the max of the scaled scores (the scale may be negative or
    // zero) and given probability 0 after the exponential.
    bool dead[C::KT][QT][16];
#pragma unroll
    for (int t = 0; t < C::KT; ++t)
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const int q = qw0 + 32 * j + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 32 * t + kappa(r, h2);
          dead[t][j][r] = MASK && (key >= N || (CAUSAL && key > q));
        }
      }
    // Row max of every q-tile first, then one wave-uniform rescale branch for the whole step.
    float mnew[QT], alpha[QT];
    bool any_upd = false;
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = dead[t][j][r] ? mx : __builtin_fmaxf(mx, s[t][j][r] * c);
      const float cand = max_halves(mx);
      const bool upd = cand > mrow[j] + kRescaleLog2;
      mnew[j] = upd ? cand : mrow[j];
      alpha[j] = fast_exp2(mrow[j] - mnew[j]);
      any_upd |= upd;
    }
    if (__builtin_amdgcn_ballot_w64(any_upd)) {
#pragma unroll
      for (int j = 0; j < QT; ++j)
#pragma unroll
        for (int u = 0; u < C::DT; ++u) acc[u][j] *= alpha[j];
    }
    Op pop[QT][C::NSK];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      mrow[j] = mnew[j];
      const float nm = -mnew[j];
      float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = dead[t][j][r] ? 0.0f : fast_exp2(__builtin_fmaf(s[t][j][r], c, nm));
          s[t][j][r] = e;
          ps[r & 3] = (t == 0 && r < 4) ? e : ps[r & 3] + e;
        }
      lrow[j] = lrow[j] * alpha[j] + ((ps[0] + ps[1]) + (ps[2] + ps[3]));
      if constexpr (C::KPL == 8) {
#pragma unroll
        for (int sg = 0; sg < C::NSK; ++sg) {
          const int t = sg >> 1, b = (sg & 1) * 8;
          typename H16<T>::V8 x;
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            const typename H16<T>::V2 pr = H16<T>::pack(s[t][j][b + i], s[t][j][b + i + 1]);
            x[i] = pr[0];
            x[i + 1] = pr[1];
          }
          pop[j][sg] = x;
        }
      } else {
#pragma unroll
        for (int sg = 0; sg < C::NSK; ++sg) pop[j][sg] = s[sg >> 4][j][sg & 15];
      }
    }
#pragma unroll
    for (int u = 0; u < C::DT; ++u) {
#pragma unroll
      for (int sg = 0; sg < C::NSK; ++sg) {
        Op vop;
        if constexpr (C::KPL == 8) {
          const int g = lane >> 4, src = lane & 15;
          const int mb = 32 * u + 16 * (g & 1);
          const int kb0 = 16 * sg + 8 * (g >> 1);
          const TATTN_LDS char* a =
              (const TATTN_LDS char*)vs + (kb0 + (src >> 2)) * C::RV + (mb + 4 * (src & 3)) * 2;
          const auto lo = lds_tr<T>(a), hi4 = lds_tr<T>(a + 4 * C::RV);
          vop = Op{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          if (D < 32 && mb >= D) vop = E::zero();
        } else {
          const int d = 32 * u + l32;
          const int key = 32 * (sg >> 4) + kappa(sg & 15, h2);
          vop = d < D ? *reinterpret_cast<const TATTN_LDS float*>(
                            (const TATTN_LDS char*)vs + key * C::RV + d * 4)
                      : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < QT; ++j) acc[u][j] = E::mfma(vop, pop[j][sg], acc[u][j]);
      }
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();
  const int wave_last = qw0 + QT * 32 - 1;
  for (int it = 0; it < nsteps; ++it) {
    const int kb = it * BN;
    if (it + 1 < nsteps) gload(kb + BN);
    const char* ks = smem + (it & 1) * C::STAGE;
    const char* vs = ks + C::KBYTES;
    const bool idle = qw0 >= N || (CAUSAL && kb > wave_last);
    if (!idle) {
      const bool need_mask = kb + BN > N || (CAUSAL && kb + BN - 1 > qw0);
      if (need_mask)
        step(ks, vs, kb, std::true_type{});
      else
        step(ks, vs, kb, std::false_type{});
    }
    if (it + 1 < nsteps) lstore((it + 1) & 1);
    __syncthreads();
  }

  // Epilogue: O = acc / l, M = m + log2(l).
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const float lt = sum_halves(lrow[j]);
    const float inv = 1.0f / lt;
    const int q = qw0 + 32 * j + l32;
    if (q < N) {
      T* orow = O + (int64_t)q * son;
#pragma unroll
      for (int u = 0; u < C::DT; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * u + 8 * g + 4 * h2;
          if (d0 < D) {
            if constexpr (C::KPL == 8) {
              typename H16<T>::V4 x;
#pragma unroll
              for (int i = 0; i < 4; ++i) x[i] = (T)(acc[u][j][4 * g + i] * inv);
              *reinterpret_cast<typename H16<T>::V4*>(orow + d0) = x;
            } else {
              f32x4 x;
#pragma unroll
              for (int i = 0; i < 4; ++i) x[i] = acc[u][j][4 * g + i] * inv;
              *reinterpret_cast<f32x4*>(orow + d0) = x;
            }
          }
        }
      if (h2 == 0 && M) M[q] = mrow[j] + __log2f(lt);
    }
  }
}

// ---- fp16: software-pipelined forward ------------------------------------------------------
//
// 32 keys per step. Each step issues 16 MFMAs that do not depend on the step's softmax:
// S_{i+1} = K_{i+1} Q^T and O^T += V_{i-1}^T P_{i-1}^T (the previous step's probabilities,
// kept in registers), so the matrix cores stay busy while the VALU runs the softmax of step i.
// Steps skip the row max: probabilities use the running max as it stands (seeded with step 0's
// row max) and a per-lane sum check sends the wave to a slow path (row max, rescale, S
// recomputed from the K tile still in LDS) only when some probability could exceed 2^12,
// which is rare. Masked steps (diagonal, sequence end) take the same path with keys hidden per
// 32x32 tile.
// LDS rings of four tiles each, filled by LDS DMA (range-checked buffer loads that write LDS
// directly, no registers): step i reads K_{i+1} (and K_i on the slow path) and V_{i-1}, and
// starts K_{i+3} and V_{i+1}, which have two steps to arrive; one barrier per step. Rows past
// the sequence end come back as zeros.
// LDS row strides: K rows D*2+16 bytes (16 consecutive rows of a 16-byte column hit distinct
// banks); V rows are an odd multiple of 64 bytes so each transposed read (4 rows x 64 bytes per
// 32 lanes) covers distinct banks of gfx950's 64-bank LDS.

template <int D>
struct PipeLayout {
  static constexpr int RK = D * 2 + 16;  // LDS row bytes of K and V tiles
  static constexpr int RV = D == 16 ? 64 : D == 32 ? 64 : D == 64 ? 192 : 320;
  // Tiles arrive by LDS DMA (buffer_load ... lds): one wave instruction writes 64 lanes x 16
  // bytes to 1 KB of consecutive LDS, so a slot holds whole 1 KB pieces; lanes that land on row
  // padding or past the 32 rows fetch a duplicate chunk into that slack.
  static constexpr int KPIECES = (32 * RK / 16 + 63) / 64;
  static constexpr int VPIECES = (32 * RV / 16 + 63) / 64;
  static constexpr int KSLOT = 1024 * KPIECES, VSLOT = 1024 * VPIECES;
  // Four-deep rings: during step i the kernel reads K_{i+1} (S of the next step), K_i (rare
  // slow softmax path) and V_{i-1}, while K_{i+2} and V_i sit landed and K_{i+3}, V_{i+1} are in
  // flight (issued at the start of step i, needed two steps later).
  static constexpr int NSLOT = 4;
  static constexpr int LDS = NSLOT * (KSLOT + VSLOT);
};

template <typename T, int D, int NW, int QT, int OCC, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, OCC) void fwd_pipe_kernel(const FwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V4 = typename H::V4;
  using V2 = typename H::V2;
  using L = PipeLayout<D>;
  constexpr int NT = NW * 64, BM = NW * QT * 32;
  constexpr int NSD = D / 16;        // 16-wide d slices of S = K Q^T
  constexpr int DT = (D + 31) / 32;  // 32-row d tiles of O^T
  constexpr int CPK = (L::KPIECES + NW - 1) / NW;  // K and V DMA instructions per wave per step
  constexpr int CPV = (L::VPIECES + NW - 1) / NW;
  constexpr int CPW = CPK + CPV;
  static_assert(CPW < 16, "vmcnt field");
  // One array per ring slot: distinct objects let the compiler see that a DMA into one slot
  // does not alias reads of another (no conservative waits on in-flight tiles).
  __shared__ __attribute__((aligned(1024))) char ks0[L::KSLOT], ks1[L::KSLOT], ks2[L::KSLOT], ks3[L::KSLOT];
  __shared__ __attribute__((aligned(1024))) char vs0[L::VSLOT], vs1[L::VSLOT], vs2[L::VSLOT], vs3[L::VSLOT];
  auto kbuf = [&](int s) -> char* { return s == 0 ? ks0 : s == 1 ? ks1 : s == 2 ? ks2 : ks3; };
  auto vbuf = [&](int s) -> char* { return s == 0 ? vs0 : s == 1 ? vs1 : s == 2 ? vs2 : vs3; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_qblocks, !CAUSAL);
  const int zh = bc.zh;
  int qb = bc.blk;
  if (CAUSAL) qb = p.n_qblocks - 1 - qb;  // longest rows first
  const int64_t z = zh / p.H, hh = zh % p.H;
  const T* Q = (const T*)p.q + z * p.sq[0] + hh * p.sq[1];
  T* O = (T*)p.o + z * p.so[0] + hh * p.so[1];
  float* M = p.m ? p.m + (int64_t)zh * N : nullptr;  // null: M not stored
  const int64_t sqn = p.sq[2], son = p.so[2];
  const __amdgpu_buffer_rsrc_t krs = slice_rsrc((const T*)p.k + z * p.sk[0] + hh * p.sk[1], slice_bytes(N, p.sk[2], D));
  const __amdgpu_buffer_rsrc_t vrs = slice_rsrc((const T*)p.v + z * p.sv[0] + hh * p.sv[1], slice_bytes(N, p.sv[2], D));
  const uint32_t k_step = uniform32((uint32_t)(p.sk[2] * 64)), v_step = uniform32((uint32_t)(p.sv[2] * 64));
  const float c = p.c;

  const int qblk = qb * BM;
  const int qw0 = qblk + w * QT * 32;

  V8 qop[QT][NSD];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int row = qw0 + 32 * j + l32;
    const T* src = Q + (int64_t)(row < N ? row : 0) * sqn + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      const V8 x = *reinterpret_cast<const V8*>(src + 16 * s);
      qop[j][s] = row < N ? x : V8{};
    }
  }

  const int hi = CAUSAL ? min(qblk + BM, N) : N;
  const int nsteps = (hi + 31) / 32;
  // Steps this wave computes: every step up to the one holding its last query row.
  const int wave_steps = qw0 >= N ? 0 : CAUSAL ? min(nsteps, (qw0 + 32 * QT - 1) / 32 + 1) : nsteps;

  // DMA work of this wave: pieces w, w + NW, ... of the step's K tile and of its V tile (indices
  // past a tile's last piece wrap around: a duplicate piece writes the same bytes again). For
  // each, the lane's HBM byte offset from the tile's first row: LDS chunk j = 64 * piece + lane
  // of the padded tile holds row j / (R / 16), chunk j % (R / 16); K rows are in perm32 order.
  const int wu = (int)uniform32((uint32_t)w);
  int kpc[CPK], vpc[CPV];
  uint32_t kgo[CPK], vgo[CPV];
  auto piece = [&](int pp, int rb, int64_t rstride, bool perm, uint32_t& go) {
    const int cpr = rb / 16;
    const int j = 64 * pp + lane;
    const int row = min(j / cpr, 31);
    const int cc = min(j % cpr, D / 8 - 1);
    go = (uint32_t)((perm ? perm32(row) : row) * rstride * 2 + cc * 16);
  };
#pragma unroll
  for (int t = 0; t < CPK; ++t) {
    const int pp = (wu + NW * t) % L::KPIECES;
    kpc[t] = 1024 * pp;
    piece(pp, L::RK, p.sk[2], true, kgo[t]);
  }
#pragma unroll
  for (int t = 0; t < CPV; ++t) {
    const int pp = (wu + NW * t) % L::VPIECES;
    vpc[t] = 1024 * pp;
    piece(pp, L::RV, p.sv[2], false, vgo[t]);
  }
  // K tile kt into K slot ks, V tile vt into V slot vs (tiles past the sequence read as zero).
  auto dma = [&](int kt, int vt, int ks, int vs) {
#pragma unroll
    for (int t = 0; t < CPK; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (TATTN_LDS void*)(kbuf(ks) + kpc[t]), 16,
                                               (int)(kgo[t] + (uint32_t)kt * k_step), 0, 0, 0);
#pragma unroll
    for (int t = 0; t < CPV; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (TATTN_LDS void*)(vbuf(vs) + vpc[t]), 16,
                                               (int)(vgo[t] + (uint32_t)vt * v_step), 0, 0, 0);
  };
  // End of a step: this wave's DMAs of the previous step have landed and its LDS reads are done
  // (this step's DMAs stay in flight), then the barrier publishes the landed tiles. The signal
  // fences keep the compiler from moving LDS reads across the barrier.
  auto step_end = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0070 | CPW);  // vmcnt(CPW), lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  const int g = lane >> 4, src = lane & 15;
  const int kop_off = l32 * L::RK + 16 * h2;
  const int vop_off = (8 * (g >> 1) + (src >> 2)) * L::RV + (16 * (g & 1) + 4 * (src & 3)) * 2;

  // S = K Q^T for the 32-key tile in K buffer kb_ (C layout: lane = query, register r = key
  // kappa(r, h2)).
  auto qk = [&](f32x16* s, int kb_) {
#pragma unroll
    for (int j = 0; j < QT; ++j) s[j] = f32x16{};
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) {
      const V8 kop = *reinterpret_cast<const TATTN_LDS V8*>((const TATTN_LDS char*)kbuf(kb_) + kop_off + 32 * sd);
#pragma unroll
      for (int j = 0; j < QT; ++j) s[j] = Elt<T>::mfma(kop, qop[j][sd], s[j]);
    }
  };

  float mrow[QT], lrow[QT];
  f32x16 acc[DT][QT];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    mrow[j] = -__builtin_inff();
    lrow[j] = 0.0f;
#pragma unroll
    for (int u = 0; u < DT; ++u) acc[u][j] = f32x16{};
  }

  // O^T += V^T P^T for the 32-key tile in V buffer vb_.
  auto pv_mma = [&](const V8 (*pp)[2], int vb_) {
#pragma unroll
    for (int u = 0; u < DT; ++u) {
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        const TATTN_LDS char* a = (const TATTN_LDS char*)vbuf(vb_) + vop_off + 16 * sg * L::RV + 64 * u;
        const V4 lo = lds_tr<T>(a), hi4 = lds_tr<T>(a + 4 * L::RV);
        V8 vop = V8{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        if (D < 32 && 32 * u + 16 * (g & 1) >= D) vop = V8{};
#pragma unroll
        for (int j = 0; j < QT; ++j) acc[u][j] = Elt<T>::mfma(vop, pp[j][sg], acc[u][j]);
      }
    }
  };

  // Softmax of scur (keys kb..kb+31): probabilities into pc, running max and sum updated;
  // returns whether any row of the wave raised its max (the accumulator then needs alpha).
  // The max is taken over the scaled scores (the scale may be negative or zero) and hidden keys
  // get probability 0 after the exponential; for a positive scale this is the same max and the
  // same probabilities as scaling the max of the raw scores.
  auto softmax = [&](f32x16* scur, V8 (*pc)[2], float* alpha, int kb, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    bool dead[QT][16];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const int q = qw0 + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + kappa(r, h2);
        dead[j][r] = MASK && (key >= N || (CAUSAL && key > q));
      }
    }
    bool any_upd = false;
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = dead[j][r] ? mx : __builtin_fmaxf(mx, scur[j][r] * c);
      const float cand = max_halves(mx);
      const bool upd = cand > mrow[j] + kRescaleLog2;
      const float mnew = upd ? cand : mrow[j];
      alpha[j] = fast_exp2(mrow[j] - mnew);
      any_upd |= upd;
      mrow[j] = mnew;
      const float nm = -mnew;
      float ps = 0.0f;
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        V8 x;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float e0 = fast_exp2(__builtin_fmaf(scur[j][8 * sg + i], c, nm));
          float e1 = fast_exp2(__builtin_fmaf(scur[j][8 * sg + i + 1], c, nm));
          e0 = dead[j][8 * sg + i] ? 0.0f : e0;
          e1 = dead[j][8 * sg + i + 1] ? 0.0f : e1;
          const V2 pr = H::pack(e0, e1);
          ps = H::sum2(pr, ps);
          x[i] = pr[0];
          x[i + 1] = pr[1];
        }
        pc[j][sg] = x;
      }
      lrow[j] = lrow[j] * alpha[j] + ps;
    }
    return any_upd;
  };
  // Unmasked steps: probabilities with the running max as it stands (no row max), summed with
  // v_dot2 (fast_probs). A lane whose 16 probabilities sum above 2^12 (some score exceeds the
  // max used in the exponent by more than 12 in base 2) sends the wave down the slow path (fast_fixup): row max, lazy update, accumulator rescale,
  // probabilities recomputed. Probabilities fed to the MFMAs therefore stay at or below 2^12,
  // far inside fp16, and rows whose max moves by less than that skip the max entirely.
  // Diagonal 32x32 tile (first key = first row): register r of the lane holds key offset
  // kappa(r, h2) of row offset l32; keys past the row are hidden.
  bool diag_hide[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) diag_hide[r] = CAUSAL && kappa(r, h2) > l32;
  // Probabilities of one 32x32 tile with the row max as it stands; with MASK, keys whose hide[r]
  // is set get probability 0 (applied after the exponential, so no inf - inf arises).
  auto tile_probs = [&](const f32x16& st, V8* pt, float nm, const bool* hide, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    float acc_s = 0.0f;
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      V8 x;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float e0 = fast_exp2(__builtin_fmaf(st[8 * sg + i], c, nm));
        float e1 = fast_exp2(__builtin_fmaf(st[8 * sg + i + 1], c, nm));
        if constexpr (MASK) {
          e0 = hide[8 * sg + i] ? 0.0f : e0;
          e1 = hide[8 * sg + i + 1] ? 0.0f : e1;
        }
        const V2 pr = H::pack(e0, e1);
        acc_s = H::sum2(pr, acc_s);
        x[i] = pr[0];
        x[i + 1] = pr[1];
      }
      pt[sg] = x;
    }
    return acc_s;
  };
  auto fast_probs = [&](f32x16* scur, V8 (*pc)[2], float* ps) {
    bool need = false;
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      ps[j] = tile_probs(scur[j], pc[j], -mrow[j], nullptr, std::false_type{});
      need |= !(ps[j] <= 4096.0f);
    }
    return need;
  };
  // Steps that need a mask (keys past the sequence end, or causal steps across the workgroup's
  // diagonal) take the same fast path per 32x32 tile, by the tile's place against the diagonal
  // (wave-uniform): keys all at or below its rows: as is; keys all above: probabilities zero, no
  // exponentials; on the diagonal (first row = first key): keys past the row hidden with the
  // fixed lane pattern diag_hide (key offset kappa(r, h2) > row offset l32). In the step holding
  // the sequence end, key offsets N - 32i and beyond are hidden as well. Hidden keys get
  // probability 0, set after the exponential (no inf - inf); the slow path masks in full.
  auto mask_probs = [&](f32x16* scur, V8 (*pc)[2], float* ps, int i) {
    bool need = false;
    const int kend = N - 32 * i - 8 * h2;  // register r is past the end if 16(r/8) + r%8 >= kend
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const int rel = CAUSAL ? qw0 + 32 * j - 32 * i : 32;
      if (rel < 0) {
        pc[j][0] = pc[j][1] = V8{};
        ps[j] = 0.0f;
        continue;
      }
      bool hide[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) hide[r] = (rel == 0 && diag_hide[r]) || 16 * (r >> 3) + (r & 7) >= kend;
      ps[j] = tile_probs(scur[j], pc[j], -mrow[j], hide, std::true_type{});
      need |= !(ps[j] <= 4096.0f);
    }
    return need;
  };
  // kc_: K buffer still holding this step's keys: the slow path recomputes S from it, so S
  // need not stay live through the fast path. The slow path is the body of a one-sided branch
  // (the fast path's state updates come first and are undone there): a two-sided branch that
  // updates the accumulators on one side only makes the register allocator double them.
  auto fast_fixup = [&](bool need, f32x16* scur, V8 (*pc)[2], const float* ps, int kc_, int kb,
                        auto mask_tag) {
    float lprev[QT];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      lprev[j] = lrow[j];
      lrow[j] += ps[j];
    }
    if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
      for (int j = 0; j < QT; ++j) lrow[j] = lprev[j];
      qk(scur, kc_);
      float alpha[QT];
      (void)softmax(scur, pc, alpha, kb, mask_tag);
#pragma unroll
      for (int j = 0; j < QT; ++j)
#pragma unroll
        for (int u = 0; u < DT; ++u) acc[u][j] *= alpha[j];
    }
  };

  // Prologue: K_0..K_2 and V_0..V_2 into slots 0..2; V slot 3 (read by a full step 0 together
  // with all-zero probabilities) cleared.
  dma(0, 0, 0, 0);
  dma(1, 1, 1, 1);
  dma(2, 2, 2, 2);
  for (int o = tid * 16; o < L::VSLOT; o += NT * 16) st16(vs3 + o, u32x4{0, 0, 0, 0});
  __syncthreads();

  f32x16 sa[QT], sb[QT];
  V8 pa[QT][2], pb[QT][2];
#pragma unroll
  for (int j = 0; j < QT; ++j) pa[j][0] = pa[j][1] = V8{};
  if (wave_steps > 0) {
    qk(sa, 0);
    // Running max seeded with step 0's row max over its visible keys (what the slow path would
    // set there), so step 0 takes the fast path like any other step.
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const int q = qw0 + 32 * j + l32;
      float mx = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kappa(r, h2);
        mx = (key < N && (!CAUSAL || key <= q)) ? __builtin_fmaxf(mx, sa[j][r] * c) : mx;
      }
      mrow[j] = max_halves(mx);
    }
  }

  // Steps before n_full need no mask for any wave of the workgroup (all keys below the
  // workgroup's first query row and inside the sequence): they run four per trip so ring
  // slots are constants and the S / P registers swap roles without copies. Tiles fetched past
  // the sequence end are harmless (zeros into a free slot). Later steps mask per tile and let
  // waves above their diagonal idle.
  const int n_full = CAUSAL ? min((qblk + 1) / 32, N / 32) : N / 32;

  // Full step i with i % 4 == IV: PV of step i-1 (pprev), S of step i+1, softmax of step i;
  // K_{i+3} and V_{i+1} start streaming into the slots freed two steps ago. The instruction
  // order within the step is left to the compiler (measured faster than pinned MFMA/VALU
  // interleave patterns).
  auto full_step = [&](int i, f32x16* scur, f32x16* snext, const V8 (*pprev)[2], V8 (*pcur)[2],
                       auto iv_tag) {
    constexpr int IV = decltype(iv_tag)::value;
    dma(i + 3, i + 1, (IV + 3) % 4, (IV + 1) % 4);
    pv_mma(pprev, (IV + 3) % 4);
    qk(snext, (IV + 1) % 4);
    float ps[QT];
    const bool need = fast_probs(scur, pcur, ps);
    fast_fixup(need, scur, pcur, ps, IV, 0, std::false_type{});
    step_end();
  };

  int i = 0;
  for (; i + 3 < n_full; i += 4) {
    full_step(i, sa, sb, pa, pb, std::integral_constant<int, 0>{});
    full_step(i + 1, sb, sa, pb, pa, std::integral_constant<int, 1>{});
    full_step(i + 2, sa, sb, pa, pb, std::integral_constant<int, 2>{});
    full_step(i + 3, sb, sa, pb, pa, std::integral_constant<int, 3>{});
  }
  // Remaining steps (masked or not) with run-time slots; state: scur = sa, pprev = pa.
  for (; i < nsteps; ++i) {
    dma(i + 3, i + 1, (i + 3) & 3, (i + 1) & 3);
    if (i > 0 && i - 1 < wave_steps) pv_mma(pa, (i + 3) & 3);
    if (i < wave_steps) {
      qk(sb, (i + 1) & 3);
      float ps[QT];
      const bool need = i >= n_full ? mask_probs(sa, pb, ps, i) : fast_probs(sa, pb, ps);
      fast_fixup(need, sa, pb, ps, i & 3, 32 * i, std::true_type{});
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        sa[j] = sb[j];
        pa[j][0] = pb[j][0];
        pa[j][1] = pb[j][1];
      }
    }
    step_end();
  }
  if (wave_steps == nsteps && nsteps > 0) pv_mma(pa, (nsteps - 1) & 3);
  // No LDS DMA may still be in flight when the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const float lt = sum_halves(lrow[j]);
    const float inv = 1.0f / lt;
    const int q = qw0 + 32 * j + l32;
    if (q < N) {
      T* orow = O + (int64_t)q * son;
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int g2 = 0; g2 < 4; ++g2) {
          const int d0 = 32 * u + 8 * g2 + 4 * h2;
          if (d0 < D) {
            V4 x;
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) x[i2] = (T)(acc[u][j][4 * g2 + i2] * inv);
            *reinterpret_cast<V4*>(orow + d0) = x;
          }
        }
      if (h2 == 0 && M) M[q] = mrow[j] + __log2f(lt);
    }
  }
}

}  // namespace tattn

#include "fwd_persist.h"

namespace tattn {

// ---- launch ------------------------------------------------------------------------------

template <typename T, int D, int I>
static int launch_fwd_entry(const FwdParams& p0, bool causal, hipStream_t st) {
  constexpr TileEntry e = FwdTable<T, D>::e[I];
  constexpr int BM = e.nw * e.tiles * 32;
  FwdParams p = p0;
  p.n_qblocks = (p.N + BM - 1) / BM;
  const int64_t blocks = (int64_t)p.n_qblocks * p.Z * p.H;
  if (blocks > 0x7fffffff) return set_error(TATTN_E_ARG, "grid too large: %lld workgroups", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(e.nw * 64);
  const bool fits32 = slice_bytes(p.N, p.sk[2], D) + (uint64_t)p.sk[2] * 128 < (1ull << 31) &&
                      slice_bytes(p.N, p.sv[2], D) + (uint64_t)p.sv[2] * 128 < (1ull << 31);
  if constexpr (sizeof(T) == 2) {  // fp16, bf16: the pipelined kernel
    static_assert(e.other == 32, "the 16-bit forward runs 32 keys per step");
    if (!fits32) {  // slices beyond 2 GiB: 64-bit addressing
      if (causal)
        fwd_generic_kernel<T, D, 4, 1, 64, true, D == 128 ? 1 : 2><<<dim3((unsigned)(((p.N + 127) / 128) * (int64_t)p.Z * p.H)), dim3(256), 0, st>>>(
            [&] { FwdParams q = p; q.n_qblocks = (p.N + 127) / 128; return q; }());
      else
        fwd_generic_kernel<T, D, 4, 1, 64, false, D == 128 ? 1 : 2><<<dim3((unsigned)(((p.N + 127) / 128) * (int64_t)p.Z * p.H)), dim3(256), 0, st>>>(
            [&] { FwdParams q = p; q.n_qblocks = (p.N + 127) / 128; return q; }());
      return check_launch("tattn_fwd");
    }
    if constexpr (e.pipe == 2) {  // persistent, where the problem fits it
      int rc = TATTN_OK;
      if (causal) {
        if constexpr (fwd_persist_causal_ok(e) && e.tiles == 2) {  // own translation unit
          if (launch_fwd_persist_causal2(p0, D, std::is_same_v<T, bf16> ? 2 : 0, I, st, &rc) == 0) return rc;
        } else if constexpr (fwd_persist_causal_ok(e)) {
          if (launch_fwd_persist<T, D, e.nw, e.tiles, e.occ, true, e.ring>(p0, st, &rc) == 0) return rc;
        }
      } else if (launch_fwd_persist<T, D, e.nw, e.tiles, e.occ, false, e.ring>(p0, st, &rc) == 0) {
        return rc;
      }
    }
    if (causal)
      fwd_pipe_kernel<T, D, e.nw, e.tiles, e.occ, true><<<grid, block, 0, st>>>(p);
    else
      fwd_pipe_kernel<T, D, e.nw, e.tiles, e.occ, false><<<grid, block, 0, st>>>(p);
  } else {
    if (causal)
      fwd_generic_kernel<T, D, e.nw, e.tiles, e.other, true, e.occ><<<grid, block, 0, st>>>(p);
    else
      fwd_generic_kernel<T, D, e.nw, e.tiles, e.other, false, e.occ><<<grid, block, 0, st>>>(p);
  }
  return check_launch("tattn_fwd");
}

template <typename T, int D, size_t... I>
static int dispatch_fwd(int id, const FwdParams& p, bool causal, hipStream_t st, std::index_sequence<I...>) {
  int rc = set_error(TATTN_E_CONFIG, "forward config id %d out of range [0, %d) for D=%d", id,
                     (int)sizeof...(I), D);
  ((id == (int)I ? (rc = launch_fwd_entry<T, D, I>(p, causal, st), 0) : 0), ...);
  return rc;
}

template <typename T, int D>
static int run_fwd_d(int id, const FwdParams& p, bool causal, hipStream_t st) {
  return dispatch_fwd<T, D>(id, p, causal, st, std::make_index_sequence<FwdTable<T, D>::n>{});
}

int launch_fwd(const FwdParams& p, int D, int dtype, bool causal, int id, hipStream_t st) {
  if (dtype == 0) {
    switch (D) {
      case 16: return run_fwd_d<f16, 16>(id, p, causal, st);
      case 32: return run_fwd_d<f16, 32>(id, p, causal, st);
      case 64: return run_fwd_d<f16, 64>(id, p, causal, st);
      case 128: return run_fwd_d<f16, 128>(id, p, causal, st);
    }
  } else if (dtype == 2) {
    switch (D) {
      case 16: return run_fwd_d<bf16, 16>(id, p, causal, st);
      case 32: return run_fwd_d<bf16, 32>(id, p, causal, st);
      case 64: return run_fwd_d<bf16, 64>(id, p, causal, st);
      case 128: return run_fwd_d<bf16, 128>(id, p, causal, st);
    }
  } else {
    switch (D) {
      case 16: return run_fwd_d<float, 16>(id, p, causal, st);
      case 32: return run_fwd_d<float, 32>(id, p, causal, st);
      case 64: return run_fwd_d<float, 64>(id, p, causal, st);
      case 128: return run_fwd_d<float, 128>(id, p, causal, st);
    }
  }
  return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %d", D);
}

int fwd_lds_bytes(int D, int dtype, const TileEntry& e) {
  if ((dtype == 0 || dtype == 2) && e.pipe == 2) {
    const int slot = 32 * (D < 32 ? 64 : 2 * D);
    return 2 * e.ring * slot + fwd_persist_ostage_bytes(D, e);
  }
  if (dtype == 0 || dtype == 2) {
    switch (D) {
      case 16: return PipeLayout<16>::LDS;
      case 32: return PipeLayout<32>::LDS;
      case 64: return PipeLayout<64>::LDS;
      case 128: return PipeLayout<128>::LDS;
    }
  }
  const int sz = dtype == 1 ? 4 : 2;
  const int rk = D * sz + 16, rv = D * sz + (sz == 2 ? 32 : 16);
  return 2 * e.other * (rk + rv);
}

}  // namespace tattn
