// dK/dV with split wave roles, 16-bit, for gfx950.
//
// Same math and rounding points as dkdv_pipe_kernel (the reference's
// src/tattn/kernels.py:151-239): P = exp2(S c - M) in fp32, dS = P (dP - delta) in fp32, both
// rounded to the element type only as MFMA operands, dK scaled by sm_scale at the store. What
// changes is who does what. A workgroup has eight waves in four pairs; pair j owns the 32 keys
// kblk + 32 j + (lane % 32). Over each 32-query step:
//   wave j     (role A): S = Q K^T, P = exp2(S c - M), dV += P^T dO
//   wave j + 4 (role B): dP - delta = dO V^T - delta, dS = P (dP - delta), dK += dS^T Q
// B takes P from A through LDS as computed (fp32), so dS has the reference's rounding. Each wave
// keeps one of K / V as its B operand and one accumulator set, about half the registers of the
// one-wave-per-tile kernel: at head dim 128 two waves share each SIMD (waves j and j + 4 sit on
// the same SIMD, so each SIMD runs one wave of each role), where dkdv_pipe_kernel needs all 512
// registers of one wave per SIMD.
//
// Schedule of step i (one barrier per step; stage = i % 4 of the 4-deep Q / dO / M / delta ring):
//   A: S_{i+1} (stage i+1) and dV += P_{i-1}^T dO_{i-1} (stage i-1) on the matrix cores while
//      the VALU computes P_i from S_i and M (stage i); P_i goes to LDS buffer i % 2.
//   B: dP_i - delta_i (stage i) on the matrix cores while the VALU forms dS_{i-1} from P_{i-1}
//      (buffer (i-1) % 2, written by A in step i-1) and dP_{i-1}; then dK += dS_{i-1}^T Q_{i-1}
//      (stage i-1).
// All waves stage the rows of step i+2 into stage (i+2) % 4.
#pragma once

#include <type_traits>

#include "bwd_pipe.h"

namespace tattn {

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(512, 2) void dkdv_split_kernel(const BwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V2 = typename H::V2;
  using B = BwdPipe<D>;
  constexpr int NW = 8, NP = 4, NT = NW * 64, BNK = NP * 32;
  constexpr int STAGE = B::DKDV_STAGE;
  constexpr int CPT = (B::CHUNKS + NT - 1) / NT;
  constexpr int NSD = B::NSD, DT = B::DT;
  constexpr int XB = 32 * 32 * 4;  // P of one pair and step, fp32
  __shared__ __attribute__((aligned(16))) char smem[B::NST * STAGE];
  __shared__ __attribute__((aligned(16))) char xbuf[2 * NP * XB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int wu = (int)uniform32((uint32_t)w);  // in a scalar register: the role branches are uniform
  const int pr = wu & (NP - 1);
  const bool role_b = wu >= NP;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_blocks, !CAUSAL);
  const int zh = bc.zh, kbi = bc.blk;  // causal: small key blocks (most work) first
  const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
  const int64_t rs = p.s[2];
  const float c = p.c;
  const int kblk = kbi * BNK;
  const int kw0 = kblk + 32 * pr;
  // Causal: query blocks below this key block never see its keys (kernels.py:206-208).
  const int lo = CAUSAL ? kblk : 0;
  const int nsteps = (N - lo + 31) / 32;

  // The wave's B operand: K rows (role A) or V rows (role B) of its pair's keys.
  V8 kv[NSD];
  {
    const int key = kw0 + l32;
    const T* src = (const T*)(role_b ? p.v : p.k) + hoff + (int64_t)(key < N ? key : 0) * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      const V8 a = *reinterpret_cast<const V8*>(src + 16 * s);
      kv[s] = key < N ? a : V8{};
    }
  }
  f32x16 acc[DT];  // dV (role A) or dK (role B)
#pragma unroll
  for (int u = 0; u < DT; ++u) acc[u] = f32x16{};

  const __amdgpu_buffer_rsrc_t qrs = slice_rsrc((const T*)p.q + hoff + (int64_t)lo * rs, slice_bytes(N - lo, rs, D));
  const __amdgpu_buffer_rsrc_t ors = slice_rsrc((const T*)p.dout + hoff + (int64_t)lo * rs, slice_bytes(N - lo, rs, D));
  const __amdgpu_buffer_rsrc_t mrs = slice_rsrc(p.m + (int64_t)zh * N + lo, (uint64_t)(N - lo) * 4);
  const __amdgpu_buffer_rsrc_t drs = slice_rsrc(p.delta + (int64_t)zh * N + lo, (uint64_t)(N - lo) * 4);
  const uint32_t step_bytes = uniform32((uint32_t)(rs * 64));

  uint32_t goff[CPT];
  int ldst[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int ch = min(tid + i * NT, B::CHUNKS - 1);
    const int row = ch / B::CPR, cb = (ch % B::CPR) * 16;
    goff[i] = (uint32_t)(row * rs * 2 + cb);
    ldst[i] = Swz<D>::addr(perm32(row), cb);
  }
  const bool md_loader = tid < 64;
  const int md_dst = 2 * B::TILE + tid * 4;

  int nat[NSD];
#pragma unroll
  for (int s = 0; s < NSD; ++s) nat[s] = Swz<D>::addr(l32, (16 * s + 8 * h2) * 2);
  int tra[2][DT][2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int u = 0; u < DT; ++u) tr_addrs<D>(sl, u, lane, tra[sl][u][0], tra[sl][u][1]);
  const int mo = 2 * B::TILE + 32 * h2;  // M of queries 8*h2.. (bytes); -delta at +128
  // P exchange: chunk k (registers 4k..4k+3) of lane l at 1024 k + 16 l (conflict-free 16-byte
  // accesses); the A and B waves of a pair share the C layout (lane = key, register = query).
  char* xpair = xbuf + pr * XB;

  // Register stage of one step's Q, dO, M and delta (the loop uses set 0; the prologue also set 1).
  u32x4 pq[2][CPT], pd[2][CPT];
  uint32_t pm[2], pdl[2];
  auto gload = [&](int step, auto set_tag) {
    constexpr int R = decltype(set_tag)::value;
    const uint32_t so = (uint32_t)step * step_bytes;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      pq[R][i] = rsrc_load(qrs, goff[i] + so);
      pd[R][i] = rsrc_load(ors, goff[i] + so);
    }
    const uint32_t mo4 = (uint32_t)(((tid & 31) + 32 * step) * 4);
    pm[R] = __builtin_amdgcn_raw_buffer_load_b32(mrs, (int)mo4, 0, 0);
    pdl[R] = __builtin_amdgcn_raw_buffer_load_b32(drs, (int)mo4, 0, 0);
  };
  auto lstore = [&](int st, auto set_tag) {
    constexpr int R = decltype(set_tag)::value;
    char* base = smem + st * STAGE;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      if (B::CHUNKS % NT == 0 || tid + i * NT < B::CHUNKS) {
        st16(base + ldst[i], pq[R][i]);
        st16(base + B::TILE + ldst[i], pd[R][i]);
      }
    // delta is staged negated: it seeds the dP accumulator, so dP - delta comes out of the MFMAs.
    if (md_loader) *reinterpret_cast<uint32_t*>(base + md_dst) = (tid & 32) ? (pdl[R] ^ 0x80000000u) : pm[R];
  };

  // Role A: S = Q K^T of stage st.  Role B: dP - delta = dO V^T - delta of stage st.
  auto mma_first = [&](f32x16& s, int st, bool b) {
    const char* base = smem + st * STAGE;
    if (b) {
      const TATTN_LDS char* nd = (const TATTN_LDS char*)base + mo + 128;
      const f32x4 n0 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd);
      const f32x4 n1 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 16);
      const f32x4 n2 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 64);
      const f32x4 n3 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 80);
      s = f32x16{n0[0], n0[1], n0[2], n0[3], n1[0], n1[1], n1[2], n1[3],
                 n2[0], n2[1], n2[2], n2[3], n3[0], n3[1], n3[2], n3[3]};
    } else {
      s = f32x16{};
    }
    const char* tile = base + (b ? B::TILE : 0);
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) s = Elt<T>::mfma(lds8<T>(tile + nat[sd]), kv[sd], s);
  };
  // Role A: dV += P^T dO.  Role B: dK += dS^T Q.  Over the 32 queries of stage st.
  auto mma_grad = [&](const V8 (&op)[2], int st, bool b) {
    const char* tile = smem + st * STAGE + (b ? 0 : B::TILE);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int u = 0; u < DT; ++u) {
        V8 x = tr_pair<T>(tile, tra[sl][u][0], tra[sl][u][1]);
        if (D < 32 && 16 * ((lane >> 4) & 1) >= D) x = V8{};
        acc[u] = Elt<T>::mfma(op[sl], x, acc[u]);
      }
  };
  // Role A: P = exp2(S c - M) of stage st (queries q0..q0+31), into LDS buffer xb (fp32) and into
  // MFMA operands.
  auto probs = [&](const f32x16& s, V8 (&pp)[2], int st, int q0, int xb, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const char* base = smem + st * STAGE;
    const int key = kw0 + l32;
    char* xo = xpair + xb * (NP * XB) + 16 * lane;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const f32x4 m0 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)base + mo + 64 * a);
      const f32x4 m1 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)base + mo + 64 * a + 16);
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = 8 * a + e;
        const float mv = e < 4 ? m0[e] : m1[e - 4];
        float x = fast_exp2(__builtin_fmaf(s[r], c, -mv));
        if constexpr (MASK) x = key > q0 + kappa(r, h2) ? 0.0f : x;
        pv[e] = x;
      }
      *reinterpret_cast<TATTN_LDS f32x4*>((TATTN_LDS char*)xo + 1024 * (2 * a)) = f32x4{pv[0], pv[1], pv[2], pv[3]};
      *reinterpret_cast<TATTN_LDS f32x4*>((TATTN_LDS char*)xo + 1024 * (2 * a + 1)) = f32x4{pv[4], pv[5], pv[6], pv[7]};
      V8 o;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const V2 ph = H::pack(pv[e], pv[e + 1]);
        o[e] = ph[0];
        o[e + 1] = ph[1];
      }
      pp[a] = o;
    }
  };
  // Role B: dS = P (dP - delta) from LDS buffer xb and dp, into MFMA operands.
  auto dsv = [&](const f32x16& dp, V8 (&dsp)[2], int xb) {
    const char* xi = xpair + xb * (NP * XB) + 16 * lane;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const f32x4 p0 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)xi + 1024 * (2 * a));
      const f32x4 p1 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)xi + 1024 * (2 * a + 1));
      V8 o;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = (e < 4 ? p0[e] : p1[e - 4]) * dp[8 * a + e];
        const float x1 = (e + 1 < 4 ? p0[e + 1] : p1[e - 3]) * dp[8 * a + e + 1];
        const V2 dh = H::pack(x0, x1);
        o[e] = dh[0];
        o[e + 1] = dh[1];
      }
      dsp[a] = o;
    }
  };

  // Prologue: steps 0 and 1 into stages 0 and 1 (both loads in flight together); stage 3 (read
  // by role A's first dV MFMAs together with all-zero P) cleared.
  gload(0, IC<0>{});
  gload(1, IC<1>{});
#pragma unroll
  for (int i = 0; i < CPT; ++i)
    if (B::CHUNKS % NT == 0 || tid + i * NT < B::CHUNKS) {
      st16(smem + 3 * STAGE + ldst[i], u32x4{0, 0, 0, 0});
      st16(smem + 3 * STAGE + B::TILE + ldst[i], u32x4{0, 0, 0, 0});
    }
  lstore(0, IC<0>{});
  lstore(1, IC<1>{});
  __syncthreads();

  // Each role runs its own copy of the step loop (the branch is wave-uniform); both copies meet
  // the same barriers.
  auto run = [&](auto role_tag) {
    constexpr bool RB_ = decltype(role_tag)::value;
    // A: S of the current step and of the next, P operands of the previous and current step.
    // B: dP - delta of the previous step and of the current one; dS operands (temporary).
    f32x16 sa = f32x16{}, sb = f32x16{};
    V8 pa[2] = {V8{}, V8{}}, pb[2] = {V8{}, V8{}};
    if (!RB_ && nsteps > 0) mma_first(sa, 0, false);
    // Step i with stage st; x0 / x1: the register sets in their roles for this step (swapped every
    // step in the unrolled loop, so no copies).
    auto step = [&](int i, int st, f32x16& x0, f32x16& x1, V8 (&q0)[2], V8 (&q1)[2], auto mask_tag) {
      const bool live_prev = !CAUSAL || i - 1 >= pr;
      const bool live_cur = !CAUSAL || i >= pr;
      gload(i + 2, IC<0>{});
      if constexpr (!RB_) {  // x0 = S_i, x1 <- S_{i+1}; q0 = P_{i-1}, q1 <- P_i
        if (!CAUSAL || i + 1 >= pr) mma_first(x1, (st + 1) & 3, false);
        if (live_prev) mma_grad(q0, (st + 3) & 3, false);
        if (live_cur) probs(x0, q1, st, lo + 32 * i, i & 1, mask_tag);
      } else {  // x0 = dP_{i-1}, x1 <- dP_i; q1: dS_{i-1}
        if (live_cur) mma_first(x1, st, true);
        if (i > 0 && live_prev) {
          dsv(x0, q1, (i - 1) & 1);
          mma_grad(q1, (st + 3) & 3, true);
        }
      }
      lstore((st + 2) & 3, IC<0>{});
      __syncthreads();
    };
    auto roll = [&]() {
      sa = sb;
      pa[0] = pb[0];
      pa[1] = pb[1];
    };
    int i = 0;
    const int n_mask = CAUSAL ? min(nsteps, NP) : 0;
    for (; i < n_mask; ++i) {
      step(i, i & 3, sa, sb, pa, pb, std::true_type{});
      roll();
    }
    for (; i + 3 < nsteps; i += 4) {  // i % 4 == 0 here
      step(i, 0, sa, sb, pa, pb, std::false_type{});
      step(i + 1, 1, sb, sa, pb, pa, std::false_type{});
      step(i + 2, 2, sa, sb, pa, pb, std::false_type{});
      step(i + 3, 3, sb, sa, pb, pa, std::false_type{});
    }
    for (; i < nsteps; ++i) {
      step(i, i & 3, sa, sb, pa, pb, std::false_type{});
      roll();
    }
    // Last step's gradients: A's dV from P_{L-1}, B's dS_{L-1} from A's last P buffer.
    if (nsteps > 0 && (!CAUSAL || nsteps - 1 >= pr)) {
      if constexpr (!RB_) {
        mma_grad(pa, (nsteps - 1) & 3, false);
      } else {
        dsv(sa, pb, (nsteps - 1) & 1);
        mma_grad(pb, (nsteps - 1) & 3, true);
      }
    }
  };
  if (role_b) run(std::true_type{});
  else run(std::false_type{});

  // Store through LDS, as dkdv_pipe_kernel: each wave writes its tile row-major into a private
  // block of the ring and stores whole 16-byte chunks of rows.
  __syncthreads();
  constexpr int RB = B::RB;
  constexpr int CPRO = D / 8;
  constexpr int SPW = (32 * CPRO + 63) / 64;
  static_assert(NW * 32 * RB <= B::NST * STAGE, "store blocks fit the ring");
  const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int l32e = ln & 31, h2e = ln >> 5;
  char* wb = smem + wu * 32 * RB;
  const float mul = role_b ? p.scale : 1.0f;
  T* dst = (T*)(role_b ? p.dk : p.dv) + hoff;
  {
    TATTN_LDS T* wl = (TATTN_LDS T*)((TATTN_LDS char*)wb + 4 * h2e * RB) + l32e;
#pragma unroll
    for (int u = 0; u < DT; ++u)
      if (32 * u + l32e < D) {
#pragma unroll
        for (int r = 0; r < 16; ++r) wl[(8 * (r >> 2) + (r & 3)) * (RB / 2) + 32 * u] = (T)(acc[u][r] * mul);
      }
#pragma unroll
    for (int it = 0; it < SPW; ++it) {
      const int j = ln + 64 * it;
      const int row = j / CPRO, cc = j % CPRO;
      const int key = kw0 + row;
      if (row < 32 && key < N) {
        const u32x4 v = *reinterpret_cast<const TATTN_LDS u32x4*>((const TATTN_LDS char*)wb + row * RB + 16 * cc);
        st16_stream(dst + (int64_t)key * rs + 8 * cc, v);
      }
    }
  }
}

// dQ with split wave roles (the reference's src/tattn/kernels.py:242-321), the same pairing: eight
// waves, four pairs; pair j owns the 32 queries qblk + 32 j + (lane % 32). Over each 32-key step:
//   wave j     (role A): S^T = K Q^T, P = exp2(S c - M) (masked), P to LDS (fp32)
//   wave j + 4 (role B): dP^T - delta = V dO^T - delta, dS = P (dP - delta),
//                        dQ^T += K^T dS^T
// B holds the dQ accumulator and both of its operands' register sets are halved against
// dq_pipe_kernel (A keeps Q, B keeps dO). Same rounding points and summation order as
// dq_pipe_kernel: the results are bitwise those of that kernel.
// Step j (stage j % 4 holds K_j and V_j): A computes S_{j+1} while its VALU forms P_j; B computes
// dP_j while its VALU forms dS_{j-1} from P_{j-1} (written by A in step j-1), then
// dQ^T += K_{j-1}^T dS_{j-1}^T.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(512, 2) void dq_split_kernel(const BwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V4 = typename H::V4;
  using V2 = typename H::V2;
  using B = BwdPipe<D>;
  constexpr int NW = 8, NP = 4, NT = NW * 64, BMQ = NP * 32;
  constexpr int STAGE = B::DQ_STAGE;
  constexpr int CPT = (B::CHUNKS + NT - 1) / NT;
  constexpr int NSD = B::NSD, DT = B::DT;
  constexpr int XB = 32 * 32 * 4;  // P of one pair and step, fp32
  __shared__ __attribute__((aligned(16))) char smem[B::NST * STAGE];
  __shared__ __attribute__((aligned(16))) char xbuf[2 * NP * XB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int wu = (int)uniform32((uint32_t)w);  // in a scalar register: the role branches are uniform
  const int pr = wu & (NP - 1);
  const bool role_b = wu >= NP;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_blocks, !CAUSAL);
  const int zh = bc.zh;
  int qb = bc.blk;
  if (CAUSAL) qb = p.n_blocks - 1 - qb;  // longest rows first
  const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
  const int64_t rs = p.s[2];
  const float c = p.c;
  const int qblk = qb * BMQ;
  const int qw0 = qblk + 32 * pr;
  const int q = qw0 + l32;

  // The wave's B operand: Q rows (role A) or dO rows (role B) of its pair's queries.
  V8 op[NSD];
  {
    const int64_t off = hoff + (int64_t)(q < N ? q : 0) * rs + 8 * h2;
    const T* src = (const T*)(role_b ? p.dout : p.q) + off;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      const V8 a = *reinterpret_cast<const V8*>(src + 16 * s);
      op[s] = q < N ? a : V8{};
    }
  }
  // Role A: -M of the lane's query. Role B: delta (computed here from O and dO when fuse_delta,
  // in the preprocess's summation order, and stored for the dK/dV kernel that follows).
  float nm = 0.0f, dl = 0.0f;
  if (!role_b) {
    nm = -(q < N ? p.m[(int64_t)zh * N + q] : 0.0f);
  } else if (p.fuse_delta) {
    float sd[NSD];
    const int64_t off = hoff + (int64_t)(q < N ? q : 0) * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) sd[s] = chunk_dot(*reinterpret_cast<const V8*>((const T*)p.o + off + 16 * s), op[s]);
    dl = row_delta(sd);
    if (q >= N) dl = 0.0f;
    else if (h2 == 0) p.delta[(int64_t)zh * N + q] = dl;
  } else {
    dl = q < N ? p.delta[(int64_t)zh * N + q] : 0.0f;
  }

  const int hi = CAUSAL ? min(qblk + BMQ, N) : N;
  const int nsteps = (hi + 31) / 32;
  // Steps this pair computes: every step up to the one holding its last query row.
  const int pair_steps = qw0 >= N ? 0 : CAUSAL ? min(nsteps, (qw0 + 31) / 32 + 1) : nsteps;
  // Steps before n_full need no mask for any pair of the workgroup.
  const int n_full = CAUSAL ? min((qblk + 1) / 32, N / 32) : N / 32;

  const __amdgpu_buffer_rsrc_t krs = slice_rsrc((const T*)p.k + hoff, slice_bytes(N, rs, D));
  const __amdgpu_buffer_rsrc_t vrs = slice_rsrc((const T*)p.v + hoff, slice_bytes(N, rs, D));
  const uint32_t step_bytes = uniform32((uint32_t)(rs * 64));
  uint32_t goff[CPT];
  int ldst[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int ch = min(tid + i * NT, B::CHUNKS - 1);
    const int row = ch / B::CPR, cb = (ch % B::CPR) * 16;
    goff[i] = (uint32_t)(row * rs * 2 + cb);
    ldst[i] = Swz<D>::addr(perm32(row), cb);
  }
  int nat[NSD];
#pragma unroll
  for (int s = 0; s < NSD; ++s) nat[s] = Swz<D>::addr(l32, (16 * s + 8 * h2) * 2);
  int tra[2][DT][2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int u = 0; u < DT; ++u) tr_addrs<D>(sl, u, lane, tra[sl][u][0], tra[sl][u][1]);
  char* xpair = xbuf + pr * XB;

  u32x4 pk[2][CPT], pv[2][CPT];
  auto gload = [&](int step, auto set_tag) {
    constexpr int R = decltype(set_tag)::value;
    const uint32_t so = (uint32_t)step * step_bytes;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      pk[R][i] = rsrc_load(krs, goff[i] + so);
      pv[R][i] = rsrc_load(vrs, goff[i] + so);
    }
  };
  auto lstore = [&](int st, auto set_tag) {
    constexpr int R = decltype(set_tag)::value;
    char* base = smem + st * STAGE;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      if (B::CHUNKS % NT == 0 || tid + i * NT < B::CHUNKS) {
        st16(base + ldst[i], pk[R][i]);
        st16(base + B::TILE + ldst[i], pv[R][i]);
      }
  };

  // Role A: S^T = K Q^T.  Role B: dP^T - delta = V dO^T - delta.  Over the 32 keys of stage st.
  auto mma_first = [&](f32x16& s, int st, bool b) {
    if (b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = -dl;
    } else {
      s = f32x16{};
    }
    const char* tile = smem + st * STAGE + (b ? B::TILE : 0);
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) s = Elt<T>::mfma(lds8<T>(tile + nat[sd]), op[sd], s);
  };
  f32x16 dq[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) dq[u] = f32x16{};
  // Role B: dQ^T += K^T dS^T over the 32 keys of stage st.
  auto dq_mma = [&](const V8 (&dsp)[2], int st) {
    const char* base = smem + st * STAGE;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int u = 0; u < DT; ++u) {
        V8 a = tr_pair<T>(base, tra[sl][u][0], tra[sl][u][1]);
        if (D < 32 && 16 * ((lane >> 4) & 1) >= D) a = V8{};
        dq[u] = Elt<T>::mfma(a, dsp[sl], dq[u]);
      }
  };
  // Role A: P of the step's keys kb.. (masked past the diagonal and the sequence end) into LDS
  // buffer xb, fp32.
  auto probs = [&](const f32x16& s, int kb, int xb, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    char* xo = xpair + xb * (NP * XB) + 16 * lane;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * a + e;
        float x = fast_exp2(__builtin_fmaf(s[r], c, nm));
        if constexpr (MASK) {
          const int key = kb + kappa(r, h2);
          x = (key >= N || (CAUSAL && key > q)) ? 0.0f : x;
        }
        v[e] = x;
      }
      *reinterpret_cast<TATTN_LDS f32x4*>((TATTN_LDS char*)xo + 1024 * a) = v;
    }
  };
  // Role B: dS = P (dP - delta) from LDS buffer xb, rounded into MFMA operands.
  auto dsv = [&](const f32x16& dp, V8 (&dsp)[2], int xb) {
    const char* xi = xpair + xb * (NP * XB) + 16 * lane;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const f32x4 p0 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)xi + 1024 * (2 * a));
      const f32x4 p1 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)xi + 1024 * (2 * a + 1));
      V8 o;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = (e < 4 ? p0[e] : p1[e - 4]) * dp[8 * a + e];
        const float x1 = (e + 1 < 4 ? p0[e + 1] : p1[e - 3]) * dp[8 * a + e + 1];
        const V2 dh = H::pack(x0, x1);
        o[e] = dh[0];
        o[e + 1] = dh[1];
      }
      dsp[a] = o;
    }
  };

  gload(0, IC<0>{});
  gload(1, IC<1>{});
#pragma unroll
  for (int i = 0; i < CPT; ++i)
    if (B::CHUNKS % NT == 0 || tid + i * NT < B::CHUNKS) st16(smem + 3 * STAGE + ldst[i], u32x4{0, 0, 0, 0});
  lstore(0, IC<0>{});
  lstore(1, IC<1>{});
  __syncthreads();

  auto run = [&](auto role_tag) {
    constexpr bool RB_ = decltype(role_tag)::value;
    // A: S of the current step and of the next (sets swapped every step).  B: dP - delta of the
    // previous step, then of the current one (sa only).
    f32x16 sa = f32x16{}, sb = f32x16{};
    V8 ds[2];
    if (!RB_ && pair_steps > 0) mma_first(sa, 0, false);
    auto step = [&](int j, int st, f32x16& x0, f32x16& x1, auto mask_tag) {
      gload(j + 2, IC<0>{});
      if constexpr (!RB_) {  // x0 = S_j, x1 <- S_{j+1}
        if (j + 1 < pair_steps) mma_first(x1, (st + 1) & 3, false);
        if (j < pair_steps) probs(x0, 32 * j, j & 1, mask_tag);
      } else {  // sa = dP_{j-1}, then dP_j (one register set: the other role's wave on the SIMD
                // overlaps this wave's VALU and MFMA work)
        if (j > 0 && j - 1 < pair_steps) {
          dsv(sa, ds, (j - 1) & 1);
          dq_mma(ds, (st + 3) & 3);
        }
        if (j < pair_steps) mma_first(sa, st, true);
      }
      lstore((st + 2) & 3, IC<0>{});
      __syncthreads();
    };
    int j = 0;
    for (; j + 3 < n_full; j += 4) {  // j % 4 == 0 here
      step(j, 0, sa, sb, std::false_type{});
      step(j + 1, 1, sb, sa, std::false_type{});
      step(j + 2, 2, sa, sb, std::false_type{});
      step(j + 3, 3, sb, sa, std::false_type{});
    }
    for (; j < nsteps; ++j) {
      if (j >= n_full)
        step(j, j & 3, sa, sb, std::true_type{});
      else
        step(j, j & 3, sa, sb, std::false_type{});
      if constexpr (!RB_) sa = sb;
    }
    // Last step's dS and dQ (role B), from A's last P buffer.
    if constexpr (RB_) {
      if (pair_steps == nsteps && nsteps > 0) {
        dsv(sa, ds, (nsteps - 1) & 1);
        dq_mma(ds, (nsteps - 1) & 3);
      }
    }
  };
  if (role_b) run(std::true_type{});
  else run(std::false_type{});

  // Store (role B): dQ rows (scaled, rounded) through the pair's rows of the ring, free once every
  // wave is past its last step, then out as whole rows with the non-temporal policy (nothing in
  // the backward reads dQ). The lane index is recomputed here (mbcnt) rather than kept live across
  // the main loop.
  static_assert(NP * 32 * B::RB <= B::NST * STAGE && B::RB == 2 * D, "dQ rows fit the ring");
  __syncthreads();
  const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int l32e = ln & 31, h2e = ln >> 5;
  if (role_b) {
    TATTN_LDS char* wt = (TATTN_LDS char*)smem + pr * 32 * B::RB;
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * u + 8 * g + 4 * h2e;
        V4 x;
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) x[i2] = (T)(dq[u][4 * g + i2] * p.scale);
        *reinterpret_cast<TATTN_LDS V4*>(wt + Swz<D>::addr(l32e, 2 * d0)) = x;
      }
    constexpr int CPRO = D / 8;  // 16-byte chunks of a row
#pragma unroll
    for (int it = 0; it < 32 * CPRO / 64; ++it) {
      const int j = ln + 64 * it;
      const int row = j / CPRO, cc = j % CPRO;
      const int qe = qw0 + row;
      const u32x4 v = *reinterpret_cast<const TATTN_LDS u32x4*>(wt + Swz<D>::addr(row, 16 * cc));
      if (qe < N) st16_stream((T*)p.dq + hoff + (int64_t)qe * rs + 8 * cc, v);
    }
  }
}

}  // namespace tattn
