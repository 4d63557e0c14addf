// Persistent 16-bit dQ kernel for gfx950: one workgroup per resident slot, each running a
// static list of query blocks back to back.
//
// Same math, rounding points, LDS layout (4-deep ring of XOR-swizzled K/V tiles), register-staged
// loads and per-step schedule as dq_pipe_kernel (bwd_pipe.h). What changes is the life of a
// workgroup, as in the persistent forward (fwd_persist.h): at 16-32 steps per block
// (N = 512-1024) the cold start of every block (its Q/dO rows and the first K/V tiles, all
// workgroups of a round at once) and its stores weighed on its time.
//   - The K/V stream runs on across blocks: the last two steps of a block already load the next
//     block's first two stages.
//   - The next block's Q, dO, M and delta are loaded in the block's second-to-last step, right
//     after the last use of Q and dO (no step recomputes from them later); the current block's
//     -M stays in its own register until the block ends.
//   - The block's dQ store overlaps the next block's first step.
// Work items: non-causal, one query block; causal, the pair of query blocks nb-1-p and p of one
// slice, whose step counts add up to the same number for every pair. Items are split per XCD as
// in the forward: XCD x takes the slices zh = x (mod 8), its workgroups consecutive items.
// (A persistent dK/dV built the same way measured slower than dkdv_pipe_kernel: its per-lane
// scattered dK/dV stores then sit inside the step sequence, and it ran out of registers.)
// Preconditions (checked by the launcher, which otherwise runs dq_pipe_kernel): Z*H a multiple
// of 8, N a multiple of the block and of 128, causal: an even number of blocks per slice, 32-bit
// slice offsets.
#pragma once

#include "bwd_pipe.h"

namespace tattn {

// ---- dQ ----------------------------------------------------------------------------------
template <typename T, int D, int NW, int OCC, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, OCC) void dq_persist_kernel(const BwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V4 = typename H::V4;
  using V2 = typename H::V2;
  using B = BwdPipe<D>;
  constexpr int NT = NW * 64, BMQ = NW * 32;
  constexpr int STAGE = B::DQ_STAGE;
  constexpr int CPT = (B::CHUNKS + NT - 1) / NT;
  constexpr int NSD = B::NSD, DT = B::DT;
  constexpr int SPI = CAUSAL ? 2 : 1;
  static_assert(NW % 4 == 0, "diagonal steps in whole groups of four");
  __shared__ __attribute__((aligned(16))) char smem[B::NST * STAGE];
  // Per wave: its 32 dQ rows on their way out (whole-row stores, below).
  __shared__ __attribute__((aligned(16))) char dqs[NW * 32 * B::RB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int nqb = p.n_blocks;
  const int xcd = blockIdx.x & 7, lw = blockIdx.x >> 3;
  const int n_items = lw < p.items_x ? (p.items_x - lw + p.gx - 1) / p.gx : 0;
  const int nseg = n_items * SPI;
  const int64_t rs = p.s[2];
  const float c = p.c;

  auto seg_of = [&](int t, int& zh, int& qb) __attribute__((always_inline)) {
    const int k = lw + p.gx * (t / SPI);
    if constexpr (CAUSAL) {
      const int half = nqb >> 1;
      zh = 8 * (k / half) + xcd;
      const int pr = k % half;
      qb = (t % SPI == 0) ? nqb - 1 - pr : pr;
    } else {
      zh = 8 * (k / nqb) + xcd;
      qb = k % nqb;
    }
  };
  struct Src {
    __amdgpu_buffer_rsrc_t k, v;
  };
  auto src_of = [&](int t) __attribute__((always_inline)) {
    Src s;
    if (t >= nseg) {
      s.k = s.v = slice_rsrc(p.k, 0);
      return s;
    }
    int zh, qb;
    seg_of(t, zh, qb);
    const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
    s.k = slice_rsrc((const T*)p.k + hoff, slice_bytes(N, rs, D));
    s.v = slice_rsrc((const T*)p.v + hoff, slice_bytes(N, rs, D));
    return s;
  };
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

  V8 qop[NSD], dop[NSD];
  float nm = 0.0f, m_next = 0.0f, dl_next = 0.0f;
  f32x16 ndl;
  // The lane's query row of block qb of slice zh: Q and dO into the B-operand registers, its M and
  // delta into m_next / dl_next (the current block's softmax still reads nm until its last step).
  auto load_q = [&](int zh, int qb) __attribute__((always_inline)) {
    const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
    const int qn = qb * BMQ + 32 * w + l32;
    const int64_t off = hoff + (int64_t)qn * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      qop[s] = *reinterpret_cast<const V8*>((const T*)p.q + off + 16 * s);
      dop[s] = *reinterpret_cast<const V8*>((const T*)p.dout + off + 16 * s);
    }
    m_next = p.m[(int64_t)zh * N + qn];
    if (p.fuse_delta) {  // delta = rowsum(dO * O) here, stored for the dK/dV kernel that follows
      float sd[NSD];
#pragma unroll
      for (int s = 0; s < NSD; ++s) sd[s] = chunk_dot(*reinterpret_cast<const V8*>((const T*)p.o + off + 16 * s), dop[s]);
      dl_next = row_delta(sd);
      if (h2 == 0) p.delta[(int64_t)zh * N + qn] = dl_next;
    } else {
      dl_next = p.delta[(int64_t)zh * N + qn];
    }
  };
  f32x16 dq[DT];
  u32x4 pk[CPT], pv[CPT];
  auto gload = [&](const Src& s, int step) __attribute__((always_inline)) {
    const uint32_t so = (uint32_t)step * step_bytes;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      pk[i] = rsrc_load(s.k, goff[i] + so);
      pv[i] = rsrc_load(s.v, goff[i] + so);
    }
  };
  auto lstore = [&](int st) __attribute__((always_inline)) {
    char* base = smem + st * STAGE;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      if (B::CHUNKS % NT == 0 || tid + i * NT < B::CHUNKS) {
        st16(base + ldst[i], pk[i]);
        st16(base + B::TILE + ldst[i], pv[i]);
      }
  };
  auto qk = [&](f32x16& s, f32x16& dp, int st) __attribute__((always_inline)) {
    const char* base = smem + st * STAGE;
    s = f32x16{};
    dp = ndl;
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) {
      s = Elt<T>::mfma(lds8<T>(base + nat[sd]), qop[sd], s);
      dp = Elt<T>::mfma(lds8<T>(base + B::TILE + nat[sd]), dop[sd], dp);
    }
  };
  auto dq_mma = [&](const V8* dsp, int st) __attribute__((always_inline)) {
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
  int q = 0;  // the lane's query in the current block
  auto dsv = [&](const f32x16& s, const f32x16& dp, V8* dsp, int kb, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      V8 x;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float dr[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int r = 8 * a + i + e;
          float pv2 = fast_exp2(__builtin_fmaf(s[r], c, nm));
          if constexpr (MASK) pv2 = kb + kappa(r, h2) > q ? 0.0f : pv2;
          dr[e] = pv2 * dp[r];
        }
        const V2 dh = H::pack(dr[0], dr[1]);
        x[i] = dh[0];
        x[i + 1] = dh[1];
      }
      dsp[a] = x;
    }
  };

  if (nseg == 0) return;

  int zh, qb;
  seg_of(0, zh, qb);
  Src cur = src_of(0), nxt = src_of(1);
  load_q(zh, qb);
  gload(cur, 0);
  lstore(0);
  gload(cur, 1);
  lstore(1);
  __syncthreads();

  f32x16 sa, da, sb, db;
  V8 ea[2] = {}, eb[2];
  const int rank = blockIdx.x / p.cus;

  for (int t = 0; t < nseg; ++t) {
    if (t % SPI == 0) {
      if (((t / SPI) + rank) & 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    const int qblk = qb * BMQ;
    const int qw0 = qblk + 32 * w;
    q = qw0 + l32;
    // -M of the lane's query; -delta in every register seeds the dP^T accumulator (dP - delta).
    nm = -m_next;
#pragma unroll
    for (int r = 0; r < 16; ++r) ndl[r] = -dl_next;
    const int nsteps = CAUSAL ? (qblk + BMQ) / 32 : N / 32;
#pragma unroll
    for (int u = 0; u < DT; ++u) dq[u] = f32x16{};
    qk(sa, da, 0);
    const bool more = t + 1 < nseg;

    // One step (local index i, i % 4 == IV). MASK: the block's last NW steps (causal), across
    // its diagonal: key step ii (of that region) lies wholly after wave w's queries when ii > w
    // (the wave only stages tiles), on its diagonal when ii == w. LASTG: the block's last group
    // (next block's first two stages, its Q/dO/M/delta loaded in step 2, no S in step 3).
    auto step = [&](int i, f32x16& scur, f32x16& dcur, f32x16& snext, f32x16& dnext, const V8* eprev, V8* ecur,
                    auto iv_tag, auto mask_tag, auto last_tag, int ii) __attribute__((always_inline)) {
      constexpr int IV = decltype(iv_tag)::value;
      constexpr bool MASK = decltype(mask_tag)::value;
      constexpr bool LASTG = decltype(last_tag)::value;
      if (LASTG && IV >= 2) gload(nxt, IV - 2);
      else gload(cur, i + 2);
      if constexpr (!(LASTG && IV == 3)) {
        if (!MASK || ii + 1 <= w) qk(snext, dnext, (IV + 1) & 3);
      }
      if (i > 0 && (!MASK || ii - 1 <= w)) dq_mma(eprev, (IV + 3) & 3);
      if constexpr (LASTG && IV == 2) {
        // Not above the S^T / dP^T MFMAs that read the current Q, dO: the new rows take their registers.
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
          int zn, qn;
          seg_of(t + 1, zn, qn);
          load_q(zn, qn);
        }
      }
      if (!MASK || ii <= w) dsv(scur, dcur, ecur, 32 * i, mask_tag);
      lstore((IV + 2) & 3);
      __syncthreads();
    };
    auto group = [&](int i, auto mask_tag, auto last_tag, int ii0) __attribute__((always_inline)) {
      step(i, sa, da, sb, db, ea, eb, IC<0>{}, mask_tag, last_tag, ii0);
      step(i + 1, sb, db, sa, da, eb, ea, IC<1>{}, mask_tag, last_tag, ii0 + 1);
      step(i + 2, sa, da, sb, db, ea, eb, IC<2>{}, mask_tag, last_tag, ii0 + 2);
      step(i + 3, sb, db, sa, da, eb, ea, IC<3>{}, mask_tag, last_tag, ii0 + 3);
    };
    const int ngroups = nsteps / 4;
    const int g_full = CAUSAL ? ngroups - NW / 4 : ngroups - 1;  // groups before the diagonal region
    int gi = 0;
    for (; gi < g_full; ++gi) group(4 * gi, std::false_type{}, std::false_type{}, -1);
    if constexpr (CAUSAL) {
      for (; gi < ngroups - 1; ++gi) group(4 * gi, std::true_type{}, std::false_type{}, 4 * gi - 4 * g_full);
      group(4 * gi, std::true_type{}, std::true_type{}, 4 * gi - 4 * g_full);
    } else {
      group(4 * gi, std::false_type{}, std::true_type{}, -1);
    }
    // Drain: dQ of the block's last step (stage 3; the last wave's diagonal), then the store.
    if (!CAUSAL || NW - 1 <= w) dq_mma(ea, 3);
    {
      // dQ (scaled, rounded) through the wave's LDS rows, then stored as whole 128-byte rows with
      // the non-temporal policy: nothing in the backward reads dQ. (Wave-local rows: no barrier.
      // The row index is computed here, not held across the block loop.)
      TATTN_LDS char* wt = (TATTN_LDS char*)dqs + w * 32 * B::RB;
      int rl = l32;
      asm volatile("" : "+v"(rl));
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * u + 8 * g + 4 * h2;
          if (d0 < D) {
            V4 x;
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) x[i2] = (T)(dq[u][4 * g + i2] * p.scale);
            *reinterpret_cast<TATTN_LDS V4*>(wt + Swz<D>::addr(rl, 2 * d0)) = x;
          }
        }
      const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
      T* base = (T*)p.dq + hoff + (int64_t)(qb * BMQ + 32 * w) * rs;
      constexpr int CPRO = D / 8;  // 16-byte chunks of a row
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int it = 0; it < 32 * CPRO / 64; ++it) {
        const int j = ln + 64 * it;
        const int row = j / CPRO, cc = j % CPRO;
        const u32x4 v = *reinterpret_cast<const TATTN_LDS u32x4*>(wt + Swz<D>::addr(row, 16 * cc));
        st16_stream(base + (int64_t)row * rs + 8 * cc, v);
      }
    }
    if (!more) break;
    seg_of(t + 1, zh, qb);
    cur = nxt;
    nxt = src_of(t + 2);
  }
}

}  // namespace tattn
