// Software-pipelined 16-bit (fp16, bf16) backward kernels for gfx950 (head dims 16, 32, 64 and
// 128; at 128 the table runs them at one wave per SIMD, with the 512-register budget).
//
// Same math and rounding points as the generic kernels in bwd.hip (the reference's
// src/tattn/kernels.py:151-321); the difference is the schedule. Each 32-row step issues
// MFMAs that do not depend on the step's elementwise work, so the matrix cores run while the
// VALU computes P and dS:
//   dK/dV step i: S_{i+1} = Q K^T, dP_{i+1} = dO V^T        (next query block)
//                 dV += P_{i-1}^T dO, dK += dS_{i-1}^T Q      (previous query block)
//                 VALU: P_i = exp2(S_i c - M), dS_i = P_i (dP_i - delta)
//   dQ    step i: S^T_{i+1} = K Q^T, dP^T_{i+1} = V dO^T      (next key block)
//                 dQ^T += K_{i-1}^T dS^T_{i-1}                (previous key block)
//                 VALU: dS^T_i
// Tiles stream through a 4-deep LDS ring (step i reads stages i-1, i, i+1 and refills stage
// i+2; one barrier per step); the main loops are unrolled by four so stage offsets are
// constants. Rows are stored in perm32 order with XOR-swizzled 16-byte chunks (Swz), which
// keeps both the natural (ds_read_b128) and the transposed (ds_read_b64_tr_b16) operand reads
// free of bank conflicts. HBM tiles come through range-checked buffer loads: rows past the
// sequence end read as zero.
#pragma once

#include <type_traits>

#include "common.h"

namespace tattn {

template <int D>
struct BwdPipe {
  static constexpr int RB = Swz<D>::RB;
  static constexpr int TILE = 32 * RB;
  static constexpr int NSD = D / 16;
  static constexpr int DT = (D + 31) / 32;
  static constexpr int CPR = D / 8;        // 16-byte data chunks per row
  static constexpr int CHUNKS = 32 * CPR;  // per 32-row tile
  static constexpr int NST = 4;            // LDS ring depth
  static constexpr int DKDV_STAGE = 2 * TILE + 256;  // Q, dO tiles + M[32], delta[32]
  static constexpr int DQ_STAGE = 2 * TILE;          // K, V tiles
};

// Addresses (within a tile) of the two 8-byte transposed reads that build one MFMA operand
// whose k index runs over the 16 rows of slice sl and whose m/n index is column 32u + lane%32.
template <int D>
__device__ __forceinline__ void tr_addrs(int sl, int u, int lane, int& a0, int& a1) {
  const int g = lane >> 4, src = lane & 15;
  const int colb = (32 * u + 16 * (g & 1) + 4 * (src & 3)) * 2;
  const int row = 16 * sl + 4 * (g >> 1) + (src >> 2);  // perm32 maps row 16sl+8h+4j+t to 16sl+8j+4h+t
  a0 = Swz<D>::addr(row, colb);
  a1 = Swz<D>::addr(row + 8, colb);
}

template <typename T>
__device__ __forceinline__ typename H16<T>::V8 tr_pair(const char* base, int a0, int a1) {
  const auto lo = lds_tr<T>((const TATTN_LDS char*)base + a0);
  const auto hi = lds_tr<T>((const TATTN_LDS char*)base + a1);
  return typename H16<T>::V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <typename T>
__device__ __forceinline__ typename H16<T>::V8 lds8(const char* p) {
  return *reinterpret_cast<const TATTN_LDS typename H16<T>::V8*>((const TATTN_LDS char*)p);
}

// ---- dK / dV --------------------------------------------------------------------------------
// KT key tiles per wave (32 KT keys): every Q / dO operand a wave reads from LDS (natural for S
// and dP, transposed for dK and dV) feeds KT MFMAs, so LDS bytes per MFMA fall by KT. KT = 2
// needs about 400 registers (K and V operands, dK and dV accumulators and the S / dP pairs of
// both tiles) and runs at one wave per SIMD.
template <typename T, int D, int NW, int KT, int OCC, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, OCC) void dkdv_pipe_kernel(const BwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V4 = typename H::V4;
  using V2 = typename H::V2;
  using B = BwdPipe<D>;
  constexpr int NT = NW * 64, BNK = NW * KT * 32;
  constexpr int STAGE = B::DKDV_STAGE;
  constexpr int CPT = (B::CHUNKS + NT - 1) / NT;
  constexpr int NSD = B::NSD, DT = B::DT;
  __shared__ __attribute__((aligned(16))) char smem[B::NST * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int zhs = p.Z * p.H;
  const BlockCoord bc = block_coord(zhs, p.n_blocks, !CAUSAL);
  const int zh = bc.zh, kbi = bc.blk;  // causal: small key blocks (most work) first
  const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
  const int64_t rs = p.s[2];
  const float c = p.c;
  const int kblk = kbi * BNK;
  const int kw0 = kblk + 32 * KT * w;  // first key of the wave; tile kt holds keys kw0 + 32 kt + l32
  // Causal: query blocks below this key block never see its keys (kernels.py:206-208).
  const int lo = CAUSAL ? kblk : 0;
  const int nsteps = (N - lo + 31) / 32;

  V8 kop[KT][NSD], vop[KT][NSD];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int key = kw0 + 32 * kt + l32;
    const int64_t off = hoff + (int64_t)(key < N ? key : 0) * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      const V8 a = *reinterpret_cast<const V8*>((const T*)p.k + off + 16 * s);
      const V8 b = *reinterpret_cast<const V8*>((const T*)p.v + off + 16 * s);
      kop[kt][s] = key < N ? a : V8{};
      vop[kt][s] = key < N ? b : V8{};
    }
  }
  f32x16 dk[KT][DT], dv[KT][DT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int u = 0; u < DT; ++u) dk[kt][u] = dv[kt][u] = f32x16{};

  // HBM: Q, dO rows and M, delta entries from query `lo` on.
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
  // Lanes 0-31 of wave 0 stage M, lanes 32-63 delta (one float each, range-checked per dword).
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
  const int mo = 2 * B::TILE + 32 * h2;  // M of queries 8*h2.. (bytes); delta at +128

  // Register stage of one step's Q, dO, M and delta (the loop uses set 0; the prologue also
  // set 1, so both of its steps are in flight at once).
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

  // S = Q K^T and dP - delta = dO V^T - delta of the stage's 32 queries for each key tile (C
  // layout: lane = key, register r = query kappa(r, h2)); the dP chains start from the stage's
  // -delta. Each Q / dO operand read from LDS feeds the KT tiles.
  auto qk = [&](f32x16 (&s)[KT], f32x16 (&dp)[KT], int st) {
    const char* base = smem + st * STAGE;
    {
      const TATTN_LDS char* nd = (const TATTN_LDS char*)base + mo + 128;
      const f32x4 n0 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd);
      const f32x4 n1 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 16);
      const f32x4 n2 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 64);
      const f32x4 n3 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 80);
      const f32x16 nd16 = f32x16{n0[0], n0[1], n0[2], n0[3], n1[0], n1[1], n1[2], n1[3],
                                 n2[0], n2[1], n2[2], n2[3], n3[0], n3[1], n3[2], n3[3]};
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        s[kt] = f32x16{};
        dp[kt] = nd16;
      }
    }
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) {
      const V8 qa = lds8<T>(base + nat[sd]);
      const V8 oa = lds8<T>(base + B::TILE + nat[sd]);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        s[kt] = Elt<T>::mfma(qa, kop[kt][sd], s[kt]);
        dp[kt] = Elt<T>::mfma(oa, vop[kt][sd], dp[kt]);
      }
    }
  };
  // dV += P^T dO, dK += dS^T Q over the stage's 32 queries (each transposed operand feeds the KT
  // tiles).
  auto grad_mma = [&](const V8 (&pp)[KT][2], const V8 (&dsp)[KT][2], int st) {
    const char* base = smem + st * STAGE;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int u = 0; u < DT; ++u) {
        V8 dob = tr_pair<T>(base + B::TILE, tra[sl][u][0], tra[sl][u][1]);
        V8 qb = tr_pair<T>(base, tra[sl][u][0], tra[sl][u][1]);
        if (D < 32 && 16 * ((lane >> 4) & 1) >= D) dob = qb = V8{};
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          dv[kt][u] = Elt<T>::mfma(pp[kt][sl], dob, dv[kt][u]);
          dk[kt][u] = Elt<T>::mfma(dsp[kt][sl], qb, dk[kt][u]);
        }
      }
  };
  // P = exp2(S c - M), dS = P (dP - delta) for the stage's queries, rounded into MFMA operands
  // (dp already holds dP - delta).
  auto pds = [&](const f32x16 (&s)[KT], const f32x16 (&dp)[KT], V8 (&pp)[KT][2], V8 (&dsp)[KT][2], int st, int q0,
                 auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const char* base = smem + st * STAGE;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const f32x4 m0 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)base + mo + 64 * a);
      const f32x4 m1 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)base + mo + 64 * a + 16);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int key = kw0 + 32 * kt + l32;
        V8 x, y;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float pr[2], dr[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int r = 8 * a + i + e;
            const float mv = (i + e) < 4 ? m0[i + e] : m1[i + e - 4];
            float pv = fast_exp2(__builtin_fmaf(s[kt][r], c, -mv));
            if constexpr (MASK) pv = key > q0 + kappa(r, h2) ? 0.0f : pv;
            pr[e] = pv;
            dr[e] = pv * dp[kt][r];
          }
          const V2 ph = H::pack(pr[0], pr[1]), dh = H::pack(dr[0], dr[1]);
          x[i] = ph[0];
          x[i + 1] = ph[1];
          y[i] = dh[0];
          y[i + 1] = dh[1];
        }
        pp[kt][a] = x;
        dsp[kt][a] = y;
      }
    }
  };

  // Prologue: steps 0 and 1 into stages 0 and 1, both loads in flight together (with the K/V
  // operand loads above); stage 3 (read by step 0 together with all-zero P and dS) cleared.
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

  f32x16 sa[KT], da[KT], sb[KT], db[KT];
  V8 pa[KT][2], dsa[KT][2], pb[KT][2], dsb[KT][2];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) pa[kt][0] = pa[kt][1] = dsa[kt][0] = dsa[kt][1] = V8{};
  qk(sa, da, 0);

  // One step: S/dP of step i+1, dV/dK of step i-1, P/dS of step i; ST = i % 4 (or -1: run time).
  auto step = [&](int i, int st, f32x16 (&scur)[KT], f32x16 (&dcur)[KT], f32x16 (&snext)[KT], f32x16 (&dnext)[KT],
                  const V8 (&pprev)[KT][2], const V8 (&dsprev)[KT][2], V8 (&pcur)[KT][2], V8 (&dscur)[KT][2],
                  auto mask_tag) {
    gload(i + 2, IC<0>{});
    qk(snext, dnext, (st + 1) & 3);
    grad_mma(pprev, dsprev, (st + 3) & 3);
    pds(scur, dcur, pcur, dscur, st, lo + 32 * i, mask_tag);
    lstore((st + 2) & 3, IC<0>{});
    __syncthreads();
  };
  auto roll = [&]() {  // next becomes current
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      sa[kt] = sb[kt];
      da[kt] = db[kt];
      pa[kt][0] = pb[kt][0];
      pa[kt][1] = pb[kt][1];
      dsa[kt][0] = dsb[kt][0];
      dsa[kt][1] = dsb[kt][1];
    }
  };

  int i = 0;
  // Causal: the workgroup's first NW KT query blocks cross its keys' diagonal; mask them. Query
  // block i below KT w lies wholly before wave w's keys (P = dS = 0): the wave skips its MFMAs
  // and softmax there and only stages tiles, leaving its SIMD to the other waves. (With KT = 2
  // the wave's second tile sees no key of block KT w either; the mask zeroes it.)
  const int wt = KT * w;
  const int n_mask = CAUSAL ? min(nsteps, NW * KT) : 0;
  for (; i < n_mask; ++i) {
    gload(i + 2, IC<0>{});
    if (i + 1 >= wt) qk(sb, db, (i + 1) & 3);
    if (i - 1 >= wt) grad_mma(pa, dsa, (i + 3) & 3);
    if (i >= wt) pds(sa, da, pb, dsb, i & 3, lo + 32 * i, std::true_type{});
    lstore((i + 2) & 3, IC<0>{});
    __syncthreads();
    roll();
  }
  for (; i + 3 < nsteps; i += 4) {  // i % 4 == 0 here (NW KT is a multiple of 4)
    step(i, 0, sa, da, sb, db, pa, dsa, pb, dsb, std::false_type{});
    step(i + 1, 1, sb, db, sa, da, pb, dsb, pa, dsa, std::false_type{});
    step(i + 2, 2, sa, da, sb, db, pa, dsa, pb, dsb, std::false_type{});
    step(i + 3, 3, sb, db, sa, da, pb, dsb, pa, dsa, std::false_type{});
  }
  for (; i < nsteps; ++i) {
    step(i, i & 3, sa, da, sb, db, pa, dsa, pb, dsb, std::false_type{});
    roll();
  }
  grad_mma(pa, dsa, (nsteps - 1) & 3);

  // Store through LDS: C register r of lane holds key 8*(r/4) + 4*h2 + r%4 of the tile, column
  // 32u + l32, so direct stores would write 2 bytes per lane and instruction. Each wave instead
  // writes its tile into a private LDS block (row-major [key][d], RB bytes per row) and stores
  // whole 16-byte chunks of rows. The blocks reuse the ring: the barrier waits until every
  // wave's last reads of it are done.
  __syncthreads();
  constexpr int RB = B::RB;
  constexpr int CPRO = D / 8;                 // 16-byte chunks per output row
  constexpr int SPW = (32 * CPRO + 63) / 64;  // chunk stores per lane and tile
  static_assert(NW * 32 * RB <= B::NST * STAGE, "store blocks fit the ring");
  char* wb = smem + w * 32 * RB;
  T* DK = (T*)p.dk + hoff;
  T* DV = (T*)p.dv + hoff;
  // The lane index is recomputed here (mbcnt) rather than kept live across the main loop, which
  // runs at the register limit.
  const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int l32e = ln & 31, h2e = ln >> 5;
  auto store_tile = [&](const f32x16 (&acc)[DT], float mul, T* dst, int key0) {
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
      const int key = key0 + row;
      if (row < 32 && key < N) {
        const u32x4 v = *reinterpret_cast<const TATTN_LDS u32x4*>((const TATTN_LDS char*)wb + row * RB + 16 * cc);
        st16_stream(dst + (int64_t)key * rs + 8 * cc, v);
      }
    }
  };
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    store_tile(dk[kt], p.scale, DK, kw0 + 32 * kt);
    store_tile(dv[kt], 1.0f, DV, kw0 + 32 * kt);
  }
}

// ---- dQ ----------------------------------------------------------------------------------
template <typename T, int D, int NW, int OCC, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, OCC) void dq_pipe_kernel(const BwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V4 = typename H::V4;
  using V2 = typename H::V2;
  using B = BwdPipe<D>;
  constexpr int NT = NW * 64, BMQ = NW * 32;
  constexpr int STAGE = B::DQ_STAGE;
  constexpr int CPT = (B::CHUNKS + NT - 1) / NT;
  constexpr int NSD = B::NSD, DT = B::DT;
  __shared__ __attribute__((aligned(16))) char smem[B::NST * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
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
  const int qw0 = qblk + 32 * w;
  const int q = qw0 + l32;

  V8 qop[NSD], dop[NSD];
  {
    const int64_t off = hoff + (int64_t)(q < N ? q : 0) * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      const V8 a = *reinterpret_cast<const V8*>((const T*)p.q + off + 16 * s);
      const V8 b = *reinterpret_cast<const V8*>((const T*)p.dout + off + 16 * s);
      qop[s] = q < N ? a : V8{};
      dop[s] = q < N ? b : V8{};
    }
  }
  const float nm = -(q < N ? p.m[(int64_t)zh * N + q] : 0.0f);
  float dl;
  if (p.fuse_delta) {  // delta = rowsum(dO * O) here, stored for the dK/dV kernel that follows
    float sd[NSD];
    const int64_t off = hoff + (int64_t)(q < N ? q : 0) * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) sd[s] = chunk_dot(*reinterpret_cast<const V8*>((const T*)p.o + off + 16 * s), dop[s]);
    dl = row_delta(sd);
    if (q >= N) dl = 0.0f;
    else if (h2 == 0) p.delta[(int64_t)zh * N + q] = dl;
  } else {
    dl = q < N ? p.delta[(int64_t)zh * N + q] : 0.0f;
  }
  // -delta of the lane's query in every register: seeds the dP^T accumulator, so the MFMAs
  // return dP - delta.
  f32x16 ndl;
#pragma unroll
  for (int r = 0; r < 16; ++r) ndl[r] = -dl;
  f32x16 dq[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) dq[u] = f32x16{};

  const int hi = CAUSAL ? min(qblk + BMQ, N) : N;
  const int nsteps = (hi + 31) / 32;
  // Steps this wave computes: every step up to the one holding its last query row.
  const int wave_steps = qw0 >= N ? 0 : CAUSAL ? min(nsteps, (qw0 + 31) / 32 + 1) : nsteps;
  // Steps before n_full need no mask for any wave of the workgroup.
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

  // Register stage of one step's K and V (the loop uses set 0; the prologue also set 1, so both
  // of its steps are in flight at once).
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
  // S^T = K Q^T and dP^T - delta = V dO^T - delta of the stage's 32 keys (C layout: lane = query,
  // register r = key kappa(r, h2)).
  auto qk = [&](f32x16& s, f32x16& dp, int st) {
    const char* base = smem + st * STAGE;
    s = f32x16{};
    dp = ndl;
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) {
      s = Elt<T>::mfma(lds8<T>(base + nat[sd]), qop[sd], s);
      dp = Elt<T>::mfma(lds8<T>(base + B::TILE + nat[sd]), dop[sd], dp);
    }
  };
  // dQ^T += K^T dS^T over the stage's 32 keys.
  auto dq_mma = [&](const V8* dsp, int st) {
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
  auto dsv = [&](const f32x16& s, const f32x16& dp, V8* dsp, int kb, auto mask_tag) {
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
          if constexpr (MASK) {
            const int key = kb + kappa(r, h2);
            pv2 = (key >= N || (CAUSAL && key > q)) ? 0.0f : pv2;
          }
          dr[e] = pv2 * dp[r];
        }
        const V2 dh = H::pack(dr[0], dr[1]);
        x[i] = dh[0];
        x[i + 1] = dh[1];
      }
      dsp[a] = x;
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

  f32x16 sa, da, sb, db;
  V8 ea[2] = {}, eb[2];
  if (wave_steps > 0) qk(sa, da, 0);

  auto full_step = [&](int i, int st, f32x16& scur, f32x16& dcur, f32x16& snext, f32x16& dnext,
                       const V8* eprev, V8* ecur) {
    gload(i + 2, IC<0>{});
    qk(snext, dnext, (st + 1) & 3);
    dq_mma(eprev, (st + 3) & 3);
    dsv(scur, dcur, ecur, 32 * i, std::false_type{});
    lstore((st + 2) & 3, IC<0>{});
    __syncthreads();
  };

  int i = 0;
  for (; i + 3 < n_full; i += 4) {
    full_step(i, 0, sa, da, sb, db, ea, eb);
    full_step(i + 1, 1, sb, db, sa, da, eb, ea);
    full_step(i + 2, 2, sa, da, sb, db, ea, eb);
    full_step(i + 3, 3, sb, db, sa, da, eb, ea);
  }
  // Remaining steps (masked or not): state scur = sa, eprev = ea.
  for (; i < nsteps; ++i) {
    gload(i + 2, IC<0>{});
    if (i - 1 < wave_steps) dq_mma(ea, (i + 3) & 3);
    if (i < wave_steps) {
      qk(sb, db, (i + 1) & 3);
      if (i >= n_full)
        dsv(sa, da, eb, 32 * i, std::true_type{});
      else
        dsv(sa, da, eb, 32 * i, std::false_type{});
      sa = sb;
      da = db;
      ea[0] = eb[0];
      ea[1] = eb[1];
    }
    lstore((i + 2) & 3, IC<0>{});
    __syncthreads();
  }
  if (wave_steps == nsteps && nsteps > 0) dq_mma(ea, (nsteps - 1) & 3);

  if (q < N) {
    T* row = (T*)p.dq + hoff + (int64_t)q * rs;
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * u + 8 * g + 4 * h2;
        if (d0 < D) {
          V4 x;
#pragma unroll
          for (int i2 = 0; i2 < 4; ++i2) x[i2] = (T)(dq[u][4 * g + i2] * p.scale);
          *reinterpret_cast<V4*>(row + d0) = x;
        }
      }
  }
}

}  // namespace tattn
