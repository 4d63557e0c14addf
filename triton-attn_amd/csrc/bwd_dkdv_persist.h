// Persistent 16-bit dK/dV kernel for gfx950: one workgroup per resident slot, each running a
// static list of key blocks back to back.
//
// Same math, rounding points, LDS ring (4 stages of Q, dO, M and -delta, XOR-swizzled rows),
// register-staged loads and per-step schedule as dkdv_pipe_kernel (bwd_pipe.h) with one 32-key
// tile per wave, so its gradients are those of that kernel bit for bit. What changes is the life of
// a workgroup. At 16-32 query steps per key block (N = 512-1024) the non-persistent kernel spends a
// fifth of a block's time outside its steps: the K and V operand rows and the first Q / dO stages
// come from HBM at the start (every workgroup of a round at once), the dK / dV stores at the end.
// Here:
//   - each wave fetches the next block's K and V rows of its own 32 keys into a private LDS
//     staging tile during the first steps of the current block, by LDS DMA (64 lanes x 16 bytes
//     per instruction, no registers: a lane's offset is the one it already holds for the ring
//     copy, the piece's row in the scalar offset); at the block's end it reads them into its
//     operand registers, which the current block no longer needs (its last S and dP are
//     computed);
//   - the Q / dO / M / delta ring runs on across blocks: the block's last two steps load the
//     next block's first two stages;
//   - dK and dV leave through the same staging tile (row-major, whole 16-byte row chunks), after
//     the next operands were read out of it, so the accumulators and the next block's operands
//     are never live together.
// Work items: non-causal, one key block; causal, the pair of key blocks p and nb-1-p of one slice
// (the causal lower bound kernels.py:206-208 gives block kb (N - kb BNK) / 32 query steps, so every
// pair has (N + BNK) / 32). XCD x takes the slices zh = x (mod 8), its workgroups consecutive
// items (workgroup b runs on XCD b % 8), so the key blocks that stream one slice's Q / dO rows run
// together on one L2.
// Preconditions (checked by the launcher, which otherwise runs dkdv_pipe_kernel): Z*H a multiple
// of 8, N a multiple of the block and of 128, causal: an even number of blocks per slice, 32-bit
// slice offsets, head dims whose K and V tiles take at most four 1 KB DMA pieces (D <= 64).
#pragma once

#include "bwd_pipe.h"

namespace tattn {

template <typename T, int D, int NW, int OCC, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, OCC) void dkdv_persist_kernel(const BwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V2 = typename H::V2;
  using B = BwdPipe<D>;
  using SW = Swz<D>;
  constexpr int NT = NW * 64, BNK = NW * 32;
  constexpr int STAGE = B::DKDV_STAGE;
  constexpr int CPT = (B::CHUNKS + NT - 1) / NT;
  constexpr int NSD = B::NSD, DT = B::DT;
  constexpr int RB = B::RB, TILE = B::TILE;
  constexpr int PIECES = TILE / 1024;  // 1 KB DMA pieces per staged tile
  constexpr int SPI = CAUSAL ? 2 : 1;  // key blocks per work item
  static_assert(NW % 4 == 0, "masked steps in whole groups of four");
  static_assert(PIECES >= 1 && PIECES <= 4, "staging DMA within a block's first group of steps");
  static_assert(D >= 32 && B::CPR == RB / 16, "staging rows without padding chunks");
  // The ring at LDS address 0 (the larger alignment places it first), so every ring access fits
  // the 16-bit immediate offset of the LDS instructions.
  __shared__ __attribute__((aligned(1024))) char smem[B::NST * STAGE];
  // Per wave: the staged K tile, then the V tile (also the dK / dV store buffer at a block's end).
  __shared__ __attribute__((aligned(16))) char kvs[NW * 2 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int wu = (int)uniform32((uint32_t)w);
  const int N = p.N;
  const int nkb = p.n_blocks;
  const int xcd = blockIdx.x & 7, lw = blockIdx.x >> 3;
  const int n_items = lw < p.items_x ? (p.items_x - lw + p.gx - 1) / p.gx : 0;
  const int nseg = n_items * SPI;
  const int64_t rs = p.s[2];
  const float c = p.c;

  // Block t of this workgroup -> (slice, key block); causal pairs run their longer block first.
  auto seg_of = [&](int t, int& zh, int& kb) __attribute__((always_inline)) {
    const int k = lw + p.gx * (t / SPI);
    if constexpr (CAUSAL) {
      const int half = nkb >> 1;
      zh = 8 * (k / half) + xcd;
      const int pr = k % half;
      kb = (t % SPI == 0) ? pr : nkb - 1 - pr;
    } else {
      zh = 8 * (k / nkb) + xcd;
      kb = k % nkb;
    }
  };
  // Buffer descriptors of a block: Q, dO rows and M, delta entries from its first query on (the
  // causal lower bound). Past the last block, descriptors of zero bytes (every load reads zeros
  // and touches no memory). Built where they are used, so that only the current block's four
  // stay in scalar registers through its steps.
  struct Src {
    __amdgpu_buffer_rsrc_t q, o, m, d;
  };
  auto src_of = [&](int t) __attribute__((always_inline)) {
    Src s;
    if (t >= nseg) {
      s.q = s.o = slice_rsrc(p.q, 0);
      s.m = s.d = slice_rsrc(p.m, 0);
      return s;
    }
    int zh, kb;
    seg_of(t, zh, kb);
    const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
    const int lo = CAUSAL ? kb * BNK : 0;
    s.q = slice_rsrc((const T*)p.q + hoff + (int64_t)lo * rs, slice_bytes(N - lo, rs, D));
    s.o = slice_rsrc((const T*)p.dout + hoff + (int64_t)lo * rs, slice_bytes(N - lo, rs, D));
    s.m = slice_rsrc(p.m + (int64_t)zh * N + lo, (uint64_t)(N - lo) * 4);
    s.d = slice_rsrc(p.delta + (int64_t)zh * N + lo, (uint64_t)(N - lo) * 4);
    return s;
  };
  // K or V rows of block t for this wave's staging DMA. Lane l of DMA piece pp fetches row
  // (64 / CPR) pp + l / CPR, chunk l % CPR of the wave's 32 keys: the ring-copy offset goff[0] of
  // thread tid covers row (64 / CPR) (w % WPT) + l / CPR with the same chunk, so the descriptor
  // starts (64 / CPR) (w % WPT) rows before the wave's first key and the piece adds
  // (64 / CPR) pp rows as its scalar offset.
  constexpr int WPT = B::CHUNKS / 64;  // waves whose lanes cover one 32-row tile once
  auto kv_src = [&](int t, const void* base) __attribute__((always_inline)) {
    int zh, kb;
    seg_of(t, zh, kb);
    const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
    const int shift = (64 / B::CPR) * (wu % WPT);
    return slice_rsrc((const T*)base + hoff + (int64_t)(kb * BNK + 32 * wu - shift) * rs,
                      slice_bytes(32 + shift, rs, D));
  };
  const uint32_t step_bytes = uniform32((uint32_t)(rs * 64));

  uint32_t goff[CPT];
  int ldst[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int ch = (tid + i * NT) % B::CHUNKS;  // threads past the tile load a duplicate (not stored)
    const int row = ch / B::CPR, cb = (ch % B::CPR) * 16;
    goff[i] = (uint32_t)(row * rs * 2 + cb);
    ldst[i] = SW::addr(perm32(row), cb);
  }
  const bool md_loader = tid < 64;
  const int md_dst = 2 * TILE + tid * 4;
  int nat[NSD];
#pragma unroll
  for (int s = 0; s < NSD; ++s) nat[s] = SW::addr(l32, (16 * s + 8 * h2) * 2);
  int tra[2][DT][2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int u = 0; u < DT; ++u) tr_addrs<D>(sl, u, lane, tra[sl][u][0], tra[sl][u][1]);
  const int mo = 2 * TILE + 32 * h2;

  char* const kv_w = kvs + wu * 2 * TILE;
  // One 1 KB piece of the staging tile (row-major [key][d], RB bytes per row, no swizzle: it is
  // read once per block): lane l's 16 bytes land at dst + 16 l. (A helper: called directly from
  // the step lambda below, the builtin kept clang from emitting the kernel's host-side stub.)
  auto dma_piece = [&](__amdgpu_buffer_rsrc_t src, char* dst, int pp) __attribute__((always_inline)) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (TATTN_LDS void*)dst, 16, (int)goff[0],
                                             (int)uniform32((uint32_t)(pp * (64 / B::CPR) * rs * 2)), 0, 0);
  };

  // Register stage of one step's Q, dO, M and delta (set 1 only in the first block's prologue).
  u32x4 pq[2][CPT], pd[2][CPT];
  uint32_t pm[2], pdl[2];
  auto gload = [&](const Src& s, int step, auto set_tag) __attribute__((always_inline)) {
    constexpr int R = decltype(set_tag)::value;
    const uint32_t so = (uint32_t)step * step_bytes;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      pq[R][i] = rsrc_load(s.q, goff[i] + so);
      pd[R][i] = rsrc_load(s.o, goff[i] + so);
    }
    const uint32_t mo4 = (uint32_t)(((tid & 31) + 32 * step) * 4);
    pm[R] = __builtin_amdgcn_raw_buffer_load_b32(s.m, (int)mo4, 0, 0);
    pdl[R] = __builtin_amdgcn_raw_buffer_load_b32(s.d, (int)mo4, 0, 0);
  };
  auto lstore = [&](int st, auto set_tag) __attribute__((always_inline)) {
    constexpr int R = decltype(set_tag)::value;
    char* base = smem + st * STAGE;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      if (B::CHUNKS % NT == 0 || tid + i * NT < B::CHUNKS) {
        st16(base + ldst[i], pq[R][i]);
        st16(base + TILE + ldst[i], pd[R][i]);
      }
    // delta is staged negated: it seeds the dP accumulator, so dP - delta comes out of the MFMAs.
    if (md_loader) *reinterpret_cast<uint32_t*>(base + md_dst) = (tid & 32) ? (pdl[R] ^ 0x80000000u) : pm[R];
  };

  V8 kop[NSD], vop[NSD];
  f32x16 dk[DT], dv[DT];
  auto qk = [&](f32x16& s, f32x16& dp, int st) __attribute__((always_inline)) {
    const char* base = smem + st * STAGE;
    {
      const TATTN_LDS char* nd = (const TATTN_LDS char*)base + mo + 128;
      const f32x4 n0 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd);
      const f32x4 n1 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 16);
      const f32x4 n2 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 64);
      const f32x4 n3 = *reinterpret_cast<const TATTN_LDS f32x4*>(nd + 80);
      s = f32x16{};
      dp = f32x16{n0[0], n0[1], n0[2], n0[3], n1[0], n1[1], n1[2], n1[3],
                  n2[0], n2[1], n2[2], n2[3], n3[0], n3[1], n3[2], n3[3]};
    }
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) {
      const V8 qa = lds8<T>(base + nat[sd]);
      const V8 oa = lds8<T>(base + TILE + nat[sd]);
      s = Elt<T>::mfma(qa, kop[sd], s);
      dp = Elt<T>::mfma(oa, vop[sd], dp);
    }
  };
  auto grad_mma = [&](const V8 (&pp)[2], const V8 (&dsp)[2], int st) __attribute__((always_inline)) {
    const char* base = smem + st * STAGE;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int u = 0; u < DT; ++u) {
        V8 dob = tr_pair<T>(base + TILE, tra[sl][u][0], tra[sl][u][1]);
        V8 qb = tr_pair<T>(base, tra[sl][u][0], tra[sl][u][1]);
        if (D < 32 && 16 * ((lane >> 4) & 1) >= D) dob = qb = V8{};
        dv[u] = Elt<T>::mfma(pp[sl], dob, dv[u]);
        dk[u] = Elt<T>::mfma(dsp[sl], qb, dk[u]);
      }
  };
  int kw0 = 0;  // the wave's first key in the current block
  auto pds = [&](const f32x16& s, const f32x16& dp, V8 (&pp)[2], V8 (&dsp)[2], int st, int q0, auto mask_tag)
      __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const char* base = smem + st * STAGE;
    const int key = kw0 + l32;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const f32x4 m0 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)base + mo + 64 * a);
      const f32x4 m1 = *reinterpret_cast<const TATTN_LDS f32x4*>((const TATTN_LDS char*)base + mo + 64 * a + 16);
      V8 x, y;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float pr[2], dr[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int r = 8 * a + i + e;
          const float mv = (i + e) < 4 ? m0[i + e] : m1[i + e - 4];
          float pv = fast_exp2(__builtin_fmaf(s[r], c, -mv));
          if constexpr (MASK) pv = key > q0 + kappa(r, h2) ? 0.0f : pv;
          pr[e] = pv;
          dr[e] = pv * dp[r];
        }
        const V2 ph = H::pack(pr[0], pr[1]), dh = H::pack(dr[0], dr[1]);
        x[i] = ph[0];
        x[i + 1] = ph[1];
        y[i] = dh[0];
        y[i + 1] = dh[1];
      }
      pp[a] = x;
      dsp[a] = y;
    }
  };
  // dK (scaled by sm_scale, kernels.py:232) and dV of the wave's 32 keys through its staging tile:
  // C register r of a lane holds key 8 (r/4) + 4 h2 + r%4, column 32 u + l32; written row-major
  // ([key][d], RB bytes per row), then stored as whole 16-byte row chunks.
  auto store_tile = [&](const f32x16 (&acc)[DT], float mul, T* dst, char* wb) __attribute__((always_inline)) {
    const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int l32e = ln & 31, h2e = ln >> 5;
    constexpr int CPRO = D / 8;
    constexpr int SPW = (32 * CPRO + 63) / 64;
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
      if (row < 32) {
        const u32x4 v = *reinterpret_cast<const TATTN_LDS u32x4*>((const TATTN_LDS char*)wb + row * RB + 16 * cc);
        st16_stream(dst + (int64_t)(kw0 + row) * rs + 8 * cc, v);
      }
    }
  };

  if (nseg == 0) return;

  // ---- first block: K / V operands straight from HBM, steps 0 and 1 staged -----------------
  int zh, kb;
  seg_of(0, zh, kb);
  Src cur = src_of(0);
  kw0 = kb * BNK + 32 * wu;
  {
    const int64_t hoff = (int64_t)(zh / p.H) * p.s[0] + (int64_t)(zh % p.H) * p.s[1];
    const int64_t off = hoff + (int64_t)(kw0 + l32) * rs + 8 * h2;
#pragma unroll
    for (int s = 0; s < NSD; ++s) {
      kop[s] = *reinterpret_cast<const V8*>((const T*)p.k + off + 16 * s);
      vop[s] = *reinterpret_cast<const V8*>((const T*)p.v + off + 16 * s);
    }
  }
  gload(cur, 0, IC<0>{});
  gload(cur, 1, IC<1>{});
  lstore(0, IC<0>{});
  lstore(1, IC<1>{});
  __syncthreads();

  f32x16 sa, da, sb, db;
  V8 pa[2], dsa[2], pb[2], dsb[2];
  const int rank = blockIdx.x / p.cus;

  for (int t = 0; t < nseg; ++t) {
    if (t % SPI == 0) {  // workgroups sharing a CU alternate issue priority item by item
      if (((t / SPI) + rank) & 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    const int kblk = kb * BNK;
    const int lo = CAUSAL ? kblk : 0;
    const int nsteps = (N - lo) / 32;
    const bool more = t + 1 < nseg;
#pragma unroll
    for (int u = 0; u < DT; ++u) dk[u] = dv[u] = f32x16{};
    if (!CAUSAL || wu == 0) qk(sa, da, 0);

    // One unmasked step (local index i, i % 4 == IV). LASTG: the block's last group (its steps 2
    // and 3 load the next block's stages 0 and 1; no S in step 3). Steps i < PIECES also start
    // piece i of the next block's K and V rows for this wave, after the step's own loads (so the
    // step's wait leaves them in flight; later steps' waits, in issue order, see them land within
    // the block).
    auto step = [&](int i, f32x16& scur, f32x16& dcur, f32x16& snext, f32x16& dnext, const V8 (&pprev)[2],
                    const V8 (&dsprev)[2], V8 (&pcur)[2], V8 (&dscur)[2], auto iv_tag,
                    auto last_tag) __attribute__((always_inline)) {
      constexpr int IV = decltype(iv_tag)::value;
      constexpr bool LASTG = decltype(last_tag)::value;
      if constexpr (LASTG && IV >= 2) gload(src_of(t + 1), IV - 2, IC<0>{});
      else gload(cur, i + 2, IC<0>{});
      if constexpr (IV < PIECES) {
        if (i < 4 && more) {
          dma_piece(kv_src(t + 1, p.k), kv_w + 1024 * IV, IV);
          dma_piece(kv_src(t + 1, p.v), kv_w + TILE + 1024 * IV, IV);
        }
      }
      if constexpr (!(LASTG && IV == 3)) qk(snext, dnext, (IV + 1) & 3);
      if (i > 0) grad_mma(pprev, dsprev, (IV + 3) & 3);
      pds(scur, dcur, pcur, dscur, IV, lo + 32 * i, std::false_type{});
      lstore((IV + 2) & 3, IC<0>{});
      __syncthreads();
    };
    auto group = [&](int i, auto last_tag) __attribute__((always_inline)) {
      step(i, sa, da, sb, db, pa, dsa, pb, dsb, IC<0>{}, last_tag);
      step(i + 1, sb, db, sa, da, pb, dsb, pa, dsa, IC<1>{}, last_tag);
      step(i + 2, sa, da, sb, db, pa, dsa, pb, dsb, IC<2>{}, last_tag);
      step(i + 3, sb, db, sa, da, pb, dsb, pa, dsa, IC<3>{}, last_tag);
    };
    // Causal: the block's first NW query steps cross its keys' diagonal (query step i lies wholly
    // before wave w's keys when i < w: the wave only stages tiles; on its diagonal when i == w).
    // They run as a rolled loop with run-time stages, as in dkdv_pipe_kernel; when the block is
    // only NW steps long, its last two steps load the next block's first stages here.
    int i = 0;
    if constexpr (CAUSAL) {
      for (; i < NW; ++i) {
        if (i + 2 >= nsteps) gload(src_of(t + 1), i + 2 - nsteps, IC<0>{});
        else gload(cur, i + 2, IC<0>{});
        if (i < PIECES && more) {
          dma_piece(kv_src(t + 1, p.k), kv_w + 1024 * i, i);
          dma_piece(kv_src(t + 1, p.v), kv_w + TILE + 1024 * i, i);
        }
        if (i + 1 >= wu && i + 1 < nsteps) qk(sb, db, (i + 1) & 3);
        if (i > 0 && i - 1 >= wu) grad_mma(pa, dsa, (i + 3) & 3);
        if (i >= wu) pds(sa, da, pb, dsb, i & 3, lo + 32 * i, std::true_type{});
        lstore((i + 2) & 3, IC<0>{});
        __syncthreads();
        sa = sb;
        da = db;
        pa[0] = pb[0];
        pa[1] = pb[1];
        dsa[0] = dsb[0];
        dsa[1] = dsb[1];
      }
    }
    const int ngroups = nsteps / 4;
    for (int gi = i / 4; gi < ngroups - 1; ++gi) group(4 * gi, std::false_type{});
    if (i < nsteps) group(4 * (ngroups - 1), std::true_type{});
    // Drain: dV / dK of the block's last step (stage 3).
    grad_mma(pa, dsa, 3);

    // The next block's K / V operands (DMA'd into this wave's staging tile during the block's
    // first steps; the compiler waits for them), then this block's dK / dV through the same tile.
    const int zh_cur = zh;
    if (more) {
      const int row0 = l32 * RB + 16 * h2;
#pragma unroll
      for (int s = 0; s < NSD; ++s) {
        kop[s] = lds8<T>(kv_w + row0 + 32 * s);
        vop[s] = lds8<T>(kv_w + TILE + row0 + 32 * s);
      }
    }
    {
      const int64_t hoff = (int64_t)(zh_cur / p.H) * p.s[0] + (int64_t)(zh_cur % p.H) * p.s[1];
      store_tile(dk, p.scale, (T*)p.dk + hoff, kv_w);
      store_tile(dv, 1.0f, (T*)p.dv + hoff, kv_w + TILE);
    }
    if (!more) break;
    seg_of(t + 1, zh, kb);
    kw0 = kb * BNK + 32 * wu;
    cur = src_of(t + 1);
  }
  // No LDS DMA is in flight here: the last block starts none, and every earlier one was read out
  // of its staging tile. The waves end without waiting for the dK / dV stores.
}

}  // namespace tattn
