// Persistent 16-bit forward for gfx950: one workgroup per resident slot, each working through a
// static list of work items, with the K/V stream running on across item boundaries.
//
// Same per-step math and rounding points as fwd_pipe_kernel (fwd.hip): 32 keys per step,
// S_{i+1} = K_{i+1} Q^T and O^T += V_{i-1}^T P_{i-1}^T issued while the VALU runs the softmax of
// step i. Two things change.
//
// The life of a workgroup. The non-persistent kernel starts every (slice, query block) with a
// cold prologue (Q and the first K/V tiles from HBM, all workgroups of a round at once) and ends
// it with the O stores; with 16-32 steps per block (N = 512-1024) that fixed cost is a third of
// the block's time. Here a workgroup runs several blocks back to back:
//   - the DMA of a block's last R - 1 steps already fetches the next block's first K and V tiles
//     (its slice's own buffer descriptor), so the next block starts on landed tiles;
//   - the next block's Q rows are loaded into the Q registers during the block's second-to-last
//     step, right after their last use (that step and the last one take the exact softmax path,
//     which never recomputes S, so the old Q is no longer needed); the loads have about two
//     steps to arrive (a workgroup's last block loads none);
//   - the O and M stores of a block overlap the next block's first steps.
//
// The ring. K and V tiles sit in R-deep LDS rings (R = 4 or 8) of unpadded 32-row tiles whose
// 16-byte chunks are XOR-swizzled per row (Swz, as in the backward): the K operand reads
// (ds_read_b128 of rows l32) and the transposed V reads (ds_read_b64_tr_b16 of rows 8h + 0..3
// and + 4..7, 4-row groups at 8 columns) both hit 64 distinct banks. The LDS DMA writes 64
// lanes x 16 bytes to 1 KB of consecutive LDS, so each lane fetches the global chunk that the
// swizzle places at its LDS position. Step i starts K_{i+R-1} and V_{i+R-2}: K has R - 2 steps and
// V R - 1 steps to arrive. At short rows half of the K/V tiles are a slice's first touch and come
// from HBM; eight slots (64 KB at head dim 64) give them six steps instead of two.
//
// Work items: non-causal, one query block of BM rows; causal, the pair of query blocks
// (nb-1-p, p) of one slice, so every item has the same number of steps ((nb+1) * BM / 32) and
// the static schedule is balanced. Items are split per XCD (workgroup b runs on XCD b % 8): XCD
// x takes the slices zh = x (mod 8), and the workgroups of an XCD take consecutive items, so the
// blocks that stream the same K/V rows run at the same time on one L2.
// Preconditions (checked by the launcher, which otherwise runs fwd_pipe_kernel): Z*H a multiple
// of 8, N a multiple of BM, of 32 R and (causal) of 2 BM, the causal diagonal region (BM / 32
// steps) one or two ring periods, 32-bit slice offsets.
#pragma once

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "tiles.h"

namespace tattn {

// LDS of the persistent forward: R K slots and R V slots of 32 unpadded rows.
template <int D, int R>
struct PersistLayout {
  static constexpr int RB = Swz<D>::RB;       // bytes per row
  static constexpr int SLOT = 32 * RB;        // bytes per tile
  static constexpr int PIECES = SLOT / 1024;  // 1 KB DMA pieces per tile
  static constexpr int LDS = 2 * R * SLOT;
};

// LDS bytes of a persistent forward entry's O staging (0: none). At head dim 64 each wave passes
// its O rows through its own LDS rows and stores them as whole 128-byte rows with the
// non-temporal policy (the direct stores wrote 8-byte pieces of rows, which that policy must not
// take: they then skip the L2's merging). Entries whose workgroups per CU would no longer fit in
// the 160 KB of LDS keep the direct stores, and so does head dim 128 (its 8 x 1 entry, one
// workgroup per CU with a 64 KB stage, measured 1.3-2.7% slower non-causal from N = 2048).
constexpr int fwd_persist_ostage_bytes(int D, const TileEntry& e) {
  const int rb = D < 32 ? 64 : 2 * D;
  const int stage = e.nw * e.tiles * 32 * rb, ring = 2 * e.ring * 32 * rb;
  const int per_cu = e.occ * 4 / e.nw;
  return D == 64 && e.pipe == 2 && per_cu >= 1 && per_cu * (ring + stage) <= 160 * 1024 ? stage : 0;
}

template <typename T, int D, int NW, int QT, int OCC, bool CAUSAL, int R, bool STREAM = false>
__global__ __launch_bounds__(NW * 64, OCC) void fwd_persist_kernel(const FwdParams p) {
  using H = H16<T>;
  using V8 = typename H::V8;
  using V4 = typename H::V4;
  using V2 = typename H::V2;
  using L = PersistLayout<D, R>;
  using SW = Swz<D>;
  constexpr int BM = NW * QT * 32;
  constexpr int NSD = D / 16;
  constexpr int DT = (D + 31) / 32;
  constexpr int CPK = (L::PIECES + NW - 1) / NW;  // K and V DMA instructions per wave per step
  constexpr int CPV = CPK;
  constexpr int CPW = CPK + CPV;
  constexpr int QL = QT * NSD;        // 16-byte Q loads per lane per block
  constexpr int SPI = CAUSAL ? 2 : 1;  // blocks per work item
  constexpr int SUB = BM / 32;         // steps of one block's own diagonal region (causal)
  constexpr int WAIT = (R - 3) * CPW;  // DMA operations a step leaves in flight at its end
  static_assert(R == 4 || R == 8, "ring depth");
  static_assert(!CAUSAL || (SUB % R == 0 && SUB / R <= 2), "causal diagonal region of one or two ring periods");
  static_assert(WAIT + QL < 64, "vmcnt field");
  // O through the wave's LDS rows and out as whole 128-byte rows with the non-temporal policy.
  // Inference forward, cold-cache medians, fp16, 16 heads, 16,384 tokens: non-causal N = 1024
  // -5.2%, 2048 -3.2%, 4096 -1.5%; causal N = 512 -10.9%, 1024 -5.2%, 2048 -2.5%; forward +
  // backward -1.7% / -2.8% at N = 512 (non-causal / causal), other shapes within +-0.4%.
  constexpr bool OSTAGE = fwd_persist_ostage_bytes(D, TileEntry{NW, QT, 32, OCC, 2, R}) > 0;
  constexpr int OCPR = L::RB / 16;  // 16-byte chunks of a staged O row
  static_assert(!OSTAGE || L::RB == 2 * D, "O staging stores whole rows without padding");
  // One array per ring slot: distinct objects let the compiler see that a DMA into one slot does
  // not alias reads of another (no conservative waits on in-flight tiles).
#define TATTN_PSLOT(name, s) __shared__ __attribute__((aligned(256))) char name[(s) < R ? L::SLOT : 16]
  TATTN_PSLOT(ks0, 0); TATTN_PSLOT(ks1, 1); TATTN_PSLOT(ks2, 2); TATTN_PSLOT(ks3, 3);
  TATTN_PSLOT(ks4, 4); TATTN_PSLOT(ks5, 5); TATTN_PSLOT(ks6, 6); TATTN_PSLOT(ks7, 7);
  TATTN_PSLOT(vs0, 0); TATTN_PSLOT(vs1, 1); TATTN_PSLOT(vs2, 2); TATTN_PSLOT(vs3, 3);
  TATTN_PSLOT(vs4, 4); TATTN_PSLOT(vs5, 5); TATTN_PSLOT(vs6, 6); TATTN_PSLOT(vs7, 7);
#undef TATTN_PSLOT
  __shared__ __attribute__((aligned(16))) char ost[OSTAGE ? NW * QT * 32 * L::RB : 16];
  auto kbuf = [&](int s) -> char* {
    return s == 0 ? ks0 : s == 1 ? ks1 : s == 2 ? ks2 : s == 3 ? ks3 : s == 4 ? ks4 : s == 5 ? ks5 : s == 6 ? ks6 : ks7;
  };
  auto vbuf = [&](int s) -> char* {
    return s == 0 ? vs0 : s == 1 ? vs1 : s == 2 ? vs2 : s == 3 ? vs3 : s == 4 ? vs4 : s == 5 ? vs5 : s == 6 ? vs6 : vs7;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h2 = lane >> 5, l32 = lane & 31;
  const int N = p.N;
  const int nb = p.n_qblocks;
  const int xcd = blockIdx.x & 7, lw = blockIdx.x >> 3;
  const int n_items = lw < p.items_x ? (p.items_x - lw + p.gx - 1) / p.gx : 0;
  const int nseg = n_items * SPI;
  const float c = p.c;
  const int wu = (int)uniform32((uint32_t)w);

  // Block t of this workgroup -> (slice, query block).
  auto seg_of = [&](int t, int& zh, int& qb) __attribute__((always_inline)) {
    const int k = lw + p.gx * (t / SPI);
    if constexpr (CAUSAL) {
      const int half = nb >> 1;
      zh = 8 * (k / half) + xcd;
      const int pr = k % half;
      qb = (t % SPI == 0) ? nb - 1 - pr : pr;
    } else {
      zh = 8 * (k / nb) + xcd;
      qb = k % nb;
    }
  };
  auto seg_steps = [&](int qb) __attribute__((always_inline)) { return CAUSAL ? (qb + 1) * SUB : N / 32; };
  // K / V buffer descriptors of a block's slice; past the last block, descriptors of zero bytes
  // (every load reads zeros and touches no memory).
  auto slice_k = [&](int t) __attribute__((always_inline)) {
    if (t >= nseg) return slice_rsrc(p.k, 0);
    int zh, qb;
    seg_of(t, zh, qb);
    return slice_rsrc((const T*)p.k + (int64_t)(zh / p.H) * p.sk[0] + (int64_t)(zh % p.H) * p.sk[1],
                      slice_bytes(N, p.sk[2], D));
  };
  auto slice_v = [&](int t) __attribute__((always_inline)) {
    if (t >= nseg) return slice_rsrc(p.v, 0);
    int zh, qb;
    seg_of(t, zh, qb);
    return slice_rsrc((const T*)p.v + (int64_t)(zh / p.H) * p.sv[0] + (int64_t)(zh % p.H) * p.sv[1],
                      slice_bytes(N, p.sv[2], D));
  };
  const uint32_t k_step = uniform32((uint32_t)(p.sk[2] * 64)), v_step = uniform32((uint32_t)(p.sv[2] * 64));

  // Cache policy of the K/V tile loads (STREAM: non-temporal, a short stay in the caches; the
  // launcher's rule says where).
  constexpr int KV_POLICY = STREAM ? 2 : 0;  // bit 1: nt

  // DMA work of this wave: pieces w, w + NW, ... of each tile (past the last piece a wave
  // repeats one: same bytes written again). LDS chunk j = 64 * piece + lane of a tile is chunk
  // j % (RB/16) of row j / (RB/16) in swizzled position, so the lane fetches global column chunk
  // (j % (RB/16)) ^ swz(row) of that row (key perm32(row) for K, the perm32 order that hands P
  // straight to the PV MFMAs; key `row` for V). Chunks past the head dim (D = 16 rows are 64
  // bytes) are padding and fetch a duplicate.
  int kpc[CPK];
  uint32_t kgo[CPK], vgo[CPV];
  auto piece = [&](int pp, int64_t rstride, bool perm, uint32_t& go) __attribute__((always_inline)) {
    const int cpr = L::RB / 16;
    const int j = 64 * pp + lane;
    const int row = j / cpr;
    const int cc = ((j % cpr) ^ SW::f(row)) & (D / 8 - 1);
    go = (uint32_t)((perm ? perm32(row) : row) * rstride * 2 + cc * 16);
  };
#pragma unroll
  for (int t = 0; t < CPK; ++t) {
    const int pp = (wu + NW * t) % L::PIECES;
    kpc[t] = 1024 * pp;
    piece(pp, p.sk[2], true, kgo[t]);
    piece(pp, p.sv[2], false, vgo[t]);
  }
  // The tile's offset (wave-uniform) goes into the scalar offset of the load, so one lane offset
  // serves every step: offsets per step position summed into VGPRs were held across the block
  // loop and spilled in the causal two-tile kernel. Every tile read lies inside its slice (N is a
  // multiple of the block and the ring period); past the last block the descriptor has zero bytes
  // and each load reads zeros.
  auto dma_k = [&](__amdgpu_buffer_rsrc_t rs, int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < CPK; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (TATTN_LDS void*)(kbuf(slot) + kpc[t]), 16, (int)kgo[t],
                                               (int)((uint32_t)kt * k_step), 0, KV_POLICY);
  };
  auto dma_v = [&](__amdgpu_buffer_rsrc_t rs, int vt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < CPV; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (TATTN_LDS void*)(vbuf(slot) + kpc[t]), 16, (int)vgo[t],
                                               (int)((uint32_t)vt * v_step), 0, KV_POLICY);
  };
  // End of a step: the DMAs of the previous step have landed (OUTSTANDING = memory operations
  // issued after them), this wave's LDS reads are done, then the barrier.
  auto step_end = [&](auto outstanding_tag) __attribute__((always_inline)) {
    constexpr int OUT = decltype(outstanding_tag)::value;
    __builtin_amdgcn_s_waitcnt((OUT & 15) | ((OUT >> 4) << 14) | 0x0070);  // vmcnt(OUT), lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };

  // Operand read offsets within a tile. K (A of S = K Q^T): row l32, bytes 32 sd + 16 h2. V^T (A of
  // O^T += V^T P^T) by transposed reads: rows 16 sg + 8 h2 + (src / 4) and + 4, column
  // 32 u + 16 (g & 1) + 4 (src & 3) (lane-group layout of ds_read_b64_tr_b16).
  // The swizzle depends on a row's index mod 16 only (Swz::f reads bits 0-3), so rows 16 sg + r
  // sit at r's pattern plus the constant 16 sg RB.
  const int g = lane >> 4, src = lane & 15;
  int kop[NSD], vlo[DT], vhi[DT];
#pragma unroll
  for (int sd = 0; sd < NSD; ++sd) kop[sd] = SW::addr(l32, 32 * sd + 16 * h2);
#pragma unroll
  for (int u = 0; u < DT; ++u) {
    const int row = 8 * h2 + (src >> 2);
    const int colb = (32 * u + 16 * (g & 1) + 4 * (src & 3)) * 2;
    vlo[u] = SW::addr(row, colb & (L::RB - 1));
    vhi[u] = SW::addr(row + 4, colb & (L::RB - 1));
  }

  V8 qop[QT][NSD];
  // Q rows of block (zh, qb) into the Q registers (plain loads; the caller decides when to wait).
  auto load_q = [&](int zh, int qb) __attribute__((always_inline)) {
    const T* Q = (const T*)p.q + (int64_t)(zh / p.H) * p.sq[0] + (int64_t)(zh % p.H) * p.sq[1];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const T* srcq = Q + (int64_t)(qb * BM + w * QT * 32 + 32 * j + l32) * p.sq[2] + 8 * h2;
#pragma unroll
      for (int s = 0; s < NSD; ++s) qop[j][s] = *reinterpret_cast<const V8*>(srcq + 16 * s);
    }
  };
  auto qk = [&](f32x16* s, int kb_) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < QT; ++j) s[j] = f32x16{};
#pragma unroll
    for (int sd = 0; sd < NSD; ++sd) {
      const V8 ka = *reinterpret_cast<const TATTN_LDS V8*>((const TATTN_LDS char*)kbuf(kb_) + kop[sd]);
#pragma unroll
      for (int j = 0; j < QT; ++j) s[j] = Elt<T>::mfma(ka, qop[j][sd], s[j]);
    }
  };
  float mrow[QT], lrow[QT];
  f32x16 acc[DT][QT];
  auto pv_mma = [&](const V8 (*pp)[2], int vb_) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < DT; ++u) {
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        const TATTN_LDS char* a = (const TATTN_LDS char*)vbuf(vb_) + 16 * sg * L::RB;
        const V4 lo = lds_tr<T>(a + vlo[u]), hi4 = lds_tr<T>(a + vhi[u]);
        V8 vop = V8{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        if (D < 32 && 32 * u + 16 * (g & 1) >= D) vop = V8{};
#pragma unroll
        for (int j = 0; j < QT; ++j) acc[u][j] = Elt<T>::mfma(vop, pp[j][sg], acc[u][j]);
      }
    }
  };

  // Diagonal 32x32 tile (first key = first row): register r holds key offset kappa(r, h2) of row
  // offset l32; keys past the row are hidden: kappa(r, h2) > l32, i.e. l32 - 8 h2 below
  // 16 (r / 8) + r % 8. One compare per use: sixteen lane masks computed once would be held
  // across the block loop in 32 SGPRs (spilled to VGPR lanes, which pushed VGPRs to scratch).
  // The empty asm keeps the compiler from hoisting the compares back out of the loop.
  const int diag_x = l32 - 8 * h2;
  auto diag_hide = [&](int r) __attribute__((always_inline)) {
    int x = diag_x;
    asm volatile("" : "+v"(x));
    return CAUSAL && x < 16 * (r >> 3) + (r & 7);
  };
  // Probabilities of one tile against the row max as it stands; hidden keys get probability 0
  // (after the exponential). Returns the lane's sum of the rounded probabilities.
  auto tile_probs = [&](const f32x16& st, V8* pt, float nm, auto diag_tag) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    float acc_s = 0.0f;
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      V8 xv;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float e0 = fast_exp2(__builtin_fmaf(st[8 * sg + i], c, nm));
        float e1 = fast_exp2(__builtin_fmaf(st[8 * sg + i + 1], c, nm));
        if constexpr (DIAG) {
          e0 = diag_hide(8 * sg + i) ? 0.0f : e0;
          e1 = diag_hide(8 * sg + i + 1) ? 0.0f : e1;
        }
        const V2 pr = H::pack(e0, e1);
        acc_s = H::sum2(pr, acc_s);
        xv[i] = pr[0];
        xv[i + 1] = pr[1];
      }
      pt[sg] = xv;
    }
    return acc_s;
  };
  // Row max of one tile over its visible keys (both lane-halves).
  auto tile_max = [&](const f32x16& st, auto diag_tag) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = (DIAG && diag_hide(r)) ? mx : __builtin_fmaxf(mx, st[r] * c);
    return max_halves(mx);
  };
  // Tile j of a step in the block's diagonal region: its place against the diagonal in 32-row
  // units (wave-uniform): < 0 above (no visible key), 0 on the diagonal, > 0 below.
  auto rel_of = [&](int j, int ii) __attribute__((always_inline)) { return wu * QT + j - ii; };

  // Softmax of step i's scores (ii: index in the causal diagonal region, or -1 outside it).
  // EXACT: row max taken first (lazy update, accumulator rescaled), never recomputes S.
  // Otherwise the max-free fast path with the slow path on a 2^12 overflow (S recomputed from
  // K buffer kc_, which needs this block's Q in the Q registers).
  auto probs = [&](f32x16* scur, V8 (*pc)[2], int ii, int kc_, auto exact_tag) __attribute__((always_inline)) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    if constexpr (EXACT) {
      float alpha[QT];
      bool any = false;
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const int rel = CAUSAL && ii >= 0 ? rel_of(j, ii) : 1;
        alpha[j] = 1.0f;
        if (rel < 0) {
          pc[j][0] = pc[j][1] = V8{};
          continue;
        }
        const float cand = rel == 0 ? tile_max(scur[j], std::true_type{}) : tile_max(scur[j], std::false_type{});
        const bool upd = cand > mrow[j] + kRescaleLog2;
        const float mnew = upd ? cand : mrow[j];
        alpha[j] = fast_exp2(mrow[j] - mnew);
        any |= upd;
        mrow[j] = mnew;
        const float ps = rel == 0 ? tile_probs(scur[j], pc[j], -mnew, std::true_type{})
                                  : tile_probs(scur[j], pc[j], -mnew, std::false_type{});
        lrow[j] = lrow[j] * alpha[j] + ps;
      }
      if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
        for (int j = 0; j < QT; ++j)
#pragma unroll
          for (int u = 0; u < DT; ++u) acc[u][j] *= alpha[j];
      }
    } else {
      bool need = false;
      float ps[QT], lprev[QT];
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const int rel = CAUSAL && ii >= 0 ? rel_of(j, ii) : 1;
        if (rel < 0) {
          pc[j][0] = pc[j][1] = V8{};
          ps[j] = 0.0f;
        } else {
          ps[j] = rel == 0 ? tile_probs(scur[j], pc[j], -mrow[j], std::true_type{})
                           : tile_probs(scur[j], pc[j], -mrow[j], std::false_type{});
        }
        need |= !(ps[j] <= 4096.0f);
        lprev[j] = lrow[j];
        lrow[j] += ps[j];
      }
      if (__builtin_amdgcn_ballot_w64(need)) {  // slow path: row max, rescale, probabilities again
#pragma unroll
        for (int j = 0; j < QT; ++j) lrow[j] = lprev[j];
        qk(scur, kc_);
        float alpha[QT];
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          const int rel = CAUSAL && ii >= 0 ? rel_of(j, ii) : 1;
          alpha[j] = 1.0f;
          if (rel < 0) continue;
          const float cand = rel == 0 ? tile_max(scur[j], std::true_type{}) : tile_max(scur[j], std::false_type{});
          const bool upd = cand > mrow[j] + kRescaleLog2;
          const float mnew = upd ? cand : mrow[j];
          alpha[j] = fast_exp2(mrow[j] - mnew);
          mrow[j] = mnew;
          const float ps2 = rel == 0 ? tile_probs(scur[j], pc[j], -mnew, std::true_type{})
                                     : tile_probs(scur[j], pc[j], -mnew, std::false_type{});
          lrow[j] = lrow[j] * alpha[j] + ps2;
        }
#pragma unroll
        for (int j = 0; j < QT; ++j)
#pragma unroll
          for (int u = 0; u < DT; ++u) acc[u][j] *= alpha[j];
      }
    }
  };

  if (nseg == 0) return;

  // ---- block 0 prologue: Q, the first K/V tiles, S_0 -------------------------------------
  int zh, qb;
  seg_of(0, zh, qb);
  int nsteps = seg_steps(qb);
  __amdgpu_buffer_rsrc_t krs = slice_k(0), vrs = slice_v(0);
  __amdgpu_buffer_rsrc_t krs_n = slice_k(1), vrs_n = slice_v(1);
  // Prologue: this block's Q, K_0, then the batches the R - 2 steps before step 0 would have
  // started (K_{j+R-1} with V_{j+R-2}). All of it lands before the first step: the compiler may
  // reorder these independent loads among themselves, so no partial vmcnt count would tell
  // which have arrived.
  load_q(zh, qb);
  dma_k(krs, 0, 0);
#pragma unroll
  for (int j = 1; j < R - 1; ++j) {
    dma_k(krs, j, j);
    dma_v(vrs, j - 1, j - 1);
  }
  step_end(IC<0>{});

  f32x16 sa[QT], sb[QT];
  V8 pa[QT][2], pb[QT][2];
  // Entering a block: state reset, S_0 from K slot 0 and the block's Q, running max seeded with
  // S_0's row max over the visible keys.
  auto begin_block = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      lrow[j] = 0.0f;
#pragma unroll
      for (int u = 0; u < DT; ++u) acc[u][j] = f32x16{};
    }
    qk(sa, 0);
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const int q = qb * BM + w * QT * 32 + 32 * j + l32;
      float mx = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = (!CAUSAL || kappa(r, h2) <= q) ? __builtin_fmaxf(mx, sa[j][r] * c) : mx;
      mrow[j] = max_halves(mx);
    }
  };
  begin_block();

  // Workgroups sharing a CU (ranks blockIdx / CUs: 0 dispatched first) alternate the issue
  // priority of their waves item by item. The SIMD arbiter favours older waves at equal
  // priority, so otherwise the first workgroup of a CU runs its items at near full speed while
  // the second crawls, and ends alone on its last item, at the lower throughput of one
  // workgroup per CU.
  const int rank = blockIdx.x / p.cus;
  // A workgroup with a single work item (causal entries with 256-row blocks: one pair of blocks
  // per slot) would keep one priority for its whole life; it switches on a global time slice of
  // 4096 ticks of the 100 MHz counter (41 us) instead, out of phase by rank.
  const bool time_prio = n_items == 1;
  for (int t = 0; t < nseg; ++t) {
    if (t % SPI == 0 && !time_prio) {
      if (((t / SPI) + rank) & 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    // One step, local index i (i % R == IV), slots constant. LASTG: the block's last group (DMA
    // reaches into the next block; its last two steps exact, the next block's Q loaded in step
    // R - 2, no S in step R - 1); ii: diagonal-region index, or -1 outside it.
    auto step = [&](int i, f32x16* scur, f32x16* snext, const V8 (*pprev)[2], V8 (*pcur)[2], auto iv_tag,
                    auto last_tag, int ii) __attribute__((always_inline)) {
      constexpr int IV = decltype(iv_tag)::value;
      constexpr bool LASTG = decltype(last_tag)::value;
      constexpr bool QLOAD = LASTG && IV == R - 2, FINAL = LASTG && IV == R - 1;
      // DMA: K of step i + R - 1 into the slot K_{i-1} left, V of step i + R - 2 into the slot
      // V_{i-2} left (tiles of the next block past this block's end).
      if (LASTG && IV >= 1) dma_k(krs_n, IV - 1, (IV + R - 1) % R);
      else dma_k(krs, i + R - 1, (IV + R - 1) % R);
      if (LASTG && IV >= 2) dma_v(vrs_n, IV - 2, (IV + R - 2) % R);
      else dma_v(vrs, i + R - 2, (IV + R - 2) % R);
      // PV of step i-1 (waves whose tiles all lie above the diagonal at i-1 skip it).
      const bool pv_live = i > 0 && (!CAUSAL || ii < 0 || ii == 0 || wu * QT + QT - 1 >= ii - 1);
      if (pv_live) pv_mma(pprev, (IV + R - 1) % R);
      const bool live = !CAUSAL || ii < 0 || wu * QT + QT - 1 >= ii;  // any tile at or below the diagonal
      if constexpr (!FINAL) {
        if (!CAUSAL || ii < 0 || wu * QT + QT - 1 >= ii + 1) qk(snext, (IV + 1) % R);
      }
      const bool more = t + 1 < nseg;  // a next block follows (wave-uniform)
      if constexpr (QLOAD) {
        // The next block's Q, into the registers the last S of this block has just read.
        if (more) {
          int zn, qn;
          seg_of(t + 1, zn, qn);
          load_q(zn, qn);
        }
      }
      if (live) {
        if constexpr (LASTG && IV >= R - 2) probs(scur, pcur, ii, IV, std::true_type{});
        else probs(scur, pcur, ii, IV, std::false_type{});
      }
      // The tiles step i+1 reads were started R - 3 steps ago: later DMA batches (and the Q loads
      // of step R - 2) stay in flight.
      if constexpr (QLOAD || FINAL) {
        if (more) step_end(IC<WAIT + QL>{});
        else step_end(IC<WAIT>{});
      } else {
        step_end(IC<WAIT>{});
      }
    };
    // R consecutive steps from i (i % R == 0); the S / P register sets alternate.
    auto group = [&](int i, auto last_tag, int ii0) __attribute__((always_inline)) {
      auto ii = [&](int k) __attribute__((always_inline)) { return ii0 < 0 ? -1 : ii0 + k; };
      if (time_prio) {
        const uint32_t slot = (uint32_t)(__builtin_amdgcn_s_memrealtime() >> 12);
        if ((slot + (uint32_t)rank) & 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      step(i, sa, sb, pa, pb, IC<0>{}, last_tag, ii(0));
      step(i + 1, sb, sa, pb, pa, IC<1>{}, last_tag, ii(1));
      step(i + 2, sa, sb, pa, pb, IC<2>{}, last_tag, ii(2));
      step(i + 3, sb, sa, pb, pa, IC<3>{}, last_tag, ii(3));
      if constexpr (R == 8) {
        step(i + 4, sa, sb, pa, pb, IC<4>{}, last_tag, ii(4));
        step(i + 5, sb, sa, pb, pa, IC<5>{}, last_tag, ii(5));
        step(i + 6, sa, sb, pa, pb, IC<6>{}, last_tag, ii(6));
        step(i + 7, sb, sa, pb, pa, IC<7>{}, last_tag, ii(7));
      }
    };

    const int ngroups = nsteps / R;
    // Groups before the causal diagonal region need no mask.
    const int g_mask = CAUSAL ? ngroups - SUB / R : ngroups;
    int gi = 0;
    for (; gi < min(g_mask, ngroups - 1); ++gi) group(R * gi, std::false_type{}, -1);
    if constexpr (CAUSAL && SUB == 2 * R) {
      if (gi < ngroups - 1) {  // first group of a two-group diagonal region
        group(R * gi, std::false_type{}, 0);
        ++gi;
      }
    }
    group(R * gi, std::true_type{}, CAUSAL ? SUB - R : -1);  // the block's last group
    // Drain: PV of the block's last step (V slot R - 1), then the block's O and M.
    if (!CAUSAL || wu * QT + QT - 1 >= SUB - 1) pv_mma(pa, R - 1);
    // The workgroup's last block: its last DMAs (zero-byte descriptors past the end, they touch no
    // memory) must land before the workgroup's LDS is released. Waiting here, before the O and M
    // stores, lets the waves end without waiting for those stores.
    if (t + 1 == nseg) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    if constexpr (OSTAGE) {
      // Wave-local rows: no barrier between the LDS writes and the reads. Row and lane indices
      // are computed here (the empty asm), not held across the block loop.
      TATTN_LDS char* wt = (TATTN_LDS char*)ost + w * QT * 32 * L::RB;
      int rl = l32;
      asm volatile("" : "+v"(rl));
      float* M = p.m ? p.m + (int64_t)zh * N : nullptr;
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const float lt = sum_halves(lrow[j]);
        const float inv = 1.0f / lt;
#pragma unroll
        for (int u = 0; u < DT; ++u)
#pragma unroll
          for (int g2 = 0; g2 < 4; ++g2) {
            const int d0 = 32 * u + 8 * g2 + 4 * h2;
            V4 xo;
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) xo[i2] = (T)(acc[u][j][4 * g2 + i2] * inv);
            *reinterpret_cast<TATTN_LDS V4*>(wt + SW::addr(32 * j + rl, 2 * d0)) = xo;
          }
        if (h2 == 0 && M) M[qb * BM + w * QT * 32 + 32 * j + rl] = mrow[j] + __log2f(lt);
      }
      T* ob = (T*)p.o + (int64_t)(zh / p.H) * p.so[0] + (int64_t)(zh % p.H) * p.so[1] +
              (int64_t)(qb * BM + w * QT * 32) * p.so[2];
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int it = 0; it < QT * 32 * OCPR / 64; ++it) {
        const int jj = ln + 64 * it;
        const int row = jj / OCPR, cc = jj % OCPR;
        const u32x4 x = *reinterpret_cast<const TATTN_LDS u32x4*>(wt + SW::addr(row, 16 * cc));
        st16_stream(ob + (int64_t)row * p.so[2] + 8 * cc, x);
      }
    } else {
      T* O = (T*)p.o + (int64_t)(zh / p.H) * p.so[0] + (int64_t)(zh % p.H) * p.so[1];
      float* M = p.m ? p.m + (int64_t)zh * N : nullptr;
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const float lt = sum_halves(lrow[j]);
        const float inv = 1.0f / lt;
        const int q = qb * BM + w * QT * 32 + 32 * j + l32;
        T* orow = O + (int64_t)q * p.so[2];
#pragma unroll
        for (int u = 0; u < DT; ++u)
#pragma unroll
          for (int g2 = 0; g2 < 4; ++g2) {
            const int d0 = 32 * u + 8 * g2 + 4 * h2;
            if (d0 < D) {
              V4 xo;
#pragma unroll
              for (int i2 = 0; i2 < 4; ++i2) xo[i2] = (T)(acc[u][j][4 * g2 + i2] * inv);
              *reinterpret_cast<V4*>(orow + d0) = xo;
            }
          }
        if (h2 == 0 && M) M[q] = mrow[j] + __log2f(lt);
      }
    }
    if (t + 1 == nseg) break;
    // Next block. K_0 (slot 0) landed before the last step's barrier; the compiler waits for the
    // Q loads of step L-2 at their first use (counting the DMA and stores issued since, which
    // stay in flight).
    seg_of(t + 1, zh, qb);
    nsteps = seg_steps(qb);
    krs = krs_n;
    vrs = vrs_n;
    krs_n = slice_k(t + 2);
    vrs_n = slice_v(t + 2);
    begin_block();
  }
}

// Persistent forward: grid of one workgroup per resident slot (at most), the work split per XCD
// into whole rounds. Returns 1 (nothing launched) when the problem does not meet the kernel's
// preconditions.
// Resident workgroups per CU of one instantiation (same on every gfx950).
template <typename T, int D, int NW, int QT, int OCC, bool CAUSAL, int R, bool STREAM>
int fwd_persist_per_cu() {
  static int per_cu = 0;
  if (per_cu <= 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fwd_persist_kernel<T, D, NW, QT, OCC, CAUSAL, R, STREAM>,
                                                     NW * 64, 0) != hipSuccess ||
        n <= 0)
      n = 1;
    per_cu = n;
  }
  return per_cu;
}

template <typename T, int D, int NW, int QT, int OCC, bool CAUSAL, int R>
int launch_fwd_persist(FwdParams p, hipStream_t st, int* rc) {
  constexpr int BM = NW * QT * 32;
  constexpr TileEntry self{NW, QT, 32, OCC, 2, R};
  const int64_t S = (int64_t)p.Z * p.H;
  if (!fwd_persist_fits(self, S, p.N, CAUSAL)) return 1;
  const int nb = p.N / BM;
  const int64_t items_x = S / 8 * (CAUSAL ? nb / 2 : nb);
  if (items_x >= (1 << 30)) return 1;
  // K/V streamed with the non-temporal policy: the inference forward (no M saved, so no backward
  // reads Q, K, V after it) at head dim 64 without a mask, whose blocks read their slice's K/V
  // once. A cold short launch then displaces less of what the caches hold: 6-8% faster at
  // N = 512, 3-4.5% at 1024, 0.5-1.4% at 2048-4096, even at longer rows (fp16, 16 heads, 16,384
  // tokens, same-box interleaved runs on three boxes). Where M is saved the backward that follows
  // re-reads K and V: with the hint the forward + backward took 3.6% / 2.9% / 1.4% longer at
  // N = 512 / 1024 / 2048. Causal blocks re-read prefixes of their slice's K/V through L2 (the hint
  // cost 4-5% at N = 1024-2048 and 16384), and at head dim 128 it cost 1-4%.
  constexpr bool CAN_STREAM = !CAUSAL && D == 64;
  const bool stream = CAN_STREAM && p.m == nullptr;
  const int per_cu = stream ? fwd_persist_per_cu<T, D, NW, QT, OCC, CAUSAL, R, CAN_STREAM>()
                            : fwd_persist_per_cu<T, D, NW, QT, OCC, CAUSAL, R, false>();
  p.cus = device_cus();
  const int64_t slots_x = std::max<int64_t>(1, (int64_t)per_cu * p.cus / 8);
  const int64_t rounds = (items_x + slots_x - 1) / slots_x;
  p.n_qblocks = nb;
  p.items_x = (int32_t)items_x;
  p.gx = (int32_t)((items_x + rounds - 1) / rounds);
  if (stream)
    fwd_persist_kernel<T, D, NW, QT, OCC, CAUSAL, R, CAN_STREAM><<<dim3(8u * (unsigned)p.gx), dim3(NW * 64), 0, st>>>(p);
  else
    fwd_persist_kernel<T, D, NW, QT, OCC, CAUSAL, R, false><<<dim3(8u * (unsigned)p.gx), dim3(NW * 64), 0, st>>>(p);
  *rc = check_launch("tattn_fwd");
  return 0;
}

}  // namespace tattn
