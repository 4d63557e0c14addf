// Host-side helpers shared by the kernel translation units: error reporting and launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "common.h"
#include "tiles.h"

#define TATTN_OK 0
#define TATTN_E_ARG 1
#define TATTN_E_CONFIG 2
#define TATTN_E_LAUNCH 3
#define TATTN_E_DEVICE 4

namespace tattn {

// Records a printf-style message as this thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Returns TATTN_OK, or TATTN_E_LAUNCH with the HIP error text if the last launch failed.
int check_launch(const char* what);

int launch_fwd(const FwdParams& p, int D, int dtype, bool causal, int config_id, hipStream_t st);
int launch_bwd_preprocess(const BwdParams& p, int D, int dtype, hipStream_t st);
int launch_bwd_dkdv(const BwdParams& p, int D, int dtype, bool causal, int config_id, hipStream_t st);
int launch_bwd_dq(const BwdParams& p, int D, int dtype, bool causal, int config_id, hipStream_t st);

int fwd_lds_bytes(int D, int dtype, const TileEntry& e);

// Kernels that get their own translation unit, compiled with the instruction scheduler that
// measured fastest for them (tattn/_build.py: SOURCE_FLAGS); dtype 0 = fp16, 2 = bf16.
// Persistent causal forward with two query tiles per wave (fwd_persist_causal.hip): runs entry
// `config_id` of the forward table; returns 1 (nothing launched) when the problem does not fit
// the kernel, else 0 with *rc the launch status.
int launch_fwd_persist_causal2(const FwdParams& p, int D, int dtype, int config_id, hipStream_t st, int* rc);
// Persistent dQ (bwd_dq_persist.hip): runs entry `config_id` of the dQ table; the caller has
// checked bwd_persist_fits and bwd_fits32.
int launch_dq_persist(const BwdParams& p, int D, int dtype, int config_id, bool causal, hipStream_t st);
// Persistent dK/dV (bwd_dkdv_persist.hip): runs entry `config_id` of the dK/dV table; the caller
// has checked bwd_persist_fits and bwd_fits32.
int launch_dkdv_persist(const BwdParams& p, int D, int dtype, int config_id, bool causal, hipStream_t st);
// Paired-wave backward (bwd_split.hip): dK/dV (dkdv = true) or dQ with 128 rows per workgroup,
// p.n_blocks set by the caller; the caller has checked bwd_fits32.
int launch_split(const BwdParams& p, int D, int dtype, bool dkdv, bool causal, hipStream_t st);

// Whether the backward's (z, h) slices fit 32-bit buffer offsets (plus two steps of look-ahead):
// the pipelined and persistent backward kernels need it, the generic ones take 64-bit addresses.
inline bool bwd_fits32(const BwdParams& p, int D) {
  return slice_bytes(p.N, p.s[2], D) + (uint64_t)p.s[2] * 128 < (1ull << 31);
}

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Whether a persistent backward entry (kind 2) runs a problem itself; otherwise the launcher
// runs the pipelined kernel of the same waves. Z*H a multiple of 8, N a multiple of the block
// and of 128 (whole groups of four steps), causal: an even number of blocks per slice (pairs).
inline bool bwd_persist_fits(const TileEntry& e, int64_t ZH, int64_t N, bool causal) {
  const int64_t blk = (int64_t)e.nw * 32;
  if (e.pipe != 2 || ZH % 8 != 0 || N % blk != 0 || N % 128 != 0) return false;
  return !causal || (N / blk) % 2 == 0;
}

// Whether a persistent forward entry (kind 2) runs a problem itself; otherwise the launcher runs
// the pipelined kernel of the same tiles. Z*H a multiple of 8 (whole slices per XCD), N a
// multiple of the block and of the ring period (whole unrolled groups), causal: an even number
// of blocks per slice (pairs), a diagonal region of one or two ring periods, and one 32-row tile
// per wave or a ring of 4 (the causal kernel with two tiles per wave and a ring of 8 does not fit
// the 256 registers a wave has at two waves per SIMD; those entries run their pipelined twin for
// causal problems).
constexpr bool fwd_persist_causal_ok(const TileEntry& e) {
  return (e.tiles == 1 || e.ring == 4) && (e.nw * e.tiles) % e.ring == 0 && e.nw * e.tiles / e.ring <= 2;
}
inline bool fwd_persist_fits(const TileEntry& e, int64_t ZH, int64_t N, bool causal) {
  const int64_t bm = (int64_t)e.nw * e.tiles * 32;
  if (e.pipe != 2 || ZH % 8 != 0 || N % bm != 0 || N % (32 * e.ring) != 0) return false;
  return !causal || ((N / bm) % 2 == 0 && fwd_persist_causal_ok(e));
}
int dkdv_lds_bytes(int D, int dtype, const TileEntry& e);
int dq_lds_bytes(int D, int dtype, const TileEntry& e);

}  // namespace tattn
