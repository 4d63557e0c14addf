// gfx950 tile tables for the tattn kernels (replaces the reference's sm75 autotune lists,
// src/tattn/kernels.py:21-54). One table per (kernel, element type, head dim); an entry is
// {waves per workgroup, 32-row tiles per wave, block of the other dimension}.
//
//   forward  : block_m = waves * tiles * 32 query rows per workgroup, block_n keys per step
//   dK/dV    : block_n = waves * tiles * 32 key rows per workgroup, block_m queries per step
//   dQ       : block_m = waves * tiles * 32 query rows per workgroup, block_n keys per step
//
// Every entry is instantiated for causal and non-causal and is reachable through the C ABI
// by index, so tests can run each one (the reference's test_configs.py:37-54 analog).
#pragma once

#include <stdint.h>

namespace tattn {

struct TileEntry {
  int nw;     // waves per workgroup
  int tiles;  // 32-row MFMA tiles per wave (queries for fwd/dQ, keys for dK/dV)
  int other;  // keys per step (fwd, dQ) or queries per step (dK/dV)
  int occ;    // waves per SIMD the kernel is compiled for (register budget 512 / occ)
  int pipe;   // 3: backward with paired waves (split roles), 2: persistent 16-bit kernel,
              // 1: software-pipelined 16-bit kernel, 0: generic kernel
  int ring = 4;  // persistent forward: LDS ring depth (K/V tiles), 4 or 8
};

// Rows (queries, or keys for dK/dV) one workgroup owns. The paired-wave backward kernels give
// each 32-row tile two waves, one per role.
constexpr int tile_rows(const TileEntry& e) { return (e.pipe == 3 ? e.nw / 2 : e.nw) * e.tiles * 32; }

// ---- forward ----------------------------------------------------------------------------
template <typename T, int D> struct FwdTable;
#define TATTN_TABLE(NAME, T, D, ...)                                    \
  template <> struct NAME<T, D> {                                       \
    static constexpr TileEntry e[] = {__VA_ARGS__};                     \
    static constexpr int n = sizeof(e) / sizeof(e[0]);                  \
  };
// The 16-bit element types (fp16, bf16) share one table: same kernels, same tiles.
#define TATTN_TABLE16(NAME, D, ...)          \
  TATTN_TABLE(NAME, _Float16, D, __VA_ARGS__) \
  TATTN_TABLE(NAME, __bf16, D, __VA_ARGS__)

// The picks per sequence length are measured and live in pick_config (abi.hip); entry 0 is the
// pick wherever no rule names another. Kinds (`pipe`): 1 software-pipelined (32 rows per step),
// 2 persistent (16-bit; where a problem does not meet its preconditions the pipelined kernel of
// the same tiles runs it), 3 paired-wave backward, 0 generic. The 16-bit entries fit their
// register budgets (512 / waves per SIMD) without scratch, except the non-causal persistent
// dK/dV (28 bytes of per-lane constants, reloaded once per key block), and reach their waves per
// SIMD within the 160 KB of LDS (a persistent forward workgroup holds a 32 KB K/V ring at D=64
// plus 16-32 KB of O rows on their way out, a 64 KB ring at D=128). Of the fp32 kernels only
// causal dK/dV at D=128 spills (32 bytes).
TATTN_TABLE16(FwdTable, 16, {4, 2, 32, 2, 1}, {4, 1, 32, 2, 1}, {8, 1, 32, 4, 1})
TATTN_TABLE16(FwdTable, 32, {4, 2, 32, 2, 1}, {4, 1, 32, 2, 1}, {8, 1, 32, 4, 1})
TATTN_TABLE16(FwdTable, 64, {4, 2, 32, 2, 1}, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {8, 2, 32, 2, 1},
              {4, 2, 32, 2, 2, 8}, {4, 1, 32, 2, 2, 4}, {8, 1, 32, 2, 2, 8}, {4, 2, 32, 2, 2, 4})
TATTN_TABLE16(FwdTable, 128, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 1, 32, 2, 2, 4}, {8, 1, 32, 2, 2, 4})
TATTN_TABLE(FwdTable, float, 16, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(FwdTable, float, 32, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(FwdTable, float, 64, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(FwdTable, float, 128, {4, 1, 32, 1, 0})

}  // namespace tattn

namespace tattn {

// ---- backward dK/dV: {waves, key tiles per wave, queries per step} -------------------------
template <typename T, int D> struct DkdvTable;
TATTN_TABLE16(DkdvTable, 16, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 1, 64, 2, 0}, {4, 1, 32, 2, 0}, {4, 2, 32, 2, 0})
TATTN_TABLE16(DkdvTable, 32, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 1, 64, 2, 0}, {4, 1, 32, 2, 0}, {4, 2, 32, 2, 0})
TATTN_TABLE16(DkdvTable, 64, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 1, 32, 2, 0}, {4, 2, 32, 1, 1}, {8, 1, 32, 2, 3},
              {4, 1, 32, 2, 2}, {8, 1, 32, 2, 2})
TATTN_TABLE16(DkdvTable, 128, {4, 1, 32, 1, 1}, {4, 1, 32, 1, 0}, {8, 1, 32, 2, 3})
TATTN_TABLE(DkdvTable, float, 16, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(DkdvTable, float, 32, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(DkdvTable, float, 64, {4, 1, 32, 2, 0})
TATTN_TABLE(DkdvTable, float, 128, {4, 1, 32, 1, 0})

// ---- backward dQ: {waves, query tiles per wave, keys per step} ------------------------------
template <typename T, int D> struct DqTable;
TATTN_TABLE16(DqTable, 16, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 2, 32, 2, 0}, {4, 1, 64, 2, 0}, {4, 1, 32, 2, 0})
TATTN_TABLE16(DqTable, 32, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 2, 32, 2, 0}, {4, 1, 64, 2, 0}, {4, 1, 32, 2, 0})
TATTN_TABLE16(DqTable, 64, {4, 1, 32, 2, 1}, {8, 1, 32, 2, 1}, {4, 1, 64, 2, 0}, {4, 1, 32, 2, 0}, {8, 1, 64, 2, 0},
              {4, 1, 32, 2, 2}, {8, 1, 32, 2, 2}, {8, 1, 32, 2, 3})
TATTN_TABLE16(DqTable, 128, {4, 1, 32, 1, 1}, {4, 1, 32, 1, 0}, {8, 1, 32, 2, 3})
TATTN_TABLE(DqTable, float, 16, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(DqTable, float, 32, {4, 1, 32, 2, 0}, {4, 1, 64, 2, 0})
TATTN_TABLE(DqTable, float, 64, {4, 1, 32, 2, 0})
TATTN_TABLE(DqTable, float, 128, {4, 1, 32, 1, 0})

}  // namespace tattn
