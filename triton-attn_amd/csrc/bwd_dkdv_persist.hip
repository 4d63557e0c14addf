// Persistent dK/dV launcher (dkdv_persist_kernel, bwd_dkdv_persist.h) in a translation unit of its
// own, built with the library's default instruction scheduler.
// Part of the backward (the dK/dV kernel, the reference's src/tattn/kernels.py:151-239).
#include <algorithm>
#include <type_traits>
#include <utility>

#include "bwd_dkdv_persist.h"
#include "launch.h"
#include "tiles.h"

namespace tattn {

namespace {

// Grid of one workgroup per resident slot (at most), the work split per XCD into whole rounds.
template <typename T, int D, int NW, int OCC, bool CAUSAL>
int run_dkdv_persist(BwdParams p, hipStream_t st) {
  auto kern = dkdv_persist_kernel<T, D, NW, OCC, CAUSAL>;
  const int nb = p.N / (NW * 32);
  const int64_t items_x = (int64_t)p.Z * p.H / 8 * (CAUSAL ? nb / 2 : nb);
  if (items_x >= (1 << 30)) return set_error(TATTN_E_ARG, "problem too large");
  static int per_cu = 0;  // resident workgroups per CU (same on every gfx950)
  if (per_cu <= 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, NW * 64, 0) != hipSuccess || n <= 0) n = 1;
    per_cu = n;
  }
  p.cus = device_cus();
  const int64_t slots_x = std::max<int64_t>(1, (int64_t)per_cu * p.cus / 8);
  const int64_t rounds = (items_x + slots_x - 1) / slots_x;
  p.n_blocks = nb;
  p.items_x = (int32_t)items_x;
  p.gx = (int32_t)((items_x + rounds - 1) / rounds);
  kern<<<dim3(8u * (unsigned)p.gx), dim3(NW * 64), 0, st>>>(p);
  return check_launch("tattn_bwd_dkdv");
}

template <typename T, int D, int I>
int dkdv_persist_entry(const BwdParams& p, bool causal, hipStream_t st) {
  constexpr TileEntry e = DkdvTable<T, D>::e[I];
  if constexpr (sizeof(T) == 2 && e.pipe == 2 && e.tiles == 1 && D <= 64)
    return causal ? run_dkdv_persist<T, D, e.nw, e.occ, true>(p, st) : run_dkdv_persist<T, D, e.nw, e.occ, false>(p, st);
  else
    return set_error(TATTN_E_CONFIG, "dK/dV config id %d is not a persistent entry", I);
}

template <typename T, int D, size_t... I>
int dkdv_persist_dispatch(int id, const BwdParams& p, bool causal, hipStream_t st, std::index_sequence<I...>) {
  int rc = set_error(TATTN_E_CONFIG, "dK/dV config id %d out of range [0, %d) for D=%d", id, (int)sizeof...(I), D);
  ((id == (int)I ? (rc = dkdv_persist_entry<T, D, I>(p, causal, st), 0) : 0), ...);
  return rc;
}

template <typename T>
int dkdv_persist_type(int D, int id, const BwdParams& p, bool causal, hipStream_t st) {
  switch (D) {
    case 16: return dkdv_persist_dispatch<T, 16>(id, p, causal, st, std::make_index_sequence<DkdvTable<T, 16>::n>{});
    case 32: return dkdv_persist_dispatch<T, 32>(id, p, causal, st, std::make_index_sequence<DkdvTable<T, 32>::n>{});
    case 64: return dkdv_persist_dispatch<T, 64>(id, p, causal, st, std::make_index_sequence<DkdvTable<T, 64>::n>{});
    case 128: return dkdv_persist_dispatch<T, 128>(id, p, causal, st, std::make_index_sequence<DkdvTable<T, 128>::n>{});
  }
  return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %d", D);
}

}  // namespace

int launch_dkdv_persist(const BwdParams& p, int D, int dtype, int config_id, bool causal, hipStream_t st) {
  if (dtype == 0) return dkdv_persist_type<f16>(D, config_id, p, causal, st);
  if (dtype == 2) return dkdv_persist_type<bf16>(D, config_id, p, causal, st);
  return set_error(TATTN_E_CONFIG, "persistent dK/dV entries are 16-bit only");
}

}  // namespace tattn
