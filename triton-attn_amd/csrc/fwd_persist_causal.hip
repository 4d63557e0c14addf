// Persistent causal forward with two query tiles per wave (fwd_persist_kernel, 16-bit), in a
// translation unit of its own: the library builds it with LLVM's iterative ILP scheduler
// (-amdgpu-sched-strategy=iterative-ilp), which was 3.5-4% faster on this kernel at the
// benchmark lengths where it is picked (N >= 4096) and slower on the other forward kernels.
// Part of the forward (the reference's src/tattn/kernels.py:57-148, causal rows).
#include <type_traits>
#include <utility>

#include "fwd_persist.h"

namespace tattn {

namespace {

template <typename T, int D, int I>
int causal2_entry(const FwdParams& p, hipStream_t st, int* rc) {
  constexpr TileEntry e = FwdTable<T, D>::e[I];
  if constexpr (sizeof(T) == 2 && e.pipe == 2 && e.tiles == 2 && fwd_persist_causal_ok(e))
    return launch_fwd_persist<T, D, e.nw, e.tiles, e.occ, true, e.ring>(p, st, rc);
  else
    return 1;
}

template <typename T, int D, size_t... I>
int causal2_dispatch(int id, const FwdParams& p, hipStream_t st, int* rc, std::index_sequence<I...>) {
  int r = 1;
  ((id == (int)I ? (r = causal2_entry<T, D, I>(p, st, rc), 0) : 0), ...);
  return r;
}

template <typename T>
int causal2_type(int D, int id, const FwdParams& p, hipStream_t st, int* rc) {
  switch (D) {
    case 16: return causal2_dispatch<T, 16>(id, p, st, rc, std::make_index_sequence<FwdTable<T, 16>::n>{});
    case 32: return causal2_dispatch<T, 32>(id, p, st, rc, std::make_index_sequence<FwdTable<T, 32>::n>{});
    case 64: return causal2_dispatch<T, 64>(id, p, st, rc, std::make_index_sequence<FwdTable<T, 64>::n>{});
    case 128: return causal2_dispatch<T, 128>(id, p, st, rc, std::make_index_sequence<FwdTable<T, 128>::n>{});
  }
  return 1;
}

}  // namespace

int launch_fwd_persist_causal2(const FwdParams& p, int D, int dtype, int config_id, hipStream_t st, int* rc) {
  if (dtype == 0) return causal2_type<f16>(D, config_id, p, st, rc);
  if (dtype == 2) return causal2_type<bf16>(D, config_id, p, st, rc);
  return 1;
}

}  // namespace tattn
