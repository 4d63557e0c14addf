// Persistent dQ launcher (dq_persist_kernel, bwd_persist.h) in a translation unit of its own:
// the library builds it with LLVM's max-ILP scheduler (-amdgpu-sched-strategy=max-ilp), which
// made this kernel 3-12% faster at the benchmark lengths (fp16, D = 64, both masks) with the
// same results bit for bit, and made the dK/dV kernels slower.
// Part of the backward (the dQ kernel, the reference's src/tattn/kernels.py:242-321).
#include <algorithm>
#include <type_traits>
#include <utility>

#include "bwd_persist.h"
#include "launch.h"
#include "tiles.h"

namespace tattn {

namespace {

// Grid of one workgroup per resident slot (at most), the work split per XCD into whole rounds.
template <typename T, int D, int NW, int OCC, bool CAUSAL>
int run_dq_persist(BwdParams p, hipStream_t st) {
  auto kern = dq_persist_kernel<T, D, NW, OCC, CAUSAL>;
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
  return check_launch("tattn_bwd_dq");
}

template <typename T, int D, int I>
int dq_persist_entry(const BwdParams& p, bool causal, hipStream_t st) {
  constexpr TileEntry e = DqTable<T, D>::e[I];
  if constexpr (sizeof(T) == 2 && e.pipe == 2)
    return causal ? run_dq_persist<T, D, e.nw, e.occ, true>(p, st) : run_dq_persist<T, D, e.nw, e.occ, false>(p, st);
  else
    return set_error(TATTN_E_CONFIG, "dQ config id %d is not a persistent entry", I);
}

template <typename T, int D, size_t... I>
int dq_persist_dispatch(int id, const BwdParams& p, bool causal, hipStream_t st, std::index_sequence<I...>) {
  int rc = set_error(TATTN_E_CONFIG, "dQ config id %d out of range [0, %d) for D=%d", id, (int)sizeof...(I), D);
  ((id == (int)I ? (rc = dq_persist_entry<T, D, I>(p, causal, st), 0) : 0), ...);
  return rc;
}

template <typename T>
int dq_persist_type(int D, int id, const BwdParams& p, bool causal, hipStream_t st) {
  switch (D) {
    case 16: return dq_persist_dispatch<T, 16>(id, p, causal, st, std::make_index_sequence<DqTable<T, 16>::n>{});
    case 32: return dq_persist_dispatch<T, 32>(id, p, causal, st, std::make_index_sequence<DqTable<T, 32>::n>{});
    case 64: return dq_persist_dispatch<T, 64>(id, p, causal, st, std::make_index_sequence<DqTable<T, 64>::n>{});
    case 128: return dq_persist_dispatch<T, 128>(id, p, causal, st, std::make_index_sequence<DqTable<T, 128>::n>{});
  }
  return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %d", D);
}

}  // namespace

int launch_dq_persist(const BwdParams& p, int D, int dtype, int config_id, bool causal, hipStream_t st) {
  if (dtype == 0) return dq_persist_type<f16>(D, config_id, p, causal, st);
  if (dtype == 2) return dq_persist_type<bf16>(D, config_id, p, causal, st);
  return set_error(TATTN_E_CONFIG, "persistent dQ entries are 16-bit only");
}

}  // namespace tattn
