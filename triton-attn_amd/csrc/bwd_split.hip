// Paired-wave backward kernels (dkdv_split_kernel, dq_split_kernel: bwd_split.h) in a translation
// unit of their own: the library builds them with LLVM's iterative ILP scheduler
// (-amdgpu-sched-strategy=iterative-ilp), which made them 6-12% faster at head dim 128 (the
// only head dim that picks them) with the same results bit for bit.
// Part of the backward (the reference's src/tattn/kernels.py:151-321).
#include <type_traits>

#include "bwd_split.h"
#include "launch.h"

namespace tattn {

namespace {

template <typename T, int D>
int run_split(const BwdParams& p, bool dkdv, bool causal, hipStream_t st) {
  const int64_t blocks = (int64_t)p.n_blocks * p.Z * p.H;
  const dim3 grid((unsigned)blocks), block(512);
  if (dkdv) {
    if (causal)
      dkdv_split_kernel<T, D, true><<<grid, block, 0, st>>>(p);
    else
      dkdv_split_kernel<T, D, false><<<grid, block, 0, st>>>(p);
    return check_launch("tattn_bwd_dkdv");
  }
  if (causal)
    dq_split_kernel<T, D, true><<<grid, block, 0, st>>>(p);
  else
    dq_split_kernel<T, D, false><<<grid, block, 0, st>>>(p);
  return check_launch("tattn_bwd_dq");
}

// The head dims whose tables hold a paired-wave entry (kind 3).
template <template <typename, int> class Table, typename T, int D>
constexpr bool has_split() {
  for (int i = 0; i < Table<T, D>::n; ++i)
    if (Table<T, D>::e[i].pipe == 3) return true;
  return false;
}

template <typename T, int D>
int split_d(const BwdParams& p, bool dkdv, bool causal, hipStream_t st) {
  if constexpr (has_split<DkdvTable, T, D>() || has_split<DqTable, T, D>())
    return run_split<T, D>(p, dkdv, causal, st);
  else
    return set_error(TATTN_E_CONFIG, "no paired-wave entry at head dim %d", D);
}

template <typename T>
int split_type(int D, const BwdParams& p, bool dkdv, bool causal, hipStream_t st) {
  switch (D) {
    case 16: return split_d<T, 16>(p, dkdv, causal, st);
    case 32: return split_d<T, 32>(p, dkdv, causal, st);
    case 64: return split_d<T, 64>(p, dkdv, causal, st);
    case 128: return split_d<T, 128>(p, dkdv, causal, st);
  }
  return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %d", D);
}

}  // namespace

int launch_split(const BwdParams& p, int D, int dtype, bool dkdv, bool causal, hipStream_t st) {
  if (dtype == 0) return split_type<f16>(D, p, dkdv, causal, st);
  if (dtype == 2) return split_type<bf16>(D, p, dkdv, causal, st);
  return set_error(TATTN_E_CONFIG, "paired-wave entries are 16-bit only");
}

}  // namespace tattn
