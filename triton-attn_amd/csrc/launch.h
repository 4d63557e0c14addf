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
int dkdv_lds_bytes(int D, int dtype, const TileEntry& e);
int dq_lds_bytes(int D, int dtype, const TileEntry& e);

}  // namespace tattn
