// C ABI of libtattn_hip.so (declared in include/tattn.h): argument checks, error strings,
// device check, tile-table introspection and the entry points that enqueue the kernels.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/tattn.h"
#include "launch.h"
#include "tiles.h"

namespace tattn {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(TATTN_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TATTN_OK;
}

namespace {

constexpr int kMaxDevices = 64;
std::once_flag g_dev_once[kMaxDevices];
int g_dev_ok[kMaxDevices];

int device_check() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(TATTN_E_DEVICE, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(TATTN_E_DEVICE, "device index %d out of range", dev);
  std::call_once(g_dev_once[dev], [dev] {
    hipDeviceProp_t prop;
    g_dev_ok[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                            strncmp(prop.gcnArchName, "gfx950", 6) == 0
                        ? 1
                        : 0;
  });
  if (!g_dev_ok[dev]) return set_error(TATTN_E_DEVICE, "device %d is not a gfx950 (MI355X)", dev);
  return TATTN_OK;
}

template <template <typename, int> class Table, typename T>
int table_size(int64_t D) {
  switch (D) {
    case 16: return Table<T, 16>::n;
    case 32: return Table<T, 32>::n;
    case 64: return Table<T, 64>::n;
    case 128: return Table<T, 128>::n;
  }
  return -1;
}

template <template <typename, int> class Table, typename T>
const TileEntry* table_entry(int64_t D, int id) {
  const TileEntry* e = nullptr;
  int n = 0;
  switch (D) {
    case 16: e = Table<T, 16>::e; n = Table<T, 16>::n; break;
    case 32: e = Table<T, 32>::e; n = Table<T, 32>::n; break;
    case 64: e = Table<T, 64>::e; n = Table<T, 64>::n; break;
    case 128: e = Table<T, 128>::e; n = Table<T, 128>::n; break;
    default: return nullptr;
  }
  return id >= 0 && id < n ? e + id : nullptr;
}

// fp16 and bf16 share the 16-bit tables (tiles.h).
int num_configs(int kernel, int64_t D, int dtype) {
  const bool h = dtype != TATTN_F32;
  switch (kernel) {
    case TATTN_K_FWD: return h ? table_size<FwdTable, _Float16>(D) : table_size<FwdTable, float>(D);
    case TATTN_K_BWD_DKDV: return h ? table_size<DkdvTable, _Float16>(D) : table_size<DkdvTable, float>(D);
    case TATTN_K_BWD_DQ: return h ? table_size<DqTable, _Float16>(D) : table_size<DqTable, float>(D);
  }
  return -1;
}

const TileEntry* config_entry(int kernel, int64_t D, int dtype, int id) {
  const bool h = dtype != TATTN_F32;
  switch (kernel) {
    case TATTN_K_FWD: return h ? table_entry<FwdTable, _Float16>(D, id) : table_entry<FwdTable, float>(D, id);
    case TATTN_K_BWD_DKDV:
      return h ? table_entry<DkdvTable, _Float16>(D, id) : table_entry<DkdvTable, float>(D, id);
    case TATTN_K_BWD_DQ: return h ? table_entry<DqTable, _Float16>(D, id) : table_entry<DqTable, float>(D, id);
  }
  return nullptr;
}

// Table pick for a problem (index into the kernel's table), keyed like the reference's autotuner
// on (sequence length, head dim, causal) (src/tattn/kernels.py:57-61), but static: the choices
// below are the fastest entries measured on an MI355X at 16,384 tokens per batch, H=16. Entry 0
// of each table is its general-purpose tile.
// ZH = Z * H: the persistent forward entries are picked where they run the problem themselves.
int pick_config(int kernel, int64_t D, int dtype, int causal, int64_t N, int64_t ZH) {
  if (dtype == TATTN_F32) return 0;  // fp16 and bf16 share the picks
  switch (kernel) {
    case TATTN_K_FWD:  // persistent where it fits (D=64, 128); else 128-row blocks short, 256 / 512 long
      if (D == 64) {
        // Persistent, ring of 4: 4 x 2 non-causal, and causal from N = 2048 (from 4096 one pair of
        // blocks per workgroup, time-sliced priority); 4 x 1 causal below. Fastest at every
        // benchmark length (cold-cache medians, 16,384 tokens x 16 heads; causal N = 2048: 4 x 2
        // 3% faster than 4 x 1 since both store O as whole rows, N = 1024: 4 x 1 2% faster).
        const int pid = causal && N < 2048 ? 5 : 7;
        if (fwd_persist_fits(FwdTable<_Float16, 64>::e[pid], ZH, N, causal != 0)) return pid;
      }
      if (D == 128) {
        // Persistent, ring of 4: 8 x 1 from N = 2048 (causal: 4096), 4 x 1 below; else 4 x 1
        // pipelined.
        const int pid = N >= (causal ? 4096 : 2048) ? 3 : 2;
        if (fwd_persist_fits(FwdTable<_Float16, 128>::e[pid], ZH, N, causal != 0)) return pid;
        return 0;
      }
      if (causal) return N >= 4096 ? 0 : 1;
      if (D == 64) return N >= 4096 ? 3 : N >= 1024 ? 0 : 1;
      return D == 16 && N < 2048 ? 1 : 0;
    case TATTN_K_BWD_DKDV:  // causal N < 4096: persistent 4 waves where it fits; else pipelined, 8 waves
                            // (256 keys), causal N < 2048: 4 waves (128 keys). Picked on the whole
                            // forward + backward: there the persistent entries lose non-causal (the
                            // dQ pass leaves this kernel's inputs in the caches).
      if (D == 128) return 2;  // paired waves: two per SIMD, where one wave per tile needs all 512 registers
      if (D != 64) return 0;
      if (causal && N < 4096 && bwd_persist_fits(DkdvTable<_Float16, 64>::e[5], ZH, N, true)) return 5;
      if (!causal) return 1;
      return N >= 2048 ? 1 : 0;
    case TATTN_K_BWD_DQ:  // persistent 4 waves where it fits; else 4 waves (8 for non-causal 2048 <= N < 8192)
      if (D == 128) return 2;  // paired waves, as dK/dV
      if (D != 64) return 0;
      if (bwd_persist_fits(DqTable<_Float16, 64>::e[5], ZH, N, causal != 0)) return 5;
      return !causal && N >= 2048 && N < 8192 ? 1 : 0;
  }
  return 0;
}

// Workspace of tattn_bwd_noalloc: the backward's delta (float32, one value per query row) in a
// fixed device array, so that entry point needs neither an allocation nor a caller-provided
// buffer. Every GPU holds its own copy (16 MiB) until the process ends. Host code must never
// pass `scratch` itself to a kernel or copy: that name is a host-side stand-in, not a device
// address. The device address is looked up once per device with hipGetSymbolAddress (with that
// device current) and kept in g_scratch_ptr.
constexpr int64_t kScratchRows = int64_t(1) << 22;  // Z * H * N <= 4,194,304
static __device__ __align__(256) float scratch[kScratchRows];

std::once_flag g_scratch_once[kMaxDevices];
float* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of this device's scratch array (the current device; device_check has run).
int scratch_for_current_device(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(TATTN_E_DEVICE, "hipGetDevice failed: %s", hipGetErrorString(e));
  std::call_once(g_scratch_once[dev], [dev] {
    void* ptr = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? static_cast<float*>(ptr) : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
    return set_error(TATTN_E_DEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(g_scratch_err[dev]));
  *out = g_scratch_ptr[dev];
  return TATTN_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_tensor(const char* name, const void* ptr, const int64_t* st, int sz) {
  if (!ptr) return set_error(TATTN_E_ARG, "%s is a null pointer", name);
  if (!st) return set_error(TATTN_E_ARG, "%s strides are null", name);
  if (st[3] != 1) return set_error(TATTN_E_ARG, "%s: d stride must be 1, got %lld", name, (long long)st[3]);
  const int64_t vec = 16 / sz;
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || st[i] % vec != 0)
      return set_error(TATTN_E_ARG, "%s: stride %d (%lld) must be a non-negative multiple of %lld elements",
                       name, i, (long long)st[i], (long long)vec);
  if (!aligned16(ptr)) return set_error(TATTN_E_ARG, "%s must be 16-byte aligned", name);
  return TATTN_OK;
}

int check_shape(int64_t Z, int64_t H, int64_t N, int64_t D, int dtype) {
  if (dtype != TATTN_F16 && dtype != TATTN_F32 && dtype != TATTN_BF16)
    return set_error(TATTN_E_ARG, "dtype must be TATTN_F16, TATTN_BF16 or TATTN_F32, got %d", dtype);
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return set_error(TATTN_E_ARG, "head dim must be 16, 32, 64 or 128, got %lld", (long long)D);
  if (Z < 1 || H < 1 || N < 1) return set_error(TATTN_E_ARG, "Z, H, N must be positive (%lld, %lld, %lld)",
                                                (long long)Z, (long long)H, (long long)N);
  if (N > (1 << 30) || Z * H > (1 << 30)) return set_error(TATTN_E_ARG, "problem too large");
  return TATTN_OK;
}

int resolve(int kernel, int64_t D, int dtype, int causal, int64_t N, int64_t ZH, int id, int* out) {
  const int n = num_configs(kernel, D, dtype);
  if (id < 0) id = pick_config(kernel, D, dtype, causal, N, ZH);
  if (id >= n) return set_error(TATTN_E_CONFIG, "config id %d out of range [0, %d)", id, n);
  *out = id;
  return TATTN_OK;
}

}  // namespace
}  // namespace tattn

using namespace tattn;

extern "C" {

int tattn_abi_version(void) { return TATTN_ABI_VERSION; }

const char* tattn_last_error(void) { return g_err; }

int tattn_device_supported(void) { return device_check() == TATTN_OK ? 1 : 0; }

int tattn_num_configs(int kernel, int64_t D, int dtype) { return num_configs(kernel, D, dtype); }

int tattn_config_desc(int kernel, int64_t D, int dtype, int config_id, tattn_config* out) {
  if (!out) return set_error(TATTN_E_ARG, "out is a null pointer");
  const TileEntry* e = config_entry(kernel, D, dtype, config_id);
  if (!e) return set_error(TATTN_E_CONFIG, "no config %d for kernel %d, D=%lld, dtype %d", config_id, kernel,
                           (long long)D, dtype);
  const int rows = tile_rows(*e);
  out->waves = e->nw;
  out->tiles = e->tiles;
  out->kind = e->pipe;
  out->ring = e->pipe == 2 ? e->ring : 0;
  if (kernel == TATTN_K_BWD_DKDV) {
    out->block_n = rows;
    out->block_m = e->other;
    out->lds_bytes = dkdv_lds_bytes((int)D, dtype, *e);
  } else {
    out->block_m = rows;
    out->block_n = e->other;
    out->lds_bytes = kernel == TATTN_K_FWD ? fwd_lds_bytes((int)D, dtype, *e) : dq_lds_bytes((int)D, dtype, *e);
  }
  return TATTN_OK;
}

int tattn_pick_config(int kernel, int64_t D, int dtype, int causal, int64_t N) {
  if (num_configs(kernel, D, dtype) < 0) return set_error(TATTN_E_ARG, "no table for kernel %d, D=%lld", kernel, (long long)D), -1;
  return pick_config(kernel, D, dtype, causal, N, 8);  // any Z * H that is a multiple of 8
}

int tattn_fwd(const void* q, const void* k, const void* v, void* o, float* m, const int64_t q_strides[4],
              const int64_t k_strides[4], const int64_t v_strides[4], const int64_t o_strides[4], int64_t Z,
              int64_t H, int64_t N, int64_t D, int dtype, int causal, float sm_scale, int config_id,
              void* stream) {
  int rc;
  if ((rc = check_shape(Z, H, N, D, dtype))) return rc;
  const int sz = dtype == TATTN_F32 ? 4 : 2;
  if ((rc = check_tensor("q", q, q_strides, sz)) || (rc = check_tensor("k", k, k_strides, sz)) ||
      (rc = check_tensor("v", v, v_strides, sz)) || (rc = check_tensor("o", o, o_strides, sz)))
    return rc;
  // m may be null: the log-sum-exp is then not stored (no backward will follow).
  int id;
  if ((rc = resolve(TATTN_K_FWD, D, dtype, causal, N, Z * H, config_id, &id))) return rc;
  if ((rc = device_check())) return rc;
  FwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = o; p.m = m;
  for (int i = 0; i < 3; ++i) {
    p.sq[i] = q_strides[i]; p.sk[i] = k_strides[i]; p.sv[i] = v_strides[i]; p.so[i] = o_strides[i];
  }
  p.Z = (int32_t)Z; p.H = (int32_t)H; p.N = (int32_t)N;
  p.c = sm_scale * kLog2e;
  return launch_fwd(p, (int)D, dtype, causal != 0, id, (hipStream_t)stream);
}

static int bwd_common(BwdParams& p, const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
                      int dtype, float sm_scale) {
  int rc;
  if ((rc = check_shape(Z, H, N, D, dtype))) return rc;
  if (!strides) return set_error(TATTN_E_ARG, "strides are null");
  p.s[0] = strides[0]; p.s[1] = strides[1]; p.s[2] = strides[2];
  p.Z = (int32_t)Z; p.H = (int32_t)H; p.N = (int32_t)N;
  p.c = sm_scale * kLog2e;
  p.scale = sm_scale;
  return TATTN_OK;
}

int tattn_bwd_preprocess(const void* o, const void* dout, float* delta, const int64_t strides[4], int64_t Z,
                         int64_t H, int64_t N, int64_t D, int dtype, void* stream) {
  BwdParams p{};
  int rc;
  if ((rc = bwd_common(p, strides, Z, H, N, D, dtype, 1.0f))) return rc;
  const int sz = dtype == TATTN_F32 ? 4 : 2;
  if ((rc = check_tensor("o", o, strides, sz)) || (rc = check_tensor("do", dout, strides, sz))) return rc;
  if (!delta) return set_error(TATTN_E_ARG, "delta is a null pointer");
  if ((rc = device_check())) return rc;
  p.o = o; p.dout = dout; p.delta = delta;
  return launch_bwd_preprocess(p, (int)D, dtype, (hipStream_t)stream);
}

int tattn_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout, void* dk, void* dv,
                   const float* m, const float* delta, const int64_t strides[4], int64_t Z, int64_t H, int64_t N,
                   int64_t D, int dtype, int causal, float sm_scale, int config_id, void* stream) {
  BwdParams p{};
  int rc;
  if ((rc = bwd_common(p, strides, Z, H, N, D, dtype, sm_scale))) return rc;
  const int sz = dtype == TATTN_F32 ? 4 : 2;
  if ((rc = check_tensor("q", q, strides, sz)) || (rc = check_tensor("k", k, strides, sz)) ||
      (rc = check_tensor("v", v, strides, sz)) || (rc = check_tensor("do", dout, strides, sz)) ||
      (rc = check_tensor("dk", dk, strides, sz)) || (rc = check_tensor("dv", dv, strides, sz)))
    return rc;
  if (!m || !delta) return set_error(TATTN_E_ARG, "m and delta must not be null");
  int id;
  if ((rc = resolve(TATTN_K_BWD_DKDV, D, dtype, causal, N, Z * H, config_id, &id))) return rc;
  if ((rc = device_check())) return rc;
  p.q = q; p.k = k; p.v = v; p.dout = dout; p.dk = dk; p.dv = dv; p.m = m; p.delta = const_cast<float*>(delta);
  return launch_bwd_dkdv(p, (int)D, dtype, causal != 0, id, (hipStream_t)stream);
}

// dQ; with o_fused (O, in the shared layout) the kernel computes delta = rowsum(dO * O) itself, in
// the preprocess's order, and stores it into `delta` for the dK/dV kernel that follows.
static int bwd_dq_call(const void* q, const void* k, const void* v, const void* dout, void* dq, const float* m,
                       const float* delta, const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
                       int dtype, int causal, float sm_scale, int config_id, void* stream, const void* o_fused) {
  BwdParams p{};
  int rc;
  if ((rc = bwd_common(p, strides, Z, H, N, D, dtype, sm_scale))) return rc;
  const int sz = dtype == TATTN_F32 ? 4 : 2;
  if ((rc = check_tensor("q", q, strides, sz)) || (rc = check_tensor("k", k, strides, sz)) ||
      (rc = check_tensor("v", v, strides, sz)) || (rc = check_tensor("do", dout, strides, sz)) ||
      (rc = check_tensor("dq", dq, strides, sz)))
    return rc;
  if (!m || !delta) return set_error(TATTN_E_ARG, "m and delta must not be null");
  int id;
  if ((rc = resolve(TATTN_K_BWD_DQ, D, dtype, causal, N, Z * H, config_id, &id))) return rc;
  if ((rc = device_check())) return rc;
  p.q = q; p.k = k; p.v = v; p.dout = dout; p.dq = dq; p.m = m; p.delta = const_cast<float*>(delta);
  if (o_fused) {
    p.o = o_fused;
    p.fuse_delta = 1;
  }
  return launch_bwd_dq(p, (int)D, dtype, causal != 0, id, (hipStream_t)stream);
}

int tattn_bwd_dq(const void* q, const void* k, const void* v, const void* dout, void* dq, const float* m,
                 const float* delta, const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
                 int dtype, int causal, float sm_scale, int config_id, void* stream) {
  return bwd_dq_call(q, k, v, dout, dq, m, delta, strides, Z, H, N, D, dtype, causal, sm_scale, config_id, stream,
                     nullptr);
}

// Checks every argument of the whole backward and resolves both kernels' table entries before
// anything is enqueued, so a nonzero return from tattn_bwd means no work was launched.
static int bwd_prepare(BwdParams& p, int* dk_id, int* dq_id, bool* fuse, const void* q, const void* k,
                       const void* v, const void* o, const void* dout, void* dq, void* dk, void* dv, const float* m,
                       float* delta, const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
                       int dtype, int causal, float sm_scale, int config_id) {
  int rc;
  if ((rc = bwd_common(p, strides, Z, H, N, D, dtype, sm_scale))) return rc;
  const int sz = dtype == TATTN_F32 ? 4 : 2;
  if ((rc = check_tensor("q", q, strides, sz)) || (rc = check_tensor("k", k, strides, sz)) ||
      (rc = check_tensor("v", v, strides, sz)) || (rc = check_tensor("o", o, strides, sz)) ||
      (rc = check_tensor("do", dout, strides, sz)) || (rc = check_tensor("dq", dq, strides, sz)) ||
      (rc = check_tensor("dk", dk, strides, sz)) || (rc = check_tensor("dv", dv, strides, sz)))
    return rc;
  if (!m || !delta) return set_error(TATTN_E_ARG, "m and delta must not be null");
  if (config_id >= 0) {
    // One id for both kernels, as the reference's `config=` (api.py:124-145): it must exist in both tables.
    if (config_id >= num_configs(TATTN_K_BWD_DKDV, D, dtype) || config_id >= num_configs(TATTN_K_BWD_DQ, D, dtype))
      return set_error(TATTN_E_CONFIG, "config id %d out of range for the backward tables", config_id);
  }
  if ((rc = resolve(TATTN_K_BWD_DKDV, D, dtype, causal, N, Z * H, config_id, dk_id)) ||
      (rc = resolve(TATTN_K_BWD_DQ, D, dtype, causal, N, Z * H, config_id, dq_id)))
    return rc;
  if ((rc = device_check())) return rc;
  // When dQ runs a pipelined, persistent or paired-wave 16-bit kernel it computes delta itself
  // (same bits as the preprocess) and stores it: dQ, then dK/dV, two launches and no separate
  // pass over dO. Otherwise preprocess, dK/dV, dQ.
  const TileEntry* e = config_entry(TATTN_K_BWD_DQ, D, dtype, *dq_id);
  *fuse = dtype != TATTN_F32 && e && e->pipe >= 1 && bwd_fits32(p, (int)D);
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout; p.dq = dq; p.dk = dk; p.dv = dv; p.m = m; p.delta = delta;
  return TATTN_OK;
}

int tattn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, void* dq, void* dk,
              void* dv, const float* m, float* delta, const int64_t strides[4], int64_t Z, int64_t H, int64_t N,
              int64_t D, int dtype, int causal, float sm_scale, int config_id, void* stream) {
  BwdParams p{};
  int rc, dk_id = -1, dq_id = -1;
  bool fuse = false;
  if ((rc = bwd_prepare(p, &dk_id, &dq_id, &fuse, q, k, v, o, dout, dq, dk, dv, m, delta, strides, Z, H, N, D,
                        dtype, causal, sm_scale, config_id)))
    return rc;
  const hipStream_t st = (hipStream_t)stream;
  if (fuse) {
    BwdParams pq = p;
    pq.fuse_delta = 1;
    if ((rc = launch_bwd_dq(pq, (int)D, dtype, causal != 0, dq_id, st))) return rc;
    return launch_bwd_dkdv(p, (int)D, dtype, causal != 0, dk_id, st);
  }
  if ((rc = launch_bwd_preprocess(p, (int)D, dtype, st))) return rc;
  if ((rc = launch_bwd_dkdv(p, (int)D, dtype, causal != 0, dk_id, st))) return rc;
  return launch_bwd_dq(p, (int)D, dtype, causal != 0, dq_id, st);
}

int tattn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const void* dout, void* dq,
                      void* dk, void* dv, const float* m, const int64_t strides[4], int64_t Z, int64_t H,
                      int64_t N, int64_t D, int dtype, int causal, float sm_scale, int config_id, void* stream) {
  int rc;
  if ((rc = check_shape(Z, H, N, D, dtype))) return rc;
  if (Z * H * N > kScratchRows)
    return set_error(TATTN_E_ARG,
                     "tattn_bwd_noalloc: Z*H*N = %lld query rows exceeds the static workspace of %lld rows; "
                     "use tattn_bwd with a caller-provided delta",
                     (long long)(Z * H * N), (long long)kScratchRows);
  if ((rc = device_check())) return rc;
  float* delta = nullptr;
  if ((rc = scratch_for_current_device(&delta))) return rc;
  // delta is written in full by the preprocess before dK/dV and dQ read it: nothing to clear.
  return tattn_bwd(q, k, v, o, dout, dq, dk, dv, m, delta, strides, Z, H, N, D, dtype, causal, sm_scale,
                   config_id, stream);
}

}  // extern "C"
