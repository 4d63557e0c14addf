/*
 * tattn: fused attention (FlashAttention-2 style) for AMD Instinct MI355X (gfx950).
 *
 * C ABI of libtattn_hip.so. Every entry point enqueues hand-written HIP kernels on the
 * caller's stream and returns immediately: no host synchronisation, no device allocation.
 * The caller owns every buffer (outputs and the float32 M / delta workspaces).
 *
 * Layouts. q, k, v, o, do, dq, dk, dv are [Z, H, N, D] tensors of one element type
 * (TATTN_F16, TATTN_BF16 or TATTN_F32). Strides are in ELEMENTS, four per tensor, ordered
 * (z, h, n, d). The d stride must be 1, rows must be 16-byte aligned. M and delta are
 * float32 [Z, H, N], contiguous. Head dims: 16, 32, 64, 128.
 *
 * Numerics (the reference's rounding points are kept): scores are scaled by
 * sm_scale * log2(e) and exponentiated in base 2 with float32 softmax state; P and dS are
 * rounded to the element type only as MFMA operands; M = max + log2(sum) per query row.
 *
 * Return value: 0 on success, a TATTN_E* code otherwise; tattn_last_error() then gives a
 * per-thread message.
 */
#ifndef TATTN_H
#define TATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TATTN_ABI_VERSION 2

/* TATTN_BF16 has no counterpart in the reference, which accepts fp16 and fp32 only
 * (src/tattn/api.py:55-56); it runs the fp16 kernels with bf16 MFMAs and bf16 rounding points. */
enum tattn_dtype { TATTN_F16 = 0, TATTN_F32 = 1, TATTN_BF16 = 2 };
enum tattn_kernel { TATTN_K_FWD = 0, TATTN_K_BWD_DKDV = 1, TATTN_K_BWD_DQ = 2 };
enum tattn_status {
  TATTN_OK = 0,
  TATTN_E_ARG = 1,      /* bad shape, dtype, head dim, stride or null pointer */
  TATTN_E_CONFIG = 2,   /* tile config id out of range for this kernel/dim/dtype */
  TATTN_E_LAUNCH = 3,   /* the HIP runtime refused the launch */
  TATTN_E_DEVICE = 4    /* current device is not a gfx950 */
};

/* One entry of the gfx950 tile table. */
typedef struct tattn_config {
  int32_t block_m;      /* query rows per workgroup */
  int32_t block_n;      /* key rows per workgroup (bwd dK/dV) or per inner step */
  int32_t waves;        /* wavefronts (64 lanes) per workgroup */
  int32_t tiles;        /* 32-row MFMA tiles each wave owns */
  int32_t lds_bytes;    /* LDS the workgroup uses */
  int32_t kind;         /* 0 generic kernel, 1 software-pipelined, 2 persistent (falls back to the
                           pipelined kernel of the same tiles where a problem does not fit it),
                           3 dK/dV with paired waves (two waves per 32-key tile, split roles) */
  int32_t ring;         /* persistent forward: K/V tiles in flight (LDS ring depth); else 0 */
} tattn_config;

/* ABI version of the loaded library; equals TATTN_ABI_VERSION of this header. */
int tattn_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* tattn_last_error(void);

/* 1 if the current HIP device is gfx950 and the kernels can run on it, else 0. */
int tattn_device_supported(void);

/*
 * Forward: o = softmax(q k^T * sm_scale [causal mask]) v, m = per-row base-2 log-sum-exp.
 * Replaces `_forward` + `_fwd_kernel` of the reference
 * (src/tattn/api.py:78-99, src/tattn/kernels.py:57-148). Arbitrary z/h/n strides per tensor
 * (api.py:95-96); m is [Z,H,N] float32 contiguous (api.py:88), or NULL when no backward will
 * follow: the log-sum-exp is then not stored (the reference always stores it, api.py:88, 161).
 * config_id = -1 picks from the table by (D, dtype, causal, N); otherwise an index into
 * the TATTN_K_FWD table (the reference's `config=` override, api.py:69-75).
 */
int tattn_fwd(const void* q, const void* k, const void* v, void* o, float* m,
              const int64_t q_strides[4], const int64_t k_strides[4],
              const int64_t v_strides[4], const int64_t o_strides[4],
              int64_t Z, int64_t H, int64_t N, int64_t D, int dtype, int causal,
              float sm_scale, int config_id, void* stream);

/*
 * delta[z,h,i] = sum_d o[z,h,i,d] * do[z,h,i,d] in float32.
 * Replaces `_bwd_preprocess` (src/tattn/kernels.py:324-337, launched at api.py:122).
 * o and do share `strides` (the reference makes them contiguous, api.py:111).
 */
int tattn_bwd_preprocess(const void* o, const void* dout, float* delta, const int64_t strides[4],
                         int64_t Z, int64_t H, int64_t N, int64_t D, int dtype, void* stream);

/*
 * dK, dV for every key block, looping over query blocks; no atomics.
 * Replaces `_bwd_dkdv_kernel` (src/tattn/kernels.py:151-239, launched at api.py:124-142).
 * q, k, v, do, dk, dv share one layout `strides` (kernels.py:180-181, api.py:111-114).
 */
int tattn_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout,
                   void* dk, void* dv, const float* m, const float* delta,
                   const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
                   int dtype, int causal, float sm_scale, int config_id, void* stream);

/*
 * dQ for every query block, looping over key blocks; no atomics.
 * Replaces `_bwd_dq_kernel` (src/tattn/kernels.py:242-321, launched at api.py:143-145).
 */
int tattn_bwd_dq(const void* q, const void* k, const void* v, const void* dout, void* dq,
                 const float* m, const float* delta, const int64_t strides[4], int64_t Z,
                 int64_t H, int64_t N, int64_t D, int dtype, int causal, float sm_scale,
                 int config_id, void* stream);

/*
 * The whole backward in stream order: preprocess, dK/dV, dQ (src/tattn/api.py:102-146).
 * delta is caller-owned float32 [Z,H,N] scratch. config_id applies to both dK/dV and dQ
 * (as the reference's `config=` does, api.py:124-145); -1 picks per kernel.
 */
int tattn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
              void* dq, void* dk, void* dv, const float* m, float* delta,
              const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
              int dtype, int causal, float sm_scale, int config_id, void* stream);

/*
 * tattn_bwd without the delta argument and without any allocation: delta lives in a static
 * device array of the library (16 MiB per GPU, held until the process ends), so the caller
 * passes only inputs and outputs. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Limit: Z*H*N <= 4,194,304 query rows, else TATTN_E_ARG and nothing
 * is enqueued. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, two threads) race on it and must be serialised by the caller.
 */
int tattn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const void* dout,
                      void* dq, void* dk, void* dv, const float* m,
                      const int64_t strides[4], int64_t Z, int64_t H, int64_t N, int64_t D,
                      int dtype, int causal, float sm_scale, int config_id, void* stream);

/*
 * Tile table introspection (the gfx950 replacement of the reference's autotune config lists,
 * src/tattn/kernels.py:21-54): number of entries for (kernel, D, dtype), the entry itself, and
 * the entry the library picks for a problem (the reference keys its autotuner on
 * (N bucket, head dim, causal), kernels.py:57-61 and api.py:59-62). tattn_pick_config reports
 * the pick for a batch x heads count that is a multiple of 8; the entry points also take the
 * batch x heads count into account (the persistent forward needs whole slices per XCD).
 */
int tattn_num_configs(int kernel, int64_t D, int dtype);
int tattn_config_desc(int kernel, int64_t D, int dtype, int config_id, tattn_config* out);
int tattn_pick_config(int kernel, int64_t D, int dtype, int causal, int64_t N);

#ifdef __cplusplus
}
#endif

#endif /* TATTN_H */
