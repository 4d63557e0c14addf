"""`tattn_bwd_noalloc` (the backward with delta in the library's static device workspace, no
allocation) against `tattn_bwd` with a caller-provided delta: the same kernels, so the same bits.
Two calls in a row, the second on a smaller problem, so the second runs on a workspace that
still holds the first call's values."""

import ctypes

import pytest
import torch

from helpers import rand

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tattn import hip_available

    assert hip_available(DEV), "libtattn_hip.so did not load or the device is not a gfx950"


def _with_delta(lib, q, k, v, o, do, m, causal, scale, code):
    from tattn import _lib

    z, h, n, d = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    delta = torch.empty((z, h, n), device=DEV, dtype=torch.float32)
    rc = lib.tattn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), dq.data_ptr(),
                       dk.data_ptr(), dv.data_ptr(), m.data_ptr(), delta.data_ptr(), _lib.strides4(q), z, h, n,
                       d, code, int(causal), scale, -1, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "tattn_bwd")
    return dq, dk, dv


def _no_alloc(lib, q, k, v, o, do, m, causal, scale, code):
    from tattn import _lib

    z, h, n, d = q.shape
    dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
    rc = lib.tattn_bwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                               dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), m.data_ptr(), _lib.strides4(q), z, h,
                               n, d, code, int(causal), scale, -1, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "tattn_bwd_noalloc")
    return dq, dk, dv


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_no_alloc_backward_gives_the_bits_of_tattn_bwd(dtype, causal, d):
    """Every call smaller than the one before. The 16-bit picks compute delta inside dQ and store
    it in the workspace: the persistent dQ at (1, 8, 512, 64), the paired-wave dQ at head dim 128."""
    from tattn import _lib
    from tattn.api import _DTYPES, _forward

    lib = _lib.load()
    code = _DTYPES[dtype]
    for i, shape in enumerate([(1, 8, 512, d), (2, 3, 333, d), (1, 2, 77, d)]):
        print(f"noalloc: dtype={dtype} causal={causal} shape={shape}", flush=True)
        q, k, v, do = (rand(shape, dtype, 900 + 10 * i + s, DEV) for s in range(4))
        o, m = _forward(q, k, v, causal, 0.125)
        want = _with_delta(lib, q, k, v, o, do, m, causal, 0.125, code)
        got = _no_alloc(lib, q, k, v, o, do, m, causal, 0.125, code)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.equal(a, b), f"{name} differs (call {i + 1}, shape {shape})"


def test_no_alloc_backward_rejects_problems_past_its_workspace():
    from tattn import _lib

    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(1 << 20, 1 << 16, 64, 1)
    # 1 x 65 heads x 65,536 rows = 4,259,840 > 4,194,304: refused before any launch.
    rc = lib.tattn_bwd_noalloc(16, 16, 16, 16, 16, 16, 16, 16, 16, st, 1, 65, 1 << 16, 64, _lib.F16, 0, 0.125,
                               -1, torch.cuda.current_stream().cuda_stream)
    assert rc == 1 and "exceeds the static workspace" in _lib.last_error()
