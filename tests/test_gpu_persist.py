"""The persistent forward entries of the tile table (kind 2) on shapes that meet their
preconditions (Z*H a multiple of 8, N a multiple of the block and of 128, an even number of
causal blocks per slice): O and M against float32 attention and against the pipelined kernel of
the same tiles, from one work item per workgroup to several (the benchmark's 32 x 16 heads of
512 tokens), fp16 and bf16, both masks. Shapes that do not fit run the pipelined kernel and are
covered by tests/test_gpu_configs.py."""

import math

import pytest
import torch

from helpers import F16_MAX, check_max
from oracle.reference import naive_attention

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SHAPES = [(1, 8, 512), (2, 8, 1024), (4, 16, 2048), (1, 8, 4096), (32, 16, 512), (2, 4, 384), (8, 16, 256)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tattn import hip_available

    assert hip_available(DEV), "libtattn_hip.so did not load or the device is not a gfx950"


def _persistent_entries():
    """(head dim, persistent entry, pipelined entry of the same tiles) for every kind-2 forward entry."""
    if not torch.cuda.is_available():
        return []
    from tattn import _lib

    out = []
    for d in (16, 32, 64, 128):
        descs = [_lib.config_desc(_lib.K_FWD, d, _lib.F16, c) for c in range(_lib.num_configs(_lib.K_FWD, d, _lib.F16))]
        for c, desc in enumerate(descs):
            if desc["kind"] == 2:
                twin = next(t for t, o in enumerate(descs)
                            if o["kind"] == 1 and (o["waves"], o["tiles"]) == (desc["waves"], desc["tiles"]))
                out.append((d, c, twin))
    return out


def _reference(q, k, v, causal, scale):
    z, h, n, _ = q.shape
    per = max(1, (1 << 27) // (z * n * n))
    o, m = [], []
    for i in range(0, h, per):
        qs, ks, vs = (t[:, i:i + per].float() for t in (q, k, v))
        s = qs @ ks.transpose(-1, -2) * scale
        if causal:
            s = s.masked_fill(torch.ones(n, n, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
        m.append(torch.logsumexp(s, -1) / math.log(2.0))
        o.append(torch.softmax(s, -1) @ vs)
    return torch.cat(o, 1), torch.cat(m, 1)


@pytest.mark.parametrize("entry", _persistent_entries(), ids=lambda e: f"d{e[0]}cfg{e[1]}")
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_persistent_forward(entry, shape, causal, dtype):
    from tattn.api import _forward

    d, cid, twin = entry
    b, h, n = shape
    scale = d ** -0.5
    print(f"persistent fwd: d={d} cfg{cid} shape={shape} causal={causal} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(n * 7 + b + int(causal))
    q, k, v = (torch.randn(b, h, n, d, device=DEV, dtype=dtype, generator=g) for _ in range(3))
    o, m = _forward(q, k, v, causal, scale, config=cid)
    o2, m2 = _forward(q, k, v, causal, scale, config=twin)
    torch.cuda.synchronize()
    want_o, want_m = _reference(q, k, v, causal, scale)
    bound = F16_MAX if dtype == torch.float16 else 8 * F16_MAX
    check_max(f"d{d} cfg{cid} {shape} causal={causal} {dtype} o", o, want_o, bound)
    check_max(f"d{d} cfg{cid} {shape} causal={causal} {dtype} M", m, want_m, 1e-3 if dtype == torch.float16 else 8e-3)
    # Same math as the pipelined kernel: equal up to the rounding of the softmax's lazy max moves.
    torch.testing.assert_close(o.float(), o2.float(), atol=2 ** -10, rtol=2 ** -9)
    torch.testing.assert_close(m, m2, atol=1e-4, rtol=0)


def test_persistent_inference_path_and_repeat():
    """M = NULL (inference) gives the same O; two calls in a row give the same bits."""
    from tattn.api import _forward

    for d in (64, 128):
        cid = next(c for dd, c, _ in _persistent_entries() if dd == d)
        q, k, v = (torch.randn(4, 16, 1024, d, device=DEV, dtype=torch.float16) for _ in range(3))
        for causal in (False, True):
            o1, _ = _forward(q, k, v, causal, d ** -0.5, config=cid)
            o2, m2 = _forward(q, k, v, causal, d ** -0.5, config=cid, save_lse=False)
            o3, _ = _forward(q, k, v, causal, d ** -0.5, config=cid)
            assert m2 is None and torch.equal(o1, o2) and torch.equal(o1, o3)


def _bwd_entries(kernel):
    if not torch.cuda.is_available():
        return []
    from tattn import _lib

    k = {"dkdv": _lib.K_BWD_DKDV, "dq": _lib.K_BWD_DQ}[kernel]
    descs = [_lib.config_desc(k, 64, _lib.F16, c) for c in range(_lib.num_configs(k, 64, _lib.F16))]
    out = []
    for d in descs:
        if d["kind"] == 2:
            twin = next(t for t in descs if t["kind"] == 1 and t["waves"] == d["waves"])
            out.append((kernel, d["id"], twin["id"]))
    return out


BWD_SHAPES = [(1, 8, 512), (32, 16, 512), (16, 16, 1024), (2, 8, 2048), (8, 16, 256), (2, 4, 384)]


@pytest.mark.parametrize("entry", _bwd_entries("dkdv") + _bwd_entries("dq"), ids=lambda e: f"{e[0]}{e[1]}")
@pytest.mark.parametrize("shape", BWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_persistent_backward_matches_pipelined(entry, shape, causal, dtype):
    """The persistent dK/dV and dQ kernels give the bits of the pipelined kernel with the same
    waves (same summation order and rounding points), from one block per workgroup to several,
    both masks; shapes that do not fit them run the pipelined kernel (same bits trivially)."""
    from tattn.api import _backward, _forward

    kernel, pid, twin = entry
    b, h, n = shape
    print(f"persistent bwd: {kernel}{pid} shape={shape} causal={causal} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(n * 3 + b + int(causal))
    q, k, v, do = (torch.randn(b, h, n, 64, device=DEV, dtype=dtype, generator=g) for _ in range(4))
    o, m = _forward(q, k, v, causal, 0.125)
    got = _backward(q, k, v, o, m, do, causal, 0.125, config={kernel: pid})
    want = _backward(q, k, v, o, m, do, causal, 0.125, config={kernel: twin})
    torch.cuda.synchronize()
    for name, a, w in zip(("dq", "dk", "dv"), got, want):
        assert torch.equal(a, w), f"{name} differs from the pipelined kernel"


@pytest.mark.parametrize("causal", [False, True])
def test_persistent_backward_against_float32(causal):
    """The library's picks at the benchmark shape (16 x 16 heads of 1,024 tokens) against float32
    autograd: the flat envelope non-causal; causal gradients bounded by the reference backward
    algorithm's own error on the same inputs (q, k, v, dO, the forward's O and M) plus the margin
    (check_grads_pinned)."""
    from helpers import check_grads_pinned
    from oracle.reference import rounded_backward
    from tattn import attention
    from tattn.api import _forward

    g = torch.Generator(device=DEV).manual_seed(1024 + int(causal))
    q, k, v, do = (torch.randn(16, 16, 1024, 64, device=DEV, dtype=torch.float16, generator=g) for _ in range(4))
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    attention(qg, kg, vg, causal=causal).backward(do)
    for i in range(0, 16, 4):
        qs, ks, vs = (t[i:i + 4].float().requires_grad_() for t in (q, k, v))
        naive_attention(qs, ks, vs, causal=causal).backward(do[i:i + 4].float())
        got = (qg.grad[i:i + 4], kg.grad[i:i + 4], vg.grad[i:i + 4])
        want = (qs.grad, ks.grad, vs.grad)
        if causal:
            qc, kc, vc, dc = (t[i:i + 4] for t in (q, k, v, do))
            o, m = _forward(qc, kc, vc, True, 0.125)
            emulated = rounded_backward(qc, kc, vc, dc, causal=True, o=o, lse=m)
            check_grads_pinned(f"batch {i}: causal", got, want, emulated, torch.float16,
                               rounded_backward(qc, kc, vc, dc, causal=True))
        else:
            for name, g_, w in zip(("dq", "dk", "dv"), got, want):
                check_max(f"batch {i}: {name} causal={causal}", g_, w, F16_MAX)
