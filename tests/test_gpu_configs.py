"""Every gfx950 tile-table entry against the definition, bypassing the table pick (the analog of
the reference's tests/test_configs.py:37-54, which runs every autotune config). Entries whose
query block differs from their key block exercise the dK/dV causal lower-bound rounding."""

import pytest
import torch

from helpers import rand
from oracle.reference import naive_attention

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
LENGTHS = (1, 37, 70, 300)


def _entries():
    if not torch.cuda.is_available():
        return []
    from tattn import _lib

    out = []
    for kernel in (_lib.K_FWD, _lib.K_BWD_DKDV, _lib.K_BWD_DQ):
        for dtype, code in ((torch.float16, _lib.F16), (torch.bfloat16, _lib.BF16), (torch.float32, _lib.F32)):
            for d in (16, 32, 64, 128):
                for c in range(_lib.num_configs(kernel, d, code)):
                    out.append((_lib.KERNEL_NAMES[kernel], dtype, d, c))
    return out


@pytest.mark.parametrize("kernel,dtype,d,cid", _entries(),
                         ids=lambda x: str(x).replace("torch.", ""))
def test_config_forward_and_backward(kernel, dtype, d, cid):
    from tattn.api import _backward, _forward

    tol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}.get(dtype, 1e-5)  # bf16: the fp16 bound x 8
    scale = d ** -0.5
    for n in LENGTHS:
        for causal in (False, True):
            q, k, v, do = (rand((1, 2, n, d), dtype, 7 * n + s, DEV) for s in range(4))
            fcfg = cid if kernel == "fwd" else None
            o, m = _forward(q, k, v, causal, scale, config=fcfg)
            ref = naive_attention(q.float(), k.float(), v.float(), causal=causal)
            torch.testing.assert_close(o.float(), ref, atol=tol, rtol=tol, msg=lambda s: f"fwd n={n} causal={causal}: {s}")
            bcfg = {"dkdv": cid} if kernel == "bwd_dkdv" else {"dq": cid} if kernel == "bwd_dq" else None
            dq, dk, dv = _backward(q, k, v, o, m, do, causal, scale, config=bcfg)
            qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
            naive_attention(qr, kr, vr, causal=causal).backward(do.float())
            for name, got, want in zip(("dq", "dk", "dv"), (dq, dk, dv), (qr.grad, kr.grad, vr.grad)):
                torch.testing.assert_close(got.float(), want, atol=tol, rtol=tol,
                                           msg=lambda s: f"{name} n={n} causal={causal}: {s}")


def test_autotune_first_use_times_once_and_stays_correct(monkeypatch):
    """With first-use timing on, the first fwd+bwd of a key times every table entry, keeps a valid
    entry per kernel and matches the definition; a second call of the same key (another length
    in the same power-of-two bucket) reuses the picks without timing again."""
    import tattn
    from tattn import _lib, api

    monkeypatch.setattr(api, "_tuned", {})
    tattn.set_autotune(True)
    timed = []
    real = _lib.num_configs
    monkeypatch.setattr(_lib, "num_configs", lambda *a: timed.append(a) or real(*a))
    try:
        for n in (600, 1000):
            for causal in (False, True):
                q, k, v, do = (rand((2, 4, n, 64), torch.float16, 11 * n + s, DEV) for s in range(4))
                qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
                o = tattn.attention(qg, kg, vg, causal=causal)
                o.backward(do)
                qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
                ref = naive_attention(qr, kr, vr, causal=causal)
                ref.backward(do.float())
                for name, got, want in zip(("o", "dq", "dk", "dv"), (o, qg.grad, kg.grad, vg.grad),
                                           (ref, qr.grad, kr.grad, vr.grad)):
                    torch.testing.assert_close(got.float(), want.detach(), atol=2e-3, rtol=2e-3,
                                               msg=lambda s: f"{name} n={n} causal={causal}: {s}")
    finally:
        tattn.set_autotune(False)
    assert len(timed) == 6  # three kernels x two masks, all at n=600; n=1000 shares the bucket
    cache = tattn.autotune_cache()
    for kernel, kid in (("fwd", _lib.K_FWD), ("bwd_dkdv", _lib.K_BWD_DKDV), ("bwd_dq", _lib.K_BWD_DQ)):
        assert len(cache[kernel]) == 2
        for cid in cache[kernel].values():
            assert 0 <= cid < real(kid, 64, _lib.F16)


def _raw_backward(kernel, q, k, v, do, m, delta, causal, cid):
    """One dK/dV or dQ launch through the C ABI with a given table entry."""
    from tattn import _lib

    lib = _lib.load()
    b, h, n, d = q.shape
    code = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[q.dtype]
    _, (st,) = _lib.stride_block(q)
    stream = torch.cuda.current_stream().cuda_stream
    if kernel == "bwd_dkdv":
        dk, dv = torch.empty_like(k), torch.empty_like(v)
        _lib.check(lib.tattn_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), dk.data_ptr(),
                                      dv.data_ptr(), m.data_ptr(), delta.data_ptr(), st, b, h, n, d, code,
                                      int(causal), 0.125, cid, stream), "tattn_bwd_dkdv")
        return dk, dv
    dq = torch.empty_like(q)
    _lib.check(lib.tattn_bwd_dq(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), dq.data_ptr(),
                                m.data_ptr(), delta.data_ptr(), st, b, h, n, d, code, int(causal), 0.125,
                                cid, stream), "tattn_bwd_dq")
    return (dq,)


@pytest.mark.parametrize("kernel", ["bwd_dkdv", "bwd_dq"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paired_wave_entries_match_pipelined_bitwise(kernel, d, dtype):
    """The paired-wave backward entries (kind 3: two waves per 32-row tile, one computing P, the
    other dS and the gradient) keep the pipelined kernels' rounding points and summation order:
    their gradients equal the 4-wave pipelined entry's bit for bit, on ragged and full lengths,
    both masks."""
    from tattn import _lib
    from tattn.api import _forward

    kid = _lib.K_BWD_DKDV if kernel == "bwd_dkdv" else _lib.K_BWD_DQ
    descs = [_lib.config_desc(kid, d, _lib.F16, c) for c in range(_lib.num_configs(kid, d, _lib.F16))]
    split = [x["id"] for x in descs if x["kind"] == 3]
    pipe = [x["id"] for x in descs if x["kind"] == 1 and x["waves"] == 4 and x["tiles"] == 1][0]
    assert split, "no paired-wave entry"
    for (b, h, n) in [(1, 3, 1), (2, 3, 17), (2, 3, 70), (2, 4, 300), (1, 8, 1024), (4, 16, 512)]:
        for causal in (False, True):
            q, k, v, do = (rand((b, h, n, d), dtype, 13 * n + s, DEV) for s in range(4))
            o, m = _forward(q, k, v, causal, 0.125)
            delta = (o.float() * do.float()).sum(-1).contiguous()
            want = _raw_backward(kernel, q, k, v, do, m, delta, causal, pipe)
            for cid in split:
                got = _raw_backward(kernel, q, k, v, do, m, delta, causal, cid)
                for g, w in zip(got, want):
                    assert torch.equal(g, w), (f"{kernel} entry {cid} vs {pipe} {(b, h, n, d)} causal={causal}: "
                                               f"max diff {(g.float() - w.float()).abs().max().item():.3e}")
