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
