"""Pins the oracle (CPU only): oracle.reference against float64 brute force, closed forms and
special cases, and oracle.exact against torch float64 autograd. Also shows the checks catch
plausible mistakes (a dropped scale, a transposed mask, swapped operands)."""

import math

import numpy as np
import pytest
import torch

from oracle import exact
from oracle.reference import LOG2E, flops, naive_attention, rounded_backward, tiled_backward, tiled_forward

SHAPES = [(1, 1, 1, 16), (1, 2, 17, 16), (2, 1, 33, 32), (1, 1, 64, 64), (1, 2, 70, 16)]


def rand(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def np64(t):
    return t.detach().double().numpy()


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_naive_matches_float64(shape, causal):
    q, k, v = (rand(shape, s) for s in (1, 2, 3))
    want, _ = exact.attention_fwd(np64(q), np64(k), np64(v), causal)
    got = naive_attention(q, k, v, causal=causal)
    np.testing.assert_allclose(got.numpy(), want, atol=2e-6, rtol=2e-6)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_tiled_forward_o_and_m_match_float64(shape, causal):
    q, k, v = (rand(shape, s) for s in (4, 5, 6))
    want_o, want_m = exact.attention_fwd(np64(q), np64(k), np64(v), causal)
    o, m = tiled_forward(q, k, v, causal)
    np.testing.assert_allclose(o.numpy(), want_o, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(m.numpy(), want_m, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_tiled_backward_matches_float64(shape, causal):
    q, k, v, do = (rand(shape, s) for s in (7, 8, 9, 10))
    o, m = tiled_forward(q, k, v, causal)
    got = tiled_backward(q, k, v, o, m, do, causal)
    want = exact.attention_bwd(np64(q), np64(k), np64(v), np64(do), causal)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g.numpy(), w, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("blocks", [(16, 16), (16, 32), (32, 16), (8, 64)])
def test_tiled_reference_is_block_size_independent(causal, blocks):
    """The reference's own check (tests/test_attention.py:80-90), at 1e-5."""
    q, k, v, do = (rand((2, 2, 45, 16), s) for s in (12, 13, 14, 15))
    o, m = tiled_forward(q, k, v, causal, block_m=blocks[0], block_n=blocks[1])
    torch.testing.assert_close(o, naive_attention(q, k, v, causal=causal), atol=1e-5, rtol=1e-5)
    grads = tiled_backward(q, k, v, o, m, do, causal, block_m=blocks[0], block_n=blocks[1])
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    naive_attention(qr, kr, vr, causal=causal).backward(do)
    for g, w in zip(grads, (qr.grad, kr.grad, vr.grad)):
        torch.testing.assert_close(g, w, atol=1e-5, rtol=1e-5)


def test_config1_tiled_matches_float64_and_float32_autograd():
    """Config 1 of the benchmark plan, the reference's CPU case: fp32 [2, 4, 128, 64] N(0,1),
    non-causal forward + backward with dO ~ N(0,1), tiled with the reference's default 16 x 16
    blocks. O, M and dq/dk/dv against float64 brute force and against float32 materialised
    attention with autograd: flat max abs error 1e-5."""
    q, k, v, do = (rand((2, 4, 128, 64), s) for s in (31, 32, 33, 34))
    o, m = tiled_forward(q, k, v, False, block_m=16, block_n=16)
    grads = tiled_backward(q, k, v, o, m, do, False, block_m=16, block_n=16)
    want_o, want_m = exact.attention_fwd(np64(q), np64(k), np64(v), False)
    want_g = exact.attention_bwd(np64(q), np64(k), np64(v), np64(do), False)
    assert np.abs(o.numpy() - want_o).max() <= 1e-5
    assert np.abs(m.numpy() - want_m).max() <= 1e-5
    for g, w in zip(grads, want_g):
        assert np.abs(g.numpy() - w).max() <= 1e-5
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    ref = naive_attention(qr, kr, vr, causal=False)
    ref.backward(do)
    assert (o - ref.detach()).abs().max().item() <= 1e-5
    for g, w in zip(grads, (qr.grad, kr.grad, vr.grad)):
        assert (g - w).abs().max().item() <= 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_exact_gradients_match_float64_autograd(causal):
    """Pins oracle.exact's closed-form gradients against torch autograd of the definition."""
    q, k, v, do = (rand((2, 3, 21, 32), s).double() for s in (30, 31, 32, 33))
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    s = (qr @ kr.transpose(-1, -2)) / math.sqrt(32)
    if causal:
        s = s.masked_fill(torch.ones(21, 21, dtype=torch.bool).triu(1), float("-inf"))
    (torch.softmax(s, -1) @ vr).backward(do)
    got = exact.attention_bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal)
    for g, w in zip(got, (qr.grad, kr.grad, vr.grad)):
        np.testing.assert_allclose(g, w.numpy(), atol=1e-12, rtol=1e-10)


def test_exact_lse_is_base2_logsumexp():
    q, k = rand((1, 1, 9, 16), 40).double(), rand((1, 1, 9, 16), 41).double()
    _, m = exact.attention_fwd(q.numpy(), k.numpy(), k.numpy())
    s = (q @ k.transpose(-1, -2)) / 4.0
    want = torch.logsumexp(s, -1) / math.log(2.0)
    np.testing.assert_allclose(m, want.numpy(), atol=1e-12)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_rounded_backward_in_float32_is_the_exact_gradient(shape, causal):
    """In float32 every rounding point of rounded_backward is the identity: it must give the
    closed-form float64 gradients (a dropped term, a wrong sign, a transposed operand or mask
    fails here). Small chunks exercise the chunking over leading dimensions."""
    q, k, v, do = (rand(shape, s) for s in (110, 111, 112, 113))
    got = rounded_backward(q, k, v, do, causal, max_scores=shape[-2] ** 2)
    want = exact.attention_bwd(np64(q), np64(k), np64(v), np64(do), causal)
    for g, w in zip(got, want):
        assert g.dtype == torch.float32
        np.testing.assert_allclose(g.numpy(), w, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_rounded_backward_in_float16_rounds_and_stays_close(causal):
    """In float16 the result is in float16, differs from the exact gradient (the roundings are
    applied) by no more than the rounding of P, dS and the store can cause, and a different
    non-default scale is honoured (against float64 at that scale)."""
    q, k, v, do = (rand((2, 3, 40, 32), s, torch.float16) for s in (120, 121, 122, 123))
    for scale in (None, 0.3):
        got = rounded_backward(q, k, v, do, causal, sm_scale=scale)
        want = exact.attention_bwd(np64(q), np64(k), np64(v), np64(do), causal, scale)
        errs = []
        for g, w in zip(got, want):
            assert g.dtype == torch.float16
            errs.append(np.abs(g.double().numpy() - w).max())
        assert max(errs) < 6e-3, errs  # a few fp16 ulps at |grad| ~ 1-4
        assert min(errs) > 1e-5, errs  # the roundings are really applied


@pytest.mark.parametrize("causal", [False, True])
def test_rounded_backward_takes_a_stored_output_and_lse(causal):
    """Given O and M (here from the tiled forward in float32, which match float64 at 1e-5), the
    float32 result is still the exact gradient; given a wrong M (one row shifted by 1 in log2
    units, i.e. that row's P doubled), that row's contributions change, so M is really used."""
    q, k, v, do = (rand((1, 2, 37, 16), s) for s in (140, 141, 142, 143))
    o, m = tiled_forward(q, k, v, causal)
    got = rounded_backward(q, k, v, do, causal, o=o, lse=m)
    want = exact.attention_bwd(np64(q), np64(k), np64(v), np64(do), causal)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g.numpy(), w, atol=2e-5, rtol=2e-5)
    m_bad = m.clone()
    m_bad[0, 0, 20] -= 1.0
    bad = rounded_backward(q, k, v, do, causal, o=o, lse=m_bad)
    assert (bad[0][0, 0, 20] - got[0][0, 0, 20]).abs().max() > 1e-3  # dq of that row
    assert torch.equal(bad[0][0, 1], got[0][0, 1])  # the other head is untouched


def test_rounded_backward_single_key():
    """One key: P = 1 exactly, so dV = dO exactly in float16 and dS = dP - delta = 0 up to the
    float32 summation order of the two dot products."""
    q, k, v, do = (rand((2, 3, 1, 64), s, torch.float16) for s in (130, 131, 132, 133))
    dq, dk, dv = rounded_backward(q, k, v, do, True)
    assert torch.equal(dv, do)
    assert dq.abs().max().item() < 1e-4 and dk.abs().max().item() < 1e-4


# ---- closed-form special cases (independent of any implementation's formula) --------------

@pytest.mark.parametrize("causal", [False, True])
def test_single_key_gives_v_and_zero_qk_grads(causal):
    q, k, v, do = (rand((2, 3, 1, 32), s) for s in (50, 51, 52, 53))
    o, m = tiled_forward(q, k, v, causal)
    torch.testing.assert_close(o, v, atol=1e-6, rtol=0)
    # one key: softmax is 1, so M is the scaled score itself
    torch.testing.assert_close(m, (q * k).sum(-1) / math.sqrt(32) * LOG2E, atol=1e-5, rtol=1e-5)
    dq, dk, dv = tiled_backward(q, k, v, o, m, do, causal)
    torch.testing.assert_close(dv, do, atol=1e-6, rtol=0)
    assert dq.abs().max() < 1e-6 and dk.abs().max() < 1e-6


def test_zero_queries_average_values():
    v = rand((1, 2, 13, 16), 60)
    q = torch.zeros_like(v)
    k = rand((1, 2, 13, 16), 61)
    o, _ = tiled_forward(q, k, v, False)
    torch.testing.assert_close(o, v.mean(-2, keepdim=True).expand_as(v), atol=1e-6, rtol=1e-6)
    oc, _ = tiled_forward(q, k, v, True)
    counts = torch.arange(1, 14, dtype=torch.float32).view(1, 1, 13, 1)
    torch.testing.assert_close(oc, v.cumsum(-2) / counts, atol=1e-6, rtol=1e-6)


def test_causal_first_row_is_first_value():
    q, k, v = (rand((1, 2, 25, 16), s) for s in (70, 71, 72))
    o, _ = tiled_forward(q, k, v, True)
    torch.testing.assert_close(o[..., 0, :], v[..., 0, :], atol=1e-6, rtol=0)


def test_noncausal_invariant_under_key_value_permutation():
    q, k, v = (rand((1, 2, 31, 32), s) for s in (80, 81, 82))
    perm = torch.randperm(31, generator=torch.Generator().manual_seed(83))
    o1, m1 = tiled_forward(q, k, v, False)
    o2, m2 = tiled_forward(q, k[..., perm, :], v[..., perm, :], False)
    torch.testing.assert_close(o1, o2, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(m1, m2, atol=1e-5, rtol=1e-6)


def test_flops_formula():
    assert flops(1, 16, 16384, 64, False, "fwd") == 4 * 16 * 16384**2 * 64
    assert flops(32, 16, 512, 64, True, "fwd") == 2 * 32 * 16 * 512**2 * 64
    assert flops(2, 16, 8192, 64, False, "fwd+bwd") == 3.5 * 4 * 2 * 16 * 8192**2 * 64
    # 16,384 tokens, H=16, D=64: fwd flops = 67,108,864 * N
    for n in (512, 1024, 16384):
        assert flops(16384 // n, 16, n, 64, False, "fwd") == 67108864 * n


# ---- the checks above are not vacuous: plausible mistakes fail them ---------------------------

def _wrong_mask(q, k, v):
    s = (q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    n = q.shape[-2]
    s = s.masked_fill(torch.ones(n, n, dtype=torch.bool).tril(-1), float("-inf"))  # transposed mask
    return torch.softmax(s, -1) @ v


def _no_scale(q, k, v):
    return torch.softmax(q @ k.transpose(-1, -2), -1) @ v


@pytest.mark.parametrize("mistake", ["mask", "scale", "swap"])
def test_planted_mistakes_are_caught(mistake):
    q, k, v = (rand((1, 2, 19, 16), s) for s in (90, 91, 92))
    causal = mistake == "mask"
    want, _ = exact.attention_fwd(np64(q), np64(k), np64(v), causal)
    if mistake == "mask":
        got = _wrong_mask(q, k, v)
    elif mistake == "scale":
        got = _no_scale(q, k, v)
    else:
        got = naive_attention(q, v, k, causal=False)  # k and v swapped
    assert np.abs(got.numpy() - want).max() > 1e-2
