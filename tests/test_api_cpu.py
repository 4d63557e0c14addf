"""Host-side behaviour of the public API that needs no GPU: argument checks with the reference's
messages (src/tattn/api.py:45-56), no CPU compute path, backend probe, length buckets."""

import pytest
import torch

from tattn import attention, hip_available, triton_available
from tattn.api import _bucket, _resolve
from tattn import _lib


def test_rejects_bad_inputs():
    """The reference's test_rejects_bad_inputs (tests/test_attention.py:67-77)."""
    x = torch.zeros(1, 1, 8, 16)
    with pytest.raises(ValueError, match="equal shape"):
        attention(x, x[..., :4, :], x)
    with pytest.raises(ValueError, match="head dim"):
        y = torch.zeros(1, 1, 8, 24)
        attention(y, y, y)
    with pytest.raises(ValueError, match="dtype"):
        attention(x, x.double(), x)
    with pytest.raises(ValueError, match="equal shape"):
        attention(x[0], x[0], x[0])


def test_rejects_mixed_devices():
    """tests/test_attention.py:134-137."""
    x = torch.zeros(1, 1, 8, 16)
    with pytest.raises(ValueError, match="one device"):
        attention(x, x.to("meta"), x)


def test_rejects_mixed_and_unsupported_dtypes():
    """tests/test_attention.py:74-75; bfloat16 is accepted (an addition to the reference),
    float64 and mixed dtypes are not."""
    x = torch.zeros(1, 1, 8, 16)
    with pytest.raises(ValueError, match="dtype"):
        attention(x.half(), x, x)
    with pytest.raises(ValueError, match="dtype"):
        attention(x.double(), x.double(), x.double())
    with pytest.raises(ValueError, match="dtype"):
        attention(x.bfloat16(), x.half(), x.bfloat16())
    with pytest.raises(RuntimeError, match="gfx950"):  # valid, but CPU tensors have no path
        attention(x.bfloat16(), x.bfloat16(), x.bfloat16())


def test_cpu_tensors_are_refused_not_computed():
    """The product has no CPU path: valid CPU inputs raise instead of silently computing."""
    x = torch.zeros(1, 1, 8, 16)
    with pytest.raises(RuntimeError, match="gfx950"):
        attention(x, x, x)


def test_backend_probe_false_on_cpu():
    assert not hip_available(torch.device("cpu"))
    assert not triton_available(torch.device("cpu"))


def test_bucket_matches_reference_rule():
    assert [_bucket(n) for n in (1, 2, 3, 17, 64, 65, 16384)] == [1, 2, 4, 32, 64, 128, 16384]


def test_config_resolution():
    assert _resolve(_lib.K_FWD, 64, torch.float16, None, False, 128) == -1
    assert _resolve(_lib.K_FWD, 64, torch.float16, 3, False, 128) == 3
    assert _resolve(_lib.K_FWD, 64, torch.float16, {"id": 2}, False, 128) == 2
    first = _lib.config_desc(_lib.K_FWD, 64, _lib.F16, 0)
    sel = {"BLOCK_M": first["block_m"], "BLOCK_N": first["block_n"], "waves": first["waves"]}
    with pytest.raises(ValueError, match="matches 0"):
        _resolve(_lib.K_FWD, 64, torch.float16, {"BLOCK_M": 7}, False, 128)
    # A persistent entry shares its tiles with a pipelined one: "kind" chooses between them.
    assert _resolve(_lib.K_FWD, 64, torch.float16, dict(sel, kind=first["kind"]), False, 128) == 0
    twin = dict(sel, kind=2)
    pid = _resolve(_lib.K_FWD, 64, torch.float16, twin, False, 128)
    desc = _lib.config_desc(_lib.K_FWD, 64, _lib.F16, pid)
    assert pid > 0 and desc["kind"] == 2 and desc["block_m"] == first["block_m"] and desc["ring"] in (4, 8)


def test_ambiguous_config_dict_is_refused_and_kind_resolves_it():
    """At head dim 64 the forward's 4 waves x 2 tiles exist as a pipelined entry (0) and as two
    persistent ones (4: ring 8, 7: ring 4). Without "kind" the dict is refused, naming the
    entries; with it, the lowest matching id of that kind is taken; "ring" narrows further."""
    with pytest.raises(ValueError, match=r"entries \[0, 4, 7\] of kinds \[1, 2\]"):
        _resolve(_lib.K_FWD, 64, torch.float16, {"waves": 4, "tiles": 2}, False, 4096)
    assert _resolve(_lib.K_FWD, 64, torch.float16, {"waves": 4, "tiles": 2, "kind": 1}, False, 4096) == 0
    assert _resolve(_lib.K_FWD, 64, torch.float16, {"waves": 4, "tiles": 2, "kind": 2}, False, 4096) == 4
    assert _resolve(_lib.K_FWD, 64, torch.float16, {"waves": 4, "tiles": 2, "kind": 2, "ring": 4}, False, 4096) == 7
    # Several matches of one kind: the lowest id (the dQ table's generic 128-row entries 2 and 3).
    assert _resolve(_lib.K_BWD_DQ, 64, torch.float16, {"BLOCK_M": 128, "kind": 0}, False, 4096) == 2
    with pytest.raises(ValueError, match="give"):
        _resolve(_lib.K_BWD_DKDV, 64, torch.float16, {"BLOCK_N": 256}, False, 4096)


def test_autotune_off_by_default_and_cache_format(monkeypatch):
    """First-use timing is opt-in (TATTN_AUTOTUNE=1 or set_autotune); while off the library's own
    pick (-1) is used and nothing is launched; the cache reports picks per kernel and key."""
    import tattn
    from tattn import api

    monkeypatch.setattr(api, "_tuned", {})
    launched = []
    monkeypatch.setattr(api, "_autotune", False)
    assert api._tuned_id(_lib.K_FWD, torch.zeros(1), 64, False, 1000, launched.append) == -1
    assert launched == [] and api._tuned == {}
    tattn.set_autotune(True)
    assert api._autotune
    tattn.set_autotune(False)
    assert not api._autotune
    api._tuned[(_lib.K_BWD_DQ, 0, api._bucket(1000), 64, _lib.F16, True)] = 2
    assert tattn.autotune_cache() == {"fwd": {}, "bwd_dkdv": {},
                                      "bwd_dq": {"device=0, n_bucket=1024, d=64, dtype=float16, causal=True": 2}}
