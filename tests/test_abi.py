"""The C-ABI library (CPU only, no kernel launches): it loads, exports every symbol that
include/tattn.h declares, agrees with the header's constants, describes its tile tables, and
rejects bad arguments with error codes and messages before touching a device."""

import ctypes
import re
from pathlib import Path

import pytest

from tattn import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "tattn.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(tattn_\w+)\s*\(", text, re.M)))


def test_library_loads_with_matching_abi():
    lib = _lib.load()
    assert lib.tattn_abi_version() == _lib.ABI_VERSION
    assert f"#define TATTN_ABI_VERSION {_lib.ABI_VERSION}" in HEADER.read_text()


def test_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared()
    assert names == sorted(_lib.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name


def test_header_constants_match_binding():
    text = HEADER.read_text()
    assert "TATTN_F16 = 0" in text and "TATTN_F32 = 1" in text
    assert "TATTN_K_FWD = 0" in text and "TATTN_K_BWD_DKDV = 1" in text and "TATTN_K_BWD_DQ = 2" in text
    assert ctypes.sizeof(_lib.TattnConfig) == 28


@pytest.mark.parametrize("kernel", [_lib.K_FWD, _lib.K_BWD_DKDV, _lib.K_BWD_DQ])
@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [_lib.F16, _lib.F32])
def test_tables_are_described(kernel, d, dtype):
    n = _lib.num_configs(kernel, d, dtype)
    assert n >= 1
    for c in range(n):
        desc = _lib.config_desc(kernel, d, dtype, c)
        assert desc["waves"] in (4, 8) and desc["tiles"] in (1, 2)
        # Paired-wave backward entries (kind 3) give each 32-row tile two waves.
        rows = (desc["waves"] // 2 if desc["kind"] == 3 else desc["waves"]) * desc["tiles"] * 32
        assert desc["kind"] in (0, 1, 2, 3) and (desc["kind"] != 3 or kernel != _lib.K_FWD)
        own = desc["block_n"] if kernel == _lib.K_BWD_DKDV else desc["block_m"]
        assert own == rows
        assert 0 < desc["lds_bytes"] <= 160 * 1024
    with pytest.raises(RuntimeError, match="no config"):
        _lib.config_desc(kernel, d, dtype, n)
    assert 0 <= _lib.pick_config(kernel, d, dtype, False, 4096) < n


def test_unsupported_head_dim_has_no_table():
    assert _lib.num_configs(_lib.K_FWD, 48, _lib.F16) == -1


def _fwd_args(**kw):
    st = (ctypes.c_int64 * 4)(16 * 64, 64, 64, 1)
    a = dict(q=16, k=16, v=16, o=16, m=16, qs=st, ks=st, vs=st, os=st, Z=1, H=1, N=16, D=64,
             dtype=_lib.F16, causal=0, scale=0.125, cfg=-1, stream=None)
    a.update(kw)
    return [a[x] for x in ("q", "k", "v", "o", "m", "qs", "ks", "vs", "os", "Z", "H", "N", "D",
                           "dtype", "causal", "scale", "cfg", "stream")]


@pytest.mark.parametrize("bad,msg", [
    (dict(D=48), "head dim"),
    (dict(dtype=7), "dtype"),
    (dict(N=0), "positive"),
    (dict(q=None), "q is a null pointer"),
    (dict(k=24), "16-byte aligned"),
    (dict(qs=(ctypes.c_int64 * 4)(1024, 64, 64, 2)), "d stride"),
    (dict(vs=(ctypes.c_int64 * 4)(1024, 64, 12, 1)), "multiple of"),
    (dict(cfg=999), "out of range"),
])
def test_fwd_rejects_bad_arguments_before_launch(bad, msg):
    lib = _lib.load()
    rc = lib.tattn_fwd(*_fwd_args(**bad))
    assert rc in (1, 2)
    assert msg in _lib.last_error()


def test_bwd_rejects_bad_config_for_both_tables():
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(1024, 64, 64, 1)
    rc = lib.tattn_bwd(16, 16, 16, 16, 16, 16, 16, 16, 16, 16, st, 1, 1, 16, 64, _lib.F16, 0,
                       0.125, 99, None)
    assert rc == 2 and "out of range" in _lib.last_error()


@pytest.mark.parametrize("bad,msg", [
    (dict(dk=24), "dk must be 16-byte aligned"),
    (dict(dv=None), "dv is a null pointer"),
    (dict(o=40), "o must be 16-byte aligned"),
    (dict(m=None), "m and delta must not be null"),
    (dict(delta=None), "m and delta must not be null"),
    (dict(cfg=999), "out of range"),
])
def test_bwd_checks_every_argument_before_any_device_work(bad, msg):
    """tattn_bwd validates all of its arguments, dK/dV's included, before it enqueues anything:
    here (no GPU) the first device call would fail with a device error, so an argument error
    that names dk, dv or o shows that no kernel (the dQ that runs first) was reached."""
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(1024, 64, 64, 1)
    a = dict(q=16, k=16, v=16, o=16, do=16, dq=16, dk=16, dv=16, m=16, delta=16, cfg=-1)
    a.update(bad)
    rc = lib.tattn_bwd(a["q"], a["k"], a["v"], a["o"], a["do"], a["dq"], a["dk"], a["dv"], a["m"], a["delta"], st,
                       1, 8, 512, 64, _lib.F16, 1, 0.125, a["cfg"], None)
    assert rc in (1, 2) and msg in _lib.last_error()


def test_bwd_noalloc_rejects_problems_past_its_workspace_before_launch():
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(1 << 20, 1 << 16, 64, 1)
    rc = lib.tattn_bwd_noalloc(16, 16, 16, 16, 16, 16, 16, 16, 16, st, 1, 65, 1 << 16, 64, _lib.F16, 0,
                               0.125, -1, None)
    assert rc == 1 and "exceeds the static workspace" in _lib.last_error()


@pytest.mark.parametrize("n", [512, 1024, 2048, 4096, 8192, 16384])
@pytest.mark.parametrize("dtype", [_lib.F16, _lib.BF16])
def test_picks_at_the_benchmark_lengths(n, dtype):
    """The static picks (tattn_pick_config, batch x heads a multiple of 8) at the benchmark
    lengths, by kind: persistent forward and dQ wherever they fit (forward at head dim 64: one tile
    per wave for causal N < 2048, two otherwise), the persistent 4-wave dK/dV at
    head dim 64 for causal N < 4096 and the pipelined 8-wave one otherwise, paired-wave backward
    at 128."""
    def kind(kernel, d, causal):
        return _lib.config_desc(kernel, d, dtype, _lib.pick_config(kernel, d, dtype, causal, n))

    for causal in (False, True):
        f64, f128 = kind(_lib.K_FWD, 64, causal), kind(_lib.K_FWD, 128, causal)
        assert f64["kind"] == 2 and f64["ring"] == 4
        assert (f64["waves"], f64["tiles"]) == ((4, 1) if causal and n < 2048 else (4, 2))
        assert f128["kind"] == 2 and f128["ring"] == 4
        assert (f128["waves"], f128["tiles"]) == ((8, 1) if n >= (4096 if causal else 2048) else (4, 1))
        dkdv64, dq64 = kind(_lib.K_BWD_DKDV, 64, causal), kind(_lib.K_BWD_DQ, 64, causal)
        if causal and n < 4096:
            assert dkdv64["kind"] == 2 and dkdv64["waves"] == 4
        else:
            assert dkdv64["kind"] == 1 and dkdv64["waves"] == 8
        assert dq64["kind"] == 2 and dq64["waves"] == 4
        assert kind(_lib.K_BWD_DKDV, 128, causal)["kind"] == 3 and kind(_lib.K_BWD_DQ, 128, causal)["kind"] == 3
