"""CPU tests of the measurement tools: the ISA parser of tattn.diagnose (on a hand-written
assembly listing and on the compiled forward kernel), the comparison suite's cell and error
assembly (tattn.benchsuite, with fake implementations and a fixed timer on the CPU), and the
markdown report of tattn.report."""

import json
from pathlib import Path

import pytest

from tattn import _build, diagnose, report

SYNTH = """\
\t.text
_Z6kernelPf:                            ; @_Z6kernelPf
; %bb.0:
\tv_mov_b32 v0, 0
\tds_write_b128 v1, v[2:5]
.LBB0_1:                                ; =>This Inner Loop Header: Depth=1
\tds_write_b128 v1, v[2:5]
\ts_cbranch_scc1 .LBB0_1
; %bb.2:
.LBB0_3:                                ; =>This Loop Header: Depth=1
                                        ;     Child Loop BB0_5 Depth 2
\tv_mov_b32 v0, 1
.LBB0_5:                                ;   Parent Loop BB0_3 Depth=1
                                        ; =>  This Inner Loop Header: Depth=2
\tbuffer_load_dword v1, v2, s[4:7], 0 offen lds
\tbuffer_load_dwordx4 v[4:7], v2, s[4:7], 0 offen
\tds_read_b64_tr_b16 v[8:9], v3
\tds_read_b128 v[10:13], v3
\tv_mfma_f32_32x32x16_f16 v[16:31], v[8:11], v[12:15], v[16:31]
\tv_mfma_f32_32x32x16_f16 v[16:31], v[8:11], v[12:15], v[16:31]
\tv_exp_f32_e32 v5, v5
\tv_fmac_f32_e32 v6, v7, v8
\ts_waitcnt vmcnt(0) lgkmcnt(0)
\ts_barrier
\tscratch_store_dword off, v9, s0
\ts_cbranch_scc0 .LBB0_5
\ts_cbranch_scc0 .LBB0_3
; %bb.4:
\tglobal_store_dwordx4 v[0:1], v[4:7], off
\ts_endpgm
                                        ; -- End function
; codeLenInByte = 96
; TotalNumSgprs: 12
; NumVgprs: 32
; NumAgprs: 0
; ScratchSize: 4
; LDSByteSize: 1024 bytes/workgroup (compile time only)
; Occupancy: 8
"""


def test_isa_parser_on_synthetic_listing():
    st = diagnose.isa_stats(SYNTH)
    assert list(st) == ["_Z6kernelPf"]
    k = st["_Z6kernelPf"]
    assert (k["code_bytes"], k["sgprs"], k["vgprs"], k["agprs"]) == (96, 12, 32, 0)
    assert (k["scratch_bytes_per_lane"], k["lds_bytes"], k["occupancy"]) == (4, 1024, 8)
    # The main loop is the inner loop of the nest (it holds the MFMAs), not the first store loop.
    ml = k["main_loop"]
    assert ml["mfma"] == 2 and ml["mfma_by_opcode"] == {"v_mfma_f32_32x32x16_f16": 2}
    assert ml["lds_dma"] == 1 and ml["global_load"] == 1
    assert ml["ds_read_tr"] == 1 and ml["ds_read"] == 1 and ml["ds_write"] == 0
    assert ml["v_exp"] == 1 and ml["v_fma"] == 1
    assert ml["wait_vmcnt0"] == 1 and ml["s_barrier"] == 1 and ml["scratch"] == 1
    assert k["all"]["ds_write"] == 2 and k["all"]["global_store"] == 1 and k["all"]["mfma"] == 2


def test_isa_parser_filters_kernels():
    assert diagnose.isa_stats(SYNTH, "other") == {}


def test_kernel_names_are_demangled():
    d = diagnose._short_demangle
    assert d("_ZN5tattn15fwd_pipe_kernelIDF16bLi128ELi4ELi1ELi2ELb1EEEvNS_9FwdParamsE") == \
        "tattn::fwd_pipe_kernel<__bf16, 128, 4, 1, 2, true>"
    assert d("_ZN5tattn18fwd_generic_kernelIfLi64ELi4ELi32ELi64ELb0EEEvNS_9FwdParamsE") == \
        "tattn::fwd_generic_kernel<float, 64, 4, 32, 64, false>"
    assert d("_Z6kernelPf") == "_Z6kernelPf"


def _have_hipcc() -> bool:
    try:
        _build.hipcc()
        return True
    except RuntimeError:
        return False


@pytest.fixture(scope="module")
def fwd_asm():
    return diagnose.compile_asm(diagnose.CSRC / "fwd.hip")


@pytest.mark.skipif(not _have_hipcc(), reason="hipcc not installed")
def test_forward_pipeline_main_loop_isa(fwd_asm):
    """The 16k-token fp16 forward kernel (8 waves, 2 query tiles per wave, d=64): one main-loop
    iteration per 4 K/V blocks with 96 MFMAs (4 blocks x 2 tiles x (QK^T 4 + PV 8)), 8 LDS DMA
    loads, one barrier per block, and neither register spills (anywhere in the kernel) nor full
    memory drains in the loop."""
    st = diagnose.isa_stats(fwd_asm, "fwd_pipe_kernelIDF16_Li64ELi8ELi2ELi2ELb0E")
    assert len(st) == 1
    (k,) = st.values()
    assert "fwd_pipe_kernel<_Float16, 64, 8, 2, 2, false>" in k["name"]
    assert k["occupancy"] >= 2 and k["scratch_bytes_per_lane"] == 0
    ml = k["main_loop"]
    assert ml["mfma"] == 96 and set(ml["mfma_by_opcode"]) == {"v_mfma_f32_32x32x16_f16"}
    assert ml["lds_dma"] == 8 and ml["global_load"] == 0
    assert ml["s_barrier"] == 4
    assert ml["scratch"] == 0 and ml["wait_vmcnt0"] == 0


def _suite_result():
    """A small tattn-suite/1 result built by the suite's own sweep and error code on the CPU, with
    fake implementations and a fixed timer."""
    import torch

    from tattn import benchsuite as bs

    def scaled(f):
        return lambda q, k, v, causal: bs.materialised(q, k, v, causal) * f

    def broken(q, k, v, causal):
        raise RuntimeError("No available kernel. Aborting execution.\nmore text")

    impls = [bs.Impl("tattn", "tattn", scaled(1.0)), bs.Impl("sdpa_flash", "flash", broken),
             bs.Impl("materialised", "materialised", bs.materialised)]
    inputs = {n: bs.make_inputs(n, 64, 2, 16, "cpu", torch.float32) for n in (16, 32)}
    times = {"tattn": 1.0, "materialised": 4.0}

    def timer(call, reset):
        call()
        reset()
        return times[current[0]], 3.0

    current = ["tattn"]
    orig = bs.call_for

    def call_for(impl, x, causal, passes):
        current[0] = impl.name
        return orig(impl, x, causal, passes)

    bs.call_for = call_for
    try:
        cells = bs.sweep_cells(impls, inputs, heads=2, dim=16, timer=timer)
    finally:
        bs.call_for = orig
    errors = bs.measure_errors(impls, inputs, grad_seqs=(32,))
    return {"schema": "tattn-suite/1",
            "device": {"name": "AMD Instinct MI355X", "arch": "gfx950:sramecc+:xnack-", "memory_gib": 288,
                       "torch": "2.10", "hip": "7.0", "python": "3.10"},
            "method": {"tokens": 64, "heads": 2, "dim": 16, "dtype": "float32", "timer": "fixed",
                       "flops": "4 n^2 d", "data": "randn"},
            "cells": cells, "errors": errors, "gemm_tflops": 1500.0,
            "picks": {"16/none": {"fwd": 1, "bwd_dkdv": 0, "bwd_dq": 0}}, "autotuned": None}


def test_suite_sweep_assembles_every_cell():
    from tattn import benchsuite as bs

    res = _suite_result()
    cells = res["cells"]
    assert len(cells) == 3 * 2 * 2 * 2  # impls x N x masks x passes
    ok = [c for c in cells if c["impl"] == "tattn"]
    assert all(c["status"] == "ok" and c["ms"] == 1.0 and c["peak_mib"] == 3.0 for c in ok)
    c = next(c for c in ok if c["n"] == 32 and c["mask"] == "causal" and c["pass"] == "fwd+bwd")
    assert c["b"] == 2 and c["tflops"] == bs.counted_flops(2, 2, 32, 16, True, "fwd+bwd") / 1e-3 / 1e12
    bad = [c for c in cells if c["impl"] == "sdpa_flash"]
    assert all(c["status"] == "unsupported" and c["note"] == "No available kernel. Aborting execution."
               for c in bad)


def test_suite_errors_cover_outputs_and_gradients():
    errs = _suite_result()["errors"]
    fwd = {(e["impl"], e["n"], e["mask"]) for e in errs if e["tensor"] == "o"}
    assert fwd == {(i, n, m) for i in ("tattn", "materialised") for n in (16, 32) for m in ("none", "causal")}
    assert all(e["max_abs"] < 1e-5 for e in errs)  # float32 inputs: same math as the reference
    grads = [(e["n"], e["mask"], e["tensor"]) for e in errs if e["tensor"] != "o"]
    assert sorted(grads) == sorted((32, m, t) for m in ("none", "causal") for t in ("dq", "dk", "dv"))


def test_report_renders_every_section():
    res = _suite_result()
    assert report.problems(res) == []
    text = report.render(res)
    for title in ("Forward, TFLOP/s", "Forward + backward, TFLOP/s", "Peak memory", "Accuracy",
                  "Cells that did not run", "Tile-table entries used"):
        assert f"## {title}" in text
    assert "| tattn ÷ fastest other |" in text and "| 4.00× |" in text  # 1 ms against 4 ms
    assert "SDPA flash, unsupported: 16/none/fwd (No available kernel. Aborting execution.)" in text
    assert "16/none: 1/0/0" in text


def test_report_check_flags_broken_files(tmp_path):
    res = _suite_result()
    good = tmp_path / "good.json"
    good.write_text(json.dumps(res))
    assert report.main([str(good), "--check"]) == 0
    res["cells"][0].pop("status")
    res["errors"][0]["max_abs"] = float("nan")
    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps(res))
    assert report.main([str(bad), "--check"]) == 1
    assert any("lacks ['status']" in p for p in report.problems(res))
    assert any("non-finite" in p for p in report.problems(res))


@pytest.mark.parametrize("name", ["gfx950.json", "gfx950_d128.json"])
def test_committed_suite_results_are_valid_and_rendered(name):
    """The suite's last runs on an MI355X (head dim 64 and 128) have the current schema, every cell
    of the grid and finite errors, and each .md next to them is its rendering."""
    path = Path(__file__).resolve().parent.parent / "results" / name
    res = json.loads(path.read_text())
    assert report.problems(res) == []
    assert {(c["impl"], c["n"], c["mask"], c["pass"]) for c in res["cells"]} >= {
        ("tattn", n, m, p) for n in (512, 1024, 2048, 4096, 8192, 16384) for m in ("none", "causal")
        for p in ("fwd", "fwd+bwd")}
    assert all(c["status"] == "ok" for c in res["cells"] if c["impl"] == "tattn")
    assert path.with_suffix(".md").read_text() == report.render(res)


@pytest.fixture(scope="module")
def bwd_asm():
    return diagnose.compile_asm(diagnose.CSRC / "bwd.hip")


@pytest.fixture(scope="module")
def own_scheduler_asm():
    """The translation units built with their own instruction scheduler."""
    return [diagnose.compile_asm(diagnose.CSRC / s) for s in ("fwd_persist_causal.hip", "bwd_dq_persist.hip", "bwd_split.hip")]


@pytest.fixture(scope="module")
def dkdv_persist_asm():
    """The persistent dK/dV kernels' own translation unit (default scheduler)."""
    return diagnose.compile_asm(diagnose.CSRC / "bwd_dkdv_persist.hip")


@pytest.mark.skipif(not _have_hipcc(), reason="hipcc not installed")
def test_no_kernel_spills_registers(fwd_asm, bwd_asm, own_scheduler_asm, dkdv_persist_asm):
    """Every kernel instantiation the tile tables reach compiles without scratch (register
    spills), except fp32 causal dK/dV at D=128 (a few bytes, not a performance path) and the
    non-causal persistent dK/dV (at most 32 bytes: per-lane constants written once at the start
    and reloaded once per key block, outside the step loop). The causal persistent forward with
    two tiles per wave, the long-row causal pick, is held to zero."""
    allowed = {"dkdv_kernel<float, 128, 4, 1, 32, true, 1>"}
    allowed_upto_32 = {f"dkdv_persist_kernel<{t}, 64, {nw}, 2, false>" for t in ("_Float16", "__bf16") for nw in (4, 8)}
    spills = []
    for asm in (fwd_asm, bwd_asm, *own_scheduler_asm, dkdv_persist_asm):
        for k in diagnose.isa_stats(asm, "_kernelI").values():
            name = k["name"].replace("tattn::", "").split("(")[0].removeprefix("void ")
            sc = k.get("scratch_bytes_per_lane")
            if sc and name not in allowed and not (name in allowed_upto_32 and sc <= 32):
                spills.append((name, sc))
    assert not spills, spills


@pytest.mark.skipif(not _have_hipcc(), reason="hipcc not installed")
def test_each_kernel_lives_in_one_translation_unit(fwd_asm, bwd_asm, own_scheduler_asm, dkdv_persist_asm):
    """A kernel instantiated by two translation units would reach the library twice, built with
    different scheduler flags; the launchers keep each family in exactly one unit."""
    import collections
    import re

    seen = collections.Counter()
    for asm in (fwd_asm, bwd_asm, *own_scheduler_asm, dkdv_persist_asm):
        seen.update(set(re.findall(r"^\s*\.amdhsa_kernel (\S+)", asm, re.M)))
    dups = [k for k, n in seen.items() if n > 1]
    assert not dups, dups
    causal2, dq_persist, split = (set(re.findall(r"^\s*\.amdhsa_kernel (\S+)", a, re.M)) for a in own_scheduler_asm)
    assert causal2 and all("fwd_persist_kernel" in k for k in causal2)
    assert dq_persist and all("dq_persist_kernel" in k for k in dq_persist)
    assert split and all("_split_kernel" in k for k in split)
    dkdv_persist = set(re.findall(r"^\s*\.amdhsa_kernel (\S+)", dkdv_persist_asm, re.M))
    assert dkdv_persist and all("dkdv_persist_kernel" in k for k in dkdv_persist)


@pytest.mark.skipif(not _have_hipcc(), reason="hipcc not installed")
def test_reported_lds_matches_the_persistent_kernels(fwd_asm, own_scheduler_asm):
    """tattn_config_desc's LDS bytes of the persistent forward and dQ entries (K/V ring, plus the
    O rows staged at head dim 64, plus the dQ rows) agree with what the compiled kernels allocate,
    up to the padding of the ring's unused slot arrays."""
    from tattn import _lib

    stats = {}
    for asm in (fwd_asm, own_scheduler_asm[0], own_scheduler_asm[1]):
        for k in diagnose.isa_stats(asm, "_kernelI").values():
            stats[k["name"].replace("tattn::", "").split("(")[0].removeprefix("void ")] = k["lds_bytes"]
    checked = 0
    for d in (64, 128):
        for cid in range(_lib.num_configs(_lib.K_FWD, d, _lib.F16)):
            e = _lib.config_desc(_lib.K_FWD, d, _lib.F16, cid)
            if e["kind"] != 2:
                continue
            for causal in ("false", "true"):
                name = f"fwd_persist_kernel<_Float16, {d}, {e['waves']}, {e['tiles']}, 2, {causal}, {e['ring']}, false>"
                if name not in stats:  # causal two-tile ring-8 entries run their pipelined twin
                    continue
                assert e["lds_bytes"] <= stats[name] <= e["lds_bytes"] + 2048, (name, e, stats[name])
                checked += 1
        for cid in range(_lib.num_configs(_lib.K_BWD_DQ, d, _lib.F16)):
            e = _lib.config_desc(_lib.K_BWD_DQ, d, _lib.F16, cid)
            if e["kind"] != 2:
                continue
            for causal in ("false", "true"):
                name = f"dq_persist_kernel<_Float16, {d}, {e['waves']}, 2, {causal}>"
                assert e["lds_bytes"] <= stats[name] <= e["lds_bytes"] + 2048, (name, e, stats[name])
                checked += 1
    assert checked >= 12
