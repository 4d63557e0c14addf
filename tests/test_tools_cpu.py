"""CPU tests of the measurement tools: the ISA parser of tattn.diagnose (on a hand-written
assembly listing and on the compiled forward kernel), and the markdown report of tattn.report."""

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


def _fake_result():
    rows = []
    for impl, f in (("tattn", 900.0), ("sdpa_flash", 400.0), ("naive", 50.0)):
        for mode in ("fwd", "fwd+bwd"):
            for causal in (False, True):
                for seq, batch in ((1024, 16), (16384, 1)):
                    rows.append({"impl": impl, "seq": seq, "batch": batch, "causal": causal, "mode": mode,
                                 "ms": 1.0, "tflops": f * (0.5 if mode == "fwd+bwd" else 1.0),
                                 "peak_extra_mib": 100.0})
    rows.append({"impl": "sdpa_math", "seq": 16384, "batch": 1, "causal": False, "mode": "fwd", "oom": True})
    return {
        "env": {"gpu": "AMD Instinct MI355X", "arch": "gfx950:sramecc+:xnack-", "memory_gib": 288,
                "torch": "2.10", "hip": "7.0", "python": "3.10"},
        "config": {"dim": 64, "heads": 16, "tokens": 16384, "timer": "median", "flops": "4 n^2 d", "data": "randn"},
        "rows": rows,
        "accuracy": [{"impl": "tattn", "seq": 1024, "causal": False, "max_abs_err": 1e-3, "mean_abs_err": 1e-5},
                     {"impl": "tattn", "seq": 1024, "causal": False, "grad": "dq", "max_abs_err": 2e-3}],
        "table_picks": {"16384": {"fwd": 3, "bwd_dkdv": 1, "bwd_dq": 1}},
        "fp16_matmul_4096_tflops": 1500.0,
    }


def test_report_renders_every_section():
    text = report.render(_fake_result())
    assert "Best tattn forward: 900.0 TFLOP/s (35.8% of" in text
    for title in ("Forward, non-causal", "Forward, causal", "Forward + backward, non-causal",
                  "Forward + backward, causal", "Peak extra memory", "Accuracy", "Table picks"):
        assert f"## {title}" in text
    # tattn over SDPA flash: 900/400 in every cell, both modes.
    assert "| SDPA flash | 2.25–2.25× | 2.25–2.25× |" in text
    assert "OOM" in text and "| 16,384 (1) |" in text
    assert "16384: 3/1/1" in text


@pytest.fixture(scope="module")
def bwd_asm():
    return diagnose.compile_asm(diagnose.CSRC / "bwd.hip")


@pytest.mark.skipif(not _have_hipcc(), reason="hipcc not installed")
def test_no_kernel_spills_registers(fwd_asm, bwd_asm):
    """Every kernel instantiation the tile tables reach compiles without scratch (register
    spills), except fp32 causal dK/dV at D=128 (a few bytes, not a performance path)."""
    allowed = {"dkdv_kernel<float, 128, 4, 1, 32, true, 1>"}
    spills = []
    for asm in (fwd_asm, bwd_asm):
        for k in diagnose.isa_stats(asm, "_kernelI").values():
            name = k["name"].replace("tattn::", "").split("(")[0].removeprefix("void ")
            if k.get("scratch_bytes_per_lane") and name not in allowed:
                spills.append((name, k["scratch_bytes_per_lane"]))
    assert not spills, spills
