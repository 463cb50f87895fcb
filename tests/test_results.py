"""CPU checks of the dashboard-format results writer (nkilab.results): the
summaries carry every field of the reference's results.json entries, kernel
names demangle, and rocprofv3 kernel traces become trace events."""
import json
import os

import pytest

from conftest import ROOT

SCHEMA = json.load(open(os.path.join(ROOT, "tests", "golden", "results_schema.json")))


def test_summary_has_every_reference_field():
    from nkilab import results as R

    s = R.summary("matmul blocked", 10.0, 6_291_456, 2 * 1024**3, compulsory=6_291_456,
                  extra={"rel_err_vs_numpy": 1e-3})
    for k in SCHEMA["matmul.variants[]"]:
        assert k in s, k
    assert s["latency_source"] == "measured"
    # 2 GFLOP in 10 us is 214.7 TFLOP/s; at 2.5166 PFLOP/s the bound is 0.853 us
    assert s["modeled_tflops"] == pytest.approx(214.748, rel=1e-4)
    assert s["roofline_regime"] == "compute"
    assert s["roofline_bound_us"] == pytest.approx(2 * 1024**3 / 2.5166e15 * 1e6)
    m = R.summary("softmax fused", 6.0, 33_554_432, 0)
    assert m["roofline_regime"] == "memory" and m["roofline_bound_us"] == pytest.approx(33_554_432 / 8e12 * 1e6)


def test_summary_takes_measured_counters():
    """With the kernel's counter entry, hbm_bytes is the measured traffic (the
    compulsory bytes stay beside it) and engine_busy_pct the MFMA busy share;
    without one, the computed bytes and an empty busy dict."""
    from nkilab import results as R

    s = R.summary("softmax fused", 6.0, 33_554_432, 0, compulsory=33_554_432,
                  counters={"bytes": 33_615_213, "mfma_busy": 0.0})
    assert s["hbm_bytes"] == 33_615_213 and s["compulsory_hbm_bytes"] == 33_554_432
    assert s["hbm_bytes_source"].startswith("measured")
    assert s["engine_busy_pct"] == {"mfma": 0.0}
    a = R.summary("flash", 24.0, 16_777_216, 8_598_323_200, counters={"bytes": 39_525_525, "mfma_busy": 0.1048})
    assert a["engine_busy_pct"] == {"mfma": 10.48}
    assert a["roofline_bound_us"] == pytest.approx(max(8_598_323_200 / 2.5166e15, 39_525_525 / 8e12) * 1e6)
    c = R.summary("swiglu fused", 9.0, 50_331_648, 0)
    assert c["hbm_bytes"] == 50_331_648 and c["hbm_bytes_source"].startswith("computed")
    assert c["engine_busy_pct"] == {}
    ctr = R.load_counters()
    assert ctr == {} or all(k in ctr for k in ("attention", "softmax", "matmul"))


def test_short_kernel_names():
    from nkilab.results import short_kernel_name as k

    assert k("_ZN3nkl17flash_bf16_kernelILi128ELi4ELi2EEEvNS_8AttnArgsENS_12_GLOBAL__N_14WorkE") == \
        "flash_bf16_kernel<128,4,2>"
    assert k("_ZN3nkl18softmax_vec_kernelIDF16bLi4EEEvPKT_PS1_iill") == "softmax_vec_kernel<bf16,4>"
    assert k("_ZN3nkl18rmsnorm_vec_kernelIDF16bDF16bLi4EEEvPKT_S3_PT0_iillff") == "rmsnorm_vec_kernel<bf16,bf16,4>"
    assert k("_ZN3nkl15gemm_dma_kernelIfLi128ELi128ELb1ELi4EEEvNS_8GemmArgsE") == "gemm_dma_kernel<float,128,128,1,4>"
    assert k("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"


def test_rocprof_kernel_trace_to_events(tmp_path):
    from nkilab.results import trace_events_from_rocprof

    f = tmp_path / "kernel_trace.csv"
    f.write_text(
        '"Kind","Agent_Id","Queue_Id","Stream_Id","Thread_Id","Dispatch_Id","Kernel_Id","Kernel_Name",'
        '"Correlation_Id","Start_Timestamp","End_Timestamp"\n'
        '"KERNEL_DISPATCH","Agent 1",1,0,9,2,7,"_ZN3nkl18softmax_vec_kernelIDF16bLi4EEEvPKT_PS1_iill",2,2000,8700\n'
        '"KERNEL_DISPATCH","Agent 1",1,0,9,1,7,"__amd_rocclr_copyBuffer",1,1000,1500\n')
    ev = trace_events_from_rocprof(str(f), {"softmax_vec_kernel<bf16,4>": (33_554_432, 0)})
    assert [e["op"] for e in ev] == ["__amd_rocclr_copyBuffer", "softmax_vec_kernel<bf16,4>"]
    assert ev[1] == {"op": "softmax_vec_kernel<bf16,4>", "lane": "queue 1", "t0": 1.0, "t1": 7.7,
                     "bytes": 33_554_432, "flops": 0}
    for e in ev:
        assert sorted(e) == SCHEMA["traces{}.events[]"]


def test_schema_gaps_finds_missing_keys():
    from nkilab import results as R

    full = {k: None for k in SCHEMA["top"]}
    gaps = R.schema_gaps(full, SCHEMA)
    assert "matmul.variants[] (empty)" in gaps and "traces.attention flash" in gaps and "hardware_model" in gaps
