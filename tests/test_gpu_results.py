"""The dashboard-format results (nkilab.results) measured on the GPU: every
field the reference's results.json carries, plausible timings, and the
correctness matrix within fp32 tolerance."""
import json
import math
import os

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

SCHEMA = json.load(open(os.path.join(ROOT, "tests", "golden", "results_schema.json")))


def test_collect_quick_matches_the_reference_schema(tmp_path):
    from nkilab import results as R

    res = R.collect(quick=True)
    assert R.schema_gaps(res, SCHEMA) == []
    text = json.dumps(res, allow_nan=False, default=float)  # finite numbers only
    assert json.loads(text)["hardware_model"]["hbm_bytes_per_s"] == 8.0e12
    for sec, key in (("matmul", "variants"), ("norm", "variants"), ("attention", "ladder")):
        for s in res[sec][key]:
            assert s["modeled_latency_us"] > 0 and s["latency_source"] == "measured", (sec, s["kernel"])
    assert all(s["rel_err_vs_torch"] < 1e-2 for s in res["attention"]["ladder"])
    assert all(s["rel_err_vs_numpy"] < 1e-2 for s in res["matmul"]["variants"])
    assert all(row["vs_torch"] < 1e-4 for row in res["correctness"]), res["correctness"]
    assert res["decoder_block"]["max_abs_err_vs_pytorch"] < 1e-3
    for name, tr in res["traces"].items():
        assert tr["events"] and all(0 <= e["t0"] < e["t1"] for e in tr["events"]), name
        assert math.isfinite(tr["latency_us"]) and tr["latency_us"] > 0
