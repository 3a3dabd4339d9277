"""The gate metrics (minicpm5_mk.gate) reproduce the reference's own recorded gate reports.

Known-answer test: tests/golden/gate_fixture.json holds, for the 4 published runs (v6e / TPU7x x
1B / 2B) and both references (FP32 golden, BF16 plugin path), the reference top-20 fixtures, the
candidate dumps, and the reports the reference harness computed from them
(results/*.json validation.logprob_gates; extracted by tests/golden/make_gate_fixture.py).
"""
import json
import math
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _runs():
    with open(os.path.join(HERE, "golden", "gate_fixture.json")) as f:
        return json.load(f)["runs"]


@pytest.mark.parametrize("idx", range(8))
def test_gate_reports_match_reference(idx):
    from minicpm5_mk.gate import score_run

    r = _runs()[idx]
    rep = score_run(r["ref_results"], r["cand_inputs"], r["cand_results"])
    for k, v in r["expected"].items():
        assert rep[k] == v, (r["run"], r["reference_label"], k, rep[k], v)


def test_gate_identity_and_verdicts():
    from minicpm5_mk.gate import compare_gate

    seq = {"top_ids": list(range(20)), "top_logprobs": [-1.0 - 0.1 * i for i in range(20)]}
    s = [{"batch_size": 1, "seq_len": 8, "seqs": [seq]}]
    rep = compare_gate(s, s)
    assert rep["gate_v2"] == "PASS" and rep["mean_abs_dlogprob"] == 0 and rep["kl_top20_mean"] == 0
    assert math.isclose(rep["cos_logprob_mean"], 1.0)
    shifted = {"top_ids": seq["top_ids"], "top_logprobs": [x - 0.12 for x in seq["top_logprobs"]]}
    rep = compare_gate(s, [{"batch_size": 1, "seq_len": 8, "seqs": [shifted]}])
    assert rep["gate_v2"] == "JUDGE" and abs(rep["mean_abs_dlogprob"] - 0.12) < 1e-9
    flipped = {"top_ids": [5] + [i for i in range(20) if i != 5], "top_logprobs": seq["top_logprobs"]}
    rep = compare_gate(s, [{"batch_size": 1, "seq_len": 8, "seqs": [flipped]}])
    assert rep["top1_agreement"] == 0.0 and rep["top1_tie_aware"] == 0.0 and rep["gate_v2"] == "FAIL"
