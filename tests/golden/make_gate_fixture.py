"""Extracts the reference's accuracy-gate data into tests/golden/gate_fixture.json.

    python tests/golden/make_gate_fixture.py   (needs /root/reference; run once, output committed)

For each published run (v6e / TPU7x, 1B / 2B) it keeps, from the reference's own files:
  * the FP32-golden and BF16-reference top-20 (ids, logprobs) per scored sequence
    (benchmark/ref/{fp32,bf16}_8192_{1b,2b}_*.json -> "results"),
  * the candidate dumps of that run (results/gate/<run>_gate*.json.gz -> "results"), and
  * the gate reports the reference computed from them (results/<run>.json -> validation.logprob_gates),
dropping the 8,192-token prompt ids.  tests/test_gate.py recomputes the reports with minicpm5_mk.gate.
"""
import gzip
import json
import os

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gate_fixture.json")


def slim(results):
    return [{"batch_size": s["batch_size"], "seq_len": s["seq_len"],
             "seqs": [{"top_ids": q["top_ids"], "top_logprobs": q["top_logprobs"],
                       **({"sampled_nolp": q["sampled_nolp"]} if "sampled_nolp" in q else {})} for q in s["seqs"]]}
            for s in results]


def main():
    runs = []
    for chip in ("v6e", "tpu7x"):
        for m in ("1b", "2b"):
            run = f"{chip}_minicpm5_{m}"
            res = json.load(open(os.path.join(REF, "results", run + ".json")))
            gates = res["validation"]["logprob_gates"]
            refs = [json.load(open(os.path.join(REF, "benchmark", "ref", f"fp32_8192_{m}_golden_logprobs.json"))),
                    json.load(open(os.path.join(REF, "benchmark", "ref", f"bf16_8192_{m}_ref_logprobs.json")))]
            dumps = [json.load(gzip.open(os.path.join(REF, "results", "gate", run + "_gate.json.gz"))),
                     json.load(gzip.open(os.path.join(REF, "results", "gate",
                                                      f"{run}_gate__bf16_8192_{m}_ref_logprobs.json.gz")))]
            for ref, dump, gate in zip(refs, dumps, gates):
                runs.append({"run": run, "reference_label": ref.get("label"),
                             "ref_results": slim(ref["results"]),
                             "cand_inputs": [{k: v for k, v in st.items() if k != "prompt_token_ids"}
                                             for st in dump["inputs"]],
                             "cand_results": slim(dump["results"]),
                             "expected": {k: v for k, v in gate.items()
                                          if k not in ("reference", "reference_sha256", "reference_label")}})
    with open(OUT, "w") as f:
        json.dump({"source": "reference benchmark/ref, results/gate and results/*.json", "runs": runs}, f)
    print(OUT, os.path.getsize(OUT))


if __name__ == "__main__":
    main()
