"""bench.py's host side on the CPU: the one-GPU contract, the percentile the reference harness reports,
and the HBM traffic figures the roofline line quotes against the committed counter summaries."""
import importlib.util
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_host_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    """`--gpus N` with N > 1 exits with status 2 and says why, before touching a GPU."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_percentile_is_numpys_linear_method():
    """p50 / p90 as the reference harness computes them (benchmark/run_benchmark.py:186-194: linear
    interpolation between closest ranks, numpy's default), pinned against numpy itself."""
    pctl = _bench().pctl
    rng = np.random.default_rng(5)
    for n in (1, 2, 3, 7, 20, 50, 51):
        xs = list(rng.uniform(10.0, 20.0, n))
        for q in (0, 10, 50, 90, 95, 99, 100):
            assert abs(pctl(xs, q) - float(np.percentile(xs, q))) < 1e-12, (n, q)


def test_attention_traffic_matches_the_counter_summaries():
    """The roofline line's `traffic` for the attention kernel is the FETCH_SIZE + WRITE_SIZE row of the
    summary it names (read MB + write MB of attn_fwd_kernel in that file)."""
    traffic = _bench().ATTN_TRAFFIC
    assert traffic
    for (arch, B, S, quant), (nbytes, src) in traffic.items():
        text = open(os.path.join(ROOT, src)).read()
        row = next(l for l in text.splitlines() if l.startswith("void attn_fwd_kernel<128, false, 8>"))
        toks = row.split()   # ... n avg_us clock MFMA readMB writeMB minMB GB/s
        read_mb, write_mb = float(toks[-4]), float(toks[-3])
        assert abs(nbytes - (read_mb + write_mb) * 1e6) < 1e3, (arch, src, row)
