"""Prefill throughput of the MI355X MiniCPM5 path: one JSON line (see --help).

A step is one whole-model prefill of B sequences x 8192 tokens (random-init weights of the named
architecture, seeded token ids already resident in HBM) through libmk: embedding -> L-1 W8A8 layers ->
last-token-only last layer -> final norm -> LM head logits, replayed from a captured hipGraph.
value = B * 8192 / mean step latency (tokens/s); p50 latency uses linear interpolation
(benchmark/run_benchmark.py:186-194, :437-440 of the reference).

Extra fields:
  roofline      the attention kernel (dominant kernel of the step) inside the model: after the timed
                loop one eager forward of the same shape runs with a HIP event pair around every launch
                on the model's stream (mk_forward_timed); achieved = algorithmic FLOPs per launch
                (4 hd n_q S(S+1)/2 per sequence and layer) / average launch time, peak = MI355X dense
                bf16 2.5 PFLOP/s.  roofline.attainable: the same against the MFMA-only rate this board
                sustains with random operands, measured live (mk_bench_mfma_peak): under MFMA load the
                shader clock falls to ~1.5-1.8 GHz (power limit), well below the 2.4 GHz of the peak.
  kernels       the same for every kernel category: QKV / gate-up GEMMs (int8 MFMA, peak 5.0 POP/s when
                quantised), O / down (bf16 unless quantised), the row kernels and the LM head (HBM GB/s).
  cpu_baseline  the oracle's FP32 CPU forward (oracle/golden.py, a restatement of the reference's
                FP32 golden) of --cpu-batch whole 8192-token sequences (default 1) of the main
                architecture with every host thread: one warm-up of the first layer, then --cpu-runs
                timed runs (median).  `per_batch` gives tokens/s and ms at B = 1..32: the timed batch,
                and the others as a linear extrapolation from it, labelled as such (the FP32 path runs
                one sequence at a time, as the reference's golden does).
  sweep         the metric's other points: tokens/s, mean and p50 latency at (B, 8192) for each
                (architecture, B) of --sweep (default: 1B at B = 4..32, 2B and 1B-hd96 at B = 1..32),
                each with `roofline_ms`, the whole model's bound at MI355X's published peaks (every linear
                at its operand type's dense MFMA peak, causal attention at the bf16 peak, the LM head's
                weight read at HBM bandwidth), and `frac_roofline` = roofline_ms / mean latency.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "minicpm5-vllm-tpu_amd")]

PEAK = {"bf16": 2516.6, "int8": 5033.2, "fp8": 5033.2, "hbm": 8000.0}   # MI355X dense TFLOP/s, TOP/s; HBM GB/s
METRIC = "prefill tokens/sec at (B,8192) B=1..32, 1B and 2B arch; p50 ms at (1,8192)"
# HBM bytes per attn_fwd_kernel launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by a
# 256 MiB copy's counters) for the default workload; (arch, B, S, quant) -> (bytes, source file)
ATTN_TRAFFIC = {("1b", 1, 8192, "auto"): (77.1e6 + 33.6e6, "profiles/mfma_util_hbm_1b_b1_s8192.txt"),
                ("2b", 1, 8192, "auto"): (77.2e6 + 33.6e6, "profiles/mfma_util_hbm_2b_b1_s8192.txt")}
DEFAULT_SWEEP = "1b:4,8,16,32;2b:1,4,8,16,32;1b-hd96:1,4,8,16,32"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pctl(xs, q):
    xs = sorted(xs)
    if len(xs) == 1:
        return xs[0]
    k = (len(xs) - 1) * q / 100.0
    f = math.floor(k)
    c = min(f + 1, len(xs) - 1)
    return xs[f] + (xs[c] - xs[f]) * (k - f)


def flops_reference(cfg, bs, seq):
    """verify_results.py:131-140: all L layers over the full sequence + causal attention + head."""
    qkv = cfg.hidden * (cfg.n_q + 2 * cfg.n_kv) * cfg.head_dim
    o = cfg.n_q * cfg.head_dim * cfg.hidden
    gu = cfg.hidden * 2 * cfg.inter
    dn = cfg.inter * cfg.hidden
    lin = 2 * (qkv + o + gu + dn) * cfg.num_layers * bs * seq
    attn = cfg.num_layers * bs * 2 * seq * seq * cfg.head_dim * cfg.n_q
    return lin + attn + 2 * cfg.hidden * cfg.vocab * bs


def roofline_ms(cfg, quant, bs, seq):
    """Lower bound of one (bs, seq) prefill at MI355X's published peaks: the plugin's actual work --
    L-1 full-sequence layers (each linear at its operand type's dense MFMA peak, causal attention
    4 hd n_q S(S+1)/2 at the bf16 peak), the last layer's K/V projection over S tokens (bf16), and the
    LM head's bf16 weight read at HBM bandwidth; the last-token GEMVs are negligible."""
    from minicpm5_mk.quant import parse_quant

    qm = parse_quant(quant)
    T = bs * seq
    H, I, hd, nq, nkv = cfg.hidden, cfg.inter, cfg.head_dim, cfg.n_q, cfg.n_kv
    lin = {"qkv": 2.0 * T * H * (nq + 2 * nkv) * hd, "o": 2.0 * T * nq * hd * H, "gu": 2.0 * T * H * 2 * I,
           "down": 2.0 * T * I * H}
    peak = lambda k: PEAK["bf16" if qm[k] == "bf16" else "int8"] * 1e12  # noqa: E731
    layer = sum(f / peak(k) for k, f in lin.items()) + 4.0 * hd * nq * seq * (seq + 1) / 2 * bs / (PEAK["bf16"] * 1e12)
    last = 2.0 * T * H * 2 * nkv * hd / (PEAK["bf16"] * 1e12)
    head = 2.0 * cfg.vocab * H / (PEAK["hbm"] * 1e9)
    return ((cfg.num_layers - 1) * layer + last + head) * 1e3


def time_steps(eng, ids, steps, warmup):
    import torch

    B, S = ids.shape
    flat = ids.reshape(-1)
    for _ in range(warmup):
        eng.model.forward(flat, B, S, logits=True, copy_out=False)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        eng.model.forward(flat, B, S, logits=True, copy_out=False)
        b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    lat = [a.elapsed_time(b) for a, b in ev]
    return wall, lat


def kernel_roofline(cfg, B, S, iters=20):
    """Times the attention kernel and the layer GEMMs alone at the step's shapes (HIP events)."""
    import ctypes

    import torch

    from minicpm5_mk import _lib
    from minicpm5_mk.mk_weights import rope_tables

    lib = _lib.load()
    dev = torch.device("cuda:0")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    hd, nq, nkv, H, I = cfg.head_dim, cfg.n_q, cfg.n_kv, cfg.hidden, cfg.inter
    D = (nq + 2 * nkv) * hd
    g = torch.Generator(device=dev).manual_seed(0)
    qkv = torch.randn(B, S, D, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = (t.to(dev) for t in rope_tables(S, hd, cfg.rope_theta))
    out = torch.empty(B, S, nq * hd, dtype=torch.bfloat16, device=dev)
    nb = int(lib.mk_attn_scratch_bytes(B, S, nkv, hd))
    scratch = torch.empty(nb, dtype=torch.uint8, device=dev)
    ms = ctypes.c_float()
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    _lib.check(lib.mk_bench_attn(P(qkv), P(cos), P(sin), P(out), P(scratch), nb, B, S, nq, nkv, hd,
                                 1.0 / math.sqrt(hd), iters, st, ctypes.byref(ms)), "mk_bench_attn")
    attn_ms = ms.value
    attn_flop = 4.0 * hd * nq * S * (S + 1) / 2 * B
    res = {"attention": {"ms": attn_ms, "flop": attn_flop, "tflops": attn_flop / attn_ms / 1e9,
                         "peak": PEAK["bf16"]}}
    del qkv, out, scratch
    T = B * S

    def bench_gemm(name, is8, epi, M, N, K, silu=False, resid=False):
        dt = torch.int8 if is8 else torch.bfloat16
        if is8:
            A = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
            Bm = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        else:
            A = torch.randn(M, K, generator=g, device=dev).to(dt)
            Bm = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(dt)
        rs = torch.rand(M, generator=g, device=dev) * 1e-3
        cs = torch.rand(N, generator=g, device=dev) * 1e-3
        nout = N // 2 if silu else N
        o = None if resid else torch.empty(M, nout, dtype=torch.bfloat16, device=dev)
        r = torch.zeros(M, N, dtype=torch.bfloat16, device=dev) if resid else None
        _lib.check(lib.mk_bench_gemm(int(is8), _lib.EPI[epi], P(A), K, P(Bm), K, M, N, K, P(o), nout if o is not None
                                     else 0, P(r), N if r is not None else 0, P(rs), P(cs), None, iters, st,
                                     ctypes.byref(ms)), "mk_bench_gemm")
        fl = 2.0 * M * N * K
        res[name] = {"ms": ms.value, "flop": fl, "tflops": fl / ms.value / 1e9,
                     "peak": PEAK["int8" if is8 else "bf16"]}

    bench_gemm("qkv_int8", True, "dq_bf16", T, D, H)
    bench_gemm("gate_up_int8", True, "dq_silu", T, 2 * I, H, silu=True)
    bench_gemm("o_bf16", False, "res_bf16add", T, H, nq * hd, resid=True)
    bench_gemm("down_bf16", False, "res_f32add", T, H, I, resid=True)
    for v in res.values():
        v["frac"] = v["tflops"] / v["peak"]
    return res


def model_roofline(eng, cfg, ids):
    """Per-kernel-category time of one eager forward (mk_forward_timed) -> achieved rate vs MI355X peak."""
    from minicpm5_mk.quant import parse_quant

    B, S = ids.shape
    T = B * S
    H, I, hd, nq, nkv, V = cfg.hidden, cfg.inter, cfg.head_dim, cfg.n_q, cfg.n_kv, cfg.vocab
    qm = parse_quant(eng.quant)
    prec = {k: ("bf16" if v == "bf16" else "fp8" if v.startswith("fp8") else "int8") for k, v in qm.items()}
    i8 = {k: v != "bf16" for k, v in prec.items()}   # 8-bit linears: TOP/s against the int8 / fp8 peak
    flat = ids.reshape(-1)
    eng.model.forward_timed(flat, B, S, logits=True)          # first eager pass: code objects, caches
    t = eng.model.forward_timed(flat, B, S, logits=True)
    work = {   # kind -> (algorithmic units per launch, unit, peak)
        "attn": (4.0 * hd * nq * S * (S + 1) / 2 * B, "TFLOP/s", PEAK["bf16"]),
        "gemm_qkv": (2.0 * T * H * (nq + 2 * nkv) * hd, "TOP/s" if i8["qkv"] else "TFLOP/s", PEAK[prec["qkv"]]),
        "gemm_o": (2.0 * T * nq * hd * H, "TOP/s" if i8["o"] else "TFLOP/s", PEAK[prec["o"]]),
        "gemm_gu": (2.0 * T * H * 2 * I, "TOP/s" if i8["gu"] else "TFLOP/s", PEAK[prec["gu"]]),
        "gemm_down": (2.0 * T * I * H, "TOP/s" if i8["down"] else "TFLOP/s", PEAK[prec["down"]]),
        # K and V read and written once: 4 S kv_dim bf16 bytes per sequence
        "attn_prep": (4.0 * T * nkv * hd * 2, "GB/s", PEAK["hbm"]),
        # per-token int8 quantisation of an H-wide bf16 row: 2 H read, H written, 4 B scale
        "norm": (T * (3.0 * H + 4), "GB/s", PEAK["hbm"]),
        "lm_head": (2.0 * V * H, "GB/s", PEAK["hbm"]),        # the bf16 weight read
    }
    out = {}
    for k, (ms, n) in t.items():
        if n == 0:
            continue
        e = {"avg_us": round(ms * 1e3 / n, 2), "launches": n, "total_ms": round(ms, 3)}
        if k in work:
            units, unit, peak = work[k]
            rate = units / (ms / n) / (1e6 if unit == "GB/s" else 1e9)   # units per ms -> GB/s or T(FL)OP/s
            e.update({"achieved": round(rate, 1), "unit": unit, "peak": peak, "frac": round(rate / peak, 4)})
        out[k] = e
    return out


def attainable_peaks(iters=3000):
    """MFMA-only throughput with random operands (mk_bench_mfma_peak) at 1 and 2 waves per SIMD: the
    rate this board sustains under its power limit, in T(FL)OP/s, with the shader clock it ran at."""
    import ctypes

    import torch

    from minicpm5_mk import _lib

    lib = _lib.load()
    nbytes = lib.mk_mfma_peak_scratch_bytes(2)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for name, in_type in (("bf16", 0), ("int8", 1)):
        best = None
        for waves in (1, 2):
            rate, clk = ctypes.c_double(), ctypes.c_double()
            _lib.check(lib.mk_bench_mfma_peak(in_type, waves, iters, ctypes.c_void_p(scratch.data_ptr()), nbytes, st,
                                              ctypes.byref(rate), ctypes.byref(clk)), "mk_bench_mfma_peak")
            r = {"rate": round(rate.value / 1e12, 1), "clock_ghz": round(clk.value, 3), "waves_per_simd": waves}
            if best is None or r["rate"] > best["rate"]:
                best = r
        out[name] = best
    return out


def cpu_baseline(cfg, runs, seq=8192, batch=1):
    """The oracle's FP32 forward (restating benchmark/f32_golden.py) of `batch` whole `seq`-token
    sequences, one after another, with every host thread: one untimed warm-up over the first layer, then
    `runs` timed runs (embedding, all L layers, final norm, LM head per sequence); value =
    batch * seq / median time."""
    import torch

    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import golden

    torch.set_num_threads(os.cpu_count() or 1)
    t0 = time.perf_counter()
    W = golden.load_f32(random_hf_state_dict(cfg), cfg)
    t_load = time.perf_counter() - t0
    ids = random_token_ids(batch, seq)
    cos, sin = golden.rope_tables(seq, cfg.head_dim, cfg.rope_theta)
    golden.forward_one(ids[0], W, cfg.replace(num_layers=1), cos, sin)      # warm-up: one layer
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for b in range(batch):
            golden.forward_one(ids[b], W, cfg, cos, sin)
        times.append(time.perf_counter() - t0)
    med = pctl(times, 50)
    tps = batch * seq / med
    per_batch = []
    for b in sorted({1, 4, 8, 16, 32, batch}):
        per_batch.append({"batch": b, "tokens_per_s": round(tps, 1), "p50_ms": round(med * 1e3 * b / batch, 1),
                          "timed": b == batch,
                          **({} if b == batch else {"extrapolated_from_batch": batch})})
    what = f"one whole {seq}-token sequence" if batch == 1 else f"{batch} whole {seq}-token sequences"
    return {"value": round(tps, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle FP32 forward (oracle/golden.py) of {what} of {cfg.name} "
                      f"({cfg.num_layers} layers + final norm + LM head each), {runs} timed runs after a one-layer "
                      f"warm-up: {', '.join(f'{t:.1f}' for t in times)} s (median {med:.1f} s); weights "
                      f"generated and upcast in {t_load:.1f} s (untimed)",
            "batch": batch, "per_batch": per_batch, "cpu_model": _cpu_model()}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # the reference harness's method: 5 untimed + 50 timed forwards per shape (run_benchmark.py:39, 92-93)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--arch", default="1b", help="1b (hd 128, reference HF config) | 1b-hd96 | 2b")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seq", type=int, default=8192)
    ap.add_argument("--quant", default="auto")
    ap.add_argument("--sweep", default=DEFAULT_SWEEP,
                    help="extra (architecture, batch) rows: 'arch:B,B;arch:B' ('B,B' = the --arch architecture; "
                         "'' = none)")
    ap.add_argument("--cpu-runs", type=int, default=2, help="timed full CPU forwards of the baseline (0 = skip)")
    ap.add_argument("--cpu-batch", type=int, default=1, help="sequences per timed CPU baseline run")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the per-kernel timing loops + a 256 MiB device copy (rocprofv3 --pmc calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (data- and "
              "sequence-parallel sharding over several GPUs is not built)", file=sys.stderr)
        sys.exit(2)

    import torch

    from minicpm5_mk.config import preset
    from minicpm5_mk.engine import MkEngine
    from minicpm5_mk.synth import random_token_ids

    cfg = preset(args.arch)
    main_arch = args.arch
    if args.kernels_only:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda:0")   # 256 MiB read + 256 MiB written
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        kern = kernel_roofline(cfg, args.batch, args.seq, iters=max(1, args.steps))
        print(json.dumps({"kernels": kern, "copy_bytes_each_way": src.numel() * 4}), flush=True)
        return
    t0 = time.perf_counter()
    eng = MkEngine(cfg, quant=args.quant, max_model_len=max(8256, args.seq + 64), log=log)
    log(f"[bench] engine built in {time.perf_counter() - t0:.1f}s quant={eng.quant}")

    def run(eng, c, B, steps, warmup):
        ids = random_token_ids(B, args.seq, seed=1234).to("cuda:0")
        wall, lat = time_steps(eng, ids, steps, warmup)
        mean = sum(lat) / len(lat)
        bound = roofline_ms(c, eng.quant, B, args.seq)
        return {"arch": c.name, "batch": B, "tokens_per_s": B * args.seq / (mean / 1e3), "mean_ms": mean,
                "p50_ms": pctl(lat, 50), "p90_ms": pctl(lat, 90), "wall_ms_per_step": wall, "steps": steps,
                "roofline_ms": bound, "frac_roofline": bound / mean,
                "tflops_reference_formula": flops_reference(c, B, args.seq) / (mean / 1e3) / 1e12}

    main_run = run(eng, cfg, args.batch, args.steps, args.warmup)
    log(f"[bench] {cfg.name} B={args.batch}: {main_run}")
    kern = attain = None
    if not args.no_kernels:
        kern = model_roofline(eng, cfg, random_token_ids(args.batch, args.seq, seed=1234).to("cuda:0"))
        log(f"[bench] in-model kernels: {json.dumps(kern)}")
        attain = attainable_peaks()
        log(f"[bench] MFMA-only random-operand throughput on this board: {attain}")
        for k, e in kern.items():
            if "peak" in e and e["unit"] != "GB/s":
                ap_ = attain["bf16" if e["unit"] == "TFLOP/s" else "int8"]["rate"]
                e["attainable"] = ap_
                e["frac_attainable"] = round(e["achieved"] / ap_, 4)
    rows = {}
    for part in [p for p in (args.sweep or "").split(";") if p.strip()]:
        arch, bs = part.split(":", 1) if ":" in part else (args.arch, part)
        rows.setdefault(arch.strip(), []).extend(int(x) for x in bs.split(",") if x.strip())
    sweep = []
    for arch, batches in rows.items():
        if arch != args.arch:
            eng.model.release_buffers()
            eng.close()
            del eng
            torch.cuda.empty_cache()
            c = preset(arch)
            t0 = time.perf_counter()
            eng = MkEngine(c, quant=args.quant, max_model_len=max(8256, args.seq + 64), log=log)
            log(f"[bench] {arch} engine built in {time.perf_counter() - t0:.1f}s quant={eng.quant}")
            args.arch, cfg_now = arch, c
        else:
            cfg_now = preset(arch)
        for b in batches:
            r = run(eng, cfg_now, b, max(3, min(args.steps, int(80 / b))), 1)
            log(f"[bench] sweep {arch} B={b}: {r}")
            sweep.append(r)
            eng.model.release_buffers()
    eng.model.release_buffers()
    eng.close()
    del eng
    torch.cuda.empty_cache()
    cpu = cpu_baseline(cfg, args.cpu_runs, args.seq, args.cpu_batch) if args.cpu_runs > 0 else None
    if cpu:
        log(f"[bench] cpu baseline: {cpu}")

    out = {
        "metric": METRIC, "value": round(main_run["tokens_per_s"], 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(main_run["mean_ms"], 4),
        "p50_ms": round(main_run["p50_ms"], 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8+bf16" if args.quant != "bf16" else "bf16",
        "data": "synthetic: random-init N(0,0.02) weights (seed 0), token ids U[1000,30000) (seed 1234)",
        "config": {"workload": f"{cfg.name} prefill/scoring ({args.batch},{args.seq}), last-token logits",
                   "arch": cfg.name, "batch": args.batch, "seq_len": args.seq, "head_dim": cfg.head_dim,
                   "quant": args.quant, "parallelism": "single GPU"},
        "tflops_reference_formula": round(main_run["tflops_reference_formula"], 1),
        "roofline_ms": round(main_run["roofline_ms"], 3), "frac_roofline": round(main_run["frac_roofline"], 4),
    }
    if kern:
        a = kern["attn"]
        traffic = ATTN_TRAFFIC.get((main_arch, args.batch, args.seq, args.quant))
        out["roofline"] = {"bound": "mfma", "achieved": a["achieved"], "peak": a["peak"], "unit": a["unit"],
                           "frac": a["frac"],
                           "traffic": traffic[0] if traffic else None,
                           "traffic_source": (f"{traffic[1]}: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this "
                                              "workload, scaled by a 256 MiB copy's counters") if traffic else
                           "not measured for this workload",
                           "kernel": "attn_fwd_kernel",
                           "avg_ms": round(a["avg_us"] / 1e3, 4), "timing": "in-model, HIP events per launch",
                           "attainable": {"peak": attain["bf16"]["rate"], "frac": a["frac_attainable"],
                                          "clock_ghz": attain["bf16"]["clock_ghz"],
                                          "how": "MFMA-only kernel, random operands, measured live (mk_bench_mfma_peak)"}}
        out["kernels"] = kern
    if cpu:
        out["cpu_baseline"] = cpu
    if sweep:
        out["sweep"] = [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()} for r in sweep]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
