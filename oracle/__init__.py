"""The oracle: a CPU restatement of the reference's algorithm for the MiniCPM5 prefill path.

TEST INFRASTRUCTURE ONLY.  Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import anything from this package, and only as the checker (or the timed CPU
baseline) -- never as the measured or shipped path.  The product (`minicpm5_mk` + `libmk.so`) does
not import it and fails loudly when its HIP library is missing.

  golden.py   FP32 forward, restating benchmark/f32_golden.py.
  emulate.py  the plugin's quantized numerics (W8A8 SmoothQuant linears, fused QKV / MLP algebra,
              attention rounding points, last-token-only last layer), restating
              plugin/minicpm5_mk/mk_jax.py, mk_mlp.py and mk_attn.py.

Pinning (what each function is checked against) is listed in each module's docstring and in the
tests that exercise it.
"""
