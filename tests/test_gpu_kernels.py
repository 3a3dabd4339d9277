"""Per-kernel parity of libmk's HIP kernels against the oracle (GPU; calls go through the C ABI).

  * attention (super_gqa_v2 numerics): vs the FP32 reference attention.  Tolerance: max |err| <= 0.02,
    mean |err| <= 5e-4 -- about 2x the error of the oracle's own bf16-rounding emulation of the same
    kernel (0.0093 / 2.3e-4 at S = 1024..4096, hd 96), and below the TPU reference's own rounding
    (0.013 / 3.0e-4 with its bf16 exp2 and bf16 RoPE products).
  * row quantisation: bit-exact int8 and f32 scales (same f32 operations).
  * int8 GEMM: bit-exact int32 accumulators (exact integer arithmetic), dequant epilogues within
    1 bf16 ulp of the oracle (f32 products identical up to the row scale's last bit).
  * bf16 GEMM: f32 accumulation in a different order than the CPU: relative error <= 1e-2 of the
    output scale, bf16 rounding of the result dominating.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _dev():
    assert torch.cuda.is_available(), "GPU test needs a visible MI355X"
    return torch.device("cuda:0")


def _attn_inputs(B, S, hd, n_q=16, n_kv=2):
    gens = [torch.Generator().manual_seed(i) for i in range(3)]
    q = torch.randn(B, S, n_q * hd, generator=gens[0])
    k = torch.randn(B, S, n_kv * hd, generator=gens[1])
    v = torch.randn(B, S, n_kv * hd, generator=gens[2])
    return torch.cat([q, k, v], -1).to(BF16)


@pytest.mark.parametrize("B,S,hd,theta", [(1, 256, 64, 1e4), (2, 512, 96, 1e4), (1, 1024, 128, 5e6),
                                           (1, 8192, 96, 1e4), (1, 8192, 128, 5e6)])
def test_attention_vs_fp32(B, S, hd, theta):
    from minicpm5_mk import ops
    from minicpm5_mk.mk_weights import rope_tables
    from oracle import emulate

    dev = _dev()
    print(f"[attn] B={B} S={S} hd={hd}", flush=True)
    qkv = _attn_inputs(B, S, hd)
    cos, sin = rope_tables(S, hd, theta)
    sm = 1.0 / math.sqrt(hd)
    out = ops.attn_prefill(qkv.to(dev), cos.to(dev), sin.to(dev), 16, 2, hd, sm_scale=sm)
    torch.cuda.synchronize()
    out = out.float().cpu()
    ref = emulate.attention_fp32(qkv, cos, sin, 16, 2, hd, sm)
    err = (out - ref).abs()
    print(f"[attn] max {err.max():.4g} mean {err.mean():.4g}", flush=True)
    assert torch.isfinite(out).all()
    assert err.max() <= 0.02 and err.mean() <= 5e-4, (float(err.max()), float(err.mean()))


def test_attention_deterministic():
    from minicpm5_mk import ops
    from minicpm5_mk.mk_weights import rope_tables

    dev = _dev()
    qkv = _attn_inputs(1, 2048, 128).to(dev)
    cos, sin = (t.to(dev) for t in rope_tables(2048, 128, 5e6))
    a = ops.attn_prefill(qkv, cos, sin, 16, 2, 128)
    b = ops.attn_prefill(qkv, cos, sin, 16, 2, 128)
    assert torch.equal(a, b)


@pytest.mark.parametrize("T,H,norm,recip,f32", [(300, 1536, True, True, False), (64, 2048, False, False, False),
                                                (129, 4608, False, True, True), (8192, 1536, True, True, False)])
def test_row_quant_bitexact(T, H, norm, recip, f32):
    from minicpm5_mk import ops
    from oracle import emulate

    dev = _dev()
    g = torch.Generator().manual_seed(T + H)
    x = torch.randn(T, H, generator=g) * 3
    x[0, :7] = 0.0
    x = x if f32 else x.to(BF16)
    a = torch.rand(H, generator=g) + 0.5
    q, sx = ops.row_quant(x.to(dev), a.to(dev), 1e-6, norm, recip)
    qr, sxr = emulate.row_quant(x.float(), a, 1e-6, norm, recip)
    assert torch.equal(q.cpu(), qr)
    if norm:   # rstd: different summation order of mean(x^2) -> a few f32 ulps
        torch.testing.assert_close(sx.cpu(), sxr, rtol=4e-7, atol=0)
    else:
        assert torch.equal(sx.cpu(), sxr)


@pytest.mark.parametrize("M,N,K", [(256, 128, 64), (300, 200, 1536), (8192, 1920, 1536), (1000, 1536, 4608)])
def test_gemm_int8_exact(M, N, K):
    from minicpm5_mk import ops
    from oracle import emulate

    dev = _dev()
    g = torch.Generator().manual_seed(M * 7 + N)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    acc = ops.gemm(a.to(dev), b.to(dev), "i32").cpu()
    ref = emulate.int_matmul(a, b.t().contiguous())
    assert torch.equal(acc.to(torch.int64), ref)


def test_gemm_int8_skinny_exact():
    from minicpm5_mk import ops
    from oracle import emulate

    dev = _dev()
    g = torch.Generator().manual_seed(5)
    for M in (1, 7, 32):
        a = torch.randint(-127, 128, (M, 2048), generator=g, dtype=torch.int8)
        b = torch.randint(-127, 128, (4096 + 96, 2048), generator=g, dtype=torch.int8)
        acc = ops.gemm(a.to(dev), b.to(dev), "i32").cpu()
        assert torch.equal(acc.to(torch.int64), emulate.int_matmul(a, b.t().contiguous()))


def test_fused_qkv_epilogue():
    """fused_qkv (mk_mlp.py:161-170) through row_quant + int8 GEMM with the DQ epilogue."""
    from minicpm5_mk import ops
    from oracle import emulate

    dev = _dev()
    g = torch.Generator().manual_seed(11)
    T, H, D = 1024, 1536, 2560
    x = torch.randn(T, H, generator=g).to(BF16)
    w = torch.randint(-127, 128, (H, D), generator=g, dtype=torch.int8)
    s_w = torch.rand(D, generator=g) * 1e-3
    a = torch.rand(H, generator=g) + 0.5
    q, sx = ops.row_quant(x.to(dev), a.to(dev), 1e-6, True, True)
    out = ops.gemm(q, w.t().contiguous().to(dev), "dq_bf16", rs=sx, cs=s_w.to(dev)).float().cpu()
    ref = emulate.fused_qkv(x, w, s_w, a, 1e-6).float()
    ulp = ref.abs().clamp(min=1e-30) * 2.0 ** -7
    assert ((out - ref).abs() <= ulp).all()


@pytest.mark.parametrize("M,N,K", [(512, 1536, 2048), (8192, 1536, 4608), (100, 512, 1536)])
def test_gemm_bf16(M, N, K):
    from minicpm5_mk import ops

    dev = _dev()
    g = torch.Generator().manual_seed(M + K)
    a = torch.randn(M, K, generator=g).to(BF16)
    b = (torch.randn(N, K, generator=g) * 0.02).to(BF16)
    out = ops.gemm(a.to(dev), b.to(dev), "f32").cpu()
    ref = a.float() @ b.float().t()
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4 * ref.abs().max().item())
    outb = ops.gemm(a.to(dev), b.to(dev), "bf16").float().cpu()
    assert ((outb - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-3 * ref.abs().max()).all()


def test_gemm_residual_epilogues():
    from minicpm5_mk import ops

    dev = _dev()
    g = torch.Generator().manual_seed(3)
    M, N, K = 512, 256, 512
    a = torch.randn(M, K, generator=g).to(BF16)
    b = (torch.randn(N, K, generator=g) * 0.05).to(BF16)
    x = torch.randn(M, N, generator=g).to(BF16)
    acc = ops.gemm(a.to(dev), b.to(dev), "f32").cpu()
    r1 = ops.gemm(a.to(dev), b.to(dev), "res_bf16add", res=x.clone().to(dev)).cpu()
    exp1 = (x.float() + acc.to(BF16).float()).to(BF16)
    assert torch.equal(r1, exp1)
    r2 = ops.gemm(a.to(dev), b.to(dev), "res_f32add", res=x.clone().to(dev)).cpu()
    exp2 = (x.float() + acc).to(BF16)
    assert torch.equal(r2, exp2)


def test_gate_up_silu_epilogue():
    """fused_mlp gate/up (mk_mlp.py:79-84): packed 32-interleave, h = silu(g) * u."""
    from minicpm5_mk import ops
    from minicpm5_mk.mk_weights import interleave_gu, mlp_chunk
    from oracle import emulate

    dev = _dev()
    g = torch.Generator().manual_seed(21)
    T, H, inter = 640, 1536, 4608
    x = torch.randn(T, H, generator=g).to(BF16)
    w = torch.randint(-127, 128, (H, 2, inter), generator=g, dtype=torch.int8)
    s = torch.rand(2, inter, generator=g) * 2e-3
    a = torch.rand(H, generator=g) + 0.5
    ic = mlp_chunk(inter)
    w_il, s_il = interleave_gu(w, s, ic)                       # reference layout (H, 2I), (1, 2I)
    wp = ops.pack_weight(w_il.to(dev), map_gu=True, ic=ic, inter=inter)     # (2I, H) packed
    # scales in packed order: row p <- reference column map(p)
    p = torch.arange(2 * inter)
    blk, half, n = p // 64, (p // 32) % 2, (p // 64) * 32 + p % 32
    src = (n // ic) * 2 * ic + half * ic + n % ic
    s_p = s_il.reshape(-1)[src].contiguous()
    q, sx = ops.row_quant(x.to(dev), a.to(dev), 1e-6, True, True)
    h = ops.gemm(q, wp, "dq_silu", rs=sx, cs=s_p.to(dev)).float().cpu()
    qr, sxr = emulate.row_quant(x.float(), a, 1e-6, True, True)
    gu = (emulate.int_matmul(qr, w.reshape(H, -1)).float() * sx.cpu()[:, None]) * s.reshape(1, -1)
    ref = emulate.silu_f32(gu[:, :inter]) * gu[:, inter:]
    err = (h - ref).abs()
    assert (err <= ref.abs() * 2.0 ** -7 + 1e-6).all(), float(err.max())


def test_lm_head():
    from minicpm5_mk import ops

    dev = _dev()
    g = torch.Generator(device=dev).manual_seed(9)
    w = (torch.randn(130560, 1536, generator=g, device=dev) * 0.02).to(BF16)
    for B in (1, 5, 40):
        hdn = torch.randn(B, 1536, generator=g, device=dev).to(BF16)
        out = ops.lm_head(hdn, w)
        ref = hdn.float() @ w.float().t()          # f32 torch reference for a floating-point kernel
        torch.testing.assert_close(out, ref, rtol=1e-4, atol=2e-4)
