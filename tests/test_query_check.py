"""The host checks of the integrated memory query (tests/query_check.py) on the CPU: an fp32 computation with the
kernels' roundings and another summation order passes them, and the mistakes they exist to catch fail them -- a
swapped BatchNorm scale and shift, a BatchNorm applied to shifted columns, the affine on the wrong column block,
mixed-up sub-key halves.  Also the direct pins of oracle/torch_path.py's attention and RMSNorm against the
library routines (F.scaled_dot_product_attention, F.rms_norm)."""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle.torch_path as TP
import query_check as QC

M, C, NQ, V, EPS = 48, 384, 2048, 384, 1e-5


def bf(t):
    return t.bfloat16().double()


def make(seed=0):
    g = torch.Generator().manual_seed(seed)
    x = bf(torch.randn(M, C, generator=g))
    gam = bf(1 + 0.1 * torch.randn(C, generator=g))
    w = bf(torch.randn(NQ + V, C, generator=g) * 0.02)
    b = bf(torch.randn(NQ + V, generator=g) * 0.02)
    mean, var = torch.randn(NQ, generator=g) * 0.1, torch.rand(NQ, generator=g) * 1.5 + 0.5
    wt, bias = torch.rand(NQ, generator=g) + 0.5, torch.randn(NQ, generator=g) * 0.1
    scale = (torch.rsqrt(var + 1e-5) * wt).float()
    shift = (-mean * scale + bias).float()
    return x, gam, w, b, scale, shift


def kernel_like(x, gam, w, b, scale, shift, n_affine=NQ):
    """What the decode linear computes, in fp32 with torch's summation order and the kernels' roundings."""
    x32 = x.float()
    h = (x32 * torch.rsqrt((x32 * x32).mean(-1, keepdim=True) + EPS) * gam.float()).bfloat16().float()
    v = (h @ w.float().T + b.float()).bfloat16().float()
    q = (v[:, :n_affine] * scale[:n_affine] + shift[:n_affine]).bfloat16().float()
    return torch.cat([q, v[:, n_affine:]], 1)


def host(x, gam, w, b, scale, shift):
    h, herr = QC.rms_norm_bf16(x, gam, EPS)
    return QC.linear_bf16(h, w, b, scale, shift, n_affine=NQ, h_err=herr)


def test_kernel_like_query_passes():
    x, gam, w, b, scale, shift = make()
    ref, bound = host(x, gam, w, b, scale, shift)
    got = kernel_like(x, gam, w, b, scale, shift)
    eq = QC.check_close(got, ref, bound, "query")
    assert eq > 0.99


@pytest.mark.parametrize("mistake", ["swap_scale_shift", "shift_columns", "affine_on_swilu", "no_bias"])
def test_planted_query_mistakes_fail(mistake):
    x, gam, w, b, scale, shift = make(1)
    ref, bound = host(x, gam, w, b, scale, shift)
    if mistake == "swap_scale_shift":
        got = kernel_like(x, gam, w, b, shift, scale)
    elif mistake == "shift_columns":                      # the affine of column j applied to column j + 1
        got = kernel_like(x, gam, w, b, scale.roll(1), shift.roll(1))
    elif mistake == "affine_on_swilu":                    # BatchNorm on the swilu block, not the query block
        wq = torch.cat([w[NQ:], w[:NQ]])
        bq = torch.cat([b[NQ:], b[:NQ]])
        got = kernel_like(x, gam, wq, bq, scale, shift, n_affine=V)
        got = torch.cat([got[:, V:], got[:, :V]], 1)
    else:
        got = kernel_like(x, gam, w, torch.zeros_like(b), scale, shift)
    with pytest.raises(AssertionError):
        QC.check_close(got, ref, bound, "query")


def test_scores_check_and_planted_half_swap():
    g = torch.Generator().manual_seed(2)
    H, NK, half = 4, 256, 256
    q = bf(torch.randn(M, H, 2 * half, generator=g))
    keys = bf(torch.randn(H, 2, NK, half, generator=g) / 16)
    s1 = torch.einsum("mhd,hkd->mhk", q[..., :half].float(), keys[:, 0].float()).bfloat16()
    s2 = torch.einsum("mhd,hkd->mhk", q[..., half:].float(), keys[:, 1].float()).bfloat16()
    QC.check_scores(q, keys, s1, s2)
    with pytest.raises(AssertionError):
        QC.check_scores(q, keys, s2, s1)                  # halves exchanged
    with pytest.raises(AssertionError):
        QC.check_scores(q, keys.flip(0), s1, s2)          # heads in the wrong order


def test_rms_norm_matches_library():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 7, 48, generator=g, dtype=torch.float64)
    w = torch.rand(48, generator=g, dtype=torch.float64) + 0.5
    torch.testing.assert_close(TP.rms_norm(x, w, 1e-5), F.rms_norm(x, (48,), w, 1e-5), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("T,cached", [(9, 0), (1, 12), (5, 10)])
def test_attention_matches_sdpa(T, cached):
    """oracle/torch_path.attention (projection, RoPE, causal softmax attention over cache + chunk, output
    projection) against F.scaled_dot_product_attention on the same rotated q, k, v: causal for a prompt, all
    cached rows plus the causal part of the chunk otherwise."""
    g = torch.Generator().manual_seed(T * 100 + cached)
    B, H, hd = 2, 4, 16
    Cm = H * hd
    cfg = {"n_heads": H, "rope_theta": 10000.0}
    sd = {"a.wqkv.weight": torch.randn(3 * Cm, Cm, generator=g, dtype=torch.float64) * 0.2,
          "a.wo.weight": torch.randn(Cm, Cm, generator=g, dtype=torch.float64) * 0.2}
    xs = torch.randn(B, cached + T, Cm, generator=g, dtype=torch.float64)
    cache = {}
    if cached:
        TP.attention(sd, "a.", xs[:, :cached], cfg, cache, 0)
    got = TP.attention(sd, "a.", xs[:, cached:], cfg, cache, cached)
    qkv = (xs @ sd["a.wqkv.weight"].T).view(B, cached + T, 3, H, hd).permute(2, 0, 3, 1, 4)
    q = TP.rope(qkv[0], 0, 10000.0)[:, :, cached:]
    k, v = TP.rope(qkv[1], 0, 10000.0), qkv[2]
    S = cached + T
    mask = torch.ones(T, S, dtype=torch.bool).tril(S - T)
    y = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=1 / math.sqrt(hd))
    ref = y.transpose(1, 2).reshape(B, T, Cm) @ sd["a.wo.weight"].T
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    assert cache["k"].shape == (B, H, S, hd)
