"""Prefill attention kernel (smlm_prefill_attention) against fp64 / fp32 CPU attention of the same bf16 inputs:
the causal F.scaled_dot_product_attention of smlm/model.py:97-105 (S == T) and its masked form for new tokens
after a filled cache (mask ones(T, S).tril(S - T)).

Tolerance: the north star's 1e-2 relative for bf16 outputs, i.e. |y - ref| <= 1e-2 * max|ref| per element, and
the mean error within 5e-3 of the mean |ref| (the kernel rounds the probabilities to bf16 for the value product and
the output to bf16, about 0.2% of an output that averages hundreds of values; a dropped key tile, a wrong mask or a
transposed operand is off by several percent).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from smlm_hip import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(msg, flush=True)


def ref_attention(q, k, v):
    """fp64 causal attention with the query offset S - T, (B, H, T, hd) -> (B, T, H, hd)."""
    q, k, v = q.double().cpu(), k.double().cpu(), v.double().cpu()
    T, S, hd = q.shape[2], k.shape[2], q.shape[3]
    s = q @ k.transpose(-1, -2) / math.sqrt(hd)
    mask = torch.ones(T, S, dtype=torch.bool).tril(S - T)
    s = s.masked_fill(~mask, float("-inf"))
    return (torch.softmax(s, -1) @ v).transpose(1, 2)


def check(got, ref, what):
    got = got.float().cpu().double()
    scale = float(ref.abs().max())
    worst = float((got - ref).abs().max())
    mean_err = float((got - ref).abs().mean())
    assert worst <= 1e-2 * scale, f"{what}: worst error {worst:.3e} vs scale {scale:.3e}"
    assert mean_err <= 5e-3 * float(ref.abs().mean()), f"{what}: mean error {mean_err:.3e}"


def rand_qkv(B, H, T, S, hd, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, T, hd, generator=g) * scale).to(torch.bfloat16)
    k = (torch.randn(B, H, S, hd, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(B, H, S, hd, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,H,T,S,hd", [
    (2, 3, 1, 1, 64),        # one token
    (1, 2, 37, 37, 64),      # one partial query tile, partial key tile
    (2, 6, 300, 300, 64),    # several query tiles, ragged
    (1, 2, 130, 700, 64),    # new tokens after 570 cached ones
    (1, 1, 1, 513, 64),      # one new token after a long prefix
    (3, 2, 256, 256, 32),
    (1, 3, 200, 333, 128),
])
def test_prefill_attention_matches_fp64(B, H, T, S, hd):
    note(f"prefill_attention B={B} H={H} T={T} S={S} hd={hd}")
    q, k, v = rand_qkv(B, H, T, S, hd, seed=B * 1000 + T + S + hd)
    y = K.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (B, T, H, hd) and y.dtype == torch.bfloat16
    check(y, ref_attention(q, k, v), f"B={B} H={H} T={T} S={S} hd={hd}")


def test_prefill_attention_sharp_scores():
    """Large logits (softmax close to one-hot, the running max moves a lot between tiles): the online rescaling."""
    note("prefill_attention sharp scores")
    q, k, v = rand_qkv(1, 2, 257, 257, 64, seed=7, scale=4.0)
    y = K.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    check(y, ref_attention(q, k, v), "sharp")


def test_prefill_attention_strided_views():
    """q, k, v as the model passes them: permuted views of one (B, T, 3, H, hd) projection, and keys / values as a
    prefix slice of a larger static cache."""
    note("prefill_attention strided views")
    B, T, H, hd = 2, 160, 6, 64
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(B, T, 3, H, hd, generator=g).to(torch.bfloat16)
    q, k, v = qkv.permute(2, 0, 3, 1, 4)
    y = K.prefill_attention(*(t for t in qkv.to(DEV).permute(2, 0, 3, 1, 4)))
    torch.cuda.synchronize()
    check(y, ref_attention(q, k, v), "permuted qkv")

    cache_k = torch.zeros(B, H, 512, hd, dtype=torch.bfloat16)
    cache_v = torch.zeros_like(cache_k)
    cache_k[:, :, :T] = k
    cache_v[:, :, :T] = v
    ck, cv = cache_k.to(DEV), cache_v.to(DEV)
    y2 = K.prefill_attention(q.to(DEV), ck[:, :, :T], cv[:, :, :T])
    torch.cuda.synchronize()
    check(y2, ref_attention(q, k, v), "cache slice")
    assert torch.equal(y2.cpu(), y.cpu())   # same values, same order of operations


def test_prefill_attention_against_sdpa_config2_shape():
    """One (batch, head) slice pair at the config-2 prefill length (2048 tokens, head_dim 64) against torch's own
    fp32 F.scaled_dot_product_attention (is_causal=True) on the CPU."""
    note("prefill_attention 2048 tokens vs CPU SDPA")
    q, k, v = rand_qkv(1, 2, 2048, 2048, 64, seed=11)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True).transpose(1, 2).double()
    y = K.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    check(y, ref, "2048 tokens")


def test_prefill_attention_out_argument_and_errors():
    note("prefill_attention out= and argument checks")
    q, k, v = rand_qkv(1, 2, 64, 64, 64, seed=5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = torch.empty(1, 64, 2, 64, dtype=torch.bfloat16, device=DEV)
    assert K.prefill_attention(qd, kd, vd, out=out) is out
    torch.cuda.synchronize()
    check(out, ref_attention(q, k, v), "out=")
    with pytest.raises(ValueError):
        K.prefill_attention(qd.float(), kd, vd)
    with pytest.raises(ValueError):
        K.prefill_attention(qd, kd[:, :, :32], vd[:, :, :32])          # S < T
    with pytest.raises(ValueError):
        K.prefill_attention(qd[..., :48], kd[..., :48], vd[..., :48])  # head_dim 48


def rope_ref(x, cos, sin, pos0):
    """fp64 rotation of the halves of x (B, H, T, hd) at positions pos0.. (smlm/model.py:63-78), tables as given."""
    T, hd = x.shape[2], x.shape[3]
    c = cos[pos0:pos0 + T].double().cpu()
    s = sin[pos0:pos0 + T].double().cpu()
    x = x.double().cpu()
    a, b = x[..., :hd // 2], x[..., hd // 2:]
    return torch.cat([a * c - b * s, a * s + b * c], dim=-1)


def assert_within_ulp(got, ref, what):
    """got (bf16) within one bf16 ulp of the fp64 ref (the kernel rounds an fp32 value once)."""
    got = got.float().cpu().double()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2 ** -120))) - 7)
    excess = float(((got - ref).abs() - ulp).max())
    assert excess <= 0, f"{what}: off by more than one bf16 ulp (excess {excess})"


@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,hd,pos0", [(2, 37, 3, 64, 5), (1, 1, 6, 64, 300), (3, 130, 2, 128, 0),
                                           (2, 17, 4, 16, 1)])
def test_rope_qkv_matches_fp64(B, T, H, hd, pos0, table_dtype):
    note(f"rope_qkv B={B} T={T} H={H} hd={hd} pos0={pos0} tables {table_dtype}")
    from smlm_hip.model import RotaryEmbedding
    rope = RotaryEmbedding(hd, 512, 10000.0)
    cos, sin = rope.cos.to(table_dtype), rope.sin.to(table_dtype)
    g = torch.Generator().manual_seed(T + hd)
    qkv = torch.randn(B, T, 3 * H * hd, generator=g).to(torch.bfloat16)
    q_ref, k_ref, v_ref = qkv.view(B, T, 3, H, hd).permute(2, 0, 3, 1, 4)
    qd = torch.empty(B, H, T, hd, dtype=torch.bfloat16, device=DEV)
    cache_k = torch.zeros(B, H, pos0 + T + 8, hd, dtype=torch.bfloat16, device=DEV)
    cache_v = torch.zeros_like(cache_k)
    K.rope_qkv(qkv.to(DEV), cos.to(DEV), sin.to(DEV), pos0, qd, cache_k[:, :, pos0:pos0 + T],
               cache_v[:, :, pos0:pos0 + T])
    torch.cuda.synchronize()
    assert_within_ulp(qd, rope_ref(q_ref, cos, sin, pos0), "q")
    assert_within_ulp(cache_k[:, :, pos0:pos0 + T], rope_ref(k_ref, cos, sin, pos0), "k")
    assert torch.equal(cache_v[:, :, pos0:pos0 + T].cpu(), v_ref)
    # slots outside [pos0, pos0 + T) untouched
    assert not cache_k[:, :, :pos0].any() and not cache_k[:, :, pos0 + T:].any()
    assert not cache_v[:, :, :pos0].any() and not cache_v[:, :, pos0 + T:].any()


def test_rope_qkv_errors():
    note("rope_qkv argument checks")
    qkv = torch.zeros(1, 8, 3 * 2 * 64, dtype=torch.bfloat16, device=DEV)
    cos = torch.zeros(16, 32, device=DEV)
    q = torch.empty(1, 2, 8, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.empty_like(q)
    with pytest.raises(ValueError):
        K.rope_qkv(qkv, cos, cos, 9, q, k)               # positions 9..16 past a 16-row table
    with pytest.raises(ValueError):
        K.rope_qkv(qkv.float(), cos, cos, 0, q, k)
    with pytest.raises(ValueError):
        K.rope_qkv(qkv, cos[:, :16], cos[:, :16], 0, q, k)


def test_model_prefill_kernels_match_torch_path():
    """A dense bf16 LM's prompt logits through the prompt-pass kernels (no autograd graph) against the torch ops of
    the same model (recorded for autograd: RoPE by chunk / cat, attention by bmm + fp32 softmax), at one and two
    prompt chunks (the second attends over a dict cache of the first)."""
    note("model prefill: kernels vs torch ops")
    from smlm_hip.model import ModelConfig, Transformer
    torch.manual_seed(0)
    cfg = ModelConfig(vocab_size=512, d_model=384, n_layers=2, n_heads=6, ffn_hidden=1024, max_seq_len=512,
                      mem_layers=[])
    model = Transformer(cfg).to(DEV).to(torch.bfloat16).eval()
    idx = torch.randint(0, 512, (2, 300), device=DEV)
    ref = model(idx)                                   # grad enabled: parameters record -> torch path
    with torch.no_grad():
        got = model(idx)
        cache = [dict() for _ in range(cfg.n_layers)]
        a = model(idx[:, :170], kv_caches=cache, pos0=0)
        b = model(idx[:, 170:], kv_caches=cache, pos0=170)
    torch.cuda.synchronize()
    ref = ref.detach().float()
    scale = float(ref.abs().max())
    for what, t in (("one pass", got), ("two chunks", torch.cat([a, b], dim=1))):
        err = float((t.float() - ref).abs().max())
        assert err <= 2e-2 * scale, f"{what}: logits off by {err:.3e} (scale {scale:.3e})"


# ----------------------------------------------------------------------------- FFN up-projection + SwiGLU (fused)
def _swiglu_rule(x, w):
    """The bf16 model's arithmetic from fp64 products: a, b = bf16 of the projection's halves, then
    bf16(bf16(silu(a)) * b) (smlm/model.py:110-118 with the bf16 roundings of the projection and the activation).
    Returns (out, a, b) as fp32 tensors of bf16 values."""
    h = (x.double() @ w.double().T).float().bfloat16().float()
    H = w.shape[0] // 2
    a, b = h[:, :H], h[:, H:]
    return _act(a, b), a, b


def _act(a, b):
    s = (a / (1.0 + torch.exp(-a))).bfloat16().float()
    return (s * b).bfloat16().float()


def _ulp_bf16(t):
    return torch.pow(2.0, torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -126))) - 7)


def _check_swiglu(got, x, w, what):
    """At least 99.9% of the outputs are the rule on the exact roundings (_swiglu_rule), and every other one lies
    within the error the kernel's arithmetic allows: a and b each off by their fp32 accumulation (2^-20 of the sum
    of |x w| over the dot product, a generous bound on K = 1024 additions) plus one bf16 ulp, carried through silu
    (|silu'| <= 1.1) and the product, plus one bf16 rounding of s and of the output.  A wrong operand (a and b
    exchanged, a feature or token shifted) misses by orders of magnitude."""
    ref, a, b = _swiglu_rule(x, w)
    miss = got != ref
    assert float(miss.double().mean()) <= 1e-3, f"{what}: {int(miss.sum())} outputs differ from the rule"
    if bool(miss.any()):
        H = w.shape[0] // 2
        mag = x.double().abs() @ w.double().abs().T
        ma, mb = mag[:, :H][miss], mag[:, H:][miss]
        am, bm, gm, rm = a[miss].double(), b[miss].double(), got[miss].double(), ref[miss].double()
        da = _ulp_bf16(am) + 2.0 ** -20 * ma
        db = _ulp_bf16(bm) + 2.0 ** -20 * mb
        sm = am / (1.0 + torch.exp(-am))
        ds = 1.1 * da + _ulp_bf16(sm)
        bound = sm.abs() * db + bm.abs() * ds + ds * db + _ulp_bf16(rm) + _ulp_bf16(gm)
        bad = (gm - rm).abs() > bound
        assert not bool(bad.any()), f"{what}: {int(bad.sum())} outputs beyond the arithmetic's error bound"


@pytest.mark.parametrize("M,Kd,H", [(16384, 384, 1024), (1000, 384, 1024), (129, 512, 64), (1, 128, 128),
                                    (300, 256, 192), (128, 1024, 512), (257, 384, 2048), (140, 64, 64),
                                    (100, 192, 320)])
def test_linear_swiglu_matches_the_bf16_rule(M, Kd, H):
    """kernels.linear_swiglu against the fp64-product restatement of the w13 projection + SwiGLU roundings
    (_check_swiglu), with partial token tiles (M not a multiple of 128) and one row; the unfused pair (the library
    GEMM + smlm_swiglu) meets the same check."""
    note(f"linear_swiglu M={M} K={Kd} H={H}")
    g = torch.Generator(device=DEV).manual_seed(M + Kd + H)
    x = torch.randn(M, Kd, generator=g, device=DEV).bfloat16()
    w = (torch.randn(2 * H, Kd, generator=g, device=DEV) * 0.05).bfloat16()
    _check_swiglu(K.linear_swiglu(x, w).float(), x, w, "fused")
    if M == 1000:   # a planted mistake fails the check: the a and b halves of the weight exchanged
        wx = torch.cat([w[H:], w[:H]])
        with pytest.raises(AssertionError):
            _check_swiglu(K.linear_swiglu(x, wx).float(), x, w, "exchanged halves")
    if M > 1:
        _check_swiglu(K.swiglu(F.linear(x, w)).float(), x, w, "library GEMM + swiglu")


def test_linear_swiglu_strided_input_and_rejects():
    """A (rows, K) view with a row stride larger than K gives the contiguous call's bits; shapes outside the
    kernel (K not a multiple of 64, hidden not of 64, fp32) are refused with ValueError."""
    note("linear_swiglu strided / rejects")
    g = torch.Generator(device=DEV).manual_seed(5)
    big = torch.randn(300, 512, generator=g, device=DEV).bfloat16()
    w = (torch.randn(256, 384, generator=g, device=DEV) * 0.05).bfloat16()
    view = big[:, :384]
    assert torch.equal(K.linear_swiglu(view, w), K.linear_swiglu(view.contiguous(), w))
    with pytest.raises(ValueError):
        K.linear_swiglu(big[:, :288], (torch.randn(256, 288, device=DEV)).bfloat16())
    with pytest.raises(ValueError):
        K.linear_swiglu(view, w[:192])
    with pytest.raises(ValueError):
        K.linear_swiglu(view.float(), w.float())


def _check_linear(got, x, w, bias, what):
    """At least 99.9% of the outputs are bf16 of the fp64 product plus the bias, and every other one lies within
    the fp32 accumulation's error (2^-20 of the sum of |x w| and |bias|, generous for K <= 1024 additions) plus
    one bf16 ulp of either value.  A wrong operand (a shifted weight row or bias entry) misses by far more."""
    exact = x.double() @ w.double().T + (bias.double() if bias is not None else 0.0)
    ref = exact.float().bfloat16().float()
    miss = got != ref
    assert float(miss.double().mean()) <= 1e-3, f"{what}: {int(miss.sum())} outputs differ from the rule"
    if bool(miss.any()):
        mag = x.double().abs() @ w.double().abs().T + (bias.double().abs() if bias is not None else 0.0)
        gm, rm = got[miss].double(), ref[miss].double()
        bound = 2.0 ** -20 * mag[miss] + _ulp_bf16(rm) + _ulp_bf16(gm)
        bad = (gm - rm).abs() > bound
        assert not bool(bad.any()), f"{what}: {int(bad.sum())} outputs beyond the arithmetic's error bound"


@pytest.mark.parametrize("M,Kd,N,with_bias", [(16384, 384, 1152, False), (16384, 384, 384, True),
                                              (16384, 1024, 384, False), (1000, 384, 384, True),
                                              (129, 512, 128, True), (1, 128, 256, False), (300, 256, 640, True),
                                              (200, 64, 128, True), (130, 192, 2048, False)])
def test_prompt_linear_matches_the_fp64_rule(M, Kd, N, with_bias):
    """kernels.prompt_linear against bf16 of the fp64 product (+ bias) (_check_linear), at the model's prompt-pass
    shapes (wqkv, wo / value_proj with its bias, w2) and partial token tiles; the library's F.linear meets the same
    check, and a bias shifted by one feature fails it."""
    note(f"prompt_linear M={M} K={Kd} N={N} bias={with_bias}")
    g = torch.Generator(device=DEV).manual_seed(M + Kd + N)
    x = torch.randn(M, Kd, generator=g, device=DEV).bfloat16()
    w = (torch.randn(N, Kd, generator=g, device=DEV) * 0.05).bfloat16()
    b = torch.randn(N, generator=g, device=DEV).bfloat16() if with_bias else None
    got = K.prompt_linear(x, w, b).float()
    _check_linear(got, x, w, b, "prompt_linear")
    if M > 1:
        _check_linear(F.linear(x, w, b).float(), x, w, b, "F.linear")
    if with_bias and M == 1000:
        with pytest.raises(AssertionError):
            _check_linear(K.prompt_linear(x, w, b.roll(1)).float(), x, w, b, "shifted bias")


def test_prompt_linear_strided_input_rejects_and_dispatch():
    """A strided (rows, K) view gives the contiguous call's bits; shapes outside the kernel are refused with
    ValueError; kernels.linear takes the kernel for a no-grad bf16 prompt (its bits) and the module itself for few
    rows, when autograd records (gradients then flow as through nn.Linear) and under an autocast that is not bf16 or
    with fp32 weights."""
    note("prompt_linear strided / rejects / dispatch")
    g = torch.Generator(device=DEV).manual_seed(6)
    big = torch.randn(300, 512, generator=g, device=DEV).bfloat16()
    w = (torch.randn(256, 384, generator=g, device=DEV) * 0.05).bfloat16()
    view = big[:, :384]
    assert torch.equal(K.prompt_linear(view, w), K.prompt_linear(view.contiguous(), w))
    with pytest.raises(ValueError):
        K.prompt_linear(big[:, :288], torch.randn(256, 288, device=DEV).bfloat16())
    with pytest.raises(ValueError):
        K.prompt_linear(view, w[:192])
    with pytest.raises(ValueError):
        K.prompt_linear(view.float(), w.float())
    with pytest.raises(ValueError):
        K.prompt_linear(view, w, torch.zeros(256, device=DEV))
    lin = torch.nn.Linear(384, 256, device=DEV).bfloat16()
    x3 = torch.randn(2, 150, 384, generator=g, device=DEV).bfloat16()
    with torch.no_grad():
        assert torch.equal(K.linear(lin, x3), K.prompt_linear(x3, lin.weight, lin.bias))
        assert torch.equal(K.linear(lin, x3[:, :60]), lin(x3[:, :60]))
    y = K.linear(lin, x3)
    assert y.requires_grad
    y.float().sum().backward()
    assert lin.weight.grad is not None and lin.bias.grad is not None
    # autocast: fp32 weights under bf16 autocast, and fp16 autocast, take the module (autocast's own casts)
    lin32 = torch.nn.Linear(384, 256, device=DEV)
    x32 = torch.randn(300, 384, generator=g, device=DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        assert torch.equal(K.linear(lin32, x32), lin32(x32))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        got = K.linear(lin, x3)
        assert got.dtype == lin(x3).dtype and torch.equal(got, lin(x3))


@pytest.mark.parametrize("M", [16384, 300])
def test_prompt_linear_affine_equals_the_two_launches(M):
    """prompt_linear with scale / shift (the memory query's projection + eval BatchNorm in one launch) gives the
    bits of the projection followed by affine_bf16 (the BatchNorm kernel of the unfused path), at the config-2
    query shape (384 -> 4 x 512) and a partial token tile; a scale without a shift is refused."""
    note(f"prompt_linear affine M={M}")
    g = torch.Generator(device=DEV).manual_seed(M)
    x = torch.randn(M, 384, generator=g, device=DEV).bfloat16()
    w = (torch.randn(2048, 384, generator=g, device=DEV) * 0.05).bfloat16()
    b = (torch.randn(2048, generator=g, device=DEV) * 0.1).bfloat16()
    scale = torch.rand(2048, generator=g, device=DEV) + 0.5
    shift = torch.randn(2048, generator=g, device=DEV) * 0.1
    fused = K.prompt_linear(x, w, b, scale, shift)
    assert torch.equal(fused, K.affine_bf16(K.prompt_linear(x, w, b), scale, shift))
    ref = ((x.double() @ w.double().T + b.double()).float().bfloat16().double() * scale.double()
           + shift.double()).float().bfloat16().float()
    assert float((fused.float() != ref).double().mean()) <= 1e-3
    with pytest.raises(ValueError):
        K.prompt_linear(x, w, b, scale, None)
