"""Fused decode-step kernels (smlm_decode_linear, smlm_argmax_finish) against fp64 CPU restatements of the
reference ops they replace: nn.Linear (smlm/model.py:90-118), the residual add + RMSNorm (model.py:156-163), the
token embedding (model.py:268), the eval BatchNorm of the memory query (smlm/pkm.py:188-191), SwiGLU
(model.py:110-118) and the greedy argmax of the decode loop (smlm/train.py:297-301).

Tolerances: bf16 outputs within 2^-7 relative of the fp64 value plus 2^-9 of the output scale (the kernel
accumulates in fp32 in its own order and rounds once); the residual stream (x + delta in bf16) is bit-exact; the
argmax token is exact wherever the best logit is separated from the runner-up, and planted exact ties resolve to
the lowest column.
"""
import ctypes

import pytest
import torch

from smlm_hip import _lib
from smlm_hip import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(msg, flush=True)


def bf(t):
    return t.to(torch.bfloat16)


def rms_ref(xs, g, eps):
    """bf16(xs * rsqrt(mean(xs^2) + eps) * g) in fp64 (xs, g bf16)."""
    x = xs.double()
    return bf(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * g.double())


def assert_bf16_close(got, ref, what):
    got, ref = got.float().cpu().double(), ref.double()
    scale = float(ref.abs().max())
    err = (got - ref).abs() - (2 ** -7 * ref.abs() + 2 ** -9 * scale)
    assert float(err.max()) <= 0, f"{what}: worst excess {float(err.max())} (scale {scale})"


def make_norm(K_, g):
    norm = torch.nn.RMSNorm(K_, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(K_, generator=g) + 0.5)
    return norm.to(DEV, torch.bfloat16)


@pytest.mark.parametrize("M,N,K_", [(1, 1152, 384), (64, 1152, 384), (5, 384, 1024), (100, 48, 64),
                                    (64, 384, 384), (130, 2432, 384)])
def test_plain_store(M, N, K_):
    note(f"decode_linear plain M={M} N={N} K={K_}")
    g = torch.Generator().manual_seed(M * 7 + N)
    x = bf(torch.randn(M, K_, generator=g))
    w = bf(torch.randn(N, K_, generator=g) * 0.05)
    b = bf(torch.randn(N, generator=g) * 0.1)
    got = K.decode_linear(w.to(DEV), x.to(DEV))
    assert_bf16_close(got, bf(x.double() @ w.double().T).double(), "plain")
    got_b = K.decode_linear(w.to(DEV), x.to(DEV), bias=b.to(DEV))
    assert_bf16_close(got_b, bf(x.double() @ w.double().T + b.double()).double(), "plain + bias")


def test_plain_strided_input():
    """x rows taken from a wider buffer (row stride > K), as the attention output of a fused qkv buffer."""
    g = torch.Generator().manual_seed(11)
    big = bf(torch.randn(8, 1152, generator=g))
    w = bf(torch.randn(384, 384, generator=g) * 0.05)
    xd = big.to(DEV)[:, 384:768]
    got = K.decode_linear(w.to(DEV), xd)
    assert_bf16_close(got, bf(big[:, 384:768].double() @ w.double().T).double(), "strided x")


@pytest.mark.parametrize("M", [1, 3, 64, 77])
@pytest.mark.parametrize("with_delta", [False, True])
def test_rmsnorm_store_affine_split(M, with_delta):
    """Residual add + RMSNorm + the memory layer's query_proj | swilu_proj with bias, eval-BatchNorm affine on
    the query columns, split into (q, pre)."""
    note(f"decode_linear rmsnorm+affine M={M} delta={with_delta}")
    g = torch.Generator().manual_seed(M + 100 * with_delta)
    K_, NQ, NP = 384, 2048, 384
    x = bf(torch.randn(M, K_, generator=g))
    d = bf(torch.randn(M, K_, generator=g)) if with_delta else None
    w = bf(torch.randn(NQ + NP, K_, generator=g) * 0.05)
    b = bf(torch.randn(NQ + NP, generator=g) * 0.1)
    scale = torch.rand(NQ, generator=g) + 0.5
    shift = torch.randn(NQ, generator=g) * 0.1
    norm = make_norm(K_, g)
    xs_ref = bf(x.double() + d.double()) if with_delta else x
    h = rms_ref(xs_ref, norm.weight.detach().cpu(), 1e-5)
    v = bf(h.double() @ w.double().T + b.double())
    q_ref = bf(v[:, :NQ].double() * scale.double() + shift.double())
    pre_ref = v[:, NQ:]
    xs, (q, pre) = K.decode_linear(w.to(DEV), x.to(DEV), delta=d.to(DEV) if d is not None else None, norm=norm,
                                   write_x=True, bias=b.to(DEV), affine=(scale.to(DEV), shift.to(DEV)), n_split=NQ)
    assert torch.equal(xs.cpu(), xs_ref)
    assert_bf16_close(q, q_ref.double(), "query (affine)")
    assert_bf16_close(pre, pre_ref.double(), "pre")


@pytest.mark.parametrize("M", [1, 64, 65])
def test_embed_rmsnorm_store(M):
    note(f"decode_linear embed M={M}")
    g = torch.Generator().manual_seed(M + 5)
    V, K_, N = 1000, 384, 1152
    emb = bf(torch.randn(V, K_, generator=g) * 0.02)
    tok = torch.randint(0, V, (M,), generator=g)
    w = bf(torch.randn(N, K_, generator=g) * 0.05)
    norm = make_norm(K_, g)
    xs, y = K.decode_linear(w.to(DEV), tok=tok.to(DEV), emb=emb.to(DEV), norm=norm, write_x=True)
    assert torch.equal(xs.cpu(), emb[tok])
    h = rms_ref(emb[tok], norm.weight.detach().cpu(), 1e-5)
    assert_bf16_close(y, bf(h.double() @ w.double().T).double(), "embed + norm + linear")


@pytest.mark.parametrize("M", [1, 64, 70])
def test_rmsnorm_swiglu(M):
    note(f"decode_linear swiglu M={M}")
    g = torch.Generator().manual_seed(M + 9)
    K_, H = 384, 1024
    x = bf(torch.randn(M, K_, generator=g))
    d = bf(torch.randn(M, K_, generator=g))
    w = bf(torch.randn(2 * H, K_, generator=g) * 0.05)
    norm = make_norm(K_, g)
    got = K.decode_linear(w.to(DEV), x.to(DEV), delta=d.to(DEV), norm=norm, swiglu=True)
    h = rms_ref(bf(x.double() + d.double()), norm.weight.detach().cpu(), 1e-5)
    ab = bf(h.double() @ w.double().T)
    a, b = ab[:, :H].double(), ab[:, H:].double()
    ref = bf(bf(torch.nn.functional.silu(a)).double() * b)
    # a and b may each sit one bf16 rounding away from the fp64 value: allow two roundings
    got, ref = got.float().cpu().double(), ref.double()
    scale = float(ref.abs().max())
    assert float(((got - ref).abs() - (2 ** -6 * ref.abs() + 2 ** -8 * scale)).max()) <= 0


@pytest.mark.parametrize("M,N", [(1, 32000), (64, 32000), (3, 128), (70, 1008)])
def test_argmax_epilogue_and_finish(M, N):
    """lm_head + greedy argmax: the token is the fp64 argmax wherever it is separated from the runner-up by more
    than the bf16 rounding of the logits; exact ties (duplicated weight rows) go to the lowest column; the
    history slot pos + 1 is written and pos advances by one."""
    note(f"decode_linear argmax M={M} N={N}")
    g = torch.Generator().manual_seed(M + N)
    K_ = 384
    x = bf(torch.randn(M, K_, generator=g))
    d = bf(torch.randn(M, K_, generator=g))
    w = bf(torch.randn(N, K_, generator=g) * 0.05)
    norm = make_norm(K_, g)
    h = rms_ref(bf(x.double() + d.double()), norm.weight.detach().cpu(), 1e-5)
    logits = h.double() @ w.double().T
    best = logits.argmax(-1)
    # plant an exact tie for row 0: a later column with the same weight row as the winner
    j = int(best[0])
    dup = N - 1 if j != N - 1 else 0
    w[j] = bf(w[j].double() * 1.5)        # a clear winner for row 0 ...
    w[dup] = w[j]                          # ... tied exactly with a later column
    logits = h.double() @ w.double().T
    top2 = logits.topk(2, -1).values
    sep = (top2[:, 0] - top2[:, 1]) > 2 ** -6 * top2[:, 0].abs()
    ref = logits.argmax(-1)            # torch.argmax: first index of the maximum
    L = 10
    hist = torch.full((M, L), -1, dtype=torch.int64, device=DEV)
    pos = torch.tensor(3, device=DEV)
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    partial = K.decode_linear(w.to(DEV), x.to(DEV), delta=d.to(DEV), norm=norm, argmax=True)
    assert partial.shape == (M, _lib.lib().smlm_linear_argmax_blocks(N))
    K.argmax_finish(partial, pos, tok, hist)
    got = tok.cpu()
    assert int(got[0]) == min(j, dup), (int(got[0]), j, dup)
    assert torch.equal(got[sep], ref[sep])
    assert int(pos) == 4
    assert torch.equal(hist[:, 4].cpu(), got) and bool((hist[:, :4] == -1).all()) and bool((hist[:, 5:] == -1).all())
    K.argmax_finish(partial, torch.tensor(L - 1, device=DEV), tok, hist)   # slot L is outside: no write
    assert bool((hist[:, 5:] == -1).all())


@pytest.mark.parametrize("M,N,pad", [(1, 32000, 0), (64, 32000, 0), (17, 640, 1), (5, 128, 1)])
def test_embed_argmax_prologue_matches_finish_then_embed(M, N, pad):
    """EMBED_ARGMAX (the token picked from the previous step's argmax keys inside the next step's first launch)
    against argmax_finish followed by the EMBED_RMSNORM launch on its tokens: bit-identical residual rows and
    outputs, the same tokens in tok_out and in hist[:, pos] (pos itself unchanged); an odd number of key blocks
    (the row stride padded to even), a row without keys (id 2^32 - 1: a NaN row in both), keys seeded as ~token
    (what the decoder's start() writes), a history slot outside the history (no write); and the lm_head launch's
    pos_advance adds one without changing the keys."""
    note(f"embed argmax prologue M={M} N={N}")
    g = torch.Generator().manual_seed(M * 7 + N)
    K_, V = 384, N
    x = bf(torch.randn(M, K_, generator=g)).to(DEV)
    w_lm = bf(torch.randn(N, K_, generator=g) * 0.05).to(DEV)
    norm = make_norm(K_, g)
    nblk = _lib.lib().smlm_linear_argmax_blocks(N)
    keys = torch.zeros(M, nblk + pad, dtype=torch.int64, device=DEV)
    partial = K.decode_linear(w_lm, x, norm=norm, argmax=True, partial_out=keys[:, :nblk])
    assert partial.data_ptr() == keys.data_ptr()
    pos = torch.tensor(5, device=DEV)
    again = torch.zeros_like(keys)
    K.decode_linear(w_lm, x, norm=norm, argmax=True, partial_out=again[:, :nblk], advance_pos=pos)
    assert int(pos) == 6 and torch.equal(again, keys)
    if M > 2:
        keys[1] = 0                                        # no keys: id 2^32 - 1
        keys[2] = 0
        keys[2, 0] = ~torch.tensor(N - 3)                  # seeded: token N - 3
    emb = bf(torch.randn(V, K_, generator=g) * 0.02).to(DEV)
    w = bf(torch.randn(1152, K_, generator=g) * 0.05).to(DEV)
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    K.argmax_finish(keys, torch.tensor(0, device=DEV), tok, advance=False)
    if M > 2:
        assert int(tok[1]) == 2 ** 32 - 1 and int(tok[2]) == N - 3
    xs_ref, y_ref = K.decode_linear(w, tok=tok, emb=emb, norm=norm, write_x=True)
    L = 12
    hist = torch.full((M, L), -1, dtype=torch.int64, device=DEV)
    tok_out = torch.full((M,), -7, dtype=torch.int64, device=DEV)
    xs, y = K.decode_linear(w, tok_partial=keys, tok_out=tok_out, hist=hist, pos=pos, emb=emb, norm=norm,
                            write_x=True)
    assert int(pos) == 6
    assert torch.equal(xs.view(torch.int16), xs_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(tok_out, tok)
    assert torch.equal(hist[:, 6], tok) and bool((hist[:, :6] == -1).all()) and bool((hist[:, 7:] == -1).all())
    if M > 2:
        assert bool(xs[1].isnan().all()) and not bool(xs[0].isnan().any())
    hist.fill_(-1)
    K.decode_linear(w, tok_partial=keys, hist=hist, pos=torch.tensor(L, device=DEV), emb=emb, norm=norm)
    assert bool((hist == -1).all())


def test_argmax_all_equal_logits_gives_column_zero():
    M, N, K_ = 4, 640, 64
    w = torch.zeros(N, K_, dtype=torch.bfloat16, device=DEV)
    x = torch.randn(M, K_, device=DEV).to(torch.bfloat16)
    partial = K.decode_linear(w, x, argmax=True)
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    pos = torch.tensor(0, device=DEV)
    K.argmax_finish(partial, pos, tok, advance=False)
    assert bool((tok == 0).all()) and int(pos) == 0


def test_decode_linear_rejects_bad_shapes():
    w = torch.zeros(100, 384, dtype=torch.bfloat16, device=DEV)      # N not a multiple of 16
    x = torch.zeros(2, 384, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.SmlmError):
        K.decode_linear(w, x)
    w2 = torch.zeros(64, 1024, dtype=torch.bfloat16, device=DEV)     # RMSNorm prologue with K > 480
    x2 = torch.zeros(2, 1024, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.SmlmError):
        K.decode_linear(w2, x2, norm=make_norm(1024, torch.Generator().manual_seed(0)))


@pytest.mark.parametrize("M,NP,swiglu", [(1, 6, True), (1, 6, False), (3, 1, True), (4, 8, False), (16, 6, True),
                                         (17, 6, False), (40, 3, True), (64, 6, False)])
def test_rmsnorm_parts_prologue_equals_summed_delta(M, NP, swiglu):
    """The RMSNORM_PARTS prologue (delta = fp32 parts summed in part order, rounded to bf16 once) gives exactly
    what the RMSNORM prologue gives on that bf16 delta: the same residual stream and the same outputs, bit for
    bit (one row per wavefront, several rows per wavefront, several token groups)."""
    note(f"decode_linear parts prologue M={M} parts={NP} swiglu={swiglu}")
    g = torch.Generator().manual_seed(M * 10 + NP)
    K_ = 384
    x = bf(torch.randn(M, K_, generator=g))
    parts = torch.randn(M, NP, K_, generator=g) * 0.5
    d = parts[:, 0].clone()
    for q in range(1, NP):
        d = d + parts[:, q]
    d = bf(d)
    norm = make_norm(K_, g)
    if swiglu:
        w = bf(torch.randn(2048, K_, generator=g) * 0.05).to(DEV)
        kw = dict(norm=norm, write_x=True, swiglu=True)
    else:
        w = bf(torch.randn(2048 + 384, K_, generator=g) * 0.05).to(DEV)
        b = bf(torch.randn(2048 + 384, generator=g) * 0.1).to(DEV)
        kw = dict(norm=norm, write_x=True, bias=b, n_split=2048)
    xs, y = K.decode_linear(w, x.to(DEV), delta=parts.to(DEV), **kw)
    xs_ref, y_ref = K.decode_linear(w, x.to(DEV), delta=d.to(DEV), **kw)
    assert torch.equal(xs, xs_ref)
    assert torch.equal(xs.cpu(), bf(x.double() + d.double()))
    if swiglu:
        assert torch.equal(y, y_ref)
    else:
        assert torch.equal(y[0], y_ref[0]) and torch.equal(y[1], y_ref[1])


def test_rmsnorm_parts_prologue_rejects():
    x = torch.zeros(2, 384, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 384, dtype=torch.bfloat16, device=DEV)
    norm = make_norm(384, torch.Generator().manual_seed(0))
    with pytest.raises(ValueError):                                   # more than 8 parts
        K.decode_linear(w, x, delta=torch.zeros(2, 9, 384, device=DEV), norm=norm)
    with pytest.raises(ValueError):                                   # parts with the argmax epilogue
        K.decode_linear(w, x, delta=torch.zeros(2, 6, 384, device=DEV), norm=norm, argmax=True)
    a = _lib.LinearArgs()                                             # the library's own check: 0 parts
    a.prologue, a.epilogue, a.M, a.N, a.K = _lib.LIN_RMSNORM_PARTS, _lib.LIN_STORE, 2, 64, 384
    parts = torch.zeros(2, 1, 384, device=DEV)
    out = torch.empty(2, 64, dtype=torch.bfloat16, device=DEV)
    a.x, a.x_stride, a.delta, a.delta_parts = x.data_ptr(), 384, parts.data_ptr(), 0
    a.norm_w, a.eps, a.w = norm.weight.data_ptr(), 1e-5, w.data_ptr()
    a.n_split, a.out, a.out_stride = 64, out.data_ptr(), 64
    assert _lib.lib().smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL


# ------------------------------------------------------------------------------------- fused selection + value bag
def _tables(kind, rows, D, seed):
    """A (rows, D) value table drawn on the device (N(0, 0.02)), in the given inference format."""
    gd = torch.Generator(device=DEV).manual_seed(seed)
    dt = torch.float32 if kind in ("fp32", "int8", "q4") else torch.bfloat16
    vals = torch.empty(rows, D, dtype=dt, device=DEV).normal_(0.0, 0.02, generator=gd)
    if kind in ("fp32", "bf16"):
        return vals, None
    return K.quantize_int8(vals) if kind == "int8" else K.quantize_q4(vals)


@pytest.mark.parametrize("N,H,NK,knn,dtype,kind,with_pre,out_bf16", [
    (1, 4, 4096, 32, torch.bfloat16, "bf16", True, True),
    (64, 4, 4096, 32, torch.bfloat16, "bf16", True, True),
    (5, 4, 1024, 32, torch.bfloat16, "int8", True, True),
    (7, 4, 512, 32, torch.bfloat16, "q4", False, False),
    (3, 2, 256, 16, torch.bfloat16, "fp32", False, False),
    (9, 3, 2048, 64, torch.bfloat16, "bf16", True, False),
    (4, 2, 2048, 32, torch.float32, "bf16", True, True),
    (2, 4, 8192, 32, torch.bfloat16, "bf16", True, True),     # rows beyond the register path: streaming search
    (3, 1, 512, 16, torch.bfloat16, "bf16", True, True),      # 2 thread slots run the 8 bf16 slots
    (4, 1, 256, 32, torch.bfloat16, "fp32", False, True),     # 1 thread slot runs the 4 fp32 slots
    (6, 1, 1024, 32, torch.bfloat16, "int8", True, False),    # 5 thread slots run the 8 int8 slots
    (3, 4, 24, 4, torch.bfloat16, "bf16", True, True),        # n_keys not a power of two
    (5, 4, 1000, 5, torch.bfloat16, "int8", True, True),      # knn not a power of two: pairs built at run time
    (2, 4, 4096, 128, torch.bfloat16, "bf16", True, True),    # knn above 64: two results per lane
    (4, 2, 256, 100, torch.float32, "bf16", False, False),
    (3, 4, 2048, 128, torch.float32, "fp32", True, False),    # the most LDS: fp32 keys, 4 heads, knn 128
    (2048, 4, 2048, 32, torch.bfloat16, "bf16", True, True),  # a prompt-sized batch (the memory layer's prefill)
])
def test_select_bag_bit_identical_to_select_then_bag(N, H, NK, knn, dtype, kind, with_pre, out_bf16):
    """pk_select_bag == pk_select followed by bag_infer, bit for bit (same selection, same bag additions in the
    canonical row-slot order, also where the fused workgroup has fewer threads than the layout and runs several
    slots per thread)."""
    note(f"select_bag N={N} H={H} NK={NK} knn={knn} {dtype} {kind}")
    g = torch.Generator().manual_seed(N * 31 + NK + knn)
    D = 384
    s1 = torch.randn(N, H, NK, generator=g).to(DEV, dtype)
    s2 = torch.randn(N, H, NK, generator=g).to(DEV, dtype)
    rows = NK * NK if NK <= 4096 else 1 << 20     # NK 8192: a smaller table, tokens reaching beyond it are NaN
    table, scales = _tables(kind, rows, D, N + NK)
    pre = torch.randn(N, D, generator=g).to(DEV, torch.bfloat16) if with_pre else None
    sc, idx, w = K.pk_select(s1, s2, knn)
    ref = K.bag_infer(idx.view(N, -1), w.view(N, -1), table, scales, pre=pre, out_bf16=out_bf16)
    out, sc2, idx2, w2 = K.pk_select_bag(s1, s2, knn, table, scales, pre=pre, out_bf16=out_bf16, record=True)
    assert torch.equal(idx2, idx) and torch.equal(sc2.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                                                  sc.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
    assert torch.equal(w2, w)
    assert torch.equal(torch.isnan(out), torch.isnan(ref))
    assert torch.equal(torch.nan_to_num(out), torch.nan_to_num(ref))
    out_only = K.pk_select_bag(s1, s2, knn, table, scales, pre=pre, out_bf16=out_bf16)
    assert torch.equal(torch.nan_to_num(out_only), torch.nan_to_num(ref))


def test_select_bag_rejects_unsupported():
    s = torch.zeros(1, 5, 64, dtype=torch.bfloat16, device=DEV)                # 5 heads
    t = torch.zeros(64 * 64, 384, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        K.pk_select_bag(s, s, 8, t)
    s1 = torch.zeros(1, 1, 64, dtype=torch.bfloat16, device=DEV)               # 1 head: 128 threads
    assert K.select_bag_supported(1, t)                                        # 48 chunks per row: fits
    wide = torch.zeros(64 * 64, 640, dtype=torch.float32, device=DEV)          # 160 chunks per row: does not
    assert not K.select_bag_supported(1, wide)
    with pytest.raises(_lib.SmlmError):
        K.pk_select_bag(s1, s1, 8, wide)


# ------------------------------------------------------------------------------------------- the fused decode step
def _bits(t):
    return t.detach().view(torch.int16).cpu().numpy().view("uint16")


def _prefilled(model, B, P, seed):
    """A _StepDecoder for model with B random prompts of P tokens prefilled; returns (decoder, prompt)."""
    dec = model._decoder(B, P + 8, DEV)
    prompt = torch.randint(0, model.cfg.vocab_size, (B, P), generator=torch.Generator().manual_seed(seed)).to(DEV)
    logits = model(prompt, kv_caches=dec.caches, pos0=0)
    dec.hist[:, :P] = prompt
    dec.hist[:, P] = logits[:, -1].argmax(-1)
    dec.tok.copy_(dec.hist[:, P:P + 1])
    dec.pos.fill_(P)
    return dec, prompt


# proj_max_batch 0: the attention output goes through its own wo launch; 64: wo is folded into the attention
# launch and summed over heads in the next launch's prologue
@pytest.mark.parametrize("proj_max", [0, 64])
@torch.no_grad()
def test_fused_step_logits_match_generic_step(monkeypatch, proj_max):
    """The fused decode step (no memory layer) against Transformer.forward's single-token static-cache step on
    the same caches and token: logits within 2e-2 of their scale (the two paths round their GEMMs in different
    orders), and the step's token is the argmax of its own logits wherever that is separated."""
    from smlm_hip.model import ModelConfig, Transformer, _FusedDecodeStep
    monkeypatch.setattr(_FusedDecodeStep, "proj_max_batch", proj_max)
    cfg = ModelConfig(vocab_size=1024, d_model=384, n_layers=3, n_heads=6, ffn_hidden=1024, max_seq_len=64)
    torch.manual_seed(0)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    assert _FusedDecodeStep.supported(m, torch.bfloat16)
    for B in (1, 5, 40):
        note(f"fused step vs generic B={B} proj_max_batch={proj_max}")
        dec, _ = _prefilled(m, B, 12, B)
        assert dec.fused is not None
        ref = m(dec.tok, kv_caches=dec.caches, pos0=dec.pos.clone()).float()[:, -1]
        got = dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist, logits=True).float()
        err = float((got - ref).abs().max() / ref.abs().max())
        assert err < 2e-2, err
        pos0 = int(dec.pos)
        dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist)
        assert int(dec.pos) == pos0 + 1
        top2 = got.topk(2, -1).values
        sep = (top2[:, 0] - top2[:, 1]) > 2 ** -6 * top2[:, 0].abs()
        assert torch.equal(dec.tok.view(-1)[sep].cpu(), got.argmax(-1)[sep].cpu())
        assert torch.equal(dec.hist[:, pos0 + 1], dec.tok.view(-1))


@pytest.mark.parametrize("n_heads", [8, 16])
@torch.no_grad()
def test_fused_step_head_counts(n_heads):
    """d_model 256 with 8 heads (head_dim 32: wo folded in as 8 parts, the most the summing prologue takes) and 16
    heads (head_dim 16: more parts than that, so the step keeps its wo launch): logits within 2e-2 of
    Transformer.forward's static-cache step."""
    from smlm_hip.model import ModelConfig, Transformer, _FusedDecodeStep
    cfg = ModelConfig(vocab_size=512, d_model=256, n_layers=2, n_heads=n_heads, ffn_hidden=512, max_seq_len=48)
    torch.manual_seed(n_heads)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    assert _FusedDecodeStep.supported(m, torch.bfloat16)
    note(f"fused step d_model=256 heads={n_heads}")
    dec, _ = _prefilled(m, 3, 10, n_heads)
    assert dec.fused is not None
    ref = m(dec.tok, kv_caches=dec.caches, pos0=dec.pos.clone()).float()[:, -1]
    got = dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist, logits=True).float()
    err = float((got - ref).abs().max() / ref.abs().max())
    assert err < 2e-2, err


@pytest.mark.parametrize("proj_max", [0, 64])
@torch.no_grad()
def test_fused_generate_multi_step_graph_matches_eager(monkeypatch, proj_max):
    """generate() on the fused step: the graphs of several steps in a row plus single-step replays (45 tokens =
    a run of 32 + a run of 8 + 5 single steps) give the eager loop's tokens exactly, on every call."""
    from smlm_hip.model import ModelConfig, Transformer, _FusedDecodeStep, _StepDecoder
    monkeypatch.setattr(_FusedDecodeStep, "proj_max_batch", proj_max)
    cfg = ModelConfig(vocab_size=1024, d_model=384, n_layers=3, n_heads=6, ffn_hidden=1024, max_seq_len=64)
    torch.manual_seed(1)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    assert _StepDecoder.run_lengths == (32, 8)
    prompt = torch.randint(0, 1024, (2, 9), generator=torch.Generator().manual_seed(5)).to(DEV)
    note(f"fused generate multi-step graph B=2 proj_max_batch={proj_max}")
    eager = m.generate(prompt, 45, use_graph=False)
    graph = m.generate(prompt, 45, use_graph=True)
    graph2 = m.generate(prompt, 45, use_graph=True)
    assert eager.shape == (2, 46)
    assert torch.equal(graph, eager) and torch.equal(graph2, eager)


@pytest.mark.parametrize("proj_max,mem_layer", [(0, 2), (64, 2), (0, 1), (64, 1)])
@torch.no_grad()
def test_fused_step_with_memory_layer_matches_torch_path(monkeypatch, proj_max, mem_layer):
    """The fused decode step with a B-style memory layer (BatchNorm, swilu) in the last or a middle block: its
    query and swilu projection match the host recomputation from the step's residual row (tests/query_check.py),
    its sub-key scores the fp64 products of that query, its selection is bit-exact against the oracle on those
    scores, and its logits are within 1e-2 of the fp32 torch path (oracle/torch_path.py) given that selection and
    the prompt pass's (so that the caches of the blocks after the memory layer agree)."""
    import numpy as np
    import oracle.pkm_oracle as O
    import oracle.torch_path as TP
    import query_check as QC
    from smlm_hip.model import ModelConfig, Transformer, _FusedDecodeStep
    monkeypatch.setattr(_FusedDecodeStep, "proj_max_batch", proj_max)
    cfg = ModelConfig(vocab_size=512, d_model=128, n_layers=3, n_heads=2, ffn_hidden=256, max_seq_len=64,
                      mem_layers=[mem_layer], mem_n_keys=128, mem_heads=4, mem_knn=16, mem_k_dim=64)
    torch.manual_seed(3)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    with torch.no_grad():
        bn = m.layers[mem_layer].ffn.query_norm
        bn.running_mean.normal_(0.0, 0.1)
        bn.running_var.uniform_(0.5, 2.0)
        bn.weight.uniform_(0.5, 1.5)
        bn.bias.normal_(0.0, 0.1)
    for kind in ("bf16", "int8"):
        m.set_memory_inference_table(kind)
        B, P = 3, 10
        note(f"fused step memory layer {mem_layer} table={kind} proj_max_batch={proj_max}")
        dec = m._decoder(B, P + 8, DEV)
        assert dec.fused is not None
        prompt = torch.randint(0, cfg.vocab_size, (B, P), generator=torch.Generator().manual_seed(7)).to(DEV)
        mem = m.layers[mem_layer].ffn
        mem.record = True
        logits = m(prompt, kv_caches=dec.caches, pos0=0)
        mem.record = False
        sel_prompt = (mem.last_indices.cpu(), mem.last_weights.cpu())
        dec.hist[:, :P] = prompt
        dec.hist[:, P] = logits[:, -1].argmax(-1)
        dec.tok.copy_(dec.hist[:, P:P + 1])
        dec.pos.fill_(P)
        rec = {}
        got = dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist, logits=True, record=rec).float().cpu()
        r = rec[mem_layer]
        s1, s2, sc, idx, w = r["s1"], r["s2"], r["scores"], r["indices"], r["weights"]
        QC.check_decode_step_query(m, mem_layer, r)
        rs, ri, rw = O.pk_select(_bits(s1), _bits(s2), cfg.mem_knn)
        assert np.array_equal(idx.cpu().numpy(), ri) and np.array_equal(_bits(sc), rs)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=0, atol=1e-6)
        sd = {k: v.float().cpu() for k, v in m.state_dict().items()}
        tables = None
        if kind == "int8":
            codes, scales = mem.values.infer_table
            tables = {mem_layer: K.dequantize_int8(codes, scales).cpu()}
        caches = [dict() for _ in range(cfg.n_layers)]
        TP.lm_forward(sd, cfg.to_dict(), prompt.cpu(), caches, 0, tables=tables, selections={mem_layer: sel_prompt})
        ref = TP.lm_forward(sd, cfg.to_dict(), dec.tok.cpu(), caches, P, tables=tables,
                            selections={mem_layer: (idx.cpu(), w.cpu())})[:, -1]
        err = float((got - ref).abs().max() / ref.abs().max())
        assert err < 1e-2, err
