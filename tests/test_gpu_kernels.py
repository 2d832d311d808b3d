"""HIP kernels against the CPU oracle (oracle/pkm_oracle.py), through the C ABI (smlm_hip.kernels).

Bars: selection (indices, scores, order) bit-exact on the same sub-key scores; softmax weights within 1e-6;
bf16 scores within 1 bf16 ulp of the fp64 scores (fp32 within 1e-5 of their scale); fp32 bag outputs within
rtol = atol = 1e-5 relative to max|reference| (the reference's close(), tests/test_kernels.py:48-53); bf16 bag
outputs within 1 bf16 ulp; quantised tables bit-exact.  Shapes follow the reference's tests
(tests/test_kernels.py:123-125, 29-35, 220-242, 323-360) and BASELINE's configs.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle.pkm_oracle as O
from smlm_hip import _lib
from smlm_hip import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bits_of(t):
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_from_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def note(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------------------------------------ selection
SELECT_SHAPES = [(4096, 4, 512, 32), (4096, 4, 1024, 32), (4096, 4, 2048, 32), (4096, 4, 4096, 32),
                 (1, 4, 1024, 32), (64, 2, 16, 4), (96, 4, 64, 8), (33, 3, 256, 64), (5, 2, 65536, 32),
                 (7, 1, 8, 1)]


def check_select(s1, s2, knn, sc, idx, w):
    rs, ri, rw = O.pk_select(s1, s2, knn)
    got_sc = bits_of(sc) if s1.dtype == np.uint16 else sc.cpu().numpy()
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.array_equal(got_sc.view(np.uint16 if s1.dtype == np.uint16 else np.uint32),
                          rs.view(np.uint16 if s1.dtype == np.uint16 else np.uint32))
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=0, atol=1e-6)


@pytest.mark.parametrize("N,H,NK,knn", SELECT_SHAPES)
def test_pk_select_bf16_bit_exact(N, H, NK, knn):
    note(f"pk_select bf16 N={N} H={H} NK={NK} knn={knn}")
    rng = np.random.default_rng(N + NK)
    s1 = O.bf16_bits_rtne(rng.standard_normal((N, H, NK)).astype(np.float32))
    s2 = O.bf16_bits_rtne(rng.standard_normal((N, H, NK)).astype(np.float32))
    sc, idx, w = K.pk_select(bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV), knn)
    torch.cuda.synchronize()
    check_select(s1, s2, knn, sc, idx, w)
    # the reference test's invariants (tests/test_kernels.py:146-151)
    t1, t2 = bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV)
    own = (t1.gather(-1, idx // NK).float() + t2.gather(-1, idx % NK).float()).to(torch.bfloat16)
    assert torch.equal(own, sc)
    srt = idx.view(-1, knn).sort(-1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all())


# shapes the reference's torch path takes (smlm/pkm.py:48-53): n_keys not a power of two (the register path when
# n_keys is a multiple of 8, else the row searched in memory; 24 and 1000 sub-keys, 3000 = 375 chunks, 4100 and
# 65535), knn not a power of two (pairs built at run time, tests/test_pkm.py:18 uses knn 5) and knn above 64 (two
# results per lane, the half top-k from the row in memory), knn = n_keys
GENERAL_SHAPES = [(100, 3, 24, 4), (64, 4, 1000, 32), (9, 2, 3000, 32), (7, 2, 4100, 16), (3, 1, 65535, 32),
                  (200, 3, 32, 5), (64, 4, 1024, 5), (40, 2, 1000, 12), (33, 3, 256, 48), (17, 2, 512, 100),
                  (9, 4, 4096, 128), (13, 2, 128, 128), (5, 2, 24, 24), (20, 3, 96, 20), (50, 2, 8, 1),
                  (6, 2, 4100, 77)]


@pytest.mark.parametrize("N,H,NK,knn", GENERAL_SHAPES)
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_pk_select_general_shapes_bit_exact(N, H, NK, knn, dtype):
    note(f"pk_select {dtype} general N={N} H={H} NK={NK} knn={knn}")
    rng = np.random.default_rng(N * 7 + NK + knn)
    f1 = rng.standard_normal((N, H, NK)).astype(np.float32)
    f2 = rng.standard_normal((N, H, NK)).astype(np.float32)
    if dtype == "bf16":
        s1, s2 = O.bf16_bits_rtne(f1), O.bf16_bits_rtne(f2)
        t1, t2 = bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV)
    else:
        s1, s2 = f1, f2
        t1, t2 = torch.from_numpy(f1).to(DEV), torch.from_numpy(f2).to(DEV)
    sc, idx, w = K.pk_select(t1, t2, knn)
    torch.cuda.synchronize()
    check_select(s1, s2, knn, sc, idx, w)
    assert bool((idx >= 0).all()) and bool((idx < NK * NK).all())
    assert abs(float(w.double().sum(-1).mean()) - 1.0) < 1e-5


def test_pk_select_general_ties():
    """The general path on tie-heavy rows (a handful of values, both signed zeros): knn 12 and 100."""
    rng = np.random.default_rng(13)
    vals = np.array([0x3F80, 0x3F00, 0x0000, 0x8000, 0xBF00, 0x3F40, 0x4000, 0xBF80], np.uint16)
    for N, H, NK, knn in ((40, 3, 64, 12), (9, 2, 1000, 100)):
        note(f"pk_select general ties N={N} NK={NK} knn={knn}")
        s1 = vals[rng.integers(0, len(vals), (N, H, NK))]
        s2 = vals[rng.integers(0, len(vals), (N, H, NK))]
        sc, idx, w = K.pk_select(bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV), knn)
        torch.cuda.synchronize()
        check_select(s1, s2, knn, sc, idx, w)


@pytest.mark.parametrize("N,H,NK,knn", [(512, 4, 1024, 32), (64, 4, 4096, 32), (40, 3, 64, 8), (9, 2, 16, 16)])
def test_pk_select_bf16_ties(N, H, NK, knn):
    """Scores from a handful of values (both signed zeros): almost every comparison is a tie."""
    note(f"pk_select ties N={N} NK={NK} knn={knn}")
    rng = np.random.default_rng(11)
    vals = np.array([0x3F80, 0x3F00, 0x0000, 0x8000, 0xBF00, 0x3F40, 0x4000, 0xBF80], np.uint16)
    s1 = vals[rng.integers(0, len(vals), (N, H, NK))]
    s2 = vals[rng.integers(0, len(vals), (N, H, NK))]
    sc, idx, w = K.pk_select(bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV), knn)
    torch.cuda.synchronize()
    check_select(s1, s2, knn, sc, idx, w)


@pytest.mark.parametrize("N,H,NK,knn", [(2048, 4, 1024, 32), (3, 2, 4096, 64), (50, 2, 16, 8)])
def test_pk_select_fp32_bit_exact(N, H, NK, knn):
    note(f"pk_select fp32 N={N} NK={NK} knn={knn}")
    rng = np.random.default_rng(N * 3 + NK)
    s1 = rng.standard_normal((N, H, NK)).astype(np.float32)
    s2 = rng.standard_normal((N, H, NK)).astype(np.float32)
    sc, idx, w = K.pk_select(torch.from_numpy(s1).to(DEV), torch.from_numpy(s2).to(DEV), knn)
    torch.cuda.synchronize()
    check_select(s1, s2, knn, sc, idx, w)


def test_pk_select_many_candidates_path():
    """Rows built so that more than 1024 elements reach the lane-maxima threshold: the kernel must take its
    exact path over the whole row.  Lane l of the 64-lane stride holds elements l, l+64, ...; lanes 0..31 get
    maxima 8 - l/32 (bf16-exact) at their first element, lanes 0..15 carry 7.5 elsewhere (above the 32nd lane
    maximum 7.03125 but below their own maximum), the rest 0."""
    note("pk_select adversarial candidate overflow")
    NK, knn = 4096, 32
    row = np.zeros(NK, np.float32)
    k = np.arange(NK)
    lane = k % 64
    row[(lane < 16) & (k >= 64)] = 7.5
    row[:32] = 8.0 - np.arange(32) / 32.0
    s1 = O.bf16_bits_rtne(np.stack([row, row[::-1].copy()]).reshape(2, 1, NK))
    rng = np.random.default_rng(12)
    s2 = O.bf16_bits_rtne(rng.standard_normal((2, 1, NK)).astype(np.float32))
    assert np.sum(O.bf16_to_f32(s1[0, 0]) >= 7.03125) > 1024
    sc, idx, w = K.pk_select(bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV), knn)
    torch.cuda.synchronize()
    check_select(s1, s2, knn, sc, idx, w)


def test_pk_select_golden():
    with open(os.path.join(GOLDEN, "select_known.json")) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        s1 = np.array(c["s1"], np.uint16).reshape(1, 1, -1)
        s2 = np.array(c["s2"], np.uint16).reshape(1, 1, -1)
        sc, idx, w = K.pk_select(bf16_from_bits(s1).to(DEV), bf16_from_bits(s2).to(DEV), c["knn"])
        assert idx[0, 0].tolist() == c["idx"], c["name"]
        if "score_bits" in c:
            assert bits_of(sc)[0, 0].tolist() == c["score_bits"], c["name"]


# ------------------------------------------------------------------------------------------------ scoring
SCORE_SHAPES = [(1, 4, 4096, 256), (64, 4, 4096, 256), (2048, 4, 1024, 256), (100, 4, 2048, 256),
                (5, 2, 16, 8), (17, 3, 64, 32), (300, 1, 512, 64), (1000, 4, 2048, 256), (200, 2, 64, 40),
                (129, 3, 16, 8), (65, 2, 384, 128), (513, 2, 192, 128), (260, 3, 100, 128),
                # enough 256-token tiles for the streaming kernels: NK % 64 == 0 takes the warp-specialised one
                # (half 256, 128 with a ragged token tile, 64 with a single sub-key block), else the plain stream
                (8192, 4, 128, 256), (8200, 4, 192, 128), (16384, 2, 64, 64), (8200, 4, 100, 128)]


def _score_inputs(N, H, NK, half, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(N, H, 2 * half, generator=g)
    keys = torch.randn(H, 2, NK, half, generator=g) / 16
    return q, keys


@pytest.mark.parametrize("N,H,NK,half", SCORE_SHAPES)
def test_pk_scores_bf16_within_one_ulp(N, H, NK, half):
    note(f"pk_scores bf16 N={N} H={H} NK={NK} half={half}")
    q, keys = _score_inputs(N, H, NK, half, N + NK)
    qb, kb = q.to(torch.bfloat16), keys.to(torch.bfloat16)
    s1, s2 = K.pk_scores(qb.to(DEV), kb.to(DEV))
    r1, r2 = O.subkey_scores(qb.float().numpy(), kb.float().numpy())
    absdot1 = np.einsum("nhd,hkd->nhk", np.abs(qb.float().numpy()[..., :half]), np.abs(kb.float().numpy()[:, 0]))
    for got, ref, mag in ((s1, r1, absdot1), (s2, r2, None)):
        g = got.float().cpu().numpy().astype(np.float64)
        # one bf16 ulp (2^-7 relative) plus fp32-accumulation slack on cancellation
        slack = 1e-5 * (mag if mag is not None else np.abs(ref).max())
        assert np.all(np.abs(g - ref) <= 2 ** -7 * np.abs(ref) + slack)
    # the result is the bf16 rounding of an fp32 sum: at most one ulp from the rounded fp64 value
    assert got.dtype == torch.bfloat16


@pytest.mark.parametrize("N,H,NK,half", SCORE_SHAPES[:4] + [(5, 2, 16, 8)])
def test_pk_scores_fp32(N, H, NK, half):
    note(f"pk_scores fp32 N={N} NK={NK}")
    q, keys = _score_inputs(N, H, NK, half, 7 * N + NK)
    s1, s2 = K.pk_scores(q.to(DEV), keys.to(DEV))
    r1, r2 = O.subkey_scores(q.numpy(), keys.numpy())
    mag = np.einsum("nhd,hkd->nhk", np.abs(q.numpy()[..., :half]).astype(np.float64),
                    np.abs(keys.numpy()[:, 0]).astype(np.float64))
    np.testing.assert_array_less(np.abs(s1.cpu().numpy() - r1), 1e-5 * mag + 1e-30)
    np.testing.assert_allclose(s2.cpu().numpy(), r2, rtol=1e-5, atol=1e-5 * np.abs(r2).max())


def test_pk_scores_rejects_mismatch():
    q = torch.zeros(2, 4, 512, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        K.pk_scores(q, torch.zeros(4, 2, 64, 128, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        K.pk_scores(q, torch.zeros(4, 2, 64, 256, dtype=torch.float32, device=DEV))


# ------------------------------------------------------------------------------------------------ value bag
def skewed_indices(rows, N, K_, rng):
    """Uniform rows plus a few hot rows (the reference's skewed_indices, tests/test_kernels.py:55-61)."""
    idx = rng.integers(0, rows, (N, K_))
    hot = rng.integers(0, rows, 8)
    m = rng.random((N, K_)) < 0.2
    idx[m] = hot[rng.integers(0, 8, int(m.sum()))]
    return idx


_TABLES = {}


def make_table(kind, rows, D, rng):
    """(device-ready torch table, torch scales, numpy table, numpy scales); cached per (kind, rows, D)."""
    key = (kind, rows, D)
    if key not in _TABLES:
        _TABLES.clear()
        _TABLES[key] = _make_table(kind, rows, D, np.random.default_rng(rows * 7 + D))
    return _TABLES[key]


def _make_table(kind, rows, D, rng):
    t32 = rng.standard_normal((rows, D), dtype=np.float32) * np.float32(D ** -0.5)
    if kind == "f32":
        return torch.from_numpy(t32), None, t32, None
    if kind == "bf16":
        b = O.bf16_bits_rtne(t32)
        return bf16_from_bits(b), None, b, None
    codes, sc = O.quantize_rows(t32, kind)
    tt = torch.from_numpy(codes)
    return tt, torch.from_numpy(sc), codes, sc


def close(a, b):
    scale = max(1.0, float(np.abs(b).max()))
    np.testing.assert_allclose(a / scale, b / scale, rtol=1e-5, atol=1e-5)


BAG_CASES = [("f32", 1 << 20, 384, 512, 128), ("bf16", 1 << 20, 384, 512, 128), ("i8", 1 << 20, 384, 512, 128),
             ("q4", 1 << 20, 384, 512, 128), ("bf16", 4096, 64, 32, 96), ("f32", 4096, 64, 32, 48),
             ("q4", 4096, 64, 32, 40), ("i8", 4096, 64, 32, 40), ("i8", 1000, 24, 16, 12), ("bf16", 1000, 24, 9, 7),
             ("f32", 2048, 96, 64, 128), ("bf16", 300, 384, 3, 1), ("bf16", 1 << 16, 384, 2, 600),
             # wide rows: 2 slots of 130 chunks, 1 slot of 200 and of 256 chunks (the row kernel's widest), 257
             # chunks (the generic kernel)
             ("bf16", 512, 1040, 3, 9), ("f32", 512, 800, 4, 17), ("f32", 512, 1024, 4, 33), ("f32", 256, 1028, 2, 5)]


@pytest.mark.parametrize("kind,rows,D,N,K_", BAG_CASES)
@pytest.mark.parametrize("idx32", [False, True])
def test_bag_matches_oracle(kind, rows, D, N, K_, idx32):
    note(f"bag {kind} rows={rows} D={D} N={N} K={K_} idx32={idx32}")
    rng = np.random.default_rng(rows + D + K_)
    t, sc, tn, scn = make_table(kind, rows, D, rng)
    idx = skewed_indices(rows, N, K_, rng)
    w = rng.random((N, K_)).astype(np.float32)
    pre = O.bf16_bits_rtne(rng.standard_normal((N, D)).astype(np.float32))
    ti = torch.from_numpy(idx.astype(np.int32 if idx32 else np.int64)).to(DEV)
    tw = torch.from_numpy(w).to(DEV)
    td, tsc = t.to(DEV), (sc.to(DEV) if sc is not None else None)
    ref = O.bag(idx, w, tn, kind, scn)
    close(K.bag_infer(ti, tw, td, tsc).cpu().numpy(), ref)
    if kind in ("f32", "bf16"):
        close(K.bag_forward(ti, tw, td).cpu().numpy(), ref)
    ref2 = O.bag(idx, w, tn, kind, scn, pre=pre)
    tpre = bf16_from_bits(pre).to(DEV)
    close(K.bag_infer(ti, tw, td, tsc, pre=tpre).cpu().numpy(), ref2)
    out = K.bag_infer(ti, tw, td, tsc, pre=tpre, out_bf16=True)
    assert out.dtype == torch.bfloat16
    refb = O.bf16_to_f32(O.bag(idx, w, tn, kind, scn, pre=pre, out_bf16=True)).astype(np.float64)
    scale = float(np.abs(ref2).max())
    np.testing.assert_allclose(out.float().cpu().numpy(), refb, rtol=2 ** -7, atol=2 ** -8 * scale)


def test_bag_out_of_range_index_gives_nan_row():
    rng = np.random.default_rng(13)
    t = torch.randn(100, 64, device=DEV)
    idx = torch.from_numpy(rng.integers(0, 100, (4, 8))).to(DEV)
    idx[2, 3] = 100
    idx[3, 0] = -1
    w = torch.rand(4, 8, device=DEV)
    out = K.bag_forward(idx, w, t)
    assert torch.isnan(out[2:]).all() and torch.isfinite(out[:2]).all()
    ref = O.bag(idx[:2].cpu().numpy(), w[:2].cpu().numpy(), t.cpu().numpy(), "f32")
    close(out[:2].cpu().numpy(), ref)


def test_bag_table_beyond_2_31_elements():
    """Row offsets past 2^31 elements (and 2^32 bytes): 6M x 384 bf16 (tests/test_kernels.py:323-360)."""
    note("bag large table 6M x 384 bf16")
    rows, D = 6 * 1024 * 1024, 384
    t = torch.empty(rows, D, dtype=torch.bfloat16, device=DEV).normal_(0, 0.05)
    rng = np.random.default_rng(14)
    idx = rng.integers(rows - 200000, rows, (64, 128))
    idx[:, 0] = rows - 1
    w = rng.random((64, 128)).astype(np.float32)
    ti = torch.from_numpy(idx).to(DEV)
    used = np.unique(idx)
    sub = bits_of(t[torch.from_numpy(used).to(DEV)])
    remap = np.searchsorted(used, idx)
    ref = O.bag(remap, w, sub, "bf16")
    close(K.bag_infer(ti, torch.from_numpy(w).to(DEV), t).cpu().numpy(), ref)
    del t
    torch.cuda.empty_cache()


def test_bag_zipf_int8_gather_sample():
    """A 2048-token sample of the config-4 stress gather: int8 table with fp16 row scales, 128 Zipf(1.1)
    lookups per token through a seeded row permutation, per-head softmax weights, fp32 out."""
    note("bag zipf int8 sample")
    rows, D, N = 1 << 20, 384, 2048
    rng = np.random.default_rng(15)
    t32 = (rng.standard_normal((rows, D)) * 0.02).astype(np.float32)
    codes, sc = O.quantize_rows(t32, "i8")
    p = 1.0 / np.arange(1, rows + 1) ** 1.1
    cdf = np.cumsum(p) / p.sum()
    ranks = np.minimum(np.searchsorted(cdf, rng.random((N, 128))), rows - 1)
    idx = rng.permutation(rows)[ranks]
    w = np.concatenate([O.softmax_f32(rng.standard_normal((N, 32)).astype(np.float32)) for _ in range(4)], 1)
    out = K.bag_infer(torch.from_numpy(idx).to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(codes).to(DEV),
                      torch.from_numpy(sc).to(DEV))
    close(out.cpu().numpy(), O.bag(idx, w, codes, "i8", sc))


# ------------------------------------------------------------------------------------------------ quantisation
@pytest.mark.parametrize("kind", ["i8", "q4"])
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_quantize_bit_exact(kind, src):
    rng = np.random.default_rng(16)
    t32 = (rng.standard_normal((5000, 384)) * 0.02).astype(np.float32)
    t32[7] = 0.0                                           # zero row -> scale 1
    t32[8, 3], t32[8, 5] = 0.5, -0.5                       # tied largest magnitude
    if src == "bf16":
        bits = O.bf16_bits_rtne(t32)
        tt, t_np = bf16_from_bits(bits), O.bf16_to_f32(bits)
    else:
        tt, t_np = torch.from_numpy(t32), t32
    fn = K.quantize_int8 if kind == "i8" else K.quantize_q4
    codes, sc = fn(tt.to(DEV))
    rc, rs = O.quantize_rows(t_np, kind)
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    deq = (K.dequantize_int8 if kind == "i8" else K.dequantize_q4)(codes, sc).cpu().numpy()
    np.testing.assert_array_equal(deq, O.dequantize(rc, rs, kind).astype(np.float32))


def test_quantize_golden():
    with open(os.path.join(GOLDEN, "quant_known.json")) as f:
        g = json.load(f)
    for case in g["i8"]:
        codes, sc = K.quantize_int8(torch.tensor([case["row"]], dtype=torch.float32, device=DEV))
        assert codes[0].tolist() == case["codes"]
        assert int(sc.cpu().view(torch.int16)[0]) & 0xFFFF == case["scale_f16_bits"]
    for case in g["q4"]:
        codes, sc = K.quantize_q4(torch.tensor([case["row"]], dtype=torch.float32, device=DEV))
        assert codes[0].tolist() == case["packed"]
        assert int(sc.cpu().view(torch.int16)[0]) & 0xFFFF == case["scale_f16_bits"]


# ------------------------------------------------------------------------------------------------ decode attention
def _attention_oracle(qkv, cos, sin, kc, vc, P, H, hd):
    """fp64 restatement: RoPE (oracle/torch_path.rope convention: rotate the two halves), then softmax attention
    of the new token over cached slots 0..P-1 and itself."""
    B = qkv.shape[0]
    C = H * hd
    q = qkv[:, :C].view(B, H, hd).double()
    k = qkv[:, C:2 * C].view(B, H, hd).double()
    v = qkv[:, 2 * C:].view(B, H, hd).double()
    c, s = cos[P].double(), sin[P].double()

    def rot(x):
        a, b = x[..., :hd // 2], x[..., hd // 2:]
        return torch.cat([a * c - b * s, a * s + b * c], -1)
    qr, kr = rot(q), rot(k)
    kr_b = kr.to(torch.bfloat16)
    keys = torch.cat([kc[:, :, :P].double(), kr_b.double().unsqueeze(2)], 2)
    vals = torch.cat([vc[:, :, :P].double(), v.unsqueeze(2)], 2)
    sc = torch.einsum("bhd,bhtd->bht", qr.to(torch.bfloat16).double(), keys) / hd ** 0.5
    y = torch.einsum("bht,bhtd->bhd", torch.softmax(sc, -1), vals)
    return y.reshape(B, C), kr_b


@pytest.mark.parametrize("B,H,hd,max_len,P,rope", [(64, 6, 64, 394, 300, "bf16"), (1, 6, 64, 394, 0, "bf16"),
                                                    (1, 6, 64, 394, 393, "f32"), (3, 4, 32, 100, 57, "f32"),
                                                    (2, 2, 16, 40, 1, "bf16"), (2, 3, 128, 300, 299, "bf16"),
                                                    (5, 6, 64, 600, 511, "f32"), (20, 6, 64, 300, 250, "bf16"),
                                                    (1, 6, 64, 1100, 1050, "f32"), (64, 6, 64, 600, 64, "bf16"),
                                                    (64, 6, 64, 600, 512, "bf16"), (64, 6, 64, 600, 513, "f32"),
                                                    (2, 6, 64, 800, 768, "bf16"), (2, 6, 64, 800, 769, "f32"),
                                                    (100, 6, 64, 300, 256, "bf16"), (100, 6, 64, 300, 257, "bf16"),
                                                    (64, 6, 64, 400, 47, "bf16"), (64, 6, 64, 400, 48, "f32"),
                                                    (64, 6, 64, 400, 49, "bf16"), (64, 6, 64, 400, 383, "bf16"),
                                                    (64, 6, 64, 400, 384, "f32"), (64, 6, 64, 400, 385, "bf16"),
                                                    (48, 6, 32, 800, 768, "bf16"), (48, 6, 32, 800, 97, "f32"),
                                                    (64, 6, 128, 400, 192, "bf16"), (64, 6, 128, 400, 193, "f32"),
                                                    (2, 6, 64, 800, 512, "bf16"), (2, 6, 64, 800, 513, "f32")])
def test_decode_attention_matches_oracle(B, H, hd, max_len, P, rope):
    """512 / 384 / 256 threads per (sequence, head) (B x H below 256, below 512, from 512), head_dim 16-128, fp32
    and bf16 rope tables, position 0, the last slot, and a cache longer than one group of row loads (the rows past
    the first group loaded in a second round trip); positions on and just past a pass or a group boundary of each
    thread count: at head_dim 64, 512 threads take 64 rows a pass and 512 a group, 384 threads 48 and 384, 256
    threads 32 and 256; at 384 threads head_dim 32 takes 96 and 768, head_dim 128 24 and 192."""
    note(f"decode attention B={B} H={H} hd={hd} max_len={max_len} P={P}")
    g = torch.Generator().manual_seed(B * 1000 + P)
    C = H * hd
    qkv = torch.randn(B, 3 * C, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, H, max_len, hd, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, H, max_len, hd, generator=g).to(torch.bfloat16)
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2).float() / hd))
    ang = torch.outer(torch.arange(max_len).float(), inv)
    dt = torch.bfloat16 if rope == "bf16" else torch.float32
    cos, sin = ang.cos().to(dt), ang.sin().to(dt)
    ref, kr = _attention_oracle(qkv, cos, sin, kc, vc, P, H, hd)
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = K.decode_attention(qkv.to(DEV), cos.to(DEV), sin.to(DEV), torch.tensor(P, device=DEV), kd, vd)
    got = out.float().cpu().double()
    torch.testing.assert_close(got, ref, rtol=2 ** -7, atol=2 ** -7 * float(ref.abs().max()))
    # the new slot holds the rotated k (within one bf16 ulp of the fp64 rotation) and v; other slots untouched
    torch.testing.assert_close(kd[:, :, P].cpu().float(), kr.float(), rtol=2 ** -7, atol=1e-6)
    assert torch.equal(vd[:, :, P].cpu(), qkv[:, 2 * C:].view(B, H, hd))
    keep = [t for t in range(max_len) if t != P]
    assert torch.equal(kd[:, :, keep].cpu(), kc[:, :, keep]) and torch.equal(vd[:, :, keep].cpu(), vc[:, :, keep])


def test_decode_attention_bad_position():
    B, H, hd, L = 2, 2, 64, 16
    qkv = torch.randn(B, 3 * H * hd, device=DEV).to(torch.bfloat16)
    kc = torch.zeros(B, H, L, hd, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    cos = torch.ones(L, hd // 2, device=DEV)
    for P in (L, -1, 10 ** 6):
        out = K.decode_attention(qkv, cos, cos, torch.tensor(P, device=DEV), kc, vc)
        assert torch.isnan(out.float()).all()
        parts = K.decode_attention_proj(qkv, cos, cos, torch.tensor(P, device=DEV), kc, vc,
                                        torch.ones(64, H * hd, dtype=torch.bfloat16, device=DEV))
        assert parts.shape == (B, H, 64) and torch.isnan(parts).all()
    assert not kc.any() and not vc.any()


# B x H picks 512 / 384 / 256 threads; the wo rows cover one or several loads of a workgroup's wo registers;
# P past 512 makes the 512-thread variant load its cache rows in two groups
@pytest.mark.parametrize("B,H,hd,max_len,P,N", [(1, 6, 64, 394, 300, 384), (4, 6, 64, 1100, 767, 384),
                                                (2, 6, 64, 1100, 1000, 1500), (64, 6, 64, 394, 200, 384),
                                                (100, 6, 64, 64, 30, 384), (3, 4, 32, 100, 57, 200),
                                                (2, 2, 16, 40, 1, 1100), (2, 3, 128, 300, 299, 384),
                                                (1, 6, 64, 394, 0, 384)])
def test_decode_attention_proj_matches_attention_then_wo(B, H, hd, max_len, P, N):
    """The attention with wo folded in: parts[b, h] = bf16(y[b, h]) @ wo[:, h*hd:(h+1)*hd].T with y what
    decode_attention writes (the same arithmetic up to y), within fp32 rounding of the fp64 products (2^-20 of
    the sum of their magnitudes), and the caches written exactly as decode_attention writes them."""
    note(f"decode attention proj B={B} H={H} hd={hd} max_len={max_len} P={P} N={N}")
    g = torch.Generator().manual_seed(B * 1000 + P + N)
    C = H * hd
    qkv = torch.randn(B, 3 * C, generator=g).to(torch.bfloat16).to(DEV)
    kc = torch.randn(B, H, max_len, hd, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, H, max_len, hd, generator=g).to(torch.bfloat16).to(DEV)
    wo = (torch.randn(N, C, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2).float() / hd))
    ang = torch.outer(torch.arange(max_len).float(), inv)
    cos, sin = ang.cos().to(DEV), ang.sin().to(DEV)
    pos = torch.tensor(P, device=DEV)
    k1, v1 = kc.clone(), vc.clone()
    y = K.decode_attention(qkv, cos, sin, pos, k1, v1)
    k2, v2 = kc.clone(), vc.clone()
    parts = K.decode_attention_proj(qkv, cos, sin, pos, k2, v2, wo)
    assert parts.shape == (B, H, N) and parts.dtype == torch.float32
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    yh = y.double().cpu().view(B, H, 1, hd)
    wh = wo.double().cpu().view(N, H, hd).permute(1, 2, 0)                   # (H, hd, N)
    ref = (yh @ wh).squeeze(2)                                              # (B, H, N)
    bound = ((yh.abs() @ wh.abs()).squeeze(2)) * 2 ** -20 + 1e-30
    err = (parts.double().cpu() - ref).abs()
    assert bool((err <= bound).all()), f"worst {float((err / bound).max())} x the bound"
    # the sum over heads is the projection of the plain path (its linear kernel takes N in multiples of 16)
    if N % 16 == 0:
        proj = K.decode_linear(wo, y)
        diff = (parts.cpu().sum(1).to(torch.bfloat16).double() - proj.double().cpu()).abs()
        assert float(diff.max()) <= 2 ** -7 * float(proj.double().abs().max())


def test_decode_attention_proj_rejects():
    B, H, hd, L = 2, 2, 64, 16
    qkv = torch.zeros(B, 3 * H * hd, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(B, H, L, hd, dtype=torch.bfloat16, device=DEV)
    cos = torch.ones(L, hd // 2, device=DEV)
    pos = torch.tensor(1, device=DEV)
    with pytest.raises(ValueError):                                   # wo columns != H * head_dim
        K.decode_attention_proj(qkv, cos, cos, pos, kc, kc.clone(), torch.zeros(8, 100, dtype=torch.bfloat16,
                                                                                  device=DEV))
    with pytest.raises(ValueError):                                   # fp32 wo
        K.decode_attention_proj(qkv, cos, cos, pos, kc, kc.clone(), torch.zeros(8, H * hd, device=DEV))
    assert _lib.lib().smlm_decode_attention_proj(
        qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), cos.data_ptr(), _lib.F32, L, pos.data_ptr(), kc.data_ptr(),
        kc.data_ptr(), B, H, hd, L, None, H * hd, 8, None, None) == _lib.EINVAL


# ------------------------------------------------------------------------------------------------ decode-step helpers
@pytest.mark.parametrize("M,hidden", [(64, 1024), (1, 1024), (7, 24), (300, 256)])
def test_swiglu_matches_reference_ops(M, hidden):
    """smlm/model.py:110-118 on bf16: F.silu(a) * b, each op rounded to bf16 -- within one bf16 ulp (the exp
    implementations may differ in the last fp32 bit)."""
    g = torch.Generator().manual_seed(M + hidden)
    h = (torch.randn(M, 2 * hidden, generator=g) * 3).to(torch.bfloat16)
    got = K.swiglu(h.to(DEV)).cpu().float()
    a, b = h.chunk(2, -1)
    ref = (torch.nn.functional.silu(a.double()).to(torch.bfloat16).double() * b.double()).to(torch.bfloat16).float()
    torch.testing.assert_close(got, ref, rtol=2 ** -7, atol=1e-30)


def test_greedy_argmax_first_index_and_history():
    g = torch.Generator().manual_seed(3)
    B, V, L = 64, 32000, 20
    logits = torch.randn(B, V, generator=g).to(torch.bfloat16)
    logits[1] = 0.0                                      # all tied -> index 0
    logits[2, 17] = logits[2, 900] = 50.0                # tied maximum -> the first
    logits[3, -1] = 60.0
    hist = torch.full((B, L), -1, dtype=torch.int64, device=DEV)
    tok = torch.empty(B, dtype=torch.int64, device=DEV)
    pos = torch.tensor(4, device=DEV)
    K.greedy_argmax(logits.to(DEV), pos, tok, hist)
    ref = logits.float().argmax(-1)
    assert torch.equal(tok.cpu(), ref) and ref[1] == 0 and ref[2] == 17 and ref[3] == V - 1
    assert torch.equal(hist[:, 5].cpu(), ref) and bool((hist[:, :5] == -1).all()) and bool((hist[:, 6:] == -1).all())
    K.greedy_argmax(logits.to(DEV), torch.tensor(L - 1, device=DEV), tok, hist)   # slot L: outside, no write
    assert bool((hist[:, 6:] == -1).all())


@pytest.mark.parametrize("M,C", [(64, 384), (1, 384), (5, 100), (4096, 384), (37, 512), (3, 64), (17, 200)])
def test_add_rmsnorm_matches_reference_ops(M, C):
    """x + delta rounded to bf16 (the residual stream), then RMSNorm with fp32 statistics and bf16 weight."""
    g = torch.Generator().manual_seed(M + C)
    x = torch.randn(M, C, generator=g).to(torch.bfloat16)
    d = torch.randn(M, C, generator=g).to(torch.bfloat16)
    norm = torch.nn.RMSNorm(C, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(C, generator=g) + 0.5)
    norm = norm.to(DEV, torch.bfloat16)
    xo, h = K.add_rmsnorm(x.to(DEV), d.to(DEV), norm)
    xs = (x.double() + d.double()).to(torch.bfloat16)
    assert torch.equal(xo.cpu(), xs)
    ref = (torch.nn.functional.rms_norm(xs.double(), (C,), eps=1e-5) * norm.weight.cpu().double()).float()
    torch.testing.assert_close(h.cpu().float(), ref, rtol=2 ** -7, atol=1e-6)
    x0, h0 = K.add_rmsnorm(x.to(DEV), None, norm)
    ref0 = (torch.nn.functional.rms_norm(x.double(), (C,), eps=1e-5) * norm.weight.cpu().double()).float()
    torch.testing.assert_close(h0.cpu().float(), ref0, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("M,C", [(1, 2048), (300, 2048), (7, 40)])
def test_affine_bf16_matches_fp64(M, C):
    """The eval BatchNorm of the memory query (smlm/pkm.py:188-191) on bf16 rows: bf16(x * scale + shift) within one
    bf16 ulp of the fp64 value (one fp32 fused multiply-add, then one rounding), and equal to torch's
    BatchNorm1d(eval) of the same rows rounded to bf16 within that ulp."""
    g = torch.Generator().manual_seed(M + C)
    x = torch.randn(M, C, generator=g).to(torch.bfloat16)
    bn = torch.nn.BatchNorm1d(C).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(C, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(C, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(C, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(C, generator=g) * 0.1)
    scale = (bn.weight / torch.sqrt(bn.running_var + bn.eps)).detach()
    shift = (bn.bias - bn.running_mean * scale).detach()
    got = K.affine_bf16(x.to(DEV), scale.to(DEV), shift.to(DEV)).cpu()
    exact = x.double() * scale.double() + shift.double()
    ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(2 ** -120))) - 7)
    assert float(((got.double() - exact).abs() - ulp).max()) <= 0
    with torch.no_grad():
        ref = bn(x.float()).to(torch.bfloat16).double()
    assert float(((got.double() - ref).abs() - 2 * ulp).max()) <= 0
    with pytest.raises(ValueError):
        K.affine_bf16(x.to(DEV), scale[:-1].to(DEV), shift.to(DEV))
