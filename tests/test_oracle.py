"""Pins the CPU oracle (oracle/pkm_oracle.py) before it is trusted as the checker of the HIP kernels.

Every oracle function is checked against something that does not share its code path: torch's own casts and
ops (library routines), brute force written with Python floats and tuples instead of packed integer keys,
brute force over all NK^2 product keys (the pattern of the reference's tests/test_pkm.py:16-37), exhaustive
enumeration, and the hand-derived fixtures of tests/golden/.  The last test plants mistakes in a copy of the
oracle and shows that these checks catch them.
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.pkm_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bf16_bits_torch(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# --------------------------------------------------------------------------------------------- number formats
def test_bf16_rounding_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 100000),
        np.array([0.0, -0.0, 1.0, -1.0, 3.4e38, -3.4e38, 1e-40, -1e-40, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    # exact ties (low half 0x8000) with even and odd upper halves, and one below / above a tie
    u = (rng.integers(0, 0x7F00, 2000, dtype=np.uint32) << 16)
    ties = np.concatenate([u | 0x8000, (u | 0x10000) | 0x8000, u | 0x7FFF, u | 0x8001]).astype(np.uint32)
    x = np.concatenate([x, ties.view(np.float32), (ties | 0x80000000).view(np.float32)])
    assert np.array_equal(O.bf16_bits_rtne(x), bf16_bits_torch(x))


def _bf16_total_order():
    """All non-NaN bf16 bit patterns sorted by value, -0 placed just below +0."""
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = O.bf16_to_f32(b)
    ok = ~np.isnan(v)
    b, v = b[ok], v[ok].astype(np.float64)
    negzero = (b == 0x8000).astype(np.float64)
    return b[np.lexsort((-negzero, v))]


def test_order16_is_monotone_on_all_bf16_values():
    b = _bf16_total_order()
    codes = O.order16(b).astype(np.int64)
    assert np.all(np.diff(codes) > 0)
    all_b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(O.unorder16(O.order16(all_b)), all_b)


def test_order32_is_monotone():
    rng = np.random.default_rng(1)
    x = np.unique(np.concatenate([rng.standard_normal(200000).astype(np.float32) * 1e3,
                                  np.array([np.inf, -np.inf, 1e-45, -1e-45, 3.4e38], np.float32)]))
    x = np.concatenate([x[x < 0], np.array([-0.0, 0.0], np.float32), x[x > 0]])
    codes = O.order32(x).astype(np.float64)
    assert np.all(np.diff(codes) > 0)
    assert np.array_equal(O.unorder32(O.order32(x)).view(np.uint32), x.view(np.uint32))


# --------------------------------------------------------------------------------------------- selection
def _rank_key(v, k):
    """Python-float ranking: larger value first, +0 before -0, then lower index."""
    return (-v, 1 if (v == 0 and math.copysign(1.0, v) < 0) else 0, k)


def _bf16_float(bits):
    return float(O.bf16_to_f32(np.uint16(bits)))


def brute_select(s1_row, s2_row, knn, bf16):
    """pk_select for one (token, head) written with floats and tuples; bf16 rounding by torch's cast."""
    NK = len(s1_row)
    val = (lambda b: _bf16_float(b)) if bf16 else (lambda f: float(f))
    r1 = sorted(range(NK), key=lambda k: _rank_key(val(s1_row[k]), k))[:knn]
    r2 = sorted(range(NK), key=lambda k: _rank_key(val(s2_row[k]), k))[:knn]
    cands = []
    for i in range(knn):
        for j in range(knn):
            if (i + 1) * (j + 1) > knn:
                continue
            s32 = np.float32(val(s1_row[r1[i]])) + np.float32(val(s2_row[r2[j]]))
            if bf16:
                s = torch.tensor(float(s32), dtype=torch.float32).to(torch.bfloat16).float().item()
                if s == 0 and s32 == 0:
                    s = math.copysign(0.0, float(s32))
            else:
                s = float(s32)
            cands.append((s, r1[i] * NK + r2[j]))
    cands.sort(key=lambda c: _rank_key(c[0], c[1]))
    top = cands[:knn]
    w = torch.softmax(torch.tensor([c[0] for c in top], dtype=torch.float32), -1).numpy()
    return [c[0] for c in top], [c[1] for c in top], w


def _tie_heavy_bf16(rng, shape):
    """bf16 scores drawn from a few values (lots of exact ties, both signed zeros)."""
    vals = np.array([0x3F80, 0x3F00, 0x0000, 0x8000, 0xBF00, 0x3F40, 0x4000, 0xBF80], np.uint16)
    return vals[rng.integers(0, len(vals), shape)]


@pytest.mark.parametrize("NK,knn,kind", [(16, 4, "bf16"), (64, 8, "bf16"), (32, 32, "bf16"), (8, 1, "bf16"),
                                         (64, 8, "ties"), (128, 16, "ties"), (64, 8, "f32"), (32, 4, "f32")])
def test_pk_select_matches_float_brute_force(NK, knn, kind):
    rng = np.random.default_rng(NK + knn)
    N, H = 6, 3
    if kind == "f32":
        s1 = rng.standard_normal((N, H, NK)).astype(np.float32)
        s2 = rng.standard_normal((N, H, NK)).astype(np.float32)
    elif kind == "bf16":
        s1 = O.bf16_bits_rtne(rng.standard_normal((N, H, NK)).astype(np.float32))
        s2 = O.bf16_bits_rtne(rng.standard_normal((N, H, NK)).astype(np.float32))
    else:
        s1, s2 = _tie_heavy_bf16(rng, (N, H, NK)), _tie_heavy_bf16(rng, (N, H, NK))
    sc, idx, w = O.pk_select(s1, s2, knn)
    bf16 = kind != "f32"
    for n in range(N):
        for h in range(H):
            bs, bi, bw = brute_select(s1[n, h], s2[n, h], knn, bf16)
            assert list(idx[n, h]) == bi
            got = [_bf16_float(b) for b in sc[n, h]] if bf16 else list(sc[n, h].astype(np.float64))
            assert got == bs
            np.testing.assert_allclose(w[n, h], bw, rtol=0, atol=1e-6)


@pytest.mark.parametrize("NK,knn", [(16, 8), (16, 16), (32, 5 + 3), (8, 1), (64, 32)])
def test_pk_select_is_exact_top_k_over_all_product_keys(NK, knn):
    """fp32 sub-key scores: the selected set equals the top-knn over all NK^2 sums s1[a] + s2[b] (rows whose
    knn-th and (knn+1)-th sums tie are skipped: there the set is not unique)."""
    rng = np.random.default_rng(NK * knn)
    N, H = 40, 2
    s1 = rng.standard_normal((N, H, NK)).astype(np.float32)
    s2 = rng.standard_normal((N, H, NK)).astype(np.float32)
    sc, idx, _ = O.pk_select(s1, s2, knn)
    checked = 0
    for n in range(N):
        for h in range(H):
            full = (s1[n, h][:, None] + s2[n, h][None, :]).astype(np.float32).reshape(-1)
            order = np.argsort(-full.astype(np.float64), kind="stable")
            if knn < full.size and full[order[knn - 1]] == full[order[knn]]:
                continue
            assert set(idx[n, h].tolist()) == set(order[:knn].tolist())
            np.testing.assert_array_equal(sc[n, h], full[idx[n, h]])
            checked += 1
    assert checked > N


def test_fp64_queries_bruteforce_pattern():
    """The reference's brute-force check (tests/test_pkm.py:16-37): scores from fp64 queries and sub-keys,
    every returned index reproduces its score from the concatenated full key and is in the exact top-k."""
    rng = np.random.default_rng(3)
    N, H, NK, half, knn = 50, 3, 16, 8, 8
    q = rng.standard_normal((N, H, 2 * half))
    keys = rng.uniform(-0.25, 0.25, (H, 2, NK, half))
    s1, s2 = O.subkey_scores(q, keys)
    sc, idx, _ = O.pk_select(s1.astype(np.float32), s2.astype(np.float32), knn)
    for h in range(H):
        full_keys = np.concatenate([np.repeat(keys[h, 0], NK, 0), np.tile(keys[h, 1], (NK, 1))], axis=1)
        bf = q[:, h] @ full_keys.T
        for n in range(N):
            recomputed = full_keys[idx[n, h]] @ q[n, h]
            np.testing.assert_allclose(recomputed, sc[n, h], rtol=1e-5, atol=1e-5)
            kth = np.sort(bf[n])[::-1][knn - 1]
            assert np.all(bf[n][idx[n, h]] >= kth - 1e-5)


def test_half_topk_matches_torch_topk_without_ties():
    rng = np.random.default_rng(4)
    s = rng.standard_normal((500, 1024)).astype(np.float32)
    v, i = O.half_topk(s, 32)
    tv, ti = torch.from_numpy(s).topk(32, dim=-1)
    assert np.array_equal(i, ti.numpy())
    assert np.array_equal(v, tv.numpy())


def test_pair_counts():
    # sum_{i=1..knn} floor(knn / i): the pair list of smlm/kernels.py:200-211 has 119 entries for knn = 32
    # (its comment says 130; the list comprehension there is what defines the candidates)
    assert len(O.pairs(32)[0]) == 119
    assert len(O.pairs(64)[0]) == 280
    assert len(O.pairs(1)[0]) == 1


def test_pruned_pairs_keep_every_top_score():
    """Math fact behind the pruning: for lists sorted descending, pair (i, j) is dominated by the (i+1)(j+1)
    pairs (i' <= i, j' <= j), so the top-knn scores over all knn^2 pairs equal those over the pruned set."""
    rng = np.random.default_rng(5)
    for knn in (1, 2, 4, 8, 16, 32, 64):
        a = -np.sort(-rng.standard_normal(knn).astype(np.float32))
        b = -np.sort(-rng.standard_normal(knn).astype(np.float32))
        allv = np.sort((a[:, None] + b[None, :]).reshape(-1))[::-1][:knn]
        pi, pj = O.pairs(knn)
        pv = np.sort(a[pi] + b[pj])[::-1][:knn]
        assert np.array_equal(allv, pv)


def test_softmax_matches_torch():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((1000, 32)) * 3).astype(np.float32)
    np.testing.assert_allclose(O.softmax_f32(x), torch.softmax(torch.from_numpy(x), -1).numpy(), rtol=0, atol=1e-6)


def test_select_golden_cases():
    with open(os.path.join(GOLDEN, "select_known.json")) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        s1 = np.array(c["s1"], np.uint16).reshape(1, 1, -1)
        s2 = np.array(c["s2"], np.uint16).reshape(1, 1, -1)
        sc, idx, w = O.pk_select(s1, s2, c["knn"])
        assert idx[0, 0].tolist() == c["idx"], c["name"]
        if "score_bits" in c:
            assert sc[0, 0].tolist() == c["score_bits"], c["name"]
        assert abs(float(w.sum()) - 1.0) < 1e-6


# --------------------------------------------------------------------------------------------- value bag
@pytest.mark.parametrize("kind", ["f32", "bf16", "i8", "q4"])
def test_bag_matches_embedding_bag(kind):
    rng = np.random.default_rng(7)
    rows, D, N, K = 1000, 64, 50, 24
    t32 = (rng.standard_normal((rows, D)) * 0.02).astype(np.float32)
    idx = rng.integers(0, rows, (N, K))
    w = rng.random((N, K)).astype(np.float32)
    scales = None
    if kind == "f32":
        table, deq = t32, t32
    elif kind == "bf16":
        table = O.bf16_bits_rtne(t32)
        deq = O.bf16_to_f32(table)
    else:
        table, scales = O.quantize_rows(t32, kind)
        deq = O.dequantize(table, scales, kind).astype(np.float32)
    ref = F.embedding_bag(torch.from_numpy(idx), torch.from_numpy(np.ascontiguousarray(deq)),
                          per_sample_weights=torch.from_numpy(w), mode="sum").numpy()
    out = O.bag(idx, w, table, kind, scales)
    scale = max(1.0, float(np.abs(ref).max()))
    np.testing.assert_allclose(out / scale, ref / scale, rtol=1e-5, atol=1e-5)


def test_silu_bf16_bit_exact_against_torch_everywhere():
    """bf16(silu(p)) of smlm/kernels.py:304-307 on every finite bf16 pattern equals torch's F.silu on bf16 (fp32
    arithmetic, one rounding to bf16), and the values are bf16 numbers (an oracle that skipped the rounding, or
    rounded by truncation, fails)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(O.bf16_to_f32(bits))
    with np.errstate(over="ignore", invalid="ignore"):
        vals = O.silu_bf16(bits)
    t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    ref = F.silu(t).view(torch.int16).numpy().view(np.uint16)
    got = O.bf16_bits_rtne(vals)
    assert np.array_equal(got[finite], ref[finite])
    assert np.array_equal(O.bf16_to_f32(got[finite]).view(np.uint32), vals[finite].view(np.uint32))


def test_bag_swilu_epilogue_matches_torch():
    rng = np.random.default_rng(8)
    rows, D, N, K = 300, 32, 20, 16
    table = (rng.standard_normal((rows, D)) * 0.1).astype(np.float32)
    idx = rng.integers(0, rows, (N, K))
    w = rng.random((N, K)).astype(np.float32)
    pre = O.bf16_bits_rtne(rng.standard_normal((N, D)).astype(np.float32) * 2)
    ref = F.embedding_bag(torch.from_numpy(idx), torch.from_numpy(table), per_sample_weights=torch.from_numpy(w),
                          mode="sum")
    pre_t = torch.from_numpy(pre.view(np.int16)).view(torch.bfloat16)
    ref = ref * F.silu(pre_t).float()
    out = O.bag(idx, w, table, "f32", pre=pre)
    np.testing.assert_allclose(out, ref.numpy(), rtol=2 ** -7, atol=1e-6)
    ob = O.bf16_to_f32(O.bag(idx, w, table, "f32", pre=pre, out_bf16=True))
    np.testing.assert_allclose(ob, ref.to(torch.bfloat16).float().numpy(), rtol=2 ** -7,
                               atol=2 ** -8 * float(ref.abs().max()))


# --------------------------------------------------------------------------------------------- table formats
def test_quantize_known_answers():
    with open(os.path.join(GOLDEN, "quant_known.json")) as f:
        g = json.load(f)
    for kind in ("i8", "q4"):
        for case in g[kind]:
            row = np.array([case["row"]], np.float32)
            codes, d = O.quantize_rows(row, kind)
            assert int(d.view(np.uint16)[0]) == case["scale_f16_bits"], (kind, case["row"])
            if kind == "i8":
                assert codes[0].tolist() == case["codes"]
            else:
                assert codes[0].tolist() == case["packed"]


@pytest.mark.parametrize("kind,lo,hi", [("i8", -128, 127), ("q4", -8, 7)])
def test_quantize_error_bound(kind, lo, hi):
    """|dequant - w| <= |d| / 2 wherever the code is not clamped; codes stay in [lo, hi]."""
    rng = np.random.default_rng(9)
    t = (rng.standard_normal((2000, 64)) * 0.02).astype(np.float32)
    codes, d = O.quantize_rows(t, kind)
    deq = O.dequantize(codes, d, kind)
    raw = O.row_values(codes, np.arange(len(codes)), kind)
    assert raw.min() >= lo and raw.max() <= hi
    inside = (raw > lo) & (raw < hi)
    err = np.abs(deq - t.astype(np.float64))
    bound = np.abs(d.astype(np.float64))[:, None] / 2 * (1 + 1e-6)
    assert np.all(err[inside] <= np.broadcast_to(bound, err.shape)[inside])


def test_planted_mistakes_are_caught(monkeypatch):
    """A plausible slip in the oracle (ties -> higher index, no bf16 rounding of candidate sums, ties of the
    quantiser's max to the last element) must fail one of the checks above."""
    rng = np.random.default_rng(10)
    s1, s2 = _tie_heavy_bf16(rng, (4, 2, 64)), _tie_heavy_bf16(rng, (4, 2, 64))

    def agrees():
        sc, idx, _ = O.pk_select(s1, s2, 8)
        for n in range(4):
            for h in range(2):
                if list(idx[n, h]) != brute_select(s1[n, h], s2[n, h], 8, True)[1]:
                    return False
        return True

    assert agrees()
    orig_keys = O.half_keys
    monkeypatch.setattr(O, "half_keys", lambda s: (O.order16(s).astype(np.uint64) << np.uint64(16))
                        | np.arange(s.shape[1], dtype=np.uint64))          # ties -> higher index
    assert not agrees()
    monkeypatch.setattr(O, "half_keys", orig_keys)
    monkeypatch.setattr(O, "bf16_bits_rtne", lambda x: (np.ascontiguousarray(x, np.float32).view(np.uint32)
                                                        >> 16).astype(np.uint16))   # truncation
    with open(os.path.join(GOLDEN, "quant_known.json")) as f:
        g = json.load(f)
    x = np.array([1.00390625 + 2 ** -9], np.float32)
    assert O.bf16_bits_rtne(x)[0] != bf16_bits_torch(x)[0]
    monkeypatch.undo()
    row = np.array([g["i8"][2]["row"]], np.float32)   # -0.5 and +0.5 tie for the largest magnitude
    t = row[0]
    last = len(t) - 1 - int(np.abs(t[::-1]).argmax())
    d_wrong = np.float16(t[last] / np.float32(-128))
    assert int(np.array([d_wrong]).view(np.uint16)[0]) != g["i8"][2]["scale_f16_bits"]
