"""The Engram oracle (oracle/engram_oracle.py) pinned on the CPU: the hash against a scalar brute force on Python
integers and the reference's own hash properties; the module's conv and norms against torch's library routines,
chunked evaluation against the full sequence, causality and the zero-conv closed form."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.engram_oracle as E


def _wrap64(v):
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >> 63 else v


def brute_rows(c, mult, orders, heads, rows):
    """Scalar hash on Python integers: products wrapped to signed 64 bits, >> as floor division by 2^17."""
    history = max(orders) - 1
    B, L = len(c), len(c[0])
    T = L - history
    out = []
    for b in range(B):
        per_t = []
        for t in range(T):
            looks = []
            for o, n in enumerate(orders):
                for h in range(heads):
                    x = 0
                    for i in range(n):
                        x ^= _wrap64(int(c[b][history + t - i]) * int(mult[o][h][i]))
                    x = _wrap64(x ^ (x // (1 << 17)))
                    looks.append(x % rows + (o * heads + h) * rows)          # Python % is non-negative here
            per_t.append(looks)
        out.append(per_t)
    return np.array(out, dtype=np.int64)


def _mult(orders, heads, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(0, 2 ** 30, (len(orders), heads, max(orders)), generator=g) * 2 + 1).numpy()


@pytest.mark.parametrize("orders,heads,rows", [((2, 3), 4, 101), ((2, 3), 8, 524287), ((1, 2, 4), 3, 97)])
def test_ngram_rows_matches_brute_force(orders, heads, rows):
    rng = np.random.default_rng(len(orders) * 10 + heads)
    mult = _mult(orders, heads, 0)
    c = rng.integers(0, 50000, (2, max(orders) - 1 + 9))
    c[0, 0] = 50000                                          # the pad id
    np.testing.assert_array_equal(E.ngram_rows(c, mult, orders, heads, rows), brute_rows(c, mult, orders, heads, rows))
    # ids large enough that products wrap around and x turns negative: the mod stays non-negative
    big = rng.integers(2 ** 40, 2 ** 62, (1, max(orders) - 1 + 5))
    got = E.ngram_rows(big, mult, orders, heads, rows)
    np.testing.assert_array_equal(got, brute_rows(big, mult, orders, heads, rows))


def test_ngram_rows_reference_properties():
    """tests/test_engram.py:35-48: head j reads its own row block, the hash is deterministic, a bigram head only
    depends on tokens t-1 and t."""
    orders, heads, rows = (2, 3), 4, 101
    mult = _mult(orders, heads, 0)
    c = np.random.default_rng(1).integers(0, 1000, (3, 2 + 50))
    r = E.ngram_rows(c, mult, orders, heads, rows)
    assert r.shape == (3, 50, 8)
    for j in range(8):
        assert ((r[..., j] >= j * rows) & (r[..., j] < (j + 1) * rows)).all()
    c2 = c.copy()
    c2[:, 0] = (c2[:, 0] + 1) % 1000                          # token t-2 of the first position
    r2 = E.ngram_rows(c2, mult, orders, heads, rows)
    np.testing.assert_array_equal(r2[:, 0, :4], r[:, 0, :4])
    assert (r2[:, 0, 4:] != r[:, 0, 4:]).any()


def _params(d, n_lookups, hd, rows, ks, seed, conv_std=0.3):
    g = torch.Generator().manual_seed(seed)
    f = lambda *s, std=1.0: torch.randn(*s, generator=g, dtype=torch.float64) * std  # noqa: E731
    return {"values": f(n_lookups * rows, hd, std=0.3), "w_k": f(d, n_lookups * hd, std=0.1),
            "w_v": f(d, n_lookups * hd, std=0.1), "h_norm": 1 + f(d, std=0.1), "k_norm": 1 + f(d, std=0.1),
            "v_norm": 1 + f(d, std=0.1), "conv": f(d, 1, ks, std=conv_std)}


def test_engram_forward_conv_and_norms_against_torch():
    d, dil, ks = 16, 3, 4
    g = torch.Generator().manual_seed(2)
    full = torch.randn(2, 9 + (ks - 1) * dil, d, generator=g, dtype=torch.float64)
    w = torch.randn(d, 1, ks, generator=g, dtype=torch.float64)
    ref = F.conv1d(full.transpose(1, 2), w, dilation=dil, groups=d).transpose(1, 2)
    torch.testing.assert_close(E.causal_depthwise_conv(full, w, dil, 9), ref, rtol=1e-12, atol=1e-12)
    x = torch.randn(3, 5, d, generator=g, dtype=torch.float64)
    norm = torch.nn.RMSNorm(d, eps=1e-5).double()
    with torch.no_grad():
        norm.weight.copy_(torch.rand(d, generator=g, dtype=torch.float64) + 0.5)
        torch.testing.assert_close(E.rms_norm(x, norm.weight, 1e-5), norm(x), rtol=1e-12, atol=1e-12)


def test_engram_forward_chunks_causality_and_zero_conv():
    d, L, hd, rows, ks, dil = 16, 6, 4, 37, 4, 3
    p = _params(d, L, hd, rows, ks, 3)
    g = torch.Generator().manual_seed(4)
    B, T = 2, 20
    h = torch.randn(B, T, d, generator=g, dtype=torch.float64)
    r = torch.randint(0, rows, (B, T, L), generator=g) + torch.arange(L) * rows
    full, _ = E.engram_forward(p, h, r, 1e-5, dil)
    past, parts = None, []
    for a, n in ((0, 7), (7, 1), (8, 1), (9, 11)):
        y, past = E.engram_forward(p, h[:, a:a + n], r[:, a:a + n], 1e-5, dil, past)
        parts.append(y)
    torch.testing.assert_close(torch.cat(parts, 1), full, rtol=1e-12, atol=1e-12)
    h2, r2 = h.clone(), r.clone()
    h2[:, 12:] += 1.0
    r2[:, 12:] = (r2[:, 12:] + 1) % rows + torch.arange(L) * rows
    y2, _ = E.engram_forward(p, h2, r2, 1e-5, dil)
    torch.testing.assert_close(y2[:, :12], full[:, :12], rtol=0, atol=0)
    p0 = dict(p, conv=torch.zeros_like(p["conv"]))
    y0, _ = E.engram_forward(p0, h, r, 1e-5, dil)
    e = p["values"][r.reshape(-1)].view(B, T, -1)
    k, v = e @ p["w_k"].T, e @ p["w_v"].T
    hn = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-5) * p["h_norm"]
    kn = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-5) * p["k_norm"]
    alpha = torch.sigmoid((hn * kn).sum(-1, keepdim=True) / math.sqrt(d))
    torch.testing.assert_close(y0, alpha * v, rtol=1e-12, atol=1e-12)   # SiLU(0) = 0: Y = v~
