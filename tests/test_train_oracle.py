"""The training-backward oracle (oracle/train_oracle.py) pinned against torch's CPU autograd, torch.optim.Adam and
the closed-form special cases of the compact Adam states.  CPU only."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.pkm_oracle as O
import oracle.train_oracle as T


def _selection(N, H, NK, knn, seed):
    g = torch.Generator().manual_seed(seed)
    s1 = torch.randn(N, H, NK, generator=g)
    s2 = torch.randn(N, H, NK, generator=g)
    _, idx, _ = O.pk_select(s1.numpy(), s2.numpy(), knn)
    return s1, s2, torch.from_numpy(idx.astype(np.int64))


@pytest.mark.parametrize("with_gs,with_gw", [(True, True), (False, True), (True, False)])
def test_select_backward_matches_autograd(with_gs, with_gw):
    """fp32 scores: PKSelect.backward equals the autograd of gather(s1) + gather(s2) -> softmax on the same
    selection (the reference's torch path, smlm/pkm.py:130-136 + 205-208)."""
    N, H, NK, knn = 5, 3, 64, 16
    s1, s2, idx = _selection(N, H, NK, knn, 1)
    s1.requires_grad_(True)
    s2.requires_grad_(True)
    scores = s1.gather(-1, idx // NK) + s2.gather(-1, idx % NK)
    w = torch.softmax(scores, -1)
    g = torch.Generator().manual_seed(2)
    Gs, Gw = torch.randn(N, H, knn, generator=g), torch.randn(N, H, knn, generator=g)
    loss = (scores * Gs).sum() * with_gs + (w * Gw).sum() * with_gw
    loss.backward()
    ds1, ds2 = T.select_backward(idx.numpy(), w.detach().numpy(), Gs.numpy() if with_gs else None,
                                 Gw.numpy() if with_gw else None, NK, bf16=False)
    np.testing.assert_allclose(ds1, s1.grad.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ds2, s2.grad.numpy(), rtol=1e-5, atol=1e-6)


def test_select_backward_bf16_rounds_before_and_after_the_scatter():
    """bf16 scores: the selected scores' gradient is rounded to bf16, summed in fp32 per sub-key (torch's
    scatter_add, a library routine, here) and rounded once more (smlm/kernels.py:260-265)."""
    N, H, NK, knn = 4, 2, 32, 32      # knn = NK: every sub-key index repeats across the Cartesian pairs
    _, _, idx = _selection(N, H, NK, knn, 3)
    g = torch.Generator().manual_seed(4)
    w = torch.softmax(torch.randn(N, H, knn, generator=g), -1)
    Gs, Gw = torch.randn(N, H, knn, generator=g), torch.randn(N, H, knn, generator=g)
    dl = w * (Gw - (w * Gw).sum(-1, keepdim=True)) + Gs
    ds = dl.to(torch.bfloat16).float()
    z = torch.zeros(N, H, NK)
    r1 = z.scatter_add(-1, idx // NK, ds).to(torch.bfloat16).float()
    r2 = z.scatter_add(-1, idx % NK, ds).to(torch.bfloat16).float()
    ds1, ds2 = T.select_backward(idx.numpy(), w.numpy(), Gs.numpy(), Gw.numpy(), NK, bf16=True)
    assert (np.bincount((idx // NK).reshape(-1).numpy()) > 1).any()
    np.testing.assert_array_equal(ds1, r1.numpy())
    np.testing.assert_array_equal(ds2, r2.numpy())


def test_bag_backward_rows_matches_embedding_bag_autograd():
    """acc / touched / per-sample-weight gradient against the autograd of F.embedding_bag (fp64)."""
    N, K, D, rows = 7, 12, 24, 50
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(0, rows, (N, K), generator=g)
    idx[0, :4] = 3                                   # repeated rows inside and across bags
    idx[1, 0] = 3
    table = torch.randn(rows, D, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.rand(N, K, generator=g, dtype=torch.float64, requires_grad=True)
    G = torch.randn(N, D, generator=g, dtype=torch.float64)
    out = F.embedding_bag(idx, table, per_sample_weights=w, mode="sum")
    (out * G).sum().backward()
    acc0 = np.random.default_rng(6).standard_normal((rows, D))
    touched0 = np.zeros(rows, dtype=bool)
    touched0[rows - 1] = True                        # a flag from an earlier micro-batch stays set
    gw, acc, touched = T.bag_backward_rows(G.numpy(), idx.numpy(), w.detach().numpy(), table.detach().numpy(),
                                           acc0, touched0)
    np.testing.assert_allclose(gw, w.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(acc - acc0, table.grad.numpy(), rtol=1e-12, atol=1e-12)
    expect = np.zeros(rows, dtype=bool)
    expect[idx.reshape(-1).numpy()] = True
    expect[rows - 1] = True
    np.testing.assert_array_equal(touched, expect)


def test_lazy_adam_matches_torch_adam_on_rows_touched_every_step():
    rows, D = 20, 16
    rng = np.random.default_rng(7)
    p = rng.standard_normal((rows, D)).astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    hot = np.array([1, 4, 5, 11, 19])
    ref = torch.from_numpy(p[hot].copy()).requires_grad_(True)
    adam = torch.optim.Adam([ref], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, foreach=False, fused=False)
    p0 = p.copy()
    for step in range(1, 4):
        acc = np.zeros_like(p)
        acc[hot] = rng.standard_normal((len(hot), D)).astype(np.float32)
        touched = np.zeros(rows, dtype=bool)
        touched[hot] = True
        scale = 0.5 if step == 2 else 1.0
        p, m, v, acc_after, touched_after = T.lazy_adam(p, m, v, acc, touched, scale, step, 1e-2, 0.9, 0.95, 1e-8)
        ref.grad = torch.from_numpy(acc[hot] * np.float32(scale))
        adam.step()
        assert not acc_after.any() and not touched_after.any()
    np.testing.assert_allclose(p[hot], ref.detach().numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(m[hot], adam.state[ref]["exp_avg"].numpy(), rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(v[hot], adam.state[ref]["exp_avg_sq"].numpy(), rtol=1e-5, atol=1e-10)
    cold = np.setdiff1d(np.arange(rows), hot)
    np.testing.assert_array_equal(p[cold], p0[cold])
    assert not m[cold].any() and not v[cold].any()


def _first_step(int8):
    rows, D = 6, 32
    rng = np.random.default_rng(8)
    p = rng.standard_normal((rows, D)).astype(np.float32)
    acc = (rng.standard_normal((rows, D)) * 1e-2).astype(np.float32)
    acc[2] = 0.0                                      # a touched row with a zero gradient
    acc[3, 5] = 0.0                                   # a zero coordinate
    touched = np.array([True, True, True, True, False, True])
    if int8:
        m, v = np.zeros((rows, D), np.int8), np.zeros((rows, D), np.uint8)
        ms, vs = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    else:
        m, v = np.zeros((rows, D), np.float32), np.zeros((rows, D), np.float32)
        ms = vs = None
    out = T.lazy_adam_lowmem(p, m, v, ms, vs, acc, touched, 1.0, 1, 1e-2, 0.9, 0.95, 1e-8, int8)
    ref = T.lazy_adam(p, np.zeros((rows, D), np.float32), np.zeros((rows, D), np.float32), acc, touched, 1.0, 1,
                      1e-2, 0.9, 0.95, 1e-8)
    return p, acc, touched, out, ref


def test_lazy_adam_bf16_first_step():
    p, acc, touched, (p1, m1, v1, _, _, acc1, t1), (pr, mr, vr, _, _) = _first_step(False)
    np.testing.assert_allclose(p1, pr, rtol=1e-6, atol=1e-9)      # the update uses the fresh fp32 moments
    np.testing.assert_array_equal(p1[~touched], p[~touched])
    for got, fresh in ((m1, mr), (v1, vr)):
        one_ulp = np.abs(T.round_to(fresh, True)) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(got - T.round_to(fresh, True)) <= one_ulp)
        np.testing.assert_array_equal(got, T.round_to(got, True))   # stored values are bf16
    assert not acc1[touched].any() and not t1.any()
    np.testing.assert_array_equal(acc1[~touched], acc[~touched])    # unread rows keep their accumulator


def test_lazy_adam_int8_first_step_codes():
    p, acc, touched, (p1, mq, vq, ms, vs, acc1, t1), (pr, mr, vr, _, _) = _first_step(True)
    np.testing.assert_allclose(p1, pr, rtol=1e-6, atol=1e-9)
    for r in np.flatnonzero(touched):
        if not acc[r].any():                          # zero row: zero codes and zero scales, no update
            assert not mq[r].any() and not vq[r].any() and ms[r] == 0 and vs[r] == 0
            np.testing.assert_array_equal(p1[r], p[r])
            continue
        j = np.argmax(np.abs(mr[r]))
        assert abs(int(mq[r, j])) == 127 and np.sign(mq[r, j]) == np.sign(mr[r, j])
        assert vq[r].max() == 255
        assert np.all(vq[r][vr[r] > 0] >= 1) and np.all(vq[r][vr[r] == 0] == 0)
        np.testing.assert_allclose(ms[r], np.abs(mr[r]).max(), rtol=1e-6)
        np.testing.assert_allclose(vs[r], np.sqrt(np.sqrt(vr[r])).max(), rtol=1e-6)
        m_dec = np.sign(mq[r]) * (mq[r].astype(np.float64) / 127) ** 2 * ms[r]
        v_dec = (vq[r].astype(np.float64) / 255 * vs[r]) ** 4
        assert np.all(np.abs(m_dec - mr[r]) <= 2.0 / 127 * ms[r])
        assert np.all(np.abs(np.sqrt(np.sqrt(v_dec)) - np.sqrt(np.sqrt(vr[r]))) <= 1.0 / 255 * vs[r])
    np.testing.assert_array_equal(p1[~touched], p[~touched])
    assert not mq[~touched].any() and not acc1[touched].any() and not t1.any()


def _rn32(x):
    """The float32 nearest to the rational x, ties to even (x zero or in the normal range)."""
    from fractions import Fraction
    if x == 0:
        return np.float32(0)
    c = np.float32(float(x))
    cands = [np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))]
    return min(cands, key=lambda t: (abs(Fraction(float(t)) - x), int(np.float32(t).view(np.uint32)) & 1))


def test_code_division_by_corrected_reciprocal_is_the_ieee_quotient():
    """The int8 lazy Adam decodes its codes with q = c * RN(1/DEN), e = fma(-q, DEN, c), q' = fma(e, RN(1/DEN), q)
    instead of an IEEE division (csrc/pkm_train.hip: div_code).  Every code of both moments, in exact rational
    arithmetic with one rounding per operation, against the correctly rounded c / DEN."""
    from fractions import Fraction
    for den, lo, hi in ((127, -127, 127), (255, 0, 255)):
        r = _rn32(Fraction(1, den))
        assert r == np.float32(1) / np.float32(den)
        for ci in range(lo, hi + 1):
            c = Fraction(ci)
            q = _rn32(c * Fraction(float(r)))
            e = _rn32(c - Fraction(float(q)) * den)
            q2 = _rn32(Fraction(float(e)) * Fraction(float(r)) + Fraction(float(q)))
            assert q2 == _rn32(Fraction(ci, den)) == np.float32(ci) / np.float32(den), (den, ci)
    # a plain product with the reciprocal is not enough: it differs for some codes of each moment
    c = np.arange(-127, 128, dtype=np.float32)
    assert np.any(c * (np.float32(1) / np.float32(127)) != c / np.float32(127))
    c = np.arange(0, 256, dtype=np.float32)
    assert np.any(c * (np.float32(1) / np.float32(255)) != c / np.float32(255))


def test_torch_path_bag_backward_matches_the_oracle():
    """oracle/torch_path.bag_backward_rows (the reference's torch branch, bench.py's CPU baseline of the bag backward)
    against the numpy restatement: the per-sample-weight gradient and the accumulator within fp32 rounding, the flags
    exact, with rows read several times in a bag and across bags."""
    import oracle.torch_path as TP
    g = torch.Generator().manual_seed(3)
    N, K, D, rows = 64, 16, 48, 200
    idx = torch.randint(0, rows, (N, K), generator=g)
    idx[0, :4] = 5
    idx[-1, 0] = 5
    w, G = torch.rand(N, K, generator=g), torch.randn(N, D, generator=g)
    table = torch.randn(rows, D, generator=g)
    acc0 = torch.randn(rows, D, generator=g) * 0.1
    t0 = torch.zeros(rows, dtype=torch.bool)
    t0[rows - 1] = True
    acc, t = acc0.clone(), t0.clone()
    gw = TP.bag_backward_rows(G, idx, w, table, acc, t)
    rgw, racc, rt = T.bag_backward_rows(G.numpy(), idx.numpy(), w.numpy(), table.numpy(), acc0.numpy(), t0.numpy())
    np.testing.assert_allclose(gw.numpy(), rgw, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(acc.numpy(), racc, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(t.numpy(), rt)


def test_torch_path_lazy_adam_fp32_matches_the_oracle():
    """oracle/torch_path.lazy_adam_fp32_step (the reference's fp32 torch path: one dense torch.optim.Adam step with the
    unread rows put back, bench.py's CPU baseline of the table optimizer) against the numpy lazy Adam over two steps
    with different touched rows: touched rows within fp32 rounding, untouched rows unchanged bit for bit."""
    import oracle.torch_path as TP
    rng = np.random.default_rng(4)
    rows, D, lr, b1, b2, eps = 50, 16, 1e-3, 0.9, 0.95, 1e-8
    p = rng.standard_normal((rows, D)).astype(np.float32)
    param = torch.nn.Parameter(torch.tensor(p))
    adam = torch.optim.Adam([param], lr=lr, betas=(b1, b2), eps=eps)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for step in (1, 2):
        touched = rng.random(rows) < 0.6
        acc = np.where(touched[:, None], rng.standard_normal((rows, D)), 0).astype(np.float32)
        before = param.detach().clone()
        acc_t, t_t = torch.tensor(acc), torch.tensor(touched)
        TP.lazy_adam_fp32_step(param, adam, acc_t, t_t)
        p, m, v, _, _ = T.lazy_adam(p, m, v, acc, touched, 1.0, step, lr, b1, b2, eps)
        got = param.detach().numpy()
        np.testing.assert_allclose(got[touched], p[touched], rtol=1e-6, atol=1e-7)
        np.testing.assert_array_equal(got[~touched], before.numpy()[~touched])
        # torch forms the first moment with lerp_, the oracle as b1 m + (1 - b1) g: equal up to fp32 rounding
        np.testing.assert_allclose(adam.state[param]["exp_avg"].numpy(), m, rtol=1e-6, atol=1e-7)
        assert not acc_t.any() and not t_t.any()


def test_torch_path_select_backward_matches_the_oracle():
    """oracle/torch_path.select_backward (the reference's PKSelect.backward in torch ops, bench.py's CPU baseline of the
    selection backward) against the numpy restatement, bf16 and fp32 scores: within one bf16 ulp / fp32 rounding of
    the per-sub-key sums, unselected sub-keys exactly zero."""
    import oracle.torch_path as TP
    g = torch.Generator().manual_seed(8)
    N, H, NK, knn = 6, 3, 64, 16
    for dtype in (torch.bfloat16, torch.float32):
        s1 = torch.randn(N, H, NK, generator=g).to(dtype)
        s2 = torch.randn(N, H, NK, generator=g).to(dtype)
        sc, idx = TP.pkm_select_torch(s1.float(), s2.float(), knn)
        w = torch.softmax(sc, -1)
        gs = torch.randn(N, H, knn, generator=g).to(dtype)
        gw = torch.randn(N, H, knn, generator=g)
        d1, d2 = TP.select_backward(idx, w, gs, gw, NK, dtype)
        bf16 = dtype == torch.bfloat16
        r1, r2 = T.select_backward(idx.numpy(), w.numpy(), gs.float().numpy(), gw.numpy(), NK, bf16)
        for got, ref in ((d1, r1), (d2, r2)):
            got = got.float().numpy()
            tol = np.abs(ref) * (2.0 ** -7 if bf16 else 1e-6) + 1e-7
            assert np.all(np.abs(got - ref) <= tol)
            assert not got[ref == 0].any()
