"""Training-side kernels against the CPU oracle (oracle/train_oracle.py, pinned in tests/test_train_oracle.py):
selection backward (smlm_pkm_select_backward), row-sparse bag backward (smlm_bag_backward_rows) and the lazy row
Adam (smlm_lazy_adam) with fp32, bf16 and int8 moments.

Bars: the lazy Adam is bit-exact (same operation order, IEEE division and square root, no fused multiply-add).
The selection backward is bit-exact up to the softmax backward's wavefront sum (the oracle sums w * g_w in
numpy's order): bf16 outputs within one bf16 ulp and fp32 outputs within 1e-5 relative, and every element whose
sub-key is not selected is exactly zero.  The bag backward's accumulator (a fixed order in the default, sorted form;
fp32 atomic adds in no fixed order in the other): within 1e-5 of the summed magnitudes; the per-sample-weight
gradient within 1e-5; the flags exact; the sorted form gives the same bits on every call."""
import numpy as np
import pytest
import torch

import oracle.train_oracle as T
from smlm_hip import kernels as KR

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(msg, flush=True)


def _ulp_bf16(x):
    return np.abs(T.round_to(x, True)) * 2.0 ** -7 + 2.0 ** -133


@pytest.mark.parametrize("N,H,NK,knn,dtype,gs,gw", [
    (5, 4, 2048, 32, torch.bfloat16, True, True),
    (9, 4, 4096, 32, torch.bfloat16, False, True),
    (3, 2, 64, 64, torch.float32, True, True),
    (7, 3, 8, 8, torch.bfloat16, True, False),
    (4, 4, 1024, 16, torch.float32, False, True),
    # shapes of the reference's torch path: non-power-of-two n_keys and knn, knn > 64
    (6, 3, 24, 4, torch.bfloat16, True, True),
    # rows that are not whole 16-byte chunks (zeros element by element, then the sums)
    (5, 2, 30, 6, torch.bfloat16, True, True),
    (4, 3, 50, 10, torch.float32, True, True),
    (5, 2, 1000, 5, torch.float32, True, True),
    (3, 4, 4096, 128, torch.bfloat16, True, True),
    (4, 2, 100, 100, torch.float32, False, True),
])
def test_select_backward_matches_oracle(N, H, NK, knn, dtype, gs, gw):
    note(f"select backward N={N} H={H} NK={NK} knn={knn} {dtype} g_scores={gs} g_w={gw}")
    g = torch.Generator().manual_seed(N * NK + knn)
    s1 = torch.randn(N, H, NK, generator=g).to(dtype).to(DEV)
    s2 = torch.randn(N, H, NK, generator=g).to(dtype).to(DEV)
    _, idx, w = KR.pk_select(s1, s2, knn)
    G_s = torch.randn(N, H, knn, generator=g).to(dtype) if gs else None
    G_w = torch.randn(N, H, knn, generator=g) if gw else None
    ds1, ds2 = KR.pk_select_backward(idx, w, None if G_s is None else G_s.to(DEV),
                                    None if G_w is None else G_w.to(DEV), NK, dtype)
    torch.cuda.synchronize()
    bf16 = dtype == torch.bfloat16
    r1, r2 = T.select_backward(idx.cpu().numpy(), w.cpu().numpy(), None if G_s is None else G_s.float().numpy(),
                               None if G_w is None else G_w.numpy(), NK, bf16)
    i = idx.cpu().numpy()
    for got, ref, sub in ((ds1, r1, i // NK), (ds2, r2, i % NK)):
        got = got.float().cpu().numpy()
        mask = np.zeros(got.shape, dtype=bool)
        np.put_along_axis(mask, sub, True, axis=-1)
        assert not got[~mask].any()                       # every unselected sub-key: exactly zero
        if bf16:
            assert np.all(np.abs(got - ref) <= _ulp_bf16(ref))
            assert (got == ref).mean() > 0.97
        else:
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7)


def test_pkselect_autograd_matches_oracle():
    note("PKSelect autograd")
    N, H, NK, knn = 6, 4, 512, 32
    g = torch.Generator().manual_seed(11)
    s1 = torch.randn(N, H, NK, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    s2 = torch.randn(N, H, NK, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    scores, idx, w = KR.PKSelect.apply(s1, s2, knn)
    Gs = torch.randn(N, H, knn, generator=g).to(torch.bfloat16)
    Gw = torch.randn(N, H, knn, generator=g)
    ((scores.float() * Gs.float().to(DEV)).sum() + (w * Gw.to(DEV)).sum()).backward()
    r1, r2 = T.select_backward(idx.cpu().numpy(), w.detach().cpu().numpy(), Gs.float().numpy(), Gw.numpy(), NK,
                               True)
    for got, ref in ((s1.grad, r1), (s2.grad, r2)):
        assert got.dtype == torch.bfloat16
        got = got.float().cpu().numpy()
        assert np.all(np.abs(got - ref) <= _ulp_bf16(ref))


@pytest.mark.parametrize("N,K,D,rows,tdtype", [(33, 128, 384, 1000, torch.float32), (5, 7, 100, 50, torch.float32),
                                               (17, 64, 384, 300, torch.bfloat16), (3, 40, 512, 20, torch.float32),
                                               # runs longer than a wavefront and across workgroups
                                               (64, 128, 384, 3, torch.float32),
                                               # K = 1: 64 tokens per workgroup; K > 512: one token per workgroup
                                               (700, 1, 64, 50, torch.float32), (3, 600, 64, 500, torch.bfloat16)])
@pytest.mark.parametrize("ordered", [True, False])
def test_bag_backward_rows_matches_oracle(N, K, D, rows, tdtype, ordered):
    note(f"bag backward N={N} K={K} D={D} rows={rows} {tdtype} ordered={ordered}")
    g = torch.Generator().manual_seed(N + K + D)
    idx = torch.randint(0, rows, (N, K), generator=g)
    idx[0, : min(K, 5)] = 1                                # a row read several times in a bag and across bags
    idx[-1, 0] = 1
    w = torch.rand(N, K, generator=g)
    table = torch.randn(rows, D, generator=g).to(tdtype)
    G = torch.randn(N, D, generator=g)
    acc0 = torch.randn(rows, D, generator=g) * 0.1
    t0 = torch.zeros(rows, dtype=torch.bool)
    t0[rows - 1] = True
    acc, touched = acc0.to(DEV), t0.to(DEV)
    gw = KR.bag_backward_rows(G.to(DEV), idx.to(DEV), w.to(DEV), table.to(DEV), acc, touched, ordered=ordered)
    torch.cuda.synchronize()
    rgw, racc, rt = T.bag_backward_rows(G.numpy(), idx.numpy(), w.numpy(), table.float().numpy(), acc0.numpy(),
                                        t0.numpy())
    mag_gw = np.abs(G.numpy()) @ np.abs(table.float().numpy()).T
    np.testing.assert_array_less(np.abs(gw.cpu().numpy() - rgw), 1e-5 * np.take_along_axis(mag_gw, idx.numpy(), 1)
                                 + 1e-6)
    mag = np.zeros((rows, D))
    np.add.at(mag, idx.reshape(-1).numpy(), (np.abs(w.numpy())[..., None] * np.abs(G.numpy())[:, None]).reshape(
        N * K, D))
    np.testing.assert_array_less(np.abs(acc.cpu().numpy() - racc), 1e-5 * (mag + np.abs(acc0.numpy())) + 1e-7)
    np.testing.assert_array_equal(touched.cpu().numpy(), rt)


@pytest.mark.parametrize("ordered", [True, False])
def test_bag_backward_rows_index_outside_table(ordered):
    note(f"bag backward: index outside the table, ordered={ordered}")
    N, K, D, rows = 2, 3, 64, 10
    idx = torch.tensor([[0, 10, 2], [3, -1, 3]])
    acc = torch.zeros(rows, D, device=DEV)
    touched = torch.zeros(rows, dtype=torch.bool, device=DEV)
    gw = KR.bag_backward_rows(torch.ones(N, D, device=DEV), idx.to(DEV), torch.ones(N, K, device=DEV),
                             torch.ones(rows, D, device=DEV), acc, touched, ordered=ordered)
    gw = gw.cpu()
    assert torch.isnan(gw[0, 1]) and torch.isnan(gw[1, 1]) and not torch.isnan(gw[:, [0, 2]]).any()
    assert touched.cpu().nonzero().view(-1).tolist() == [0, 2, 3]
    np.testing.assert_array_equal(acc.cpu().sum(1).numpy(), [64, 0, 64, 128, 0, 0, 0, 0, 0, 0])


@pytest.mark.parametrize("N,K,rows,hot", [(256, 128, 1000, 0.5), (1, 5, 10, 0.0), (1, 64, 3, 0.0), (5, 13, 7, 0.9),
                                          (1, 65, 2, 0.0), (300, 1, 40, 0.0),
                                          # one run over ~28 whole 32-chunk groups (added by their group sums)
                                          (512, 128, 50, 0.9)])
def test_bag_backward_ordered_is_repeatable_and_matches_oracle(N, K, rows, hot):
    """The ordered bag backward gives the same bits on every call (each accumulator row has one writer, runs across
    64-lookup chunks add their partial sums in a fixed order), matches the oracle, and covers a row read by half of
    all lookups (its run spans hundreds of chunks), one read by 90% of 65,536 lookups (whole 32-chunk groups),
    lookups fewer than a chunk, exactly one chunk and one more."""
    note(f"ordered bag backward N={N} K={K} rows={rows} hot={hot}")
    D = 384
    g = torch.Generator().manual_seed(N * K + rows)
    idx = torch.randint(0, rows, (N, K), generator=g)
    idx[torch.rand(N, K, generator=g) < hot] = 7 % rows
    w = torch.rand(N, K, generator=g)
    table = torch.randn(rows, D, generator=g)
    G = torch.randn(N, D, generator=g)
    acc0 = torch.randn(rows, D, generator=g) * 0.1
    outs = []
    for _ in range(2):
        acc, touched = acc0.to(DEV), torch.zeros(rows, dtype=torch.bool, device=DEV)
        gw = KR.bag_backward_rows(G.to(DEV), idx.to(DEV), w.to(DEV), table.to(DEV), acc, touched)
        outs.append((gw.cpu(), acc.cpu(), touched.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][2], outs[1][2])
    rgw, racc, rt = T.bag_backward_rows(G.numpy(), idx.numpy(), w.numpy(), table.numpy(), acc0.numpy(),
                                        np.zeros(rows, dtype=bool))
    gw, acc, touched = (t.numpy() for t in outs[0])
    mag_gw = np.abs(G.numpy()) @ np.abs(table.numpy()).T
    np.testing.assert_array_less(np.abs(gw - rgw), 1e-5 * np.take_along_axis(mag_gw, idx.numpy(), 1) + 1e-6)
    mag = np.zeros((rows, D))
    np.add.at(mag, idx.reshape(-1).numpy(), (np.abs(w.numpy())[..., None] * np.abs(G.numpy())[:, None]).reshape(
        N * K, D))
    np.testing.assert_array_less(np.abs(acc - racc), 1e-5 * (mag + np.abs(acc0.numpy())) + 1e-7)
    np.testing.assert_array_equal(touched, rt)


@pytest.mark.parametrize("N,K,D,rows,weighted,offset", [
    (700, 1, 24, 50, False, 0),        # the Engram width: 2.7 rows per wavefront, many repeated rows
    (300, 3, 24, 100000, True, 0),     # K > 1 (lookup i reads gradient row i / K), weights
    (50, 2, 100, 30, True, 0),
    (40, 1, 256, 20, False, 0),
    (33, 2, 98, 40, True, 0),
    (20, 1, 384, 10, False, 0),
    (64, 1, 24, 30, False, 1),         # gradient rows not 16-byte aligned
])
def test_bag_backward_without_weight_grad_matches_oracle(N, K, D, rows, weighted, offset):
    """weight_grad=False (smlm_bag_backward_rows with gw NULL, the Engram backward): the lookups' w * g scattered
    with fp32 atomic adds and no table read; the accumulator within 1e-5 of the summed magnitudes, the flags exact,
    an index outside the table adding nothing."""
    note(f"bag backward without weight grad N={N} K={K} D={D} rows={rows} weighted={weighted} offset={offset}")
    g = torch.Generator().manual_seed(N * D + K)
    idx = torch.randint(0, rows, (N, K), generator=g)
    idx[0, 0] = -1
    idx[-1, -1] = rows                                      # outside the table: no update
    w = torch.rand(N, K, generator=g) if weighted else torch.ones(N, K)
    G = torch.randn(N, D, generator=g)
    acc0 = torch.randn(rows, D, generator=g) * 0.1
    t0 = torch.zeros(rows, dtype=torch.bool)
    acc, touched = acc0.to(DEV), t0.to(DEV)
    store = torch.zeros(N * D + offset, device=DEV)
    gd = store[offset:].view(N, D)
    gd.copy_(G.to(DEV))
    out = KR.bag_backward_rows(gd, idx.to(DEV), w.to(DEV) if weighted else None, torch.empty(rows, D, device=DEV),
                               acc, touched, ordered=False, weight_grad=False)
    torch.cuda.synchronize()
    assert out is None
    ok = (idx >= 0) & (idx < rows)
    _, racc, rt = T.bag_backward_rows(G.numpy(), torch.where(ok, idx, 0).numpy(), (w * ok).numpy(),
                                      np.zeros((rows, D), np.float32), acc0.numpy(), t0.numpy())
    rt[:] = False
    rt[idx[ok].numpy()] = True
    mag = np.zeros((rows, D))
    np.add.at(mag, idx[ok].numpy(), (np.abs(w.numpy())[..., None] * np.abs(G.numpy())[:, None])[ok.numpy()])
    np.testing.assert_array_less(np.abs(acc.cpu().numpy() - racc), 1e-5 * (mag + np.abs(acc0.numpy())) + 1e-7)
    np.testing.assert_array_equal(touched.cpu().numpy(), rt)


def test_bag_backward_without_weight_grad_arguments():
    """The C-ABI's null-pointer rules for the weight-gradient-free form, and the wrapper's refusal of weights=None
    where a weight gradient or the ordered form is asked for."""
    note("bag backward without weight grad: arguments")
    from smlm_hip import _lib
    L = _lib.lib()
    g = torch.ones(4, 24, device=DEV)
    idx = torch.zeros(4, 1, dtype=torch.int64, device=DEV)
    acc = torch.zeros(10, 24, device=DEV)
    touched = torch.zeros(10, dtype=torch.uint8, device=DEV)
    gw = torch.empty(4, 1, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    assert L.smlm_bag_backward_rows(g.data_ptr(), idx.data_ptr(), None, 4, 1, None, _lib.F32, 10, 24,
                                    acc.data_ptr(), touched.data_ptr(), None, s) == _lib.OK
    assert L.smlm_bag_backward_rows(g.data_ptr(), idx.data_ptr(), None, 4, 1, acc.data_ptr(), _lib.F32, 10, 24,
                                    acc.data_ptr(), touched.data_ptr(), gw.data_ptr(), s) == _lib.EINVAL
    torch.cuda.synchronize()
    assert acc[0].sum().item() == 4 * 24 and touched.cpu().tolist() == [1] + [0] * 9
    for kw in ({"ordered": True, "weight_grad": False}, {"ordered": False, "weight_grad": True}):
        with pytest.raises(ValueError):
            KR.bag_backward_rows(g, idx, None, acc, acc, touched.bool(), **kw)


def test_bag_backward_ordered_hot_run_with_indices_outside_the_table():
    """A run over whole 32-chunk groups next to lookups whose index is outside the table (they sort after every row,
    so they share the last chunks with the hot run's end): the valid lookups match the oracle, the others add
    nothing and get a NaN weight gradient, and two calls give the same bits."""
    note("ordered bag backward: hot run over chunk groups and indices outside the table")
    N, K, D, rows = 512, 128, 384, 50
    g = torch.Generator().manual_seed(21)
    idx = torch.randint(0, rows, (N, K), generator=g)
    idx[torch.rand(N, K, generator=g) < 0.9] = rows - 1          # the hot row sorts last among the valid ones
    bad = torch.rand(N, K, generator=g) < 0.003
    idx[bad] = rows                                              # outside the table
    w = torch.rand(N, K, generator=g)
    table = torch.randn(rows, D, generator=g)
    G = torch.randn(N, D, generator=g)
    acc0 = torch.randn(rows, D, generator=g) * 0.1
    outs = []
    for _ in range(2):
        acc, touched = acc0.to(DEV), torch.zeros(rows, dtype=torch.bool, device=DEV)
        gw = KR.bag_backward_rows(G.to(DEV), idx.to(DEV), w.to(DEV), table.to(DEV), acc, touched)
        outs.append((gw.cpu(), acc.cpu(), touched.cpu()))
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])
    assert torch.equal(torch.isnan(outs[0][0]), bad) and torch.equal(outs[0][0][~bad], outs[1][0][~bad])
    ok = ~bad
    rgw, racc, rt = T.bag_backward_rows(G.numpy(), torch.where(ok, idx, 0).numpy(), (w * ok).numpy(), table.numpy(),
                                        acc0.numpy(), np.zeros(rows, dtype=bool))
    rt[:] = False
    rt[idx[ok].numpy()] = True
    gw, acc, touched = (t.numpy() for t in outs[0])
    mag_gw = np.abs(G.numpy()) @ np.abs(table.numpy()).T
    okn = ok.numpy()
    lim = 1e-5 * np.take_along_axis(mag_gw, torch.where(ok, idx, 0).numpy(), 1) + 1e-6
    assert np.all(np.abs(gw[okn] - rgw[okn]) < lim[okn])
    mag = np.zeros((rows, D))
    np.add.at(mag, idx[ok].numpy(), (np.abs(w.numpy())[..., None] * np.abs(G.numpy())[:, None])[okn])
    np.testing.assert_array_less(np.abs(acc - racc), 1e-5 * (mag + np.abs(acc0.numpy())) + 1e-7)
    np.testing.assert_array_equal(touched, rt)


def test_bag_backward_sorted_workspace_checks():
    """The workspace query and its use: a too-small or unaligned workspace is refused before any launch."""
    note("ordered bag backward workspace checks")
    import ctypes
    from smlm_hip import _lib
    L = _lib.lib()
    size = ctypes.c_size_t(0)
    assert L.smlm_bag_backward_sorted_workspace(4, 8, 100, 64, ctypes.byref(size)) == _lib.OK and size.value > 0
    assert L.smlm_bag_backward_sorted_workspace(4, 8, 100, 600, ctypes.byref(size)) == _lib.EUNSUPPORTED
    g = torch.zeros(4, 64, device=DEV)
    idx = torch.zeros(4, 8, dtype=torch.int64, device=DEV)
    w = torch.zeros(4, 8, device=DEV)
    table = torch.zeros(100, 64, device=DEV)
    acc = torch.zeros(100, 64, device=DEV)
    touched = torch.zeros(100, dtype=torch.uint8, device=DEV)
    gw = torch.empty(4, 8, device=DEV)
    L.smlm_bag_backward_sorted_workspace(4, 8, 100, 64, ctypes.byref(size))
    ws = torch.empty(size.value + 256, dtype=torch.uint8, device=DEV)
    args = (g.data_ptr(), idx.data_ptr(), w.data_ptr(), 4, 8, table.data_ptr(), _lib.F32, 100, 64, acc.data_ptr(),
            touched.data_ptr(), gw.data_ptr())
    s = torch.cuda.current_stream().cuda_stream
    assert L.smlm_bag_backward_sorted(*args, ws.data_ptr(), size.value - 1, s) == _lib.EINVAL
    assert L.smlm_bag_backward_sorted(*args, ws.data_ptr() + 16, size.value, s) == _lib.EINVAL
    assert L.smlm_bag_backward_sorted(*args, ws.data_ptr(), size.value, s) == _lib.OK
    torch.cuda.synchronize()


def _adam_case(rows, D, seed):
    rng = np.random.default_rng(seed)
    p = rng.standard_normal((rows, D)).astype(np.float32)
    return rng, p


# D % 4 == 0 takes 4 adjacent columns per lane (one or two chunks of 256); other widths one column per lane
@pytest.mark.parametrize("rows,D", [(300, 384), (40, 100), (64, 512), (50, 98), (20, 510), (45, 300)])
def test_lazy_adam_fp32_bit_exact(rows, D):
    note(f"lazy adam fp32 rows={rows} D={D}")
    rng, p = _adam_case(rows, D, rows + D)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    P, M, V = (torch.from_numpy(a.copy()).to(DEV) for a in (p, m, v))
    for step in range(1, 4):
        acc = (rng.standard_normal((rows, D)) * 1e-2).astype(np.float32)
        touched = rng.random(rows) < 0.6
        scale = 0.7 if step == 2 else 1.0
        A, Tt = torch.from_numpy(acc.copy()).to(DEV), torch.from_numpy(touched.copy()).to(DEV)
        KR.lazy_adam_step(P, M, V, A, Tt, torch.tensor(scale), step, 1e-3, 0.9, 0.95, 1e-8)
        p, m, v, acc_r, t_r = T.lazy_adam(p, m, v, acc, touched, scale, step, 1e-3, 0.9, 0.95, 1e-8)
        torch.cuda.synchronize()
        for got, ref in ((P, p), (M, m), (V, v), (A, acc_r)):
            np.testing.assert_array_equal(got.cpu().numpy(), ref)
        assert not Tt.cpu().any()


@pytest.mark.parametrize("state,rows,D", [("bf16", 200, 384), ("int8", 200, 384), ("int8", 33, 100),
                                          ("bf16", 30, 130), ("int8", 30, 98), ("int8", 40, 512), ("int8", 50, 300), ("bf16", 45, 300)])
def test_lazy_adam_lowmem_bit_exact(state, rows, D):
    note(f"lazy adam {state} rows={rows} D={D}")
    rng, p = _adam_case(rows, D, 7 * rows + D)
    int8 = state == "int8"
    if int8:
        m, v = np.zeros((rows, D), np.int8), np.zeros((rows, D), np.uint8)
        ms, vs = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
        M = torch.zeros(rows, D, dtype=torch.int8, device=DEV)
        V = torch.zeros(rows, D, dtype=torch.uint8, device=DEV)
        MS, VS = torch.zeros(rows, device=DEV), torch.zeros(rows, device=DEV)
    else:
        m, v = np.zeros((rows, D), np.float32), np.zeros((rows, D), np.float32)
        ms = vs = None
        M = torch.zeros(rows, D, dtype=torch.bfloat16, device=DEV)
        V = torch.zeros(rows, D, dtype=torch.bfloat16, device=DEV)
        MS = VS = None
    P = torch.from_numpy(p.copy()).to(DEV)
    for step in range(1, 5):
        acc = (rng.standard_normal((rows, D)) * 1e-2).astype(np.float32)
        acc[0] = 0.0                                       # a touched row with a zero gradient
        touched = rng.random(rows) < 0.7
        touched[0] = True
        A, Tt = torch.from_numpy(acc.copy()).to(DEV), torch.from_numpy(touched.copy()).to(DEV)
        KR.lazy_adam_step_lowmem(P, M, V, A, Tt, 1.0, step, 1e-3, 0.9, 0.95, 1e-8, state, MS, VS)
        p, m, v, ms, vs, acc_r, _ = T.lazy_adam_lowmem(p, m, v, ms, vs, acc, touched, 1.0, step, 1e-3, 0.9, 0.95,
                                                       1e-8, int8)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(P.cpu().numpy(), p)
        np.testing.assert_array_equal(A.cpu().numpy(), acc_r)
        if int8:
            np.testing.assert_array_equal(M.cpu().numpy(), m)
            np.testing.assert_array_equal(V.cpu().numpy(), v)
            np.testing.assert_array_equal(MS.cpu().numpy(), ms)
            np.testing.assert_array_equal(VS.cpu().numpy(), vs)
        else:
            np.testing.assert_array_equal(M.float().cpu().numpy(), m)
            np.testing.assert_array_equal(V.float().cpu().numpy(), v)
        assert not Tt.cpu().any()


def _ref_grads(mem, x, G, idx):
    """fp64 CPU autograd of the layer given the kernels' selection idx: q = x Wq^T + b, s1/s2 = einsum, scores =
    gathered sums, softmax, embedding_bag (smlm/pkm.py:117-148, 186-228)."""
    sd = {k: v.detach().double().cpu().requires_grad_(True) for k, v in mem.named_parameters()}
    xd = x.double().cpu()
    N = xd.shape[0]
    H, kd, NK = mem.heads, mem.k_dim, mem.n_keys
    q = (xd @ sd["query_proj.weight"].T + sd["query_proj.bias"]).view(N, H, kd)
    s1 = torch.einsum("nhd,hkd->nhk", q[..., :kd // 2], sd["keys"][:, 0])
    s2 = torch.einsum("nhd,hkd->nhk", q[..., kd // 2:], sd["keys"][:, 1])
    i = idx.cpu()
    scores = s1.gather(-1, i // NK) + s2.gather(-1, i % NK)
    if "log_score_scale" in sd:          # score_scale="learned" (smlm/pkm.py:205-208)
        scores = scores * sd["log_score_scale"].exp().view(1, H, 1)
    w = torch.softmax(scores, -1)
    out = torch.nn.functional.embedding_bag(i.view(N, -1), sd["values.weight"], per_sample_weights=w.view(N, -1),
                                            mode="sum")
    (out * G.double().cpu()).sum().backward()
    return {k: v.grad for k, v in sd.items()}


@pytest.mark.parametrize("value_grad,score_scale", [("row_sparse", "none"), ("dense", "none"),
                                                     ("row_sparse", "learned")])
def test_layer_training_step_matches_fp64_autograd(value_grad, score_scale):
    """A training forward + backward of ProductKeyMemory (fp32, no BatchNorm, no swilu) on the kernels: query /
    key gradients through the selection backward and the einsum, value gradients in the row store (row_sparse) or
    as a dense .grad, against fp64 autograd on the CPU given the same selection; then one LazyRowAdam step equals
    the oracle on the accumulated rows.  With score_scale="learned" the per-head scale (0.5 and 3 here) multiplies
    the selected scores before the softmax and receives its own gradient."""
    from smlm_hip.pkm import ProductKeyMemory
    from smlm_hip.sparse_values import LazyRowAdam, row_store
    note(f"layer training step value_grad={value_grad} score_scale={score_scale}")
    torch.manual_seed(0)
    N, d, H, kd, NK, knn = 48, 32, 2, 32, 64, 8
    mem = ProductKeyMemory(d, d, n_keys=NK, heads=H, knn=knn, k_dim=kd, query_norm="none", swilu=False,
                           value_grad=value_grad, score_scale=score_scale).to(DEV).train()
    if score_scale == "learned":
        with torch.no_grad():
            mem.log_score_scale.copy_(torch.tensor([0.5, 3.0]).log())
    g = torch.Generator().manual_seed(1)
    x = torch.randn(N, d, generator=g).to(DEV)
    G = torch.randn(N, d, generator=g)
    mem.record = True
    out = mem(x)
    (out * G.to(DEV)).sum().backward()
    idx = mem.last_indices
    ref = _ref_grads(mem, x, G, idx)
    names = ("query_proj.weight", "query_proj.bias", "keys") + (("log_score_scale",) if score_scale == "learned" else ())
    for name in names:
        got = dict(mem.named_parameters())[name].grad.double().cpu()
        scale = ref[name].abs().max()
        assert float((got - ref[name]).abs().max()) <= 1e-5 * float(scale), name
    table = mem.values.weight
    if value_grad == "dense":
        assert float((table.grad.double().cpu() - ref["values.weight"]).abs().max()) <= 1e-6
        return
    assert table.grad is None
    st = row_store(table)
    acc = st.acc.double().cpu()
    assert float((acc - ref["values.weight"]).abs().max()) <= 1e-6
    expect = torch.zeros(NK * NK, dtype=torch.bool)
    expect[idx.reshape(-1).cpu()] = True
    assert torch.equal(st.touched.cpu(), expect)
    p0, acc0, t0 = table.detach().cpu().numpy().copy(), st.acc.cpu().numpy().copy(), st.touched.cpu().numpy()
    opt = LazyRowAdam([table], lr=1e-2)
    opt.step()
    torch.cuda.synchronize()
    z = np.zeros_like(p0)
    p1, m1, v1, _, _ = T.lazy_adam(p0, z, z, acc0, t0, 1.0, 1, 1e-2, 0.9, 0.95, 1e-8)
    np.testing.assert_array_equal(table.detach().cpu().numpy(), p1)
    np.testing.assert_array_equal(opt.state[table]["exp_avg"].cpu().numpy(), m1)
    assert not st.touched.any() and not st.acc.any()
