"""CPU oracle of the product-key-memory training backward -- TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, as the checker; the product path (smlm_hip) never calls it.

A numpy restatement of the reference's training-side lookup ops:
  select_backward      smlm/kernels.py:253-266   PKSelect.backward: softmax backward, the selected scores'
                                                  gradient rounded to the scores' dtype, scattered to both halves
                                                  (fp32 sums in selection order, rounded once to the dtype)
  bag_backward_rows    smlm/kernels.py:90-104    row-sparse bag backward: acc[idx[n,k]] += w[n,k] * g[n] (fp64 sums),
                        smlm/sparse_values.py:94-113   touched[idx] = True, per-sample-weight gradient
                                                  gw[n,k] = g[n] . table[idx[n,k]] (fp64)
  lazy_adam            smlm/kernels.py:392-433   lazy Adam on touched rows, fp32 moments, global step for the bias
                                                  correction; the rows' accumulator and flags cleared
  lazy_adam_lowmem     smlm/kernels.py:445-515   the same with bf16 moments, or int8 companded moments (signed
                        smlm/sparse_values.py:204-236  sqrt first moment, fourth-root second moment, fp32 row scales)

How each is pinned (tests/test_train_oracle.py): select_backward against torch autograd through a gather-based
selection of the same indices on the CPU; bag_backward_rows against torch autograd of F.embedding_bag with
per-sample weights (fp64); lazy_adam against torch.optim.Adam (CPU, fp32) on rows that are touched at every step,
with untouched rows unchanged bit for bit; lazy_adam_lowmem at step 1 against lazy_adam's parameter update (the
update uses the fresh fp32 moments) and its stored codes against the bf16 rounding oracle / the companding's
closed-form special cases (largest |m| -> +-127, largest v -> 255, zero rows -> zero codes, positive v never a
zero code) and decode error bounds.
"""
import numpy as np

from .pkm_oracle import bf16_bits_rtne, bf16_to_f32

F32 = np.float32


def round_to(x, bf16):
    x = np.asarray(x, dtype=F32)
    return bf16_to_f32(bf16_bits_rtne(x)) if bf16 else x


def select_backward(idx, w, g_scores, g_w, nk, bf16):
    """PKSelect.backward (smlm/kernels.py:253-266).  idx (N, H, knn) int64 table indices, w (N, H, knn) fp32
    softmax weights, g_scores (N, H, knn) or None (gradient of the returned scores, any float dtype), g_w
    (N, H, knn) fp32 or None.  Returns ds1, ds2 (N, H, nk) fp32 arrays holding values of the scores' dtype."""
    w = np.asarray(w, dtype=F32)
    dl = np.zeros_like(w)
    if g_w is not None:
        gw = np.asarray(g_w, dtype=F32)
        s = (w * gw).sum(-1, keepdims=True, dtype=F32)
        dl = (w * (gw - s)).astype(F32)
    if g_scores is not None:
        dl = (dl + np.asarray(g_scores, dtype=F32)).astype(F32)
    ds = round_to(dl, bf16)
    N, H, knn = idx.shape
    ds1 = np.zeros((N, H, nk), dtype=F32)
    ds2 = np.zeros((N, H, nk), dtype=F32)
    i1, i2 = idx // nk, idx % nk
    for n in range(N):
        for h in range(H):
            for k in range(knn):                  # fp32 sums in selection order
                ds1[n, h, i1[n, h, k]] = F32(ds1[n, h, i1[n, h, k]] + ds[n, h, k])
                ds2[n, h, i2[n, h, k]] = F32(ds2[n, h, i2[n, h, k]] + ds[n, h, k])
    return round_to(ds1, bf16), round_to(ds2, bf16)


def bag_backward_rows(grad_out, idx, w, table, acc, touched):
    """Row-sparse bag backward (smlm/kernels.py:90-104, smlm/sparse_values.py:94-113), in place on acc (fp64
    copy returned) and touched.  grad_out (N, D), idx (N, K), w (N, K), table (rows, D).  Returns (gw (N, K)
    fp64, acc fp64, touched bool)."""
    g = np.asarray(grad_out, dtype=np.float64)
    t = np.asarray(table, dtype=np.float64)
    wv = np.asarray(w, dtype=np.float64)
    acc = np.array(acc, dtype=np.float64)
    touched = np.array(touched, dtype=bool)
    N, K = idx.shape
    gw = np.einsum("nd,nkd->nk", g, t[idx])
    np.add.at(acc, idx.reshape(-1), (wv[..., None] * g[:, None, :]).reshape(N * K, -1))
    touched[idx.reshape(-1)] = True
    return gw, acc, touched


def lazy_adam(p, m, v, acc, touched, grad_scale, step, lr, b1, b2, eps):
    """Lazy Adam, fp32 moments (smlm/kernels.py:392-433): on touched rows g = acc * scale,
    m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g g, p -= (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps); their acc
    rows are zeroed and the flags cleared.  Returns new (p, m, v, acc, touched) as fp32 / bool arrays."""
    p, m, v, acc = (np.array(a, dtype=F32) for a in (p, m, v, acc))
    t = np.array(touched, dtype=bool)
    step_size = F32(lr / (1 - b1 ** step))
    bc2_sqrt = F32((1 - b2 ** step) ** 0.5)
    b1, b2, eps = F32(b1), F32(b2), F32(eps)
    g = acc[t] * F32(grad_scale)
    mt = b1 * m[t] + (F32(1) - b1) * g
    vt = b2 * v[t] + (F32(1) - b2) * g * g
    p[t] = p[t] - step_size * mt / (np.sqrt(vt) / bc2_sqrt + eps)
    m[t], v[t], acc[t] = mt, vt, 0
    return p, m, v, acc, np.zeros_like(t)


def _rtne_int(x):
    """Round half to even (np.rint does so)."""
    return np.rint(x).astype(F32)


def lazy_adam_lowmem(p, m, v, m_scale, v_scale, acc, touched, grad_scale, step, lr, b1, b2, eps, int8):
    """Lazy Adam with compact moments (smlm/kernels.py:445-515).  bf16: m, v stored as bf16 (RTNE); int8: m as
    int8 codes of sign(m) sqrt(|m| / max|m|) * 127, v as uint8 codes of v^(1/4) / max v^(1/4) * 255 (>= 1 where
    v > 0), fp32 row scales max|m|, max v^(1/4).  The parameter update uses the fresh fp32 moments.  m, v are
    the stored arrays (bf16 values as fp32, or integer codes); returns new (p, m, v, m_scale, v_scale, acc,
    touched)."""
    p, acc = np.array(p, dtype=F32), np.array(acc, dtype=F32)
    m, v = np.array(m), np.array(v)
    m_scale = None if m_scale is None else np.array(m_scale, dtype=F32)
    v_scale = None if v_scale is None else np.array(v_scale, dtype=F32)
    t = np.array(touched, dtype=bool)
    step_size = F32(lr / (1 - b1 ** step))
    bc2_sqrt = F32((1 - b2 ** step) ** 0.5)
    omb1, omb2 = F32(1 - b1), F32(1 - b2)     # 1 - beta in double, then fp32, as the reference passes them
    b1, b2, eps = F32(b1), F32(b2), F32(eps)
    g = acc[t] * F32(grad_scale)
    mt = m[t].astype(F32)
    vt = v[t].astype(F32)
    if int8:
        mt = mt / F32(127)
        mt = np.where(mt < 0, F32(-1), F32(1)) * mt * mt * m_scale[t][:, None]
        vt = vt / F32(255) * v_scale[t][:, None]
        vt = vt * vt
        vt = vt * vt
    mt = (b1 * mt + omb1 * g).astype(F32)
    vt = (b2 * vt + omb2 * g * g).astype(F32)
    denom = np.sqrt(vt) / bc2_sqrt + eps
    p[t] = p[t] - (step_size * mt) / denom
    if int8:
        ms = np.abs(mt).max(axis=1)
        vroot = np.sqrt(np.sqrt(vt))
        vs = vroot.max(axis=1)
        mq = np.sqrt(np.abs(mt) / np.where(ms > 0, ms, F32(1))[:, None])
        mq = np.where(mt < 0, F32(-1), F32(1)) * mq * F32(127)
        vq = vroot / np.where(vs > 0, vs, F32(1))[:, None] * F32(255)
        mq = _rtne_int(np.clip(mq, -127, 127))
        vq = _rtne_int(np.clip(vq, 0, 255))
        vq = np.where(vt > 0, np.maximum(vq, 1), 0)
        m[t] = mq.astype(m.dtype)
        v[t] = vq.astype(v.dtype)
        m_scale[t], v_scale[t] = ms, vs
    else:
        m[t] = round_to(mt, True)
        v[t] = round_to(vt, True)
    acc[t] = 0
    return p, m, v, m_scale, v_scale, acc, np.zeros_like(t)
