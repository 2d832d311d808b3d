"""CPU oracle of the Engram n-gram memory -- TEST INFRASTRUCTURE ONLY.

Only tests/ (as the checker) and bench.py's CPU baseline may import this module; the product path (smlm_hip) never
calls it.

  ngram_rows       smlm/engram.py:60-73    row of every hash head for every position: XOR over the n-gram's
                                            tokens of token x multiplier (int64, wrap-around), x ^= x >> 17
                                            (arithmetic), (x mod rows) + (order * heads + head) * rows
  engram_forward   smlm/engram.py:111-131  the module in fp64: rows gathered and concatenated, k / v projections,
                                            sigmoid gate of RMSNorm(h) . RMSNorm(k) / sqrt(d), v~ = alpha v,
                                            u = RMSNorm(v~), depthwise causal conv over [past, u] (no padding,
                                            dilation), Y = SiLU(conv) + v~; returns Y and the conv's new past

How each is pinned (tests/test_engram_oracle.py): ngram_rows against a scalar brute force on Python integers with
explicit two's-complement wrap and floor-division shift, and the reference's own test properties (each head in its
own row block, determinism, a bigram head independent of token t-2; tests/test_engram.py:35-48); engram_forward's
conv against torch's F.conv1d, its norms against nn.RMSNorm, chunked evaluation with the returned past against the
full sequence, causality, and the zero-conv closed form Y = alpha v (tests/test_engram.py:81-92).
"""
import math

import numpy as np
import torch
import torch.nn.functional as F


def ngram_rows(c, mult, orders, heads, rows):
    """c (B, history + T) int64 compressed ids, mult (len(orders), heads, max(orders)) -> (B, T, len * heads)."""
    c = np.asarray(c, dtype=np.int64)
    mult = np.asarray(mult, dtype=np.int64)
    history = max(orders) - 1
    B, L = c.shape
    T = L - history
    out = np.empty((B, T, len(orders) * heads), dtype=np.int64)
    for o, n in enumerate(orders):
        x = np.zeros((B, T, heads), dtype=np.int64)
        for i in range(n):                                  # token t - i
            tok = c[:, history - i:history - i + T]
            x ^= tok[:, :, None] * mult[o, :, i]            # numpy int64 products wrap around
        x ^= x >> 17
        out[:, :, o * heads:(o + 1) * heads] = np.mod(x, rows) + (o * heads + np.arange(heads)) * rows
    return out


def rms_norm(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def causal_depthwise_conv(full, weight, dilation, T):
    """y[:, t, ch] = sum_j weight[ch, 0, j] * full[:, t + j * dilation, ch] for t < T (no padding)."""
    y = torch.zeros(full.shape[0], T, full.shape[2], dtype=full.dtype)
    for j in range(weight.shape[-1]):
        y = y + weight[:, 0, j] * full[:, j * dilation:j * dilation + T]
    return y


def engram_forward(p, h, rows, eps, dilation, past=None):
    """p: fp64 tensors {"values" (rows, hd), "w_k", "w_v" (d, d_mem), "h_norm", "k_norm", "v_norm" (d,), "conv"
    (d, 1, ks)}; h (B, T, d) fp64; rows (B, T, n_lookups) int64.  Returns (Y (B, T, d), new past (B, P, d))."""
    B, T, d = h.shape
    e = p["values"][torch.as_tensor(rows).reshape(-1)].view(B, T, -1)
    k = e @ p["w_k"].T
    v = e @ p["w_v"].T
    alpha = torch.sigmoid((rms_norm(h, p["h_norm"], eps) * rms_norm(k, p["k_norm"], eps)).sum(-1, keepdim=True)
                          / math.sqrt(d))
    vt = alpha * v
    u = rms_norm(vt, p["v_norm"], eps)
    P = (p["conv"].shape[-1] - 1) * dilation
    if past is None:
        past = torch.zeros(B, P, d, dtype=h.dtype)
    full = torch.cat([past, u], 1)
    y = causal_depthwise_conv(full, p["conv"], dilation, T)
    return F.silu(y) + vt, full[:, full.shape[1] - P:]
