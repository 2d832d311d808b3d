"""CPU oracle of the product-key-memory lookup -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker (or as the timed CPU baseline); the product path (smlm_hip) never calls it.

A numpy restatement of the reference's forward lookup, bit-exact where the reference defines bits:
  bf16_bits_rtne / order16 / unorder16    smlm/kernels.py:106-126  (integer RTNE, order-preserving codes)
  half_topk                               smlm/kernels.py:128-144  (top-knn, ties -> lower sub-key index)
  pairs                                   smlm/kernels.py:200-211  ((i+1)(j+1) <= knn candidates)
  pk_select                               smlm/kernels.py:146-177  (Cartesian top-knn, ties -> lower table index,
                                                                    fp32 softmax); fp32 scores: the same rules
                                                                    with 32-bit codes (smlm/pkm.py:125-136)
  subkey_scores                           smlm/pkm.py:117-123       (fp64)
  bag                                     smlm/kernels.py:179-194, 313-361 (fp64 accumulation, row scales,
                                                                    swilu epilogue, bf16 output)
  quantize_rows / dequantize              scripts/quantize_table_eval.py:55-61 (int8), smlm/kernels.py:280-300 (q4)

How each function is pinned (tests/test_oracle.py): bf16 rounding against torch's own fp32->bf16 cast and
hand-made ties; order codes exhaustively over all 65536 bf16 patterns; half_topk / pk_select against a
brute force written with Python tuples and floats (no packed keys), against brute force over all NK^2 product
keys (tests/test_pkm.py:16-37 pattern) and against torch.topk on tie-free rows; softmax against torch.softmax;
bag against torch's F.embedding_bag; quantisation against hand-derived known answers (tests/golden/) and its
error bounds.
"""
import numpy as np

U64 = np.uint64


# ---------------------------------------------------------------------------------------------- number formats
def bf16_bits_rtne(x):
    """fp32 values -> uint16 bf16 bit patterns, round to nearest even on the integer bits (kernels.py:106-112)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x):
    return bf16_to_f32(bf16_bits_rtne(x))


def order16(bits):
    """bf16 bits -> order-preserving unsigned 16-bit code (kernels.py:114-119), -0 just below +0."""
    b = np.asarray(bits).astype(np.uint32)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def unorder16(code):
    o = np.asarray(code).astype(np.uint32)
    return np.where(o & 0x8000, o ^ 0x8000, (~o) & 0xFFFF).astype(np.uint16)


def order32(f):
    """fp32 values -> order-preserving unsigned 32-bit code."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000).astype(np.uint64)


def unorder32(code):
    o = np.asarray(code).astype(np.uint64)
    u = np.where(o & 0x80000000, o ^ 0x80000000, (~o) & 0xFFFFFFFF).astype(np.uint32)
    return u.view(np.float32)


# ---------------------------------------------------------------------------------------------- selection
def _is_bf16(s):
    return s.dtype == np.uint16


def half_keys(s):
    """(R, NK) scores (bf16 bit patterns as uint16, or fp32) -> uint64 keys, larger = better, ties -> lower k."""
    R, NK = s.shape
    k = np.arange(NK, dtype=np.uint64)
    if _is_bf16(s):
        return (order16(s).astype(np.uint64) << U64(16)) | (U64(0xFFFF) - k)
    return (order32(s) << U64(32)) | (U64(0xFFFFFFFF) - k)


def _top_keys(keys, knn):
    """The knn largest keys of every row, descending (keys are distinct within a row)."""
    n = keys.shape[1]
    part = np.partition(keys, n - knn, axis=1)[:, n - knn:]
    return np.sort(part, axis=1)[:, ::-1]


def half_topk(s, knn):
    """Top-knn of each row of s (R, NK): values (fp32) and sub-key indices (int64), descending
    (kernels.py:128-144)."""
    top = _top_keys(half_keys(s), knn)
    if _is_bf16(s):
        vals = bf16_to_f32(unorder16(top >> U64(16)))
        idx = (U64(0xFFFF) - (top & U64(0xFFFF))).astype(np.int64)
    else:
        vals = unorder32(top >> U64(32))
        idx = (U64(0xFFFFFFFF) - (top & U64(0xFFFFFFFF))).astype(np.int64)
    return vals.astype(np.float32), idx


def pairs(knn):
    """Cartesian candidates (i, j) with (i+1)(j+1) <= knn (kernels.py:200-211); 130 for knn = 32."""
    pi = [i for i in range(knn) for j in range(knn) if (i + 1) * (j + 1) <= knn]
    pj = [j for i in range(knn) for j in range(knn) if (i + 1) * (j + 1) <= knn]
    return np.array(pi, dtype=np.int64), np.array(pj, dtype=np.int64)


def softmax_f32(x):
    """fp32 softmax over the last axis (max subtracted)."""
    x = np.asarray(x, dtype=np.float32)
    e = np.exp(x - x.max(axis=-1, keepdims=True)).astype(np.float32)
    return (e / e.sum(axis=-1, dtype=np.float32, keepdims=True)).astype(np.float32)


def pk_select(s1, s2, knn):
    """s1, s2 (N, H, NK) bf16 bit patterns (uint16) or fp32 -> scores (N, H, knn) (same representation),
    idx (N, H, knn) int64, w (N, H, knn) fp32 (kernels.py:146-177)."""
    N, H, NK = s1.shape
    R = N * H
    v1, i1 = half_topk(s1.reshape(R, NK), knn)
    v2, i2 = half_topk(s2.reshape(R, NK), knn)
    pi, pj = pairs(knn)
    summ = (v1[:, pi] + v2[:, pj]).astype(np.float32)          # fp32 add, as the kernel's v1 + v2
    if _is_bf16(s1):
        code = order16(bf16_bits_rtne(summ)).astype(np.uint64)
    else:
        code = order32(summ)
    full = (i1[:, pi] * NK + i2[:, pj]).astype(np.uint64)
    top = _top_keys((code << U64(32)) | (U64(0xFFFFFFFF) - full), knn)
    idx = (U64(0xFFFFFFFF) - (top & U64(0xFFFFFFFF))).astype(np.int64)
    if _is_bf16(s1):
        scores = unorder16(top >> U64(32))
        sval = bf16_to_f32(scores)
    else:
        sval = unorder32(top >> U64(32))
        scores = sval
    w = softmax_f32(sval)
    return scores.reshape(N, H, knn), idx.reshape(N, H, knn), w.reshape(N, H, knn)


# ---------------------------------------------------------------------------------------------- scoring
def subkey_scores(q, keys):
    """q (N, H, k_dim), keys (H, 2, NK, half) -> s1, s2 (N, H, NK) in fp64 (pkm.py:117-123)."""
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    half = keys.shape[-1]
    s1 = np.einsum("nhd,hkd->nhk", q[..., :half], keys[:, 0])
    s2 = np.einsum("nhd,hkd->nhk", q[..., half:], keys[:, 1])
    return s1, s2


# ---------------------------------------------------------------------------------------------- value bag
def row_values(table, rows, kind, scales=None):
    """fp64 values of table rows `rows` (any shape) -> rows.shape + (D,). kind: f32, bf16 (uint16 bits), i8, q4."""
    if kind == "f32":
        return np.asarray(table, dtype=np.float32)[rows].astype(np.float64)
    if kind == "bf16":
        return bf16_to_f32(table[rows]).astype(np.float64)
    if kind == "i8":
        return table[rows].astype(np.float64)
    if kind == "q4":
        b = table[rows].astype(np.int64)
        return np.concatenate([(b & 15) - 8, (b >> 4) - 8], axis=-1).astype(np.float64)
    raise ValueError(kind)


def silu_bf16(pre_bits):
    """bf16(silu(p)) in fp32 for bf16 bit patterns p (kernels.py:304-307)."""
    p = bf16_to_f32(pre_bits)
    return round_bf16((p / (np.float32(1) + np.exp(-p))).astype(np.float32))


def bag(idx, w, table, kind, scales=None, pre=None, out_bf16=False):
    """out[n] = sum_j w'[n, j] * row(idx[n, j]) accumulated in fp64, with w' = w * scale[row] in fp32 for
    quantised tables (kernels.py:328-335); optional epilogue * bf16(silu(pre)); optional bf16 rounding.
    Returns fp64 (N, D), or uint16 bf16 bit patterns with out_bf16."""
    idx = np.asarray(idx, dtype=np.int64)
    w = np.asarray(w, dtype=np.float32)
    if kind in ("i8", "q4"):
        sc = np.asarray(scales, dtype=np.float16)[idx].astype(np.float32)
        w = (w * sc).astype(np.float32)
    vals = row_values(table, idx, kind)
    out = np.einsum("nj,njd->nd", w.astype(np.float64), vals)
    if pre is not None:
        out = out * silu_bf16(pre).astype(np.float64)
    if out_bf16:
        return bf16_bits_rtne(out.astype(np.float32))
    return out


# ---------------------------------------------------------------------------------------------- table formats
def quantize_rows(table, kind):
    """(rows, D) fp32 -> (codes, scales fp16): int8 codes (rows, D), or q4 bytes (rows, D/2) holding column i in
    the low nibble and column i + D/2 in the high nibble as code + 8 (quantize_table_eval.py:55-61,
    kernels.py:280-300)."""
    t = np.asarray(table, dtype=np.float32)
    lo, hi = (-128, 127) if kind == "i8" else (-8, 7)
    m = t[np.arange(t.shape[0]), np.abs(t).argmax(axis=1)]
    d = (m / np.float32(lo)).astype(np.float32).astype(np.float16)
    d = np.where(d == 0, np.float16(1.0), d)
    c = np.clip(np.rint(t / d.astype(np.float32)[:, None]), lo, hi).astype(np.int64)
    if kind == "i8":
        return c.astype(np.int8), d
    half = t.shape[1] // 2
    packed = ((c[:, :half] + 8) | ((c[:, half:] + 8) << 4)).astype(np.uint8)
    return packed, d


def dequantize(codes, scales, kind):
    vals = row_values(codes, np.arange(codes.shape[0]), kind)
    return vals * np.asarray(scales, dtype=np.float16).astype(np.float64)[:, None]
