"""Product-key-memory kernels on MI355X (gfx950), with the forward API of smlm/kernels.py.

Same names, argument meaning, shapes, dtypes and error behaviour as the reference's Triton wrappers; the work
is done by the hand-written HIP kernels of libsmlm_pkm.so (include/smlm_pkm.h), launched on torch's current
stream, so every op can be recorded into a HIP graph.  Outputs are allocated with torch; the library itself
never allocates.

    pk_scores(q, keys)                      -> s1, s2            (new: replaces the einsum of smlm/pkm.py:117-123)
    pk_select(s1, s2, knn)                  -> scores, idx, w    (smlm/kernels.py:214-226)
    PKSelect.apply(s1, s2, knn)             -> scores, idx, w    (smlm/kernels.py:240-251, forward only)
    pk_select_bag(s1, s2, knn, table, ...)  -> out [, scores, idx, w]  (new: pk_select + bag_infer in one launch)
    bag_forward(indices, weights, table)    -> (N, D) fp32       (smlm/kernels.py:229-237)
    bag_infer(indices, weights, table, scales=None, pre=None, out_bf16=False)   (smlm/kernels.py:364-378)
    quantize_q4(table) / dequantize_q4      (smlm/kernels.py:280-300)
    quantize_int8(table) / dequantize_int8  (new: the int8 scheme of scripts/quantize_table_eval.py:55-61)
    decode_attention(qkv, cos, sin, pos, k_cache, v_cache)        (new: one-token attention of smlm/model.py:90-107)
    decode_attention_proj(qkv, ..., v_cache, wo)  (new: the same with wo (model.py:107) folded in, per-head parts)
    swiglu(h13)                             (new: silu(a) * b of smlm/model.py:110-118 in one launch)
    greedy_argmax(logits, pos, tok, hist)   (new: the argmax of the decode loop, smlm/train.py:297-299)
    add_rmsnorm(x, delta, norm)             (new: residual add + the next RMSNorm, smlm/model.py:156-163)
    affine_bf16(x, scale, shift)            (new: the eval BatchNorm of the memory query, smlm/pkm.py:188-191)
    rope_qkv(qkv, cos, sin, pos0, q, k, v)  (new: RoPE of a prompt pass, smlm/model.py:63-78, in one launch)
    prefill_attention(q, k, v)              (new: causal attention of a prompt pass, F.scaled_dot_product_attention
                                             of smlm/model.py:97-105, flash-style on the matrix cores)
    decode_linear(weight, x, ...)           (new: small-M linear of the decode step with fused norm / bias /
                                             BatchNorm / SwiGLU / argmax, smlm/model.py:90-118, smlm/pkm.py:188-224)
    argmax_finish(partial, pos, tok, hist)  (new: token choice + history + position step of the decode loop)
"""
import ctypes
import math

import torch

from . import _lib

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _stream(t):
    return _lib.stream_handle(t.device)


def _need_cuda(name, *tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(f"{name}: all tensors must be on a HIP (cuda) device, got {t.device}")


def _table_ptr(t, name):
    """Address the kernels read a value table (or its scales) at: device memory, or pinned host memory read over
    the host link (zero-copy; smlm_host_table_pointer).  Host tables must be contiguous: a copy would be pageable."""
    if t is None:
        return None
    if t.is_cuda:
        return t.data_ptr()
    if t.device.type == "cpu" and t.is_pinned():
        if not t.is_contiguous():
            raise ValueError(f"{name}: a table in pinned host memory must be contiguous")
        return _lib.host_device_pointer(t.data_ptr())
    raise ValueError(f"{name}: the value table must be on the GPU or in pinned host memory, got {t.device}"
                     + (" (pageable)" if t.device.type == "cpu" else ""))


MAX_N_KEYS = 65536    # sub-key indices fit the 16-bit index field of the selection keys
MAX_KNN = 128         # the selection's result lists (csrc/pkm_select.hip: kMaxKnnGen)


def pk_scores(q, keys):
    """q (N, H, k_dim), keys (H, 2, NK, k_dim/2) of the same dtype (bf16 or fp32) -> s1, s2 (N, H, NK) of that
    dtype: s1[n,h,k] = q[n,h,:half] . keys[h,0,k], s2 with q[n,h,half:] and keys[h,1] (smlm/pkm.py:117-123).
    bf16 accumulates in fp32 on the matrix cores and rounds once to bf16."""
    _need_cuda("pk_scores", q, keys)
    if q.dtype not in _DT or keys.dtype != q.dtype:
        raise ValueError(f"pk_scores: q and keys must both be bf16 or fp32, got {q.dtype} and {keys.dtype}")
    if q.dim() != 3 or keys.dim() != 4 or keys.shape[1] != 2:
        raise ValueError(f"pk_scores: expected q (N, H, k_dim) and keys (H, 2, NK, k_dim/2), got "
                         f"{tuple(q.shape)} and {tuple(keys.shape)}")
    N, H, k_dim = q.shape
    _, _, NK, half = keys.shape
    if keys.shape[0] != H or 2 * half != k_dim:
        raise ValueError(f"pk_scores: q {tuple(q.shape)} does not match keys {tuple(keys.shape)}")
    q = q.contiguous()
    keys = keys.contiguous()
    s1 = torch.empty(N, H, NK, dtype=q.dtype, device=q.device)
    s2 = torch.empty(N, H, NK, dtype=q.dtype, device=q.device)
    rc = _lib.lib().smlm_pkm_score(q.data_ptr(), H * k_dim, keys.data_ptr(), _DT[q.dtype], N, H, NK, half,
                                   s1.data_ptr(), s2.data_ptr(), _stream(q))
    _lib.check(rc, "smlm_pkm_score")
    return s1, s2


def pk_select(s1, s2, knn, ch=128, num_warps=4):
    """s1, s2 (N, H, n_keys) bf16 (or fp32) sub-key scores -> scores (N, H, knn) (same dtype), indices
    (N, H, knn) int64 into the n_keys^2 table, softmax weights (N, H, knn) fp32.  `ch` and `num_warps` are the
    reference's Triton tuning knobs and are accepted for compatibility only."""
    _need_cuda("pk_select", s1, s2)
    if s1.dtype not in _DT or s1.dtype != s2.dtype or s1.shape != s2.shape or s1.dim() != 3:
        raise ValueError(f"pk_select: s1, s2 must be (N, H, n_keys) tensors of one dtype (bf16 or fp32), got "
                         f"{s1.dtype} {tuple(s1.shape)} and {s2.dtype} {tuple(s2.shape)}")
    N, H, NK = s1.shape
    if not (1 <= knn <= min(NK, MAX_KNN) and NK <= MAX_N_KEYS):
        raise ValueError(f"pk_select needs 1 <= knn <= min(n_keys, {MAX_KNN}) and n_keys <= {MAX_N_KEYS}, got "
                         f"n_keys={NK}, knn={knn}")
    s1, s2 = s1.contiguous(), s2.contiguous()
    scores = torch.empty(N, H, knn, dtype=s1.dtype, device=s1.device)
    idx = torch.empty(N, H, knn, dtype=torch.int64, device=s1.device)
    w = torch.empty(N, H, knn, dtype=torch.float32, device=s1.device)
    rc = _lib.lib().smlm_pkm_select(s1.data_ptr(), s2.data_ptr(), _DT[s1.dtype], N, H, NK, knn, scores.data_ptr(),
                                    idx.data_ptr(), w.data_ptr(), _stream(s1))
    _lib.check(rc, "smlm_pkm_select")
    return scores, idx, w


def _table_kind(table, scales, name):
    """(smlm_dtype of the table format, row width D) of a value table, checking its scales."""
    if table.dim() != 2:
        raise ValueError(f"{name}: the table must be 2-d (rows, D)")
    if scales is None:
        if table.dtype not in _DT:
            raise ValueError(f"{name}: a table without scales must be fp32 or bf16, got {table.dtype}")
        kind, D = _DT[table.dtype], table.shape[1]
    elif table.dtype == torch.int8:
        kind, D = _lib.I8, table.shape[1]
    elif table.dtype == torch.uint8:
        kind, D = _lib.Q4, table.shape[1] * 2
    else:
        raise ValueError(f"{name}: a table with scales must be int8 codes or q4-packed uint8, got {table.dtype}")
    if scales is not None and (scales.dtype != torch.float16 or scales.numel() != table.shape[0]):
        raise ValueError(f"{name}: scales must be fp16 with one entry per table row")
    return kind, D


def _bag(indices, weights, table, scales, pre, out_bf16, name):
    _need_cuda(name, indices, weights, pre)
    if indices.dim() != 2 or weights.shape != indices.shape:
        raise ValueError(f"{name}: indices and weights must be (N, K) of one shape, got {tuple(indices.shape)} and "
                         f"{tuple(weights.shape)}")
    if indices.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"{name}: indices must be int64 or int32, got {indices.dtype}")
    N, K = indices.shape
    kind, D = _table_kind(table, scales, name)
    if pre is not None and (pre.dtype != torch.bfloat16 or tuple(pre.shape) != (N, D)):
        raise ValueError(f"{name}: pre must be a bf16 (N, D) = ({N}, {D}) tensor, got {pre.dtype} "
                         f"{tuple(pre.shape)}")
    if table.is_cuda:
        table = table.contiguous()
    tptr, sptr = _table_ptr(table, name), _table_ptr(scales, name)
    indices = indices.contiguous()
    weights = weights.to(torch.float32).contiguous()
    pre = pre.contiguous() if pre is not None else None
    out = torch.empty(N, D, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=indices.device)
    rc = _lib.lib().smlm_pkm_bag(
        indices.data_ptr(), _lib.I64 if indices.dtype == torch.int64 else _lib.I32, weights.data_ptr(), N, K,
        tptr, kind, table.shape[0], D, sptr, pre.data_ptr() if pre is not None else None, out.data_ptr(),
        _lib.BF16 if out_bf16 else _lib.F32, _stream(indices))
    _lib.check(rc, "smlm_pkm_bag")
    return out


def bag_threads(row_bytes):
    """Threads of the value bag's canonical row-slot layout for rows of row_bytes (a multiple of 16): as many whole
    rows of 16-byte chunks as fit in 192 threads for rows of up to 32 chunks, in 384 for wider rows, one at least
    (bag_threads of csrc/pkm_bag_dev.h)."""
    cpr = row_bytes // 16
    budget = 192 if cpr <= 32 else 384
    return (1 if cpr >= budget else budget // cpr) * cpr


def select_bag_supported(heads, table, scales=None):
    """Whether pk_select_bag takes this head count and table (at most 4 heads; a row's 16-byte chunks must not
    outnumber the 2 * heads wavefronts' threads)."""
    if heads > 4 or table.dim() != 2:
        return False
    row_bytes = table.shape[1] * table.element_size()
    return row_bytes % 16 == 0 and row_bytes // 16 <= 2 * heads * 64


def pk_select_bag(s1, s2, knn, table, scales=None, pre=None, out_bf16=False, record=False):
    """pk_select followed by bag_infer on its (indices, weights), in one launch per call (smlm_pkm_select_bag): the
    memory layer's no-grad bf16 lookup at every batch size (decode steps and prompts).  Same arguments and results as
        scores, idx, w = pk_select(s1, s2, knn)
        out = bag_infer(idx.view(N, -1), w.view(N, -1), table, scales, pre, out_bf16)
    Returns out, or (out, scores, idx, w) with record=True.  H (= s1.shape[1]) <= 4."""
    _need_cuda("pk_select_bag", s1, s2, pre)
    if s1.dtype not in _DT or s1.dtype != s2.dtype or s1.shape != s2.shape or s1.dim() != 3:
        raise ValueError(f"pk_select_bag: s1, s2 must be (N, H, n_keys) tensors of one dtype (bf16 or fp32), got "
                         f"{s1.dtype} {tuple(s1.shape)} and {s2.dtype} {tuple(s2.shape)}")
    N, H, NK = s1.shape
    if not (1 <= knn <= min(NK, MAX_KNN) and NK <= MAX_N_KEYS) or H > 4:
        raise ValueError(f"pk_select_bag needs 1 <= knn <= min(n_keys, {MAX_KNN}), n_keys <= {MAX_N_KEYS} and "
                         f"at most 4 heads, got n_keys={NK}, knn={knn}, heads={H}")
    kind, D = _table_kind(table, scales, "pk_select_bag")
    if pre is not None and (pre.dtype != torch.bfloat16 or tuple(pre.shape) != (N, D)):
        raise ValueError(f"pk_select_bag: pre must be a bf16 (N, D) = ({N}, {D}) tensor")
    s1, s2 = s1.contiguous(), s2.contiguous()
    if table.is_cuda:
        table = table.contiguous()
    tptr, sptr = _table_ptr(table, "pk_select_bag"), _table_ptr(scales, "pk_select_bag")
    pre = pre.contiguous() if pre is not None else None
    out = torch.empty(N, D, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=s1.device)
    scores = idx = w = None
    if record:
        scores = torch.empty(N, H, knn, dtype=s1.dtype, device=s1.device)
        idx = torch.empty(N, H, knn, dtype=torch.int64, device=s1.device)
        w = torch.empty(N, H, knn, dtype=torch.float32, device=s1.device)
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    rc = _lib.lib().smlm_pkm_select_bag(
        s1.data_ptr(), s2.data_ptr(), _DT[s1.dtype], N, H, NK, knn, tptr, kind, table.shape[0], D, sptr, ptr(pre),
        out.data_ptr(), _lib.BF16 if out_bf16 else _lib.F32, ptr(scores), ptr(idx), ptr(w),
        _stream(s1))
    _lib.check(rc, "smlm_pkm_select_bag")
    return (out, scores, idx, w) if record else out


def bag_forward(indices, weights, table, block_j=32, block_d=128):
    """out[n] = sum_k weights[n, k] * table[indices[n, k]] (fp32); table fp32 / bf16.  The block sizes are the
    reference's Triton knobs, accepted for compatibility only."""
    return _bag(indices, weights, table, None, None, False, "bag_forward")


def bag_infer(indices, weights, table, scales=None, pre=None, out_bf16=False, block_j=64, block_d=None):
    """Inference value bag.  table: fp32 / bf16 (scales None), int8 codes (rows, D) or q4-packed uint8
    (rows, D/2), both with fp16 row scales.  pre: optional (N, D) bf16 swilu pre-activation ->
    out = bag * bf16(silu(pre)).  Returns (N, D) fp32, or bf16 (rounded to nearest even) with out_bf16."""
    return _bag(indices, weights, table, scales, pre, out_bf16, "bag_infer")


def _quantize(table, kind, name):
    _need_cuda(name, table)
    if table.dim() != 2 or table.dtype not in _DT:
        raise ValueError(f"{name}: table must be a (rows, D) fp32 or bf16 tensor, got {table.dtype} "
                         f"{tuple(table.shape)}")
    rows, D = table.shape
    if kind == _lib.Q4 and D % 2:
        raise ValueError(f"{name}: D must be even, got {D}")
    table = table.contiguous()
    codes = torch.empty(rows, D // 2 if kind == _lib.Q4 else D, dtype=torch.uint8 if kind == _lib.Q4 else torch.int8,
                        device=table.device)
    scales = torch.empty(rows, dtype=torch.float16, device=table.device)
    rc = _lib.lib().smlm_pkm_quantize(table.data_ptr(), _DT[table.dtype], rows, D, kind, codes.data_ptr(),
                                      scales.data_ptr(), _stream(table))
    _lib.check(rc, "smlm_pkm_quantize")
    return codes, scales


def quantize_q4(table, chunk=1 << 18):
    """table (rows, D) -> packed (rows, D/2) uint8, scales (rows,) fp16 (smlm/kernels.py:280-300).  `chunk` is
    accepted for compatibility; the kernel streams the rows itself."""
    return _quantize(table, _lib.Q4, "quantize_q4")


def quantize_int8(table):
    """table (rows, D) -> codes (rows, D) int8, scales (rows,) fp16: per row d = fp16(m / -128) with m the value
    of largest magnitude (1 if d is 0), codes clamp(round(w / d), -128, 127)."""
    return _quantize(table, _lib.I8, "quantize_int8")


def dequantize_q4(packed, scales):
    """(rows, D/2) packed nibbles + fp16 scales -> (rows, D) fp32 values scale * code."""
    codes = torch.cat([packed & 0xF, packed >> 4], dim=1).to(torch.float32) - 8.0
    return codes * scales.to(torch.float32).unsqueeze(1)


def dequantize_int8(codes, scales):
    """(rows, D) int8 codes + fp16 scales -> (rows, D) fp32 values scale * code."""
    return codes.to(torch.float32) * scales.to(torch.float32).unsqueeze(1)


def _check_decode_attention(name, qkv, rope_cos, rope_sin, pos, k_cache, v_cache):
    _need_cuda(name, qkv, rope_cos, rope_sin, pos, k_cache, v_cache)
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError(f"{name}: k_cache and v_cache must be (B, H, max_len, head_dim) of one shape")
    B, H, max_len, hd = k_cache.shape
    if qkv.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise ValueError(f"{name}: qkv and the caches must be bf16")
    if tuple(qkv.shape) != (B, 3 * H * hd) or qkv.stride(1) != 1:
        raise ValueError(f"{name}: qkv must be ({B}, {3 * H * hd}) with unit column stride, got {tuple(qkv.shape)}")
    if rope_cos.dtype not in _DT or rope_sin.dtype != rope_cos.dtype or rope_cos.shape != rope_sin.shape \
            or rope_cos.dim() != 2 or rope_cos.shape[1] != hd // 2:
        raise ValueError(f"{name}: rope tables must be (max_seq_len, head_dim/2) fp32 or bf16")
    if pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError(f"{name}: pos must be a one-element int64 tensor")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError(f"{name}: the caches must be contiguous")
    return rope_cos.contiguous(), rope_sin.contiguous()


def decode_attention(qkv, rope_cos, rope_sin, pos, k_cache, v_cache):
    """One decode step of causal self-attention for one new token per sequence, over a static KV cache:
    RoPE on the new q and k, k and v written into the caches at slot `pos`, softmax(q k^T / sqrt(head_dim)) v
    over slots 0..pos (smlm/model.py:63-107 for T = 1).
    qkv (B, 3*H*hd) bf16 (the qkv projection of the new tokens), rope_cos / rope_sin (max_seq_len, hd/2) fp32 or
    bf16, pos a 0-d / 1-element int64 device tensor, k_cache / v_cache (B, H, max_len, hd) bf16.
    Returns (B, H*hd) bf16."""
    rope_cos, rope_sin = _check_decode_attention("decode_attention", qkv, rope_cos, rope_sin, pos, k_cache, v_cache)
    B, H, max_len, hd = k_cache.shape
    out = torch.empty(B, H * hd, dtype=torch.bfloat16, device=qkv.device)
    rc = _lib.lib().smlm_decode_attention(
        qkv.data_ptr(), qkv.stride(0), rope_cos.data_ptr(), rope_sin.data_ptr(), _DT[rope_cos.dtype],
        rope_cos.shape[0], pos.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), B, H, hd, max_len,
        out.data_ptr(), _stream(qkv))
    _lib.check(rc, "smlm_decode_attention")
    return out


def decode_attention_proj(qkv, rope_cos, rope_sin, pos, k_cache, v_cache, wo):
    """decode_attention followed by the output projection per head (smlm/model.py:107): returns parts (B, H, N)
    fp32 with parts[b, h] = bf16(y[b, h]) @ wo[:, h*hd:(h+1)*hd].T for wo (N, H*hd) bf16 (nn.Linear.weight);
    bf16(parts.sum(1)) is wo(y).  decode_linear(..., delta=parts, norm=...) adds that sum to the residual stream
    in its prologue, so the projection costs no launch of its own."""
    rope_cos, rope_sin = _check_decode_attention("decode_attention_proj", qkv, rope_cos, rope_sin, pos, k_cache,
                                                 v_cache)
    B, H, max_len, hd = k_cache.shape
    _need_cuda("decode_attention_proj", wo)
    if wo.dtype != torch.bfloat16 or wo.dim() != 2 or wo.shape[1] != H * hd or wo.stride(1) != 1 \
            or wo.stride(0) % 8 or wo.data_ptr() % 16:
        raise ValueError(f"decode_attention_proj: wo must be a (N, {H * hd}) bf16 tensor with unit column stride, "
                         "16-byte aligned rows")
    N = wo.shape[0]
    parts = torch.empty(B, H, N, dtype=torch.float32, device=qkv.device)
    rc = _lib.lib().smlm_decode_attention_proj(
        qkv.data_ptr(), qkv.stride(0), rope_cos.data_ptr(), rope_sin.data_ptr(), _DT[rope_cos.dtype],
        rope_cos.shape[0], pos.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), B, H, hd, max_len,
        wo.data_ptr(), wo.stride(0), N, parts.data_ptr(), _stream(qkv))
    _lib.check(rc, "smlm_decode_attention_proj")
    return parts


def affine_bf16(x, scale, shift):
    """bf16(x * scale + shift) per column in one pass (fp32 fused multiply-add): the eval-mode BatchNorm of the
    memory query (smlm/pkm.py:188-191) on the bf16 query projection.  x (M, C) bf16 with unit column stride,
    scale / shift (C,) fp32; C a multiple of 8.  Returns (M, C) bf16."""
    _need_cuda("affine_bf16", x, scale, shift)
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("affine_bf16: x must be a (M, C) bf16 tensor with unit column stride")
    M, C = x.shape
    if scale.dtype != torch.float32 or shift.dtype != torch.float32 or scale.numel() != C or shift.numel() != C:
        raise ValueError(f"affine_bf16: scale and shift must be ({C},) fp32")
    if C % 8 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    scale, shift = scale.contiguous(), shift.contiguous()
    out = torch.empty(M, C, dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().smlm_affine_bf16(x.data_ptr(), x.stride(0), scale.data_ptr(), shift.data_ptr(), M, C,
                                     out.data_ptr(), C, _stream(x))
    _lib.check(rc, "smlm_affine_bf16")
    return out


def _strides3(t):
    return (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))


def rope_qkv(qkv, rope_cos, rope_sin, pos0, q_out, k_out, v_out=None):
    """RoPE of a prompt pass (smlm/model.py:63-78 on q, k of the qkv projection, smlm/model.py:92-93) in one launch.
    qkv (B, T, 3*H*hd) bf16 with unit column stride and rows b*T + t evenly spaced; token t is at position pos0 + t
    (an int).  Rotated q and k are written into q_out, k_out (B, H, T, hd) bf16 -- any strides over (B, H, T) with a
    contiguous last dimension, e.g. slots of a static KV cache -- and v is copied into v_out if given.  Rotation in
    fp32 with one bf16 rounding per output, the formula of decode_attention."""
    _need_cuda("rope_qkv", qkv, rope_cos, rope_sin, q_out, k_out, v_out)
    B, H, T, hd = q_out.shape
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 3 or tuple(qkv.shape) != (B, T, 3 * H * hd) or qkv.stride(2) != 1 \
            or (T > 1 and qkv.stride(0) != T * qkv.stride(1)):
        raise ValueError(f"rope_qkv: qkv must be ({B}, {T}, {3 * H * hd}) bf16 with evenly spaced rows, got "
                         f"{tuple(qkv.shape)} {qkv.dtype}")
    outs = [t for t in (q_out, k_out, v_out) if t is not None]
    for t in outs:
        if t.shape != q_out.shape or t.dtype != torch.bfloat16 or t.stride(3) != 1:
            raise ValueError(f"rope_qkv: outputs must be ({B}, {H}, {T}, {hd}) bf16 with a contiguous last dim")
    if rope_cos.dtype not in _DT or rope_sin.dtype != rope_cos.dtype or rope_cos.shape != rope_sin.shape \
            or rope_cos.dim() != 2 or rope_cos.shape[1] != hd // 2:
        raise ValueError("rope_qkv: rope tables must be (max_seq_len, head_dim/2) fp32 or bf16")
    if pos0 < 0 or pos0 + T > rope_cos.shape[0]:
        raise ValueError(f"rope_qkv: positions {pos0}..{pos0 + T - 1} are outside the rope table "
                         f"({rope_cos.shape[0]} rows)")
    rope_cos, rope_sin = rope_cos.contiguous(), rope_sin.contiguous()
    row_stride = qkv.stride(1) if T > 1 else qkv.stride(0)
    rc = _lib.lib().smlm_rope_qkv(
        qkv.data_ptr(), row_stride, rope_cos.data_ptr(), rope_sin.data_ptr(), _DT[rope_cos.dtype],
        rope_cos.shape[0], pos0, q_out.data_ptr(), _strides3(q_out), k_out.data_ptr(), _strides3(k_out),
        v_out.data_ptr() if v_out is not None else None, _strides3(v_out) if v_out is not None else None,
        B, T, H, hd, _stream(qkv))
    _lib.check(rc, "smlm_rope_qkv")


def prefill_attention(q, k, v, out=None):
    """Causal attention of T new tokens after S - T earlier ones (smlm/model.py:97-105: F.scaled_dot_product_attention
    with is_causal=True for S == T, with the mask ones(T, S).tril(S - T) otherwise):
    q (B, H, T, hd), k, v (B, H, S, hd) bf16 with any strides over (B, H, T) and a contiguous last dimension
    (permuted views of the qkv projection and slices of a KV cache work as they are).  Returns (B, T, H, hd) bf16
    (or writes `out` of that shape), i.e. the (B, T, H*hd) input of the output projection.  Forward only."""
    _need_cuda("prefill_attention", q, k, v, out)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("prefill_attention: q, k and v must be bf16")
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError(f"prefill_attention: expected q (B, H, T, hd) and k, v (B, H, S, hd), got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    B, H, T, hd = q.shape
    S = k.shape[2]
    if k.shape[0] != B or k.shape[1] != H or k.shape[3] != hd or S < T:
        raise ValueError(f"prefill_attention: k {tuple(k.shape)} does not fit q {tuple(q.shape)} (need S >= T)")
    if hd not in (32, 64, 128):
        raise ValueError(f"prefill_attention: head_dim {hd} not in (32, 64, 128)")
    ins = []
    for t in (q, k, v):
        if t.stride(3) != 1 or any(st % 8 for st in t.stride()[:3]) or t.data_ptr() % 16:
            t = t.contiguous()
        ins.append(t)
    q, k, v = ins
    if out is None:
        out = torch.empty(B, T, H, hd, dtype=torch.bfloat16, device=q.device)
    elif out.shape != (B, T, H, hd) or out.dtype != torch.bfloat16 or out.stride(3) != 1:
        raise ValueError(f"prefill_attention: out must be ({B}, {T}, {H}, {hd}) bf16 with a contiguous last dim")
    ys = (ctypes.c_int64 * 3)(out.stride(0), out.stride(2), out.stride(1))   # (b, h, t) strides of (B, T, H, hd)
    rc = _lib.lib().smlm_prefill_attention(q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k), v.data_ptr(),
                                           _strides3(v), out.data_ptr(), ys, B, H, T, S, hd, _stream(q))
    _lib.check(rc, "smlm_prefill_attention")
    return out


def swiglu(h13):
    """h13 (..., 2*hidden) bf16, the w13 projection -> (..., hidden) bf16 = bf16(bf16(silu(a)) * b) with a, b its
    two halves (smlm/model.py:110-118)."""
    _need_cuda("swiglu", h13)
    if h13.dtype != torch.bfloat16 or h13.shape[-1] % 16:
        raise ValueError("swiglu: input must be bf16 with a last dimension that is a multiple of 16")
    hidden = h13.shape[-1] // 2
    x2 = h13.reshape(-1, 2 * hidden)
    if x2.stride(1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    out = torch.empty(x2.shape[0], hidden, dtype=torch.bfloat16, device=h13.device)
    rc = _lib.lib().smlm_swiglu(x2.data_ptr(), x2.stride(0), out.data_ptr(), x2.shape[0], hidden, _stream(h13))
    _lib.check(rc, "smlm_swiglu")
    return out.view(*h13.shape[:-1], hidden)


def linear_swiglu_supported(x, w13):
    """Whether linear_swiglu takes these operands (bf16 tensors on one CUDA device, K a multiple of 64, hidden of
    64)."""
    return (x.is_cuda and w13.device == x.device and x.dtype == torch.bfloat16 and w13.dtype == torch.bfloat16
            and w13.dim() == 2 and x.shape[-1] == w13.shape[1] and w13.shape[0] % 128 == 0
            and w13.shape[1] % 64 == 0)


def linear_swiglu(x, w13):
    """bf16(bf16(silu(a)) * b) with a | b = the halves of bf16(x @ w13.T): the w13 projection and the SwiGLU
    activation of smlm/model.py:110-118 in one launch (smlm_linear_swiglu), for prompt passes.  x (..., K) bf16,
    w13 (2 * hidden, K) bf16 with K a multiple of 64 and hidden of 64.  Returns (..., hidden) bf16."""
    _need_cuda("linear_swiglu", x, w13)
    if not linear_swiglu_supported(x, w13):
        raise ValueError(f"linear_swiglu: x (..., K) and w13 (2*hidden, K) must be bf16 with K a multiple of 64 "
                         f"and hidden of 64, got {x.dtype} {tuple(x.shape)} and {w13.dtype} {tuple(w13.shape)}")
    K, hidden = w13.shape[1], w13.shape[0] // 2
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    if w13.stride(1) != 1 or w13.stride(0) % 8 or w13.data_ptr() % 16:
        w13 = w13.contiguous()
    out = torch.empty(x2.shape[0], hidden, dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().smlm_linear_swiglu(x2.data_ptr(), x2.stride(0), w13.data_ptr(), w13.stride(0), x2.shape[0], K,
                                       hidden, out.data_ptr(), hidden, _stream(x))
    _lib.check(rc, "smlm_linear_swiglu")
    return out.view(*x.shape[:-1], hidden)


def prompt_linear_supported(x, w, bias=None):
    """Whether prompt_linear takes these operands (bf16 tensors on one CUDA device, K a multiple of 64 and N of 128,
    bias bf16 or None)."""
    return (x.is_cuda and w.device == x.device and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
            and w.dim() == 2 and x.shape[-1] == w.shape[1] and w.shape[0] % 128 == 0 and w.shape[1] % 64 == 0
            and (bias is None or (bias.device == x.device and bias.dtype == torch.bfloat16
                                  and bias.shape == (w.shape[0],))))


def prompt_linear(x, w, bias=None, scale=None, shift=None):
    """bf16(x @ w.T + bias) with fp32 accumulation (smlm_prompt_linear): an nn.Linear of a prompt pass on the
    matrix cores.  x (..., K) bf16, w (N, K) bf16 with K a multiple of 64 and N of 128, bias (N,) bf16 or None.
    scale, shift (N,) fp32 (both or neither): the result is bf16(bf16(x @ w.T + bias) * scale + shift), the eval
    BatchNorm of the memory query (affine_bf16's arithmetic) in the same launch.  Returns (..., N) bf16."""
    _need_cuda("prompt_linear", x, w, bias, scale, shift)
    if not prompt_linear_supported(x, w, bias):
        raise ValueError(f"prompt_linear: x (..., K), w (N, K) and bias (N,) must be bf16 with K a multiple of 64 "
                         f"and N of 128, got {x.dtype} {tuple(x.shape)}, {w.dtype} {tuple(w.shape)}")
    N, K = w.shape
    if (scale is None) != (shift is None):
        raise ValueError("prompt_linear: give scale and shift together")
    if scale is not None:
        if scale.shape != (N,) or shift.shape != (N,) or scale.device != x.device or shift.device != x.device:
            raise ValueError(f"prompt_linear: scale and shift must be ({N},) tensors on {x.device}")
        scale = scale.float().contiguous()
        shift = shift.float().contiguous()
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    if w.stride(1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
        w = w.contiguous()
    bias = bias.contiguous() if bias is not None else None
    out = torch.empty(x2.shape[0], N, dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().smlm_prompt_linear(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0),
                                       bias.data_ptr() if bias is not None else None,
                                       scale.data_ptr() if scale is not None else None,
                                       shift.data_ptr() if shift is not None else None, x2.shape[0], K, N,
                                       out.data_ptr(), N, _stream(x))
    _lib.check(rc, "smlm_prompt_linear")
    return out.view(*x.shape[:-1], N)


def linear(mod, x, min_rows=128, max_n=1152):
    """mod(x) for an nn.Linear, through prompt_linear when that applies (bf16 weights and activations, no autograd
    recording, at least min_rows rows, at most max_n outputs, K a multiple of 64 and N of 128, bf16 or no autocast): the
    same roundings (bf16 out of the fp32 accumulation, the bias added in fp32).  max_n: wider projections keep the
    library GEMM, as fast or faster there on MI355X (16,384 x 384 rows: 2048 outputs 32-35 against 35-38 us, the
    lm_head's 32,000 outputs 400-470 against 680-690 us)."""
    w, b = mod.weight, mod.bias
    if (x.is_cuda and x.dtype == torch.bfloat16 and w.shape[0] <= max_n and x.numel() >= min_rows * x.shape[-1]
            and prompt_linear_supported(x, w, b)
            and not (torch.is_grad_enabled() and (x.requires_grad or w.requires_grad
                                                  or (b is not None and b.requires_grad)))
            and not (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") != torch.bfloat16)):
        return prompt_linear(x, w, b)
    return mod(x)


def greedy_argmax(logits, pos=None, tok=None, hist=None):
    """logits (B, V) bf16 -> tok (B,) int64, the first index of each row's largest logit (torch.argmax's rule),
    written into `tok` if given; with `hist` (B, L) int64 and a device int64 `pos`, also hist[b, pos + 1] = tok[b]
    (skipped when that slot is outside the history)."""
    _need_cuda("greedy_argmax", logits, pos, tok, hist)
    if logits.dim() != 2 or logits.dtype != torch.bfloat16 or logits.stride(1) != 1:
        raise ValueError("greedy_argmax: logits must be (B, V) bf16 with unit column stride")
    B, V = logits.shape
    if tok is None:
        tok = torch.empty(B, dtype=torch.int64, device=logits.device)
    if tok.dtype != torch.int64 or tok.numel() != B or not tok.is_contiguous():
        raise ValueError("greedy_argmax: tok must be a contiguous int64 tensor with one entry per row")
    if hist is not None and (pos is None or hist.dtype != torch.int64 or hist.dim() != 2 or hist.shape[0] != B
                             or hist.stride(1) != 1 or pos.dtype != torch.int64 or pos.numel() != 1):
        raise ValueError("greedy_argmax: hist must be (B, L) int64 with a one-element int64 pos")
    rc = _lib.lib().smlm_greedy_argmax(
        logits.data_ptr(), logits.stride(0), B, V, pos.data_ptr() if pos is not None else None, tok.data_ptr(),
        hist.data_ptr() if hist is not None else None, hist.stride(0) if hist is not None else 0,
        hist.shape[1] if hist is not None else 0, _stream(logits))
    _lib.check(rc, "smlm_greedy_argmax")
    return tok


def add_rmsnorm(x, delta, norm):
    """Residual add and RMSNorm in one launch: returns (x + delta, norm(x + delta)) in bf16, with fp32 statistics
    (smlm/model.py:124-126, 156-163); with delta None returns (x, norm(x)).  x, delta (..., C) bf16; norm an
    nn.RMSNorm over C with bf16 weight."""
    _need_cuda("add_rmsnorm", x, delta, norm.weight)
    C = x.shape[-1]
    if x.dtype != torch.bfloat16 or (delta is not None and (delta.dtype != torch.bfloat16 or delta.shape != x.shape)):
        raise ValueError("add_rmsnorm: x and delta must be bf16 tensors of one shape")
    if norm.weight is None or norm.weight.dtype != torch.bfloat16 or norm.weight.numel() != C:
        raise ValueError("add_rmsnorm: the norm needs a bf16 weight of size C")
    x = x.contiguous()
    delta = delta.contiguous() if delta is not None else None
    eps = norm.eps if norm.eps is not None else torch.finfo(torch.bfloat16).eps
    h = torch.empty_like(x)
    x_out = torch.empty_like(x) if delta is not None else x
    rc = _lib.lib().smlm_add_rmsnorm(x.data_ptr(), delta.data_ptr() if delta is not None else None,
                                     norm.weight.data_ptr(), float(eps), x.numel() // C, C,
                                     x_out.data_ptr() if delta is not None else None, h.data_ptr(), _stream(x))
    _lib.check(rc, "smlm_add_rmsnorm")
    return x_out, h


def _rms_eps(norm):
    return norm.eps if norm.eps is not None else torch.finfo(torch.bfloat16).eps


def decode_linear(weight, x=None, *, delta=None, norm=None, tok=None, emb=None, write_x=False, bias=None,
                  affine=None, n_split=None, swiglu=False, argmax=False, tok_partial=None, tok_out=None, hist=None,
                  pos=None, partial_out=None, advance_pos=None):
    """Fused small-M linear layer of the decode step (smlm_decode_linear): y = h @ weight.T on the matrix cores.

    h is x (M, K) bf16 (unit column stride); with `norm` (an nn.RMSNorm over K with a bf16 weight) it is
    norm(xs), xs = bf16(x + delta) (delta (M, K) bf16 or None; or (M, P, K) fp32 parts from decode_attention_proj,
    then delta = bf16(sum over P in order), P <= 8, not with argmax), or xs = emb[tok] when `tok` (M,) int64 and
    `emb` (V, K) bf16 are given instead of x.  With `tok_partial` (M, nblk) int64 instead of tok, the tokens are
    the greedy choice from those argmax partial keys (the previous step's), and the launch also writes them to
    `tok_out` (M,) int64 and to hist[:, pos] (hist (M, L) int64 with pos a one-element int64 tensor; skipped
    outside the history) when given.  The epilogue is one of
      default   bf16(y + bias) (bias (N,) bf16 or None); `affine` = (scale, shift) fp32 tensors applied as
                bf16(v * scale + shift) to the first len(scale) columns; with `n_split`, columns [0, n_split) and
                [n_split, N) are returned as two tensors;
      swiglu    bf16(bf16(silu(a)) * b) with a | b the two halves of y (weight (2*hidden, K)) -> (M, hidden);
      argmax    no logits: (M, smlm_linear_argmax_blocks(N)) int64 tensor of uint64 partial keys for
                argmax_finish or the next step's tok_partial (written into `partial_out` when given); with
                `advance_pos` (one-element int64 tensor) the launch also adds 1 to it.
    With write_x (an RMSNorm prologue) returns (xs, result)."""
    _need_cuda("decode_linear", weight, x, delta, tok, emb, bias, tok_partial, tok_out, hist, pos, partial_out,
               advance_pos)
    if weight.dtype != torch.bfloat16 or weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("decode_linear: weight must be a contiguous (N, K) bf16 tensor")
    N, K = weight.shape
    args = _lib.LinearArgs()
    args.N, args.K = N, K
    keep = []
    if tok is not None or tok_partial is not None:
        if norm is None or emb is None or x is not None or delta is not None or (tok is not None
                                                                                and tok_partial is not None):
            raise ValueError("decode_linear: tok or tok_partial needs emb and norm, and excludes x and delta")
        if emb.dtype != torch.bfloat16 or emb.dim() != 2 or emb.shape[1] != K or not emb.is_contiguous():
            raise ValueError("decode_linear: emb must be a contiguous (V, K) bf16 tensor")
        args.emb, args.emb_rows = emb.data_ptr(), emb.shape[0]
        if tok is not None:
            if tok.dtype != torch.int64 or tok.dim() != 1:
                raise ValueError("decode_linear: tok must be (M,) int64")
            tok = tok.contiguous()
            M, dev = tok.shape[0], tok.device
            args.prologue, args.tok = _lib.LIN_EMBED_RMSNORM, tok.data_ptr()
        else:
            if tok_partial.dtype != torch.int64 or tok_partial.dim() != 2 or tok_partial.stride(1) != 1 \
                    or tok_partial.stride(0) % 2 or tok_partial.data_ptr() % 16:
                raise ValueError("decode_linear: tok_partial must be (M, nblk) int64 with an even row stride, "
                                 "16-byte aligned")
            M, dev = tok_partial.shape[0], tok_partial.device
            args.prologue = _lib.LIN_EMBED_ARGMAX
            args.tok_partial, args.tok_partial_stride = tok_partial.data_ptr(), tok_partial.stride(0)
            args.tok_blocks = tok_partial.shape[1]
            if tok_out is not None:
                if tok_out.dtype != torch.int64 or tok_out.numel() != M or not tok_out.is_contiguous():
                    raise ValueError("decode_linear: tok_out must be (M,) int64 contiguous")
                args.tok_out = tok_out.data_ptr()
            if hist is not None:
                if hist.dtype != torch.int64 or hist.dim() != 2 or hist.shape[0] != M or hist.stride(1) != 1 \
                        or pos is None or pos.dtype != torch.int64 or pos.numel() != 1:
                    raise ValueError("decode_linear: hist must be (M, L) int64 with unit column stride, with pos "
                                     "one int64")
                args.hist, args.hist_stride, args.hist_len = hist.data_ptr(), hist.stride(0), hist.shape[1]
                args.pos = pos.data_ptr()
        keep += [tok, tok_partial, emb]
    elif tok_out is not None or hist is not None or pos is not None:
        raise ValueError("decode_linear: tok_out, hist and pos come with tok_partial")
    else:
        if x is None or x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != K:
            raise ValueError(f"decode_linear: x must be a (M, {K}) bf16 tensor")
        if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
            x = x.contiguous()
        M, dev = x.shape[0], x.device
        args.prologue = _lib.LIN_RMSNORM if norm is not None else _lib.LIN_PLAIN
        args.x, args.x_stride = x.data_ptr(), x.stride(0)
        if delta is not None:
            if norm is not None and delta.dtype == torch.float32 and delta.dim() == 3 \
                    and tuple(delta.shape[::2]) == (M, K) and 1 <= delta.shape[1] <= 8 and not argmax:
                args.prologue, args.delta_parts = _lib.LIN_RMSNORM_PARTS, delta.shape[1]
            elif norm is None or delta.dtype != torch.bfloat16 or tuple(delta.shape) != (M, K):
                raise ValueError("decode_linear: delta must be (M, K) bf16 or (M, <= 8, K) fp32 parts (no argmax) "
                                 "and comes with a norm")
            delta = delta.contiguous()
            args.delta = delta.data_ptr()
    args.M = M
    x_out = None
    if norm is not None:
        if norm.weight is None or norm.weight.dtype != torch.bfloat16 or norm.weight.numel() != K:
            raise ValueError("decode_linear: the norm needs a bf16 weight of size K")
        args.norm_w, args.eps = norm.weight.data_ptr(), float(_rms_eps(norm))
        if write_x:
            x_out = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
            args.x_out = x_out.data_ptr()
    elif write_x:
        raise ValueError("decode_linear: write_x needs an RMSNorm prologue")
    args.w = weight.data_ptr()
    keep += [x, delta, weight]
    if (partial_out is not None or advance_pos is not None) and not argmax:
        raise ValueError("decode_linear: partial_out and advance_pos belong to argmax")
    if argmax:
        nblk = _lib.lib().smlm_linear_argmax_blocks(N)
        if partial_out is None:
            res = torch.empty(M, nblk, dtype=torch.int64, device=dev)
        elif partial_out.dtype != torch.int64 or partial_out.dim() != 2 or partial_out.shape[0] != M \
                or partial_out.shape[1] < nblk or partial_out.stride(1) != 1:
            raise ValueError(f"decode_linear: partial_out must be (M, >= {nblk}) int64 with unit column stride")
        else:
            res = partial_out
        args.epilogue, args.partial, args.partial_stride = _lib.LIN_ARGMAX, res.data_ptr(), res.stride(0)
        if advance_pos is not None:
            if advance_pos.dtype != torch.int64 or advance_pos.numel() != 1:
                raise ValueError("decode_linear: advance_pos must be one int64")
            args.pos_advance = advance_pos.data_ptr()
    elif swiglu:
        res = torch.empty(M, N // 2, dtype=torch.bfloat16, device=dev)
        args.epilogue, args.out, args.out_stride = _lib.LIN_SWIGLU, res.data_ptr(), N // 2
    else:
        args.epilogue = _lib.LIN_STORE
        if bias is not None:
            if bias.dtype != torch.bfloat16 or bias.numel() != N:
                raise ValueError("decode_linear: bias must be (N,) bf16")
            bias = bias.contiguous()
            args.bias = bias.data_ptr()
            keep.append(bias)
        if affine is not None:
            scale, shift = (t.to(torch.float32).contiguous() for t in affine)
            if scale.shape != shift.shape or scale.dim() != 1 or scale.numel() > N:
                raise ValueError("decode_linear: affine scale and shift must be 1-d fp32 of one size <= N")
            args.scale, args.shift, args.n_affine = scale.data_ptr(), shift.data_ptr(), scale.numel()
            keep += [scale, shift]
        split = N if n_split is None else n_split
        out1 = torch.empty(M, split, dtype=torch.bfloat16, device=dev) if split > 0 else None
        out2 = torch.empty(M, N - split, dtype=torch.bfloat16, device=dev) if split < N else None
        args.n_split = split
        if out1 is not None:
            args.out, args.out_stride = out1.data_ptr(), split
        if out2 is not None:
            args.out2, args.out2_stride = out2.data_ptr(), N - split
        res = out1 if n_split is None else (out1, out2)
    rc = _lib.lib().smlm_decode_linear(ctypes.byref(args), _stream(weight))
    _lib.check(rc, "smlm_decode_linear")
    del keep
    return (x_out, res) if write_x else res


def linear_argmax_blocks(N):
    """Columns of the argmax partial keys decode_linear(..., argmax=True) writes for N output features."""
    return int(_lib.lib().smlm_linear_argmax_blocks(int(N)))


def argmax_finish(partial, pos, tok, hist=None, advance=True):
    """End of a greedy decode step from decode_linear(..., argmax=True) partial keys: tok[m] = the column of row m's
    largest key; hist[m, pos + 1] = tok[m] when hist (M, L) int64 is given (skipped outside the history); then
    pos += 1 if `advance` (smlm/train.py:297-301)."""
    _need_cuda("argmax_finish", partial, pos, tok, hist)
    M, nblk = partial.shape
    if partial.dtype != torch.int64 or not partial.is_contiguous() or pos.dtype != torch.int64 \
            or pos.numel() != 1 or tok.dtype != torch.int64 or tok.numel() != M or not tok.is_contiguous():
        raise ValueError("argmax_finish: partial (M, nblk) int64, pos one int64, tok (M,) int64 contiguous")
    if hist is not None and (hist.dtype != torch.int64 or hist.dim() != 2 or hist.shape[0] != M
                             or hist.stride(1) != 1):
        raise ValueError("argmax_finish: hist must be (M, L) int64 with unit column stride")
    rc = _lib.lib().smlm_argmax_finish(
        partial.data_ptr(), nblk, nblk, M, pos.data_ptr(), tok.data_ptr(),
        hist.data_ptr() if hist is not None else None, hist.stride(0) if hist is not None else 0,
        hist.shape[1] if hist is not None else 0, 1 if advance else 0, _stream(partial))
    _lib.check(rc, "smlm_argmax_finish")
    return tok


# ---------------------------------------------------------------------------------------------------------------
# Training side: selection backward, row-sparse bag backward, lazy row Adam (smlm/kernels.py:1-104, 240-266,
# 380-515 of the reference)
# ---------------------------------------------------------------------------------------------------------------
def pk_select_backward(idx, w, g_scores, g_w, nk, dtype):
    """PKSelect.backward (smlm/kernels.py:253-266): dense (N, H, nk) gradients of s1 and s2 of `dtype` (bf16 or
    fp32) from the selection's idx (N, H, knn) int64 and weights w (N, H, knn) fp32 and the incoming gradients
    of the returned scores (g_scores, or None) and weights (g_w, or None)."""
    _need_cuda("pk_select_backward", idx, w, g_scores, g_w)
    if dtype not in _DT:
        raise ValueError(f"pk_select_backward: scores must be bf16 or fp32, got {dtype}")
    if idx.dtype != torch.int64 or idx.dim() != 3 or w.shape != idx.shape:
        raise ValueError("pk_select_backward: idx must be (N, H, knn) int64 and w of the same shape")
    N, H, knn = idx.shape
    idx, w = idx.contiguous(), w.float().contiguous()
    if g_scores is not None:
        g_scores = g_scores.to(dtype).contiguous()
    if g_w is not None:
        g_w = g_w.float().contiguous()
    ds1 = torch.empty(N, H, nk, dtype=dtype, device=idx.device)
    ds2 = torch.empty(N, H, nk, dtype=dtype, device=idx.device)
    rc = _lib.lib().smlm_pkm_select_backward(
        idx.data_ptr(), w.data_ptr(), g_scores.data_ptr() if g_scores is not None else None,
        g_w.data_ptr() if g_w is not None else None, _DT[dtype], N, H, nk, knn, ds1.data_ptr(), ds2.data_ptr(),
        _stream(idx))
    _lib.check(rc, "smlm_pkm_select_backward")
    return ds1, ds2


class PKSelect(torch.autograd.Function):
    """Differentiable pk_select (smlm/kernels.py:240-266): forward = the selection kernel; backward = the softmax
    backward and the scatter of every selected score's gradient to its two sub-key scores, dense (N, H, NK), in
    one kernel (smlm_pkm_select_backward)."""

    @staticmethod
    def forward(ctx, s1, s2, knn):
        scores, idx, w = pk_select(s1, s2, knn)
        ctx.save_for_backward(idx, w)
        ctx.nk, ctx.dtype = s1.shape[-1], s1.dtype
        ctx.mark_non_differentiable(idx)
        return scores, idx, w

    @staticmethod
    def backward(ctx, g_scores, g_idx, g_w):
        idx, w = ctx.saved_tensors
        ds1, ds2 = pk_select_backward(idx, w, g_scores, g_w, ctx.nk, ctx.dtype)
        return ds1, ds2, None


def bag_backward_rows(grad_out, indices, weights, table, acc, touched, ordered=True, weight_grad=True):
    """Row-sparse bag backward (smlm/kernels.py:90-104): acc[indices[n, k]] += weights[n, k] * grad_out[n] and
    touched[indices] = True, in place; returns the per-sample-weight gradient (N, K) fp32.  table fp32 / bf16
    (rows, D), acc (rows, D) fp32, touched (rows,) bool.  ordered (default): the lookups sorted by row and each row
    written by one wavefront in a fixed order (smlm_bag_backward_sorted: the same result on every call, no
    atomics); ordered=False: fp32 atomic adds in no fixed order (smlm_bag_backward_rows).
    weight_grad=False with ordered=False: the per-sample-weight gradient is not computed (returns None) and the
    table is not read; weights may then be None (unit weights, the Engram lookups of smlm/engram.py:118).  The
    lookups are scattered with fp32 atomic adds and no sort (smlm_bag_backward_rows with gw NULL)."""
    scatter = not weight_grad and not ordered
    if weights is None and not scatter:
        raise ValueError("bag_backward_rows: weights=None needs weight_grad=False and ordered=False")
    _need_cuda("bag_backward_rows", grad_out, indices, table, acc, touched, *(() if weights is None else (weights,)))
    N, K = indices.shape
    rows, D = table.shape
    if table.dtype not in _DT or acc.dtype != torch.float32 or tuple(acc.shape) != (rows, D) \
            or not acc.is_contiguous() or touched.dtype != torch.bool or touched.numel() != rows:
        raise ValueError("bag_backward_rows: table fp32/bf16 (rows, D), acc contiguous fp32 (rows, D), touched "
                         "(rows,) bool")
    if tuple(grad_out.shape) != (N, D) or (weights is not None and tuple(weights.shape) != (N, K)):
        raise ValueError("bag_backward_rows: grad_out must be (N, D) and weights (N, K)")
    g = grad_out.float().contiguous()
    idx = indices.to(torch.int64).contiguous()
    w = None if weights is None else weights.float().contiguous()
    L = _lib.lib()
    if scatter:
        rc = L.smlm_bag_backward_rows(g.data_ptr(), idx.data_ptr(), None if w is None else w.data_ptr(), N, K, None,
                                      _DT[table.dtype], rows, D, acc.data_ptr(), touched.data_ptr(), None, _stream(g))
        _lib.check(rc, "smlm_bag_backward_rows")
        return None
    table = table.contiguous()
    gw = torch.empty(N, K, dtype=torch.float32, device=g.device)
    if ordered and rows < 0xFFFFFFFF and N * K < 0x7FFFFFFF:
        size = ctypes.c_size_t(0)
        _lib.check(L.smlm_bag_backward_sorted_workspace(N, K, rows, D, ctypes.byref(size)),
                   "smlm_bag_backward_sorted_workspace")
        ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device=g.device)
        rc = L.smlm_bag_backward_sorted(g.data_ptr(), idx.data_ptr(), w.data_ptr(), N, K, table.data_ptr(),
                                        _DT[table.dtype], rows, D, acc.data_ptr(), touched.data_ptr(), gw.data_ptr(),
                                        ws.data_ptr(), size.value, _stream(g))
        _lib.check(rc, "smlm_bag_backward_sorted")
        return gw
    rc = L.smlm_bag_backward_rows(g.data_ptr(), idx.data_ptr(), w.data_ptr(), N, K, table.data_ptr(),
                                  _DT[table.dtype], rows, D, acc.data_ptr(), touched.data_ptr(), gw.data_ptr(),
                                  _stream(g))
    _lib.check(rc, "smlm_bag_backward_rows")
    return gw


def _scale_tensor(grad_scale, device):
    if torch.is_tensor(grad_scale):
        return grad_scale.reshape(1).to(device=device, dtype=torch.float32)
    return torch.tensor([float(grad_scale)], dtype=torch.float32, device=device)


def _adam(param, exp_avg, exp_avg_sq, acc, touched, grad_scale, step, lr, beta1, beta2, eps, state, ms, vs, name):
    _need_cuda(name, param, exp_avg, exp_avg_sq, acc, touched, ms, vs)
    if param.dtype != torch.float32 or param.dim() != 2 or not param.is_contiguous():
        raise ValueError(f"{name}: param must be a contiguous (rows, D) fp32 table")
    rows, D = param.shape
    for t in (exp_avg, exp_avg_sq, acc):
        if tuple(t.shape) != (rows, D) or not t.is_contiguous():
            raise ValueError(f"{name}: moments and accumulator must be contiguous ({rows}, {D})")
    if touched.dtype != torch.bool or touched.numel() != rows:
        raise ValueError(f"{name}: touched must be ({rows},) bool")
    scale = _scale_tensor(grad_scale, param.device)
    bc1, bc2 = 1 - beta1 ** step, 1 - beta2 ** step
    rc = _lib.lib().smlm_lazy_adam(
        param.data_ptr(), exp_avg.data_ptr(), exp_avg_sq.data_ptr(), ms.data_ptr() if ms is not None else None,
        vs.data_ptr() if vs is not None else None, state, acc.data_ptr(), touched.data_ptr(), scale.data_ptr(),
        rows, D, lr / bc1, bc2 ** 0.5, beta1, beta2, 1 - beta1, 1 - beta2, eps, _stream(param))
    _lib.check(rc, name)


def lazy_adam_step(param, exp_avg, exp_avg_sq, acc, touched, grad_scale, step, lr, beta1, beta2, eps):
    """In-place lazy Adam step with fp32 moments on the rows flagged in `touched` (smlm/kernels.py:418-433);
    afterwards their accumulator rows are zero and the flags cleared.  grad_scale: 0-d tensor or float; step:
    the step number after this update (1 for the first)."""
    if exp_avg.dtype != torch.float32 or exp_avg_sq.dtype != torch.float32:
        raise ValueError("lazy_adam_step: fp32 moments")
    _adam(param, exp_avg, exp_avg_sq, acc, touched, grad_scale, step, lr, beta1, beta2, eps, _lib.ADAM_F32, None,
          None, "lazy_adam_step")


def lazy_adam_step_lowmem(param, exp_avg, exp_avg_sq, acc, touched, grad_scale, step, lr, beta1, beta2, eps,
                          state_dtype, exp_avg_scale=None, exp_avg_sq_scale=None):
    """Lazy Adam with bf16 moments or int8 / uint8 companded moments and fp32 row scales (smlm/kernels.py:
    494-515), in fp32, in place."""
    if state_dtype not in ("bf16", "int8"):
        raise ValueError("low-memory Adam state_dtype must be 'bf16' or 'int8'")
    if state_dtype == "int8":
        if exp_avg_scale is None or exp_avg_sq_scale is None:
            raise ValueError("int8 Adam needs exp_avg_scale and exp_avg_sq_scale")
        if exp_avg.dtype != torch.int8 or exp_avg_sq.dtype != torch.uint8 or exp_avg_scale.dtype != torch.float32 \
                or exp_avg_sq_scale.dtype != torch.float32:
            raise ValueError("int8 Adam: exp_avg int8, exp_avg_sq uint8, fp32 scales")
        state = _lib.ADAM_INT8
    else:
        if exp_avg.dtype != torch.bfloat16 or exp_avg_sq.dtype != torch.bfloat16:
            raise ValueError("bf16 Adam: bf16 moments")
        state = _lib.ADAM_BF16
        exp_avg_scale = exp_avg_sq_scale = None
    _adam(param, exp_avg, exp_avg_sq, acc, touched, grad_scale, step, lr, beta1, beta2, eps, state, exp_avg_scale,
          exp_avg_sq_scale, "lazy_adam_step_lowmem")


def engram_hash(c, mult, orders, rows_per_head):
    """NgramHash.forward (smlm/engram.py:60-73): c (B, T + max(orders) - 1) int64 compressed ids, mult
    (len(orders), heads, max_order) int64 -> (B, T, len(orders) * heads) int64 row indices, head h of order o in
    rows [(o * heads + h) * rows_per_head, ... + rows_per_head)."""
    _need_cuda("engram_hash", c, mult)
    if c.dtype != torch.int64 or mult.dtype != torch.int64 or c.dim() != 2 or mult.dim() != 3:
        raise ValueError("engram_hash: c must be (B, L) int64 and mult (orders, heads, max_order) int64")
    orders = [int(n) for n in orders]
    n_orders, heads, max_order = mult.shape
    if len(orders) != n_orders:
        raise ValueError(f"engram_hash: {len(orders)} orders for mult of {n_orders}")
    B, L = c.shape
    T = L - (max(orders) - 1)
    if T < 0:
        raise ValueError(f"engram_hash: c has {L} columns, fewer than the history of {max(orders) - 1}")
    c, mult = c.contiguous(), mult.contiguous()
    rows = torch.empty(B, T, n_orders * heads, dtype=torch.int64, device=c.device)
    arr = (ctypes.c_int * n_orders)(*orders)
    rc = _lib.lib().smlm_engram_hash(c.data_ptr(), B, T, L, mult.data_ptr(), ctypes.cast(arr, ctypes.c_void_p),
                                     n_orders, heads, max_order, int(rows_per_head), rows.data_ptr(), _stream(c))
    _lib.check(rc, "smlm_engram_hash")
    return rows


def row_gather(rows, table):
    """table[rows] for int64 rows of any shape and a (table_rows, D) fp32 / bf16 table -> rows.shape + (D,) of the
    table's dtype (F.embedding; a row outside the table gives a NaN output row)."""
    _need_cuda("row_gather", rows, table)
    if rows.dtype != torch.int64 or table.dim() != 2 or table.dtype not in _DT:
        raise ValueError("row_gather: int64 rows and a (rows, D) fp32 or bf16 table")
    flat, table = rows.reshape(-1).contiguous(), table.contiguous()
    out = torch.empty(flat.numel(), table.shape[1], dtype=table.dtype, device=table.device)
    rc = _lib.lib().smlm_row_gather(flat.data_ptr(), flat.numel(), table.data_ptr(), _DT[table.dtype],
                                    table.shape[0], table.shape[1], out.data_ptr(), _stream(table))
    _lib.check(rc, "smlm_row_gather")
    return out.view(*rows.shape, table.shape[1])
