"""Host recomputation of a memory layer's query and sub-key scores from the input the kernels saw, for the tests
that pin the integrated lookup (smlm/pkm.py:186-201): fp64 arithmetic with the bf16 roundings a bf16 model makes,

    h   = bf16(x * rsqrt(mean(x^2) + eps) * g)          the ffn_norm in front of the memory layer (decode step)
    v   = bf16(h W^T + b)                                query_proj | swilu_proj (bias added before rounding)
    q   = bf16(v * scale + shift)                        eval BatchNorm on the query columns, fp32 scale / shift
    s_p = q[..., p half] . keys[h, p]                    the two sub-key score rows

and the error bounds that separate the kernels' fp32 accumulation (and a bf16 rounding that lands on the other
side of a tie) from a wrong operand: every value must lie within the bound, and nearly every value must be
bit-equal to the host's, which a swapped scale and shift or a column mix-up cannot meet (tests/test_query_check.py
shows both on the CPU).
"""
import torch


def to_bf16(t):
    """fp64 -> the bf16 value (through fp32, as the kernels round their fp32 results), as fp64."""
    return t.float().bfloat16().double()


def ulp_bf16(t):
    """Spacing of bf16 values at magnitude |t| (8 significant bits)."""
    a = t.abs().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - 7)


def rms_norm_bf16(x, g, eps):
    """h = bf16(x rsqrt(mean(x^2) + eps) g) in fp64 from the bf16 residual row x; returns (h, elementwise bound of
    |h_kernel - h|: one bf16 ulp)."""
    x, g = x.double(), g.double()
    h = to_bf16(x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * g)
    return h, ulp_bf16(h)


def linear_bf16(h, w, b, scale=None, shift=None, n_affine=0, h_err=None, extra_ulps=0):
    """v = bf16(h W^T + b), and on the first n_affine columns q = bf16(v scale + shift); returns (out, bound) with
    bound[m, n] the largest |kernel - host| of a kernel that accumulates in fp32 (any order) from an h within h_err
    of this one and rounds where this does (extra_ulps: further bf16 roundings the kernel may make, e.g. of the
    product before the bias)."""
    h, w = h.double(), w.double()
    K = h.shape[-1]
    mag = h.abs() @ w.abs().T
    err = K * 2.0 ** -23 * mag
    if h_err is not None:
        err = err + h_err.double() @ w.abs().T
    v = to_bf16(h @ w.T + (b.double() if b is not None else 0.0))
    bound = err + (1 + extra_ulps) * ulp_bf16(v.abs() + err)
    if n_affine:
        s, t = scale.double()[:n_affine], shift.double()[:n_affine]
        qa = to_bf16(v[:, :n_affine] * s + t)
        qb = bound[:, :n_affine] * s.abs()
        qb = qb + ulp_bf16(qa.abs() + qb)
        v = torch.cat([qa, v[:, n_affine:]], 1)
        bound = torch.cat([qb, bound[:, n_affine:]], 1)
    return v, bound


def check_close(got, ref, bound, what, min_equal=0.99):
    """Every value within its bound, and at least min_equal of them bit-equal to the host's."""
    d = (got.double() - ref).abs()
    over = d > bound
    assert not bool(over.any()), (f"{what}: {int(over.sum())} of {d.numel()} values beyond the bound (worst "
                                  f"{float((d / bound).max()):.2f} x bound)")
    eq = float((d == 0).double().mean())
    assert eq >= min_equal, f"{what}: only {eq:.4f} of the values are bit-equal to the host's"
    return eq


def check_scores(q, keys, s1, s2, what="sub-key scores"):
    """s1, s2 (M, H, NK) against the fp64 products of the kernel's own q (M, H, k_dim) with the sub-keys
    (H, 2, NK, half): within one bf16 ulp of the exact value plus fp32 accumulation slack."""
    q, keys = q.double(), keys.double()
    half = q.shape[-1] // 2
    for p, s in ((0, s1), (1, s2)):
        qp = q[..., p * half:(p + 1) * half]
        ref = torch.einsum("mhd,hkd->mhk", qp, keys[:, p])
        mag = torch.einsum("mhd,hkd->mhk", qp.abs(), keys[:, p].abs())
        d = (s.double() - ref).abs()
        bound = 2.0 ** -7 * ref.abs() + 1e-5 * mag
        assert bool((d <= bound).all()), f"{what} (half {p}): {int((d > bound).sum())} values off"


@torch.no_grad()
def randomize_batchnorm(bn, seed):
    """Eval statistics and affine parameters away from the identity (running mean N(0, 0.1), variance U(0.5, 2),
    weight U(0.5, 1.5), bias N(0, 0.1)), so that every query column gets its own scale and shift and a column
    mix-up changes the result."""
    g = torch.Generator().manual_seed(seed)
    n = bn.num_features
    for t, v in ((bn.running_mean, torch.randn(n, generator=g) * 0.1),
                 (bn.running_var, torch.rand(n, generator=g) * 1.5 + 0.5),
                 (bn.weight, torch.rand(n, generator=g) + 0.5), (bn.bias, torch.randn(n, generator=g) * 0.1)):
        t.copy_(v.to(t.dtype))


def batchnorm_affine(bn):
    """fp64 (scale, shift) of an eval BatchNorm1d from its stored (bf16) parameters and statistics."""
    scale = torch.rsqrt(bn.running_var.double().cpu() + bn.eps) * bn.weight.double().cpu()
    return scale, bn.bias.double().cpu() - bn.running_mean.double().cpu() * scale


def memory_weights(mem):
    """query_proj | swilu_proj weights and biases of a memory layer (host fp64), the query width and the affine."""
    w = torch.cat([mem.query_proj.weight, mem.swilu_proj.weight]).double().cpu()
    b = torch.cat([mem.query_proj.bias, mem.swilu_proj.bias]).double().cpu()
    scale, shift = batchnorm_affine(mem.query_norm)
    return w, b, mem.heads * mem.k_dim, scale, shift


def check_decode_step_query(model, layer, r):
    """One fused decode step's memory layer (r = _FusedDecodeStep.run's record[layer]): the query and swilu
    projection recomputed from the residual row r["x"] through the ffn_norm, query_proj | swilu_proj and the
    BatchNorm, then the sub-key scores from the kernel's own query."""
    blk = model.layers[layer]
    mem = blk.ffn
    h, herr = rms_norm_bf16(r["x"].cpu(), blk.ffn_norm.weight.cpu(), model.cfg.norm_eps)
    w, b, nq, scale, shift = memory_weights(mem)
    ref, bound = linear_bf16(h, w, b, scale, shift, n_affine=nq, h_err=herr)
    check_close(r["q"].cpu(), ref[:, :nq], bound[:, :nq], "memory query")
    check_close(r["pre"].cpu(), ref[:, nq:], bound[:, nq:], "swilu projection")
    B = r["x"].shape[0]
    check_scores(r["q"].view(B, mem.heads, mem.k_dim).cpu(), mem.keys.detach().cpu(), r["s1"].cpu(),
                 r["s2"].cpu())


def check_layer_query(mem, rows, min_equal=0.5):
    """A memory layer's recorded no-grad lookup (mem.last_lookup, record=True) on the token rows `rows`: the query
    recomputed from the layer's input through query_proj and the BatchNorm, and the sub-key scores from the
    kernel's own query.  The projection there is a library GEMM whose rounding of the bias is not known (one more
    bf16 rounding is allowed, and half of the values must be bit-equal)."""
    L = mem.last_lookup
    x = L["x"].index_select(0, rows).cpu()
    w, b, nq, scale, shift = memory_weights(mem)
    ref, bound = linear_bf16(x.double(), w[:nq], b[:nq], scale, shift, n_affine=nq, extra_ulps=1)
    q = L["q"].index_select(0, rows)
    check_close(q.reshape(len(rows), nq).cpu(), ref, bound, "memory query", min_equal=min_equal)
    check_scores(q.cpu(), mem.keys.detach().cpu(), L["s1"].index_select(0, rows).cpu(),
                 L["s2"].index_select(0, rows).cpu())
