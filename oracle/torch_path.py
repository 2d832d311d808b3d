"""Reference PyTorch path on the CPU -- TEST INFRASTRUCTURE ONLY (the LM-level checker and the timed CPU
baseline of bench.py; the product path never calls it).

A functional restatement of the reference's torch implementation, driven by a state_dict with the
reference's key names:
  pkm_forward     smlm/pkm.py:117-148, 186-228 with impl="torch": query_proj, BatchNorm (eval), two einsums,
                  topk per half, Cartesian topk over all knn^2 sums, softmax, F.embedding_bag, swilu
  lm_forward      smlm/model.py:63-118, 156-163, 266-293: RMSNorm, RoPE, causal attention with a dict KV cache,
                  SwiGLU, tied lm_head
  greedy_decode   the decode loop of smlm/train.py:283-301 (prefill, then one token per step, argmax)
  select_backward        PKSelect.backward, smlm/kernels.py:253-266 (torch ops in the reference too)
  bag_backward_rows      the torch branch of the row-sparse bag backward, smlm/sparse_values.py:66-104
  lazy_adam_fp32_step    the fp32 torch path of LazyRowAdam.step, smlm/sparse_values.py:271-306
Everything runs in the dtype of the given weights (fp32 or fp64).  torch.topk breaks ties in an unspecified
order, exactly like the reference's torch path; on tie-free scores it selects what pk_select selects.
"""
import math

import torch
import torch.nn.functional as F


def rms_norm(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope(x, pos0, theta):
    hd = x.shape[-1]
    T = x.shape[-2]
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    ang = torch.outer(torch.arange(pos0, pos0 + T, dtype=torch.float32), inv)
    cos, sin = ang.cos().to(x.dtype), ang.sin().to(x.dtype)
    a, b = x[..., :hd // 2], x[..., hd // 2:]
    return torch.cat([a * cos - b * sin, a * sin + b * cos], dim=-1)


def attention(sd, p, x, cfg, cache, pos0):
    B, T, C = x.shape
    H = cfg["n_heads"]
    hd = C // H
    qkv = (x @ sd[p + "wqkv.weight"].T).view(B, T, 3, H, hd).permute(2, 0, 3, 1, 4)
    q, k, v = rope(qkv[0], pos0, cfg["rope_theta"]), rope(qkv[1], pos0, cfg["rope_theta"]), qkv[2]
    if cache is not None:
        if "k" in cache:
            k = torch.cat([cache["k"], k], 2)
            v = torch.cat([cache["v"], v], 2)
        cache["k"], cache["v"] = k, v
    S = k.shape[2]
    s = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
    if T > 1:
        mask = torch.ones(T, S, dtype=torch.bool).tril(S - T)
        s = s.masked_fill(~mask, float("-inf"))
    y = torch.softmax(s, -1) @ v
    return y.transpose(1, 2).reshape(B, T, C) @ sd[p + "wo.weight"].T


def pkm_select_torch(s1, s2, knn):
    """get_indices of smlm/pkm.py:125-136 on given sub-key scores (N, H, NK)."""
    N, H, NK = s1.shape
    a1, i1 = s1.topk(knn, -1)
    a2, i2 = s2.topk(knn, -1)
    alls = (a1.unsqueeze(-1) + a2.unsqueeze(-2)).reshape(N, H, knn * knn)
    alli = (i1.unsqueeze(-1) * NK + i2.unsqueeze(-2)).reshape(N, H, knn * knn)
    sc, best = alls.topk(knn, -1)
    return sc, alli.gather(-1, best)


def pkm_forward(sd, p, x, mcfg, table=None, selection=None):
    """One memory layer: x (N, d_in) -> (N, d_out).  mcfg: heads, knn, k_dim, n_keys, query_norm, swilu.
    `table` overrides the value table (e.g. a dequantised inference table); `selection` = (indices, weights),
    each (N, heads, knn), replaces the scoring and selection (to check everything downstream of a given
    selection)."""
    N = x.shape[0]
    H, knn, k_dim = mcfg["heads"], mcfg["knn"], mcfg["k_dim"]
    if selection is None:
        q = x @ sd[p + "query_proj.weight"].T + sd[p + "query_proj.bias"]
        if mcfg["query_norm"] == "batchnorm":
            q = (q - sd[p + "query_norm.running_mean"]) / torch.sqrt(sd[p + "query_norm.running_var"] + 1e-5)
            q = q * sd[p + "query_norm.weight"] + sd[p + "query_norm.bias"]
        q = q.view(N, H, k_dim)
        keys = sd[p + "keys"]
        half = k_dim // 2
        s1 = torch.einsum("nhd,hkd->nhk", q[..., :half], keys[:, 0])
        s2 = torch.einsum("nhd,hkd->nhk", q[..., half:], keys[:, 1])
        scores, idx = pkm_select_torch(s1, s2, knn)
        w = torch.softmax(scores, -1)
    else:
        idx, w = selection[0], selection[1].to(x.dtype)
    values = sd[p + "values.weight"] if table is None else table
    if values.dtype == x.dtype:
        out = F.embedding_bag(idx.view(N, -1), values, per_sample_weights=w.view(N, -1), mode="sum")
    else:
        # a table stored in another dtype (bf16): the reference's value_impl="gather" form (smlm/pkm.py:147-148)
        out = torch.einsum("nj,njd->nd", w.view(N, -1), F.embedding(idx.view(N, -1), values).to(x.dtype))
    if mcfg["swilu"]:
        pre = x @ sd[p + "swilu_proj.weight"].T + sd[p + "swilu_proj.bias"]
        out = (out * F.silu(pre)) @ sd[p + "value_proj.weight"].T + sd[p + "value_proj.bias"]
    return out


def lm_forward(sd, cfg, idx, caches=None, pos0=0, tables=None, last_only=False, selections=None, positions=None):
    """Logits (B, T, vocab) of the decoder with the memory layers cfg["mem_layers"] (only the last position's,
    (B, 1, vocab), with last_only; only those at the chunk offsets `positions`, (B, len, vocab), with a
    positions index tensor).  selections: {layer: (indices, weights)} given to pkm_forward."""
    x = sd["tok_emb.weight"][idx]
    mcfg = dict(heads=cfg["mem_heads"], knn=cfg["mem_knn"], k_dim=cfg["mem_k_dim"], n_keys=cfg["mem_n_keys"],
                query_norm=cfg["mem_query_norm"], swilu=cfg["mem_swilu"])
    eps = cfg["norm_eps"]
    for i in range(cfg["n_layers"]):
        p = f"layers.{i}."
        x = x + attention(sd, p + "attn.", rms_norm(x, sd[p + "attn_norm.weight"], eps), cfg,
                          None if caches is None else caches[i], pos0)
        h = rms_norm(x, sd[p + "ffn_norm.weight"], eps)
        if i in cfg["mem_layers"]:
            B, T, C = h.shape
            t = None if tables is None else tables.get(i)
            sel = None if selections is None else selections.get(i)
            x = x + pkm_forward(sd, p + "ffn.", h.reshape(B * T, C), mcfg, t, sel).view(B, T, -1)
        else:
            a, b = (h @ sd[p + "ffn.w13.weight"].T).chunk(2, -1)
            x = x + (F.silu(a) * b) @ sd[p + "ffn.w2.weight"].T
    if last_only:
        x = x[:, -1:]
    elif positions is not None:
        x = x[:, positions]
    return rms_norm(x, sd["norm.weight"], eps) @ sd["tok_emb.weight"].T


def greedy_decode(sd, cfg, prompt, new_tokens):
    """Prefill + new_tokens greedy steps with a dict KV cache -> generated ids (B, new_tokens + 1)."""
    caches = [dict() for _ in range(cfg["n_layers"])]
    logits = lm_forward(sd, cfg, prompt, caches, 0)
    nxt = logits[:, -1:].argmax(-1)
    out = [nxt]
    P = prompt.shape[1]
    for i in range(new_tokens):
        logits = lm_forward(sd, cfg, nxt, caches, P + i)
        nxt = logits[:, -1:].argmax(-1)
        out.append(nxt)
    return torch.cat(out, 1)


def select_backward(idx, w, g_scores, g_w, nk, dtype):
    """PKSelect.backward (smlm/kernels.py:253-266): the softmax backward of the knn weights plus the scores' own
    gradient, rounded to the scores' dtype, scattered (fp32 sums) into dense (N, H, nk) gradients of both halves and
    rounded once.  idx (N, H, knn) int64, w (N, H, knn) fp32, g_scores of dtype or None, g_w fp32 or None."""
    dl = torch.zeros_like(w)
    if g_w is not None:
        dl = w * (g_w - (w * g_w).sum(-1, keepdim=True))
    if g_scores is not None:
        dl = dl + g_scores.float()
    ds = dl.to(dtype).float()
    N, H, _ = idx.shape
    z = torch.zeros(N, H, nk, dtype=torch.float32)
    ds1 = z.scatter_add(-1, idx // nk, ds).to(dtype)
    ds2 = z.scatter_add_(-1, idx % nk, ds).to(dtype)
    return ds1, ds2


ACC_CHUNK = 1 << 18     # lookups per accumulation chunk (smlm/sparse_values.py:23)


def bag_backward_rows(grad_out, idx, w, table, acc, touched):
    """The reference's torch branch of the row-sparse bag backward (smlm/sparse_values.py:66-104), in place on acc and
    touched: the bags' offsets and lookup -> bag map as its forward builds them (76-81), the per-sample-weight
    gradient by aten's embedding-bag backward (98-99), each lookup's w * g added into acc by index_put_ with
    accumulation in chunks of 2^18 lookups (100-102), then the rows flagged (103).  grad_out (N, D), idx (N, K)
    int64, w (N, K), table (rows, D), acc (rows, D), touched (rows,) bool.  Returns gw (N, K)."""
    n, j = idx.shape
    flat = idx.reshape(-1).contiguous()
    wf = w.reshape(-1).to(table.dtype).contiguous()
    offsets = torch.arange(0, n * j, j)
    offset2bag = torch.arange(n).repeat_interleave(j)
    g = grad_out.contiguous().to(acc.dtype)
    gw = torch.ops.aten._embedding_bag_per_sample_weights_backward(g.to(table.dtype), table, flat, offsets,
                                                                   offset2bag, 0, -1)
    for a in range(0, flat.numel(), ACC_CHUNK):
        contrib = g.index_select(0, offset2bag[a:a + ACC_CHUNK]).mul_(wf[a:a + ACC_CHUNK, None].to(g.dtype))
        acc.index_put_((flat[a:a + ACC_CHUNK],), contrib, accumulate=True)
    touched[flat] = True
    return gw.view(n, j)


def lazy_adam_fp32_step(param, adam, acc, touched, grad_scale=1.0):
    """The fp32 torch path of LazyRowAdam.step (smlm/sparse_values.py:271-306) for one table: param an
    nn.Parameter, adam its torch.optim.Adam; the unread rows' parameters and moments are kept aside (287-290), the
    accumulator (scaled) becomes the gradient of one dense Adam step (291-296), the kept rows are put back (297-303)
    and the accumulator and flags cleared (306, RowStore.reset at 34-41)."""
    if not bool(touched.any()):
        return
    state = adam.state[param]
    unread = (~touched).nonzero().squeeze(1)
    keep = [param.data.index_select(0, unread)]
    if state:
        keep += [state["exp_avg"].index_select(0, unread), state["exp_avg_sq"].index_select(0, unread)]
    if grad_scale != 1.0:
        acc.mul_(grad_scale)
    param.grad = acc
    adam.step()
    param.grad = None
    param.data.index_put_((unread,), keep[0])
    if len(keep) == 3:
        state["exp_avg"].index_put_((unread,), keep[1])
        state["exp_avg_sq"].index_put_((unread,), keep[2])
    else:
        state["exp_avg"].index_fill_(0, unread, 0.0)
        state["exp_avg_sq"].index_fill_(0, unread, 0.0)
    acc.zero_()
    touched.zero_()
