"""Product-key memory layer with the module API of smlm/pkm.py (constructor, parameters and state_dict keys,
forward, get_indices, subkey_scores, read_values, score_scale, macs_per_token, record / last_* and the decode
graph switch), whose lookup runs on the gfx950 kernels of smlm_hip.kernels:

    query_proj -> BatchNorm (fp32, eval statistics) -> pk_scores (MFMA) -> pk_select -> softmax
    -> bag_infer (value gather, swilu epilogue, bf16 out) -> value_proj
(with bf16 activations, swilu, at most 4 heads and a table in device or pinned memory, pk_select and bag_infer are
one launch, pk_select_bag, with the same results)

impl: "hip", or the reference's names "torch" and "triton" (smlm/pkm.py:48), which a reference config carries;
every name runs the same kernels (there is one implementation here) and is kept in self.impl for the config.
Shapes: any n_keys <= 65536 and knn <= min(n_keys, 128) (the reference's torch path takes any); "triton" keeps
the reference's power-of-two rule for it.

A forward that autograd records (training) takes the reference's differentiable path with the HIP kernels where the
reference uses its Triton ones (smlm/pkm.py:186-228): torch query projection and BatchNorm, sub-key scores by
torch.einsum (its backward is two library GEMMs), the selection and its backward on the kernels (kernels.PKSelect),
and the values through the row-sparse bag (smlm_hip.sparse_values: fp32 accumulator + touched flags for
LazyRowAdam) or, with value_grad="dense", F.embedding_bag.
"""
import math

import torch
import torch.nn.functional as F
from torch import nn

from . import kernels
from .sparse_values import check_impl, row_sparse_embedding_bag


def _pow2(n):
    return n > 0 and n & (n - 1) == 0


def _autocast_bf16(x):
    return x.is_cuda and torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


def inference_tables(values):
    """(table, scales) that the inference kernels read for this values module: its inference table (a tuple, or
    the device / pinned-host tensors of a smlm_hip.offload table), else the weights; None when the table stages
    every call through the host (then infer_table.bag() runs the value bag)."""
    t = getattr(values, "infer_table", None)
    if t is None:
        return values.weight.detach(), None
    if hasattr(t, "bag"):
        return t.device_tables()
    return t


def state_tensors(module):
    """The parameters and buffers of `module`, as a list to keep: walking the module tree costs ~0.3 ms of host time
    per call on the configs' LM, checking a kept list ~20 us."""
    return list(module.parameters()) + list(module.buffers())


def state_tag(tensors):
    """(data_ptr, _version) of every tensor of `tensors` (state_tensors).  It changes whenever one of them is
    written in place or has its storage replaced (an optimizer step, load_state_dict, new BatchNorm statistics,
    .to()), so a captured HIP graph, which reads the tensors and the derived copies (cast sub-keys, BatchNorm
    affine) it was captured with, is valid only while the tag it was captured under holds.  A parameter or buffer
    replaced by another object is not in a list kept from before: drop the graphs after such a change."""
    return tuple((t.data_ptr(), t._version) for t in tensors)


class ProductKeyMemory(nn.Module):
    """Same constructor as smlm/pkm.py:33-92 (impl defaults to "hip"; "torch" and "triton" are accepted)."""

    def __init__(self, d_in, d_out, n_keys=512, heads=4, knn=32, k_dim=256, v_dim=-1,
                 query_norm="batchnorm", swilu=True, value_impl="embedding_bag",
                 keys_weight_decay=True, score_scale="none", score_scale_init=1.0, shared_values=None,
                 value_grad="dense", impl="hip"):
        super().__init__()
        if k_dim % 2 or knn > n_keys:
            raise ValueError(f"k_dim must be even and knn <= n_keys, got k_dim={k_dim}, knn={knn}, n_keys={n_keys}")
        check_impl(impl, "ProductKeyMemory")
        if impl == "triton" and not (_pow2(n_keys) and n_keys <= 65536 and _pow2(knn)):
            # the reference's rule for its Triton kernels (smlm/pkm.py:49-53), kept for configs that name them
            raise ValueError(f"mem_impl='triton' needs n_keys and knn to be powers of two and n_keys <= 65536, "
                             f"got n_keys={n_keys}, knn={knn}. Use mem_impl='torch' for other sizes.")
        if n_keys > kernels.MAX_N_KEYS or knn > kernels.MAX_KNN:
            # the selection keys hold sub-key indices in 16 bits; the result lists hold up to 128 entries
            raise ValueError(f"the HIP kernels take n_keys <= {kernels.MAX_N_KEYS} and knn <= {kernels.MAX_KNN}, "
                             f"got n_keys={n_keys}, knn={knn} (mem_impl={impl!r}).")
        if value_grad not in ("dense", "row_sparse"):
            raise ValueError(value_grad)
        self.d_in, self.d_out = d_in, d_out
        self.n_keys, self.heads, self.knn, self.k_dim = n_keys, heads, knn, k_dim
        self.size = n_keys ** 2
        self.v_dim = v_dim if v_dim > 0 else d_out
        self.swilu = swilu
        self.value_impl = value_impl
        self.value_grad = value_grad
        self.impl = impl
        self.score_scale_init = score_scale_init

        self.keys = nn.Parameter(torch.empty(heads, 2, n_keys, k_dim // 2))
        if not keys_weight_decay:
            self.keys.no_weight_decay = True
        if score_scale == "learned":
            if score_scale_init <= 0:
                raise ValueError("score_scale_init must be > 0")
            self.log_score_scale = nn.Parameter(torch.empty(heads))
        elif score_scale == "none":
            self.log_score_scale = None
        else:
            raise ValueError(score_scale)
        self.query_proj = nn.Linear(d_in, heads * k_dim, bias=True)
        if query_norm == "batchnorm":
            self.query_norm = nn.BatchNorm1d(heads * k_dim)
        elif query_norm == "none":
            self.query_norm = None
        else:
            raise ValueError(query_norm)
        if shared_values is not None:
            if tuple(shared_values.weight.shape) != (self.size, self.v_dim):
                raise ValueError(f"shared value table must be ({self.size}, {self.v_dim}), got "
                                 f"{tuple(shared_values.weight.shape)}")
            self.values = shared_values
        else:
            self.values = nn.Embedding(self.size, self.v_dim)
        if swilu:
            self.swilu_proj = nn.Linear(d_in, self.v_dim)
            self.value_proj = nn.Linear(self.v_dim, d_out)
        elif self.v_dim != d_out:
            raise ValueError("without swilu the value width must equal d_out")
        self.record = False
        self.last_indices = None
        self.last_scores = None
        self.last_weights = None
        self.last_lookup = None     # with record, also the no-grad lookup's input, query and sub-key scores
        self.decode_graph = False
        self._graph = None
        self._graph_state = None    # state_tensors(self), kept for the graph's state_tag
        self._keys_cache = {}
        self._bn_cache = None
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        """The reference's initialisation (smlm/pkm.py:94-109)."""
        lim = 1.0 / math.sqrt(self.k_dim)
        self.keys.uniform_(-lim, lim)
        self.values.weight.normal_(0.0, self.v_dim ** -0.5)
        nn.init.xavier_uniform_(self.query_proj.weight)
        self.query_proj.bias.zero_()
        if self.swilu:
            std = self.d_out ** -0.5
            self.swilu_proj.weight.normal_(0.0, std)
            self.value_proj.weight.normal_(0.0, std)
            self.swilu_proj.bias.zero_()
            self.value_proj.bias.zero_()
        if self.log_score_scale is not None:
            self.log_score_scale.fill_(math.log(self.score_scale_init))
        self.values.weight.pk_value_param = True

    def score_scale(self):
        """Per-head multiplier of the selected scores before the softmax (ones if disabled)."""
        if self.log_score_scale is None:
            return torch.ones(self.heads, device=self.keys.device)
        return self.log_score_scale.exp()

    # ---- lookup pieces -----------------------------------------------------------------------------------
    def _keys_as(self, dtype):
        """The sub-keys in the scoring dtype; a cast copy per dtype is cached until the parameter changes (one per
        dtype, so that asking for another dtype does not free a copy a captured graph reads)."""
        k = self.keys
        if k.dtype == dtype:
            return k.detach()
        tag = (k.data_ptr(), k._version)
        hit = self._keys_cache.get(dtype)
        if hit is None or hit[0] != tag:
            hit = self._keys_cache[dtype] = (tag, k.detach().to(dtype).contiguous())
        return hit[1]

    def subkey_scores(self, query):
        """query (N, heads, k_dim) -> scores against both sub-key sets, each (N, heads, n_keys)."""
        return kernels.pk_scores(query, self._keys_as(query.dtype))

    def get_indices(self, query):
        """query (N, heads, k_dim) -> scores, indices (N, heads, knn): exact top-knn over all n_keys^2 keys."""
        s1, s2 = self.subkey_scores(query)
        scores, indices, _ = kernels.pk_select(s1, s2, self.knn)
        return scores, indices

    def read_values(self, indices, weights):
        """indices, weights (N, heads*knn) -> (N, v_dim) = sum_j weights[:, j] * values[indices[:, j]]"""
        table = self.values.weight.detach()
        return kernels.bag_forward(indices, weights, table).to(table.dtype)

    # ---- forward -------------------------------------------------------------------------------------------
    def forward(self, x):
        shape = x.shape
        x = x.reshape(-1, self.d_in)
        if (self.decode_graph and not self.record and not torch.is_grad_enabled() and x.is_cuda
                and not torch.cuda.is_current_stream_capturing() and inference_tables(self.values) is not None):
            return self._graph_forward(x).view(*shape[:-1], self.d_out)
        return self._forward(x).view(*shape[:-1], self.d_out)

    def _graph_forward(self, x):
        """Replay a HIP graph of _forward captured for this input shape (any token count): the same kernels as
        the eager path without the per-op launch cost.  Re-captured when the shape, dtype, autocast state or
        inference table changes, or when a parameter or buffer was written (state_tag); after replacing one by
        another object, set self._graph = None."""
        ac = torch.is_autocast_enabled("cuda")
        if self._graph_state is None:
            self._graph_state = state_tensors(self)
        tag = (tuple(x.shape), x.dtype, ac, torch.get_autocast_dtype("cuda") if ac else None,
               id(getattr(self.values, "infer_table", None)), state_tag(self._graph_state))
        if self._graph is None or self._graph[0] != tag:
            static_x = x.clone()
            ctx = (torch.autocast("cuda", dtype=tag[3], cache_enabled=False) if ac
                   else torch.autocast("cuda", enabled=False))
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side), ctx:
                for _ in range(2):
                    self._forward(static_x)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph), ctx:
                static_out = self._forward(static_x)
            self._graph = (tag, graph, static_x, static_out)
        _, graph, static_x, static_out = self._graph
        static_x.copy_(x)
        graph.replay()
        return static_out.clone()

    def _query(self, x):
        bn = self.query_norm
        if bn is not None and bn.training:
            raise NotImplementedError("smlm_hip is inference-only: put the model in eval() mode")
        w, b = self.query_proj.weight, self.query_proj.bias
        if (bn is not None and x.is_cuda and x.dtype == torch.bfloat16 and x.numel() >= 128 * x.shape[-1]
                and kernels.prompt_linear_supported(x, w, b)
                and not (torch.is_grad_enabled() and (x.requires_grad or w.requires_grad))
                and not (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") != torch.bfloat16)):
            # prompt passes: the projection and the BatchNorm below in one launch (the same roundings)
            scale, shift = self._bn_affine()
            return kernels.prompt_linear(x, w, b, scale, shift)
        q = self.query_proj(x)
        if bn is not None:
            # BatchNorm with the running statistics, in fp32 whatever the parameter dtype: q * scale + shift
            scale, shift = self._bn_affine()
            if q.is_cuda and q.dtype == torch.bfloat16 and q.shape[-1] % 8 == 0 and not (
                    torch.is_grad_enabled() and q.requires_grad):
                return kernels.affine_bf16(q, scale, shift)     # straight to the bf16 the scores are computed on
            q = torch.addcmul(shift, q, scale)
        return q

    def _bn_affine(self):
        """fp32 (scale, shift) of the eval-mode BatchNorm, cached until its parameters or statistics change."""
        bn = self.query_norm
        parts = (bn.running_mean, bn.running_var, bn.weight, bn.bias)
        tag = tuple((t.data_ptr(), t._version) if t is not None else None for t in parts)
        if self._bn_cache is None or self._bn_cache[0] != tag:
            inv = torch.rsqrt(bn.running_var.float() + bn.eps)
            scale = inv * bn.weight.float() if bn.weight is not None else inv
            shift = -bn.running_mean.float() * scale
            if bn.bias is not None:
                shift = shift + bn.bias.float()
            self._bn_cache = (tag, scale, shift)
        return self._bn_cache[1], self._bn_cache[2]

    def _train_forward(self, x):
        """The differentiable lookup (smlm/pkm.py:186-228 with impl="triton"): the kernels' selection with its
        backward (kernels.PKSelect), row-sparse or dense value gradients."""
        N = x.shape[0]
        q = self.query_proj(x)
        if self.query_norm is not None:
            q = self.query_norm(q.to(self.query_norm.weight.dtype))     # BN in fp32 under autocast
        q = q.view(N, self.heads, self.k_dim)
        if _autocast_bf16(x):
            q = q.to(torch.bfloat16)
        half = self.k_dim // 2
        k1, k2 = self.keys[:, 0], self.keys[:, 1]
        s1 = torch.einsum("nhd,hkd->nhk", q[..., :half], k1)
        s2 = torch.einsum("nhd,hkd->nhk", q[..., half:], k2)
        if s1.dtype not in (torch.bfloat16, torch.float32):
            s1, s2 = s1.float(), s2.float()
        scores, indices, weights = kernels.PKSelect.apply(s1, s2, self.knn)
        if self.log_score_scale is not None:
            logits = scores.float() * self.log_score_scale.float().exp().view(1, self.heads, 1)
            weights = torch.softmax(logits, dim=-1)
        if self.record:
            self.last_indices = indices.detach()
            self.last_scores = scores.detach()
            self.last_weights = weights.detach()
        idx, w = indices.view(N, -1), weights.view(N, -1)
        table = self.values.weight
        if self.value_grad == "row_sparse":
            out = row_sparse_embedding_bag(idx, w, table, "hip")
        else:
            out = F.embedding_bag(idx, table, per_sample_weights=w.to(table.dtype), mode="sum")
        if self.swilu:
            out = self.value_proj(out * F.silu(self.swilu_proj(x)).to(out.dtype))
        return out

    def _forward(self, x):
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return self._train_forward(x)
        N = x.shape[0]
        bf16 = _autocast_bf16(x) or x.dtype == torch.bfloat16
        sdt = torch.bfloat16 if (bf16 or self.keys.dtype == torch.bfloat16) else torch.float32
        q = self._query(x).to(sdt).view(N, self.heads, self.k_dim)
        s1, s2 = kernels.pk_scores(q, self._keys_as(sdt))
        tables = inference_tables(self.values) if self.swilu and bf16 else None
        if (tables is not None and self.log_score_scale is None
                and kernels.select_bag_supported(self.heads, tables[0], tables[1])):
            # selection, value bag and swilu epilogue in one launch (the same results as pk_select then bag_infer;
            # different workgroups overlap the selection's vector work with the gather's memory traffic)
            pre = kernels.linear(self.swilu_proj, x).to(torch.bfloat16)
            res = kernels.pk_select_bag(s1, s2, self.knn, tables[0], tables[1], pre=pre, out_bf16=True,
                                        record=self.record)
            out = res[0] if self.record else res
            if self.record:
                self.last_scores, self.last_indices, self.last_weights = res[1], res[2], res[3]
                self.last_lookup = {"x": x, "q": q, "s1": s1, "s2": s2}
            return kernels.linear(self.value_proj,
                                  out.to(self.value_proj.weight.dtype) if not _autocast_bf16(x) else out)
        scores, indices, weights = kernels.pk_select(s1, s2, self.knn)
        if self.log_score_scale is not None:
            # a positive per-head scale keeps the selection; only the softmax sharpness changes
            scale = self.log_score_scale.detach().float().exp().view(1, self.heads, 1)
            weights = torch.softmax(scores.float() * scale, dim=-1)
        if self.record:
            self.last_indices, self.last_scores, self.last_weights = indices, scores, weights
            self.last_lookup = {"x": x, "q": q, "s1": s1, "s2": s2}
        idx, w = indices.view(N, -1), weights.view(N, -1)
        if self.swilu and bf16:
            # fused inference bag: value rows (bf16 / fp32 / int8 / q4 table) * bf16(silu(pre)), bf16 out
            pre = kernels.linear(self.swilu_proj, x).to(torch.bfloat16)
            tables = inference_tables(self.values)
            if tables is None:                  # a table tier that stages every call (smlm_hip.offload)
                out = self.values.infer_table.bag(idx, w, pre)
            else:
                out = kernels.bag_infer(idx, w, tables[0], tables[1], pre=pre, out_bf16=True)
            return kernels.linear(self.value_proj,
                                  out.to(self.value_proj.weight.dtype) if not _autocast_bf16(x) else out)
        out = self.read_values(idx, w)
        if self.swilu:
            out = self.value_proj(out * F.silu(self.swilu_proj(x)).to(out.dtype))
        return out

    def macs_per_token(self):
        """Multiply-accumulates per token (analytic): query, sub-key scoring, value bag, swilu."""
        m = self.d_in * self.heads * self.k_dim
        m += self.heads * 2 * self.n_keys * (self.k_dim // 2)
        m += self.heads * self.knn * self.v_dim
        if self.swilu:
            m += self.d_in * self.v_dim + self.v_dim * self.d_out + self.v_dim
        return m
