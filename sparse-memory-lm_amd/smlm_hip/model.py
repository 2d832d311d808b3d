"""Llama-style decoder with product-key memory layers: the entry points of smlm/model.py (ModelConfig,
Transformer.forward(idx, targets, kv_caches, pos0), set_memory_decode_graphs, set_memory_inference_table),
with the memory layers on the gfx950 lookup of smlm_hip.pkm, plus a whole-decode-step HIP graph
(Transformer.generate) over a static KV cache.

The dense parts (RMSNorm, RoPE, attention, SwiGLU, tied lm_head) are PyTorch ops with the reference's arithmetic,
except the single-token decode step over the static cache, whose RoPE + cache write + attention is one HIP kernel
(smlm_hip.kernels.decode_attention); state_dict keys are the reference's, so a reference checkpoint of a supported
config loads as is.
"""
import math
from dataclasses import asdict, dataclass, field

import torch
import torch.nn.functional as F
from torch import nn

from . import kernels
from .engram import EngramMemory, NgramHash
from .pkm import ProductKeyMemory, inference_tables, state_tag, state_tensors


@dataclass
class ModelConfig:
    """Fields and defaults of smlm/model.py:13-60 (mem_impl defaults to "hip"; a reference config's "torch" or
    "triton" runs the same kernels)."""
    vocab_size: int = 50304
    d_model: int = 384
    n_layers: int = 12
    n_heads: int = 6
    ffn_hidden: int = 1024
    max_seq_len: int = 1024
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    init_std: float = 0.02
    mem_layers: list = field(default_factory=list)
    mem_n_keys: int = 512
    mem_heads: int = 4
    mem_knn: int = 32
    mem_k_dim: int = 256
    mem_v_dim: int = -1
    mem_query_norm: str = "batchnorm"
    mem_swilu: bool = True
    mem_value_impl: str = "embedding_bag"
    mem_keys_weight_decay: bool = True
    mem_score_scale: str = "none"
    mem_score_scale_init: float = 1.0
    mem_share_values: bool = False
    mem_round_layers: list = field(default_factory=list)
    mem_value_grad: str = "dense"
    mem_impl: str = "hip"
    eng_layers: list = field(default_factory=list)
    eng_orders: list = field(default_factory=lambda: [2, 3])
    eng_heads: int = 8
    eng_head_dim: int = 24
    eng_rows: int = 524287
    eng_conv_kernel: int = 4
    eng_hash_seed: int = 0
    eng_impl: str = "triton"
    eng_value_grad: str = "row_sparse"

    def to_dict(self):
        return asdict(self)


class RotaryEmbedding(nn.Module):
    """RoPE on the two halves of each head (smlm/model.py:63-78).  pos0 is an int, or a 0-d / 1-element
    device tensor (single-token decode inside a captured graph)."""

    def __init__(self, head_dim, max_seq_len, theta):
        super().__init__()
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
        ang = torch.outer(torch.arange(max_seq_len).float(), inv)
        self.register_buffer("cos", ang.cos(), persistent=False)
        self.register_buffer("sin", ang.sin(), persistent=False)

    def forward(self, x, pos0=0):
        if torch.is_tensor(pos0):
            cos = self.cos.index_select(0, pos0.view(1)).to(x.dtype)
            sin = self.sin.index_select(0, pos0.view(1)).to(x.dtype)
        else:
            T = x.shape[-2]
            cos = self.cos[pos0:pos0 + T].to(x.dtype)
            sin = self.sin[pos0:pos0 + T].to(x.dtype)
        a, b = x.chunk(2, dim=-1)
        return torch.cat([a * cos - b * sin, a * sin + b * cos], dim=-1)


class StaticKVCache:
    """Preallocated (B, heads, max_len, head_dim) key/value buffers of one attention layer, written in place, so
    a decode step has fixed shapes and addresses and can be captured in a HIP graph."""

    def __init__(self, B, n_heads, max_len, head_dim, dtype, device):
        self.k = torch.zeros(B, n_heads, max_len, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.slots = torch.arange(max_len, device=device)
        self.max_len = max_len
        self.extra = {}                     # per-layer decode state of other modules (Engram: "eng_u", "eng_hist")

    def get(self, key, default=None):
        return self.extra.get(key, default)

    def __getitem__(self, key):
        return self.extra[key]

    def __setitem__(self, key, value):
        self.extra[key] = value


class Attention(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.n_heads = cfg.n_heads
        self.head_dim = cfg.d_model // cfg.n_heads
        self.wqkv = nn.Linear(cfg.d_model, 3 * cfg.d_model, bias=False)
        self.wo = nn.Linear(cfg.d_model, cfg.d_model, bias=False)
        self.rope = RotaryEmbedding(self.head_dim, cfg.max_seq_len, cfg.rope_theta)

    def forward(self, x, kv_cache=None, pos0=0):
        B, T, C = x.shape
        if (T == 1 and torch.is_tensor(pos0) and isinstance(kv_cache, StaticKVCache) and x.is_cuda
                and kv_cache.k.dtype == torch.bfloat16 and self.head_dim in (16, 32, 64, 128)):
            # one decode step: RoPE, cache write and attention in one kernel (smlm_hip.kernels.decode_attention)
            qkv = self.wqkv(x).view(B, 3 * C).to(torch.bfloat16)
            y = kernels.decode_attention(qkv, self.rope.cos, self.rope.sin, pos0, kv_cache.k, kv_cache.v)
            return self.wo(y.view(B, 1, C).to(x.dtype))
        # prompt passes: the projections through kernels.linear (smlm_prompt_linear from 128 rows on, no autograd)
        qkv = kernels.linear(self.wqkv, x)
        if not torch.is_tensor(pos0) and _use_attention_kernels(qkv, self.head_dim):
            return kernels.linear(self.wo, self._prefill_kernels(qkv, kv_cache, pos0).reshape(B, T, C))
        q, k, v = qkv.view(B, T, 3, self.n_heads, self.head_dim).permute(2, 0, 3, 1, 4)
        q, k = self.rope(q, pos0), self.rope(k, pos0)
        if isinstance(kv_cache, StaticKVCache):
            y = self._static(q, k, v, kv_cache, pos0)
        else:
            if kv_cache is not None:
                if kv_cache.get("k") is not None:
                    k = torch.cat([kv_cache["k"], k], dim=2)
                    v = torch.cat([kv_cache["v"], v], dim=2)
                kv_cache["k"], kv_cache["v"] = k, v
            y = _causal_attention(q, k, v)
        return kernels.linear(self.wo, y.reshape(B, T, C))

    def _prefill_kernels(self, qkv, kv_cache, pos0):
        """RoPE (smlm_rope_qkv, written straight into the static cache's slots when there is one) and causal
        attention (smlm_prefill_attention) of T new tokens at positions pos0.. -> (B, T, H, hd)."""
        B, T, _ = qkv.shape
        H, hd = self.n_heads, self.head_dim
        q = torch.empty(B, H, T, hd, dtype=qkv.dtype, device=qkv.device)
        if isinstance(kv_cache, StaticKVCache):
            S = pos0 + T
            if S > kv_cache.max_len:
                raise ValueError(f"{T} new tokens at position {pos0} overflow the static cache ({kv_cache.max_len})")
            kernels.rope_qkv(qkv, self.rope.cos, self.rope.sin, pos0, q, kv_cache.k[:, :, pos0:S],
                             kv_cache.v[:, :, pos0:S])
            return kernels.prefill_attention(q, kv_cache.k[:, :, :S], kv_cache.v[:, :, :S])
        k = torch.empty_like(q)
        kernels.rope_qkv(qkv, self.rope.cos, self.rope.sin, pos0, q, k)
        v = qkv.view(B, T, 3, H, hd)[:, :, 2].transpose(1, 2)
        if kv_cache is not None:
            if kv_cache.get("k") is not None:
                k = torch.cat([kv_cache["k"], k], dim=2)
                v = torch.cat([kv_cache["v"], v], dim=2)
            kv_cache["k"], kv_cache["v"] = k, v
        return kernels.prefill_attention(q, k, v)

    def _static(self, q, k, v, cache, pos0):
        T = q.shape[2]
        if torch.is_tensor(pos0):
            # one token at a device-side position: write the slot, attend over the filled prefix
            if T != 1:
                raise ValueError("a device-side position is for single-token decode steps")
            cache.k.index_copy_(2, pos0.view(1), k)
            cache.v.index_copy_(2, pos0.view(1), v)
            return _attention(q, cache.k, cache.v, (cache.slots <= pos0).view(1, 1, 1, -1)).transpose(1, 2)
        cache.k[:, :, pos0:pos0 + T] = k
        cache.v[:, :, pos0:pos0 + T] = v
        S = pos0 + T
        return _causal_attention(q, cache.k[:, :, :S], cache.v[:, :, :S])


def _causal_mask(T, S, device):
    """Token i of T new tokens after S - T cached ones sees keys 0 .. S - T + i (None: sees everything)."""
    if T == 1:
        return None
    return torch.ones(T, S, dtype=torch.bool, device=device).tril(S - T)


def _use_attention_kernels(t, head_dim):
    """bf16 on the GPU without an autograd graph to record: the prompt-pass kernels (forward only) apply."""
    return (t.is_cuda and t.dtype == torch.bfloat16 and head_dim in (32, 64, 128)
            and not (torch.is_grad_enabled() and t.requires_grad))


def _causal_attention(q, k, v):
    """Token i of the T new tokens (q) after S - T earlier ones sees keys 0 .. S - T + i; returns (B, T, H, hd).
    bf16 on the GPU without an autograd graph: the flash-attention kernel (smlm_prefill_attention), which reads the
    permuted / sliced views as they are; otherwise (training, fp32) the torch ops of _attention."""
    if (_use_attention_kernels(q, q.shape[-1]) and k.dtype == v.dtype == torch.bfloat16
            and not (torch.is_grad_enabled() and (k.requires_grad or v.requires_grad))):
        return kernels.prefill_attention(q, k, v)
    return _attention(q, k, v, _causal_mask(q.shape[2], k.shape[2], q.device)).transpose(1, 2)


def _attention(q, k, v, mask):
    """softmax(q k^T / sqrt(head_dim), masked) v for q (B, H, T, hd), k, v (B, H, S, hd); softmax in fp32.
    Both products are bmm calls whose right operand is contiguous (single-token steps compute k q, so the
    cache is never transposed)."""
    B, H, T, hd = q.shape
    S = k.shape[2]
    if T == 1:
        s = torch.bmm(k.reshape(B * H, S, hd), q.reshape(B * H, hd, 1)).view(B, H, 1, S)
    else:
        kt = k.reshape(B * H, S, hd).transpose(1, 2).contiguous()
        s = torch.bmm(q.reshape(B * H, T, hd), kt).view(B, H, T, S)
    s = s.float() * (hd ** -0.5)
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1).to(v.dtype)
    y = torch.bmm(p.view(B * H, T, S), v.reshape(B * H, S, hd).contiguous())
    return y.view(B, H, T, hd)


class SwiGLU(nn.Module):
    def __init__(self, d, hidden):
        super().__init__()
        self.w13 = nn.Linear(d, 2 * hidden, bias=False)
        self.w2 = nn.Linear(hidden, d, bias=False)

    fused_min_rows = 128   # prompt passes: rows from which the projection and activation are one launch

    def forward(self, x):
        """w2(silu(a) * b) with a | b = w13(x).  On bf16 GPU tensors the activation is one kernel
        (smlm_hip.kernels.swiglu) with the same roundings; without autograd, from fused_min_rows rows on, the w13
        projection and the activation are one launch (kernels.linear_swiglu: the same roundings, and the
        projection's products on the matrix cores in fp32), and w2 runs through kernels.linear."""
        w = self.w13.weight
        if (x.is_cuda and x.dtype == torch.bfloat16 and x.numel() >= self.fused_min_rows * x.shape[-1]
                and self.w13.bias is None and kernels.linear_swiglu_supported(x, w)
                and not (torch.is_grad_enabled() and (x.requires_grad or w.requires_grad))
                and not (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") != torch.bfloat16)):
            return kernels.linear(self.w2, kernels.linear_swiglu(x, w))
        h = self.w13(x)
        if h.is_cuda and h.dtype == torch.bfloat16 and h.shape[-1] % 16 == 0:
            act = kernels.swiglu(h)
        else:
            a, b = h.chunk(2, dim=-1)
            act = F.silu(a) * b
        return kernels.linear(self.w2, act)


def _memory(cfg, shared):
    return ProductKeyMemory(
        cfg.d_model, cfg.d_model, n_keys=cfg.mem_n_keys, heads=cfg.mem_heads, knn=cfg.mem_knn, k_dim=cfg.mem_k_dim,
        v_dim=cfg.mem_v_dim, query_norm=cfg.mem_query_norm, swilu=cfg.mem_swilu, value_impl=cfg.mem_value_impl,
        keys_weight_decay=cfg.mem_keys_weight_decay, score_scale=cfg.mem_score_scale,
        score_scale_init=cfg.mem_score_scale_init, shared_values=shared, value_grad=cfg.mem_value_grad,
        impl=cfg.mem_impl)


class Block(nn.Module):
    def __init__(self, cfg, layer_id, shared_values=None):
        super().__init__()
        self.attn_norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.attn = Attention(cfg)
        self.ffn_norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.is_memory = layer_id in cfg.mem_layers
        self.ffn = _memory(cfg, shared_values) if self.is_memory else SwiGLU(cfg.d_model, cfg.ffn_hidden)
        self.ffn_r2 = None
        if layer_id in cfg.mem_round_layers:
            if not (self.is_memory and shared_values is not None):
                raise ValueError("a second read needs a memory layer with a shared value table")
            self.ffn_norm_r2 = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
            self.ffn_r2 = _memory(cfg, shared_values)
        self.engram = None
        if layer_id in cfg.eng_layers:
            self.engram = EngramMemory(cfg.d_model, len(cfg.eng_orders) * cfg.eng_heads, cfg.eng_head_dim,
                                       cfg.eng_rows, conv_kernel=cfg.eng_conv_kernel, dilation=max(cfg.eng_orders),
                                       eps=cfg.norm_eps, impl=cfg.eng_impl, value_grad=cfg.eng_value_grad)

    def forward(self, x, kv_cache=None, pos0=0, eng_rows=None):
        if self.engram is not None:
            x = x + self.engram(x, eng_rows, kv_cache)
        x = x + self.attn(self.attn_norm(x), kv_cache, pos0)
        x = x + self.ffn(self.ffn_norm(x))
        if self.ffn_r2 is not None:
            x = x + self.ffn_r2(self.ffn_norm_r2(x))
        return x


class Transformer(nn.Module):
    def __init__(self, cfg, ngram_canon=None):
        """ngram_canon: the token compression table of the Engram hash ((vocab_size,) int64), needed for Engram
        layers where the GPT-2 tokenizer (tiktoken) is not installed; None computes it with canonical_ids."""
        super().__init__()
        self.cfg = cfg
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        shared = None
        if cfg.mem_share_values and cfg.mem_layers:
            shared = nn.Embedding(cfg.mem_n_keys ** 2, cfg.mem_v_dim if cfg.mem_v_dim > 0 else cfg.d_model)
        self.layers = nn.ModuleList([Block(cfg, i, shared) for i in range(cfg.n_layers)])
        self.norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.tok_emb.weight
        self.ngram = (NgramHash(cfg.vocab_size, cfg.eng_orders, cfg.eng_heads, cfg.eng_rows, cfg.eng_hash_seed,
                                canon=ngram_canon) if cfg.eng_layers else None)
        self._decoders = {}
        self._fwd_graphs = {}
        self._fwd_graphs_tag = None
        self._state = None              # state_tensors(self), kept for the graphs' state_tag
        self._init_weights()

    @torch.no_grad()
    def _init_weights(self):
        """The reference's initialisation (smlm/model.py:196-206); memory layers keep their own."""
        std = self.cfg.init_std
        out_std = std / math.sqrt(2 * self.cfg.n_layers)
        self.tok_emb.weight.normal_(0.0, std)
        for blk in self.layers:
            blk.attn.wqkv.weight.normal_(0.0, std)
            blk.attn.wo.weight.normal_(0.0, out_std)
            if not blk.is_memory:
                blk.ffn.w13.weight.normal_(0.0, std)
                blk.ffn.w2.weight.normal_(0.0, out_std)

    def memory_layers(self):
        """All product-key reads in forward order (a second read follows its layer's first)."""
        out = []
        for b in self.layers:
            if b.is_memory:
                out.append(b.ffn)
                if b.ffn_r2 is not None:
                    out.append(b.ffn_r2)
        return out

    def engram_layers(self):
        return [b.engram for b in self.layers if b.engram is not None]

    def memory_sites(self):
        out = []
        for i, b in enumerate(self.layers):
            if b.is_memory:
                out.append(f"L{i}")
                if b.ffn_r2 is not None:
                    out.append(f"L{i}r2")
        return out

    def set_memory_decode_graphs(self, enabled=True):
        """No-grad forwards of the memory layers replay a captured HIP graph per input shape."""
        for m in self.memory_layers():
            m.decode_graph = enabled
            m._graph = None

    @torch.no_grad()
    def set_memory_inference_table(self, kind="fp32"):
        """Inference copy of the value table(s) read by the fused bf16 bag: "fp32" (the weights themselves),
        "bf16", "q4" (4 bit + fp16 row scale) or "int8" (8 bit + fp16 row scale).  Call again after the weights
        change; captured graphs are dropped."""
        seen = set()
        for m in self.memory_layers():
            m._graph = None
            v = m.values
            if id(v) in seen:
                continue
            seen.add(id(v))
            w = v.weight.detach()
            if kind == "fp32":
                v.infer_table = None
            elif kind == "bf16":
                v.infer_table = (w if w.dtype == torch.bfloat16 else w.to(torch.bfloat16), None)
            elif kind == "q4":
                v.infer_table = kernels.quantize_q4(w)
            elif kind == "int8":
                v.infer_table = kernels.quantize_int8(w)
            else:
                raise ValueError(kind)
        self._decoders.clear()
        self._fwd_graphs.clear()

    def forward(self, idx, targets=None, kv_caches=None, pos0=0):
        """Logits (B, T, vocab), or (logits, loss) with targets (smlm/model.py:266-293)."""
        x = self.tok_emb(idx)
        rows = self._ngram_rows(idx, kv_caches) if self.ngram is not None else None
        if (x.is_cuda and x.dtype == torch.bfloat16 and not torch.is_autocast_enabled("cuda")
                and self.ngram is None):
            logits = self.lm_head(self._blocks_fused_norms(x, kv_caches, pos0))
        else:
            for i, blk in enumerate(self.layers):
                x = blk(x, None if kv_caches is None else kv_caches[i], pos0, rows)
            logits = self.lm_head(self.norm(x))
        if targets is None:
            return logits
        loss = F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.reshape(-1))
        return logits, loss

    @torch.no_grad()
    def forward_graphed(self, idx):
        """forward(idx) (logits, no cache, no targets) from a HIP graph captured once per input shape, device and
        autocast state and replayed: the same kernels as the eager forward without a host launch per op (a prompt
        pass of ~60 launches).  The returned logits are the graph's static output, overwritten by the next call
        with the same shape; clone them to keep them.  A graph reads the tensors it was captured with, among them
        derived copies (cast sub-keys, the BatchNorm affine), so every graph is dropped and captured again when a
        parameter or buffer has been written since (state_tag: an optimizer step, load_state_dict, new BatchNorm
        statistics); set_memory_inference_table drops them too, and so must drop_graphs() after a parameter or
        buffer is replaced by another object."""
        tag = state_tag(self.state_tensors())
        if tag != self._fwd_graphs_tag:
            self._fwd_graphs.clear()
            self._fwd_graphs_tag = tag
        ac = torch.is_autocast_enabled("cuda")
        key = (tuple(idx.shape), str(idx.device), ac, torch.get_autocast_dtype("cuda") if ac else None)
        entry = self._fwd_graphs.get(key)
        if entry is None:
            static_idx = idx.clone()
            ctx = (torch.autocast("cuda", dtype=key[3], cache_enabled=False) if ac
                   else torch.autocast("cuda", enabled=False))
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side), ctx:
                for _ in range(2):             # lazily built state (library handles, cached affines) first
                    self(static_idx)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph), ctx:
                static_out = self(static_idx)
            entry = self._fwd_graphs[key] = (graph, static_idx, static_out)
        graph, static_idx, static_out = entry
        static_idx.copy_(idx)
        graph.replay()
        return static_out

    def state_tensors(self):
        """The parameters and buffers, listed once (state_tensors) and kept until drop_graphs()."""
        if self._state is None:
            self._state = state_tensors(self)
        return self._state

    def drop_graphs(self):
        """Forget the captured graphs (forward_graphed's, the decoders' and the memory layers') and the kept
        parameter list: needed after a parameter or buffer is replaced by another object."""
        self._fwd_graphs.clear()
        self._fwd_graphs_tag = None
        self._state = None
        self._decoders.clear()
        for m in self.memory_layers():
            m._graph = None
            m._graph_state = None

    def _ngram_rows(self, idx, kv_caches):
        """Engram rows of this chunk (smlm/model.py:270-279): the hash sees the last history tokens before the
        chunk, the pad id at the start of a sequence, else the ones kept in the first layer's cache."""
        c = self.ngram.canon[idx]
        hist = kv_caches[0].get("eng_hist") if kv_caches is not None else None
        if hist is None:
            hist = torch.full((c.shape[0], self.ngram.history), self.ngram.pad, dtype=c.dtype, device=c.device)
        c = torch.cat([hist, c], 1)
        if kv_caches is not None:
            kv_caches[0]["eng_hist"] = c[:, -self.ngram.history:]
        return self.ngram(c)

    def _blocks_fused_norms(self, x, kv_caches, pos0):
        """The blocks of forward() on bf16 GPU tensors with every residual add fused into the RMSNorm that follows
        it (smlm_hip.kernels.add_rmsnorm): the same sequence x = x + sublayer(norm(x)) per sublayer, ending with
        the final norm.  Returns the normed last hidden state."""
        norms, subs = [], []
        for i, blk in enumerate(self.layers):
            cache = None if kv_caches is None else kv_caches[i]
            norms += [blk.attn_norm, blk.ffn_norm]
            subs += [lambda h, blk=blk, cache=cache: blk.attn(h, cache, pos0), blk.ffn]
            if blk.ffn_r2 is not None:
                norms.append(blk.ffn_norm_r2)
                subs.append(blk.ffn_r2)
        norms.append(self.norm)
        x, h = kernels.add_rmsnorm(x, None, norms[0])
        for sub, norm in zip(subs, norms[1:]):
            x, h = kernels.add_rmsnorm(x, sub(h), norm)
        return h

    # ---- whole-step graph decode -------------------------------------------------------------------------
    @torch.no_grad()
    def generate(self, prompt, new_tokens, use_graph=True, sync_every_step=False):
        """Greedy decoding: prefill `prompt` (B, P) into a static KV cache, then `new_tokens` single-token
        steps, each one forward + argmax (the loop of smlm/train.py:283-301).  With use_graph the whole step
        (embedding, every block, lm_head, argmax, cache write, position update) is captured in a HIP graph, and
        runs of _StepDecoder.run_lengths steps are one replay each.
        Returns the generated ids (B, new_tokens + 1): the prompt's next token, then one per step."""
        B, P = prompt.shape
        dec = self._decoder(B, P + new_tokens + 1, prompt.device)
        tokens = dec.run(prompt, new_tokens, use_graph, sync_every_step)
        return tokens

    def _decoder(self, B, max_len, device):
        key = (B, max_len, str(device), torch.is_autocast_enabled("cuda"), torch.get_autocast_dtype("cuda"))
        if key not in self._decoders:
            self._decoders[key] = _StepDecoder(self, B, max_len, device)
        return self._decoders[key]


class _FusedDecodeStep:
    """One greedy decode step of a bf16 model on the fused decode kernels of smlm_hip.kernels.  Per dense block
        [residual add + attn_norm + wqkv] [RoPE + cache write + attention] [wo]
        [residual add + ffn_norm + w13 + SwiGLU] [w2]
    and per memory block, after the attention,
        [residual add + ffn_norm + query_proj | swilu_proj + eval BatchNorm] [sub-key scores]
        [selection + value bag + swilu] [value_proj]
    then [residual add + final norm + lm_head + argmax partials] [token, history slot, position + 1]; the first
    block's prologue gathers the token embeddings.  Chained steps (run(..., chain=keys), as _StepDecoder runs them)
    drop the last launch: the first launch of the next step picks the token from the argmax partials, writes it and
    its history slot, and the lm_head launch advances the position.  These are the ops of Transformer.forward on bf16 weights
    (smlm/model.py:63-118, 156-163, 266-293; smlm/pkm.py:186-228) with the same bf16 roundings: 5 launches per
    dense block, 7 per memory block and 2 for the head, instead of the ~10 PyTorch launches per block.

    At batches up to proj_max_batch the attention launch also does wo, per head (decode_attention_proj), and the
    next launch's prologue sums the heads: 4 launches per dense block, 6 per memory block (MI355X, config 3:
    0.155 -> 0.144 ms per step at batch 1).  Larger batches keep the wo launch: the summing prologue works on
    4-token groups, which re-read the weights per group, and with the wo launch on 8-token groups the fold loses
    from batch 20 up (139.4 -> 133.3 us per step at batch 16 folded, 147.3 -> 150.4 at 24, 150.1 -> 153.8 at 32).
    Summing the heads in the attention launch itself (the last of a sequence's head workgroups adding the parts
    after agent-scope release / acquire fences, no workgroup waiting) measured 176 -> 414 us per batch-64 step:
    the fences' cache writebacks and invalidations cost ~40 us per launch.  Running value_proj in the selection + bag launch the same way
    (one workgroup per token and 64-column slice of the bag output, each with the token's whole selection, the next
    block's first launch summing the slices) measured no gain at batch 1: that launch went from 10.7-11.1 to 13.6
    us (value_proj rows loaded at its start) or 14.3 us (loaded after the half top-ks), against the 4.1-4.4 us
    value_proj launch it saves and 0.9 us more in the summing prologue (123.2-123.7 -> 123.8-124.3 us per step).

    Derived weights (the concatenated query_proj | swilu_proj and its bias) are built at construction and rebuilt
    on an eager run after a parameter changed; a captured graph keeps what it was captured with."""

    proj_max_batch = 16

    @staticmethod
    def supported(model, dtype):
        """Whether the model's shapes and options are covered by the fused kernels (else the step runs
        Transformer.forward)."""
        cfg = model.cfg
        w = model.tok_emb.weight
        if dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or not w.is_cuda or model.ngram is not None:
            return False
        C, hd = cfg.d_model, cfg.d_model // cfg.n_heads
        if C % 32 or C > 480 or C % cfg.n_heads or hd not in (16, 32, 64, 128) or cfg.ffn_hidden % 16 \
                or cfg.vocab_size % 16:
            return False
        for blk in model.layers:
            if blk.ffn_r2 is not None:
                return False
            if blk.is_memory:
                m = blk.ffn
                tables = inference_tables(m.values)
                if tables is None:          # staged table tier: every call synchronises, no fused step
                    return False
                table = tables[0]
                if (not m.swilu or m.log_score_scale is not None or m.record or m.heads > 4
                        or (m.heads * m.k_dim) % 16 or (m.k_dim // 2) % 8 or m.v_dim % 32
                        or m.query_proj.weight.dtype != torch.bfloat16
                        or (m.query_norm is not None and m.query_norm.training)
                        or not kernels.select_bag_supported(m.heads, table)):
                    return False
        return True

    def __init__(self, model):
        self.model = model
        self._tag = None
        self._prepare()

    def _params_tag(self):
        return state_tag(self.model.state_tensors())

    def _prepare(self):
        self.mem = {}
        for i, blk in enumerate(self.model.layers):
            if blk.is_memory:
                m = blk.ffn
                w = torch.cat([m.query_proj.weight.detach(), m.swilu_proj.weight.detach()]).contiguous()
                b = torch.cat([m.query_proj.bias.detach(), m.swilu_proj.bias.detach()]).contiguous()
                self.mem[i] = (w, b)
        self._tag = self._params_tag()

    def run(self, tok, pos, caches, hist, logits=False, record=None, chain=None):
        """The step for tok (B, 1) at device position pos: writes the next token to tok and hist[:, pos + 1] and
        advances pos.  With logits=True it returns the (B, vocab) bf16 logits instead and changes none of tok,
        hist and pos (the KV caches get the same slot written).  With a dict `record`, record[layer] holds each
        memory layer's lookup: "x" the residual stream entering its ffn_norm (B, d_model), "q" the query after the
        BatchNorm and "pre" the swilu projection (bf16, as the kernels computed them), "s1", "s2" the sub-key scores,
        "scores", "indices", "weights" the selection.

        With `chain` ((B, >= argmax blocks) int64 argmax keys, even row stride; not with logits) the step's token
        is the greedy choice from the keys the previous chained step left in chain (or that _StepDecoder seeded):
        the first launch writes it to tok and hist[:, pos]; the step then leaves its own keys in chain and advances
        pos.  The next token reaches tok and hist in the next chained step (or in _StepDecoder.finish)."""
        if chain is not None and logits:
            raise ValueError("run: a chained step ends with argmax keys, not logits")
        model = self.model
        if not torch.cuda.is_current_stream_capturing() and self._params_tag() != self._tag:
            self._prepare()
        B = tok.shape[0]
        proj = B <= self.proj_max_batch and model.cfg.n_heads <= 8
        x = delta = None
        for i, blk in enumerate(model.layers):
            at = blk.attn
            if x is None and chain is not None:
                x, qkv = kernels.decode_linear(at.wqkv.weight, tok_partial=chain, tok_out=tok.view(-1), hist=hist,
                                               pos=pos, emb=model.tok_emb.weight, norm=blk.attn_norm, write_x=True)
            elif x is None:
                x, qkv = kernels.decode_linear(at.wqkv.weight, tok=tok.view(-1), emb=model.tok_emb.weight,
                                               norm=blk.attn_norm, write_x=True)
            else:
                x, qkv = kernels.decode_linear(at.wqkv.weight, x, delta=delta, norm=blk.attn_norm, write_x=True)
            if proj:
                delta = kernels.decode_attention_proj(qkv, at.rope.cos, at.rope.sin, pos, caches[i].k, caches[i].v,
                                                      at.wo.weight)
            else:
                y = kernels.decode_attention(qkv, at.rope.cos, at.rope.sin, pos, caches[i].k, caches[i].v)
                delta = kernels.decode_linear(at.wo.weight, y)
            if blk.is_memory:
                m = blk.ffn
                w, b = self.mem[i]
                nq = m.heads * m.k_dim
                affine = m._bn_affine() if m.query_norm is not None else None
                x, (q, pre) = kernels.decode_linear(w, x, delta=delta, norm=blk.ffn_norm, write_x=True, bias=b,
                                                    affine=affine, n_split=nq)
                s1, s2 = kernels.pk_scores(q.view(B, m.heads, m.k_dim), m._keys_as(torch.bfloat16))
                table, scales = inference_tables(m.values)
                res = kernels.pk_select_bag(s1, s2, m.knn, table, scales, pre=pre, out_bf16=True,
                                            record=record is not None)
                out, sel = (res[0], res[1:]) if record is not None else (res, None)
                delta = kernels.decode_linear(m.value_proj.weight, out, bias=m.value_proj.bias)
                if record is not None:
                    record[i] = {"x": x, "q": q, "pre": pre, "s1": s1, "s2": s2, "scores": sel[0], "indices": sel[1],
                                 "weights": sel[2]}
            else:
                f = blk.ffn
                x, act = kernels.decode_linear(f.w13.weight, x, delta=delta, norm=blk.ffn_norm, write_x=True,
                                               swiglu=True)
                delta = kernels.decode_linear(f.w2.weight, act)
        if logits:
            return kernels.decode_linear(model.lm_head.weight, x, delta=delta, norm=model.norm)
        if chain is not None:
            kernels.decode_linear(model.lm_head.weight, x, delta=delta, norm=model.norm, argmax=True,
                                  partial_out=chain, advance_pos=pos)
            return None
        partial = kernels.decode_linear(model.lm_head.weight, x, delta=delta, norm=model.norm, argmax=True)
        kernels.argmax_finish(partial, pos, tok.view(-1), hist)
        return None


class _StepDecoder:
    """Static buffers and the captured graphs of one decode step and of runs of `run_lengths` steps in a row for
    batch B, sequences up to max_len.  A step reads its position and token from device memory and advances them
    itself, so a run of steps is one graph replay: the replay boundary (about 15 us on MI355X) is paid once per
    run (32-step runs: 124.3 -> 123.5 us per step at batch 1 against 8-step runs, batch 64 unchanged).

    On the fused kernels the steps are chained through `chain`, the lm_head's argmax keys: a step's first launch
    picks its token from the previous step's keys.  start() seeds the keys with the first token, finish() turns
    the last step's keys into tok and its history slot; replay() and steps() end with it.

    The graphs read the model's tensors and derived copies as they were at capture, so replay() captures them again
    when a parameter or buffer has changed since (state_tag), and captures them at its first call if nothing did
    before; a capture leaves the decoder's state (position, token, history, argmax keys, KV caches) as it found it."""

    run_lengths = (32, 8)   # graphs of this many steps in a row, longest first; then single steps

    def __init__(self, model, B, max_len, device):
        cfg = model.cfg
        if max_len > cfg.max_seq_len:
            raise ValueError(f"prompt + new tokens = {max_len} exceed max_seq_len = {cfg.max_seq_len}")
        self.model, self.B, self.max_len = model, B, max_len
        dtype = model.tok_emb.weight.dtype
        if torch.is_autocast_enabled("cuda"):
            dtype = torch.get_autocast_dtype("cuda")
        hd = cfg.d_model // cfg.n_heads
        self.caches = [StaticKVCache(B, cfg.n_heads, max_len, hd, dtype, device) for _ in range(cfg.n_layers)]
        self.tok = torch.zeros(B, 1, dtype=torch.long, device=device)
        self.pos = torch.zeros((), dtype=torch.long, device=device)
        self.hist = torch.zeros(B, max_len, dtype=torch.long, device=device)
        self.graph = None
        self.graph_runs = {}
        self._graph_tag = None
        self.fused = _FusedDecodeStep(model) if _FusedDecodeStep.supported(model, dtype) else None
        self.chain = None
        if self.fused is not None:
            nblk = kernels.linear_argmax_blocks(cfg.vocab_size)
            self.chain = torch.zeros(B, nblk + nblk % 2, dtype=torch.long, device=device)   # even row stride

    def _seed(self):
        """Argmax keys whose greedy choice is tok: ~tok (above every logit key) in column 0, no key elsewhere."""
        self.chain.zero_()
        self.chain[:, 0] = ~self.tok.view(-1)

    def start(self, first, P):
        """The state a run of steps starts from: the first sampled token `first` (B,) at position P."""
        self.hist[:, P] = first.view(-1)
        self.tok.copy_(first.view(self.B, 1))
        self.pos.fill_(P)
        if self.chain is not None:
            self._seed()

    def finish(self):
        """After chained steps: the last step's greedy token to tok and hist[:, pos] (pos is already advanced)."""
        if self.chain is not None:
            kernels.argmax_finish(self.chain, self.pos - 1, self.tok.view(-1), self.hist, advance=False)

    def steps(self, n):
        """n decode steps run eagerly (no graph), then finish()."""
        for _ in range(n):
            self._step()
        self.finish()

    def _step(self):
        if self.fused is not None:
            self.fused.run(self.tok, self.pos, self.caches, self.hist, chain=self.chain)
            return
        logits = self.model(self.tok, kv_caches=self.caches, pos0=self.pos)
        last = logits[:, -1]
        if last.is_cuda and last.dtype == torch.bfloat16:
            # argmax, next token and its history slot in one kernel
            kernels.greedy_argmax(last, self.pos, self.tok.view(-1), self.hist)
        else:
            nxt = last.argmax(-1, keepdim=True)
            self.hist.index_copy_(1, (self.pos + 1).view(1), nxt)
            self.tok.copy_(nxt)
        self.pos.add_(1)

    def _capture(self):
        """Capture the single-step graph and the run graphs.  Two eager warm-up steps run first (library loads,
        derived weights, allocator) from position 0; what they write -- position, token, history, argmax keys and
        the KV cache slots 0 and 1 -- is saved before and restored after, so the state a caller set up (a prefilled
        prompt, start()) survives a capture."""
        ac = torch.is_autocast_enabled("cuda")
        ctx = (torch.autocast("cuda", dtype=torch.get_autocast_dtype("cuda"), cache_enabled=False) if ac
               else torch.autocast("cuda", enabled=False))
        warm = min(2, self.max_len)
        saved = (self.pos.clone(), self.tok.clone(), self.hist.clone(),
                 None if self.chain is None else self.chain.clone(),
                 [(c.k[:, :, :warm].clone(), c.v[:, :, :warm].clone(), dict(c.extra)) for c in self.caches])
        self.pos.fill_(0)
        self.tok.zero_()
        if self.chain is not None:
            self._seed()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), ctx:
            for _ in range(warm):                   # warm-up: library loads, cached casts, allocator
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        pos, tok, hist, chain, kv = saved
        self.pos.copy_(pos)
        self.tok.copy_(tok)
        self.hist.copy_(hist)
        if chain is not None:
            self.chain.copy_(chain)
        for c, (k, v, extra) in zip(self.caches, kv):
            c.k[:, :, :warm].copy_(k)
            c.v[:, :, :warm].copy_(v)
            c.extra.clear()
            c.extra.update(extra)
        del saved, kv
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph), ctx:
            self._step()
        self.graph = graph
        self.graph_runs = {}
        for k in self.run_lengths:
            if k > 1:
                run = torch.cuda.CUDAGraph()
                with torch.cuda.graph(run), ctx:
                    for _ in range(k):
                        self._step()
                self.graph_runs[k] = run
        self._graph_tag = state_tag(self.model.state_tensors())

    def _graphs_current(self):
        return self.graph is not None and self._graph_tag == state_tag(self.model.state_tensors())

    def replay(self, n):
        """n decode steps as graph replays: as many runs of the longest run length as fit, then of the next, then
        single steps; then finish().  Captures the graphs first if there are none or the model changed."""
        if not self._graphs_current():
            self._capture()
        for k in sorted(self.graph_runs, reverse=True):
            for _ in range(n // k):
                self.graph_runs[k].replay()
            n -= n // k * k
        for _ in range(n):
            self.graph.replay()
        self.finish()

    def run(self, prompt, new_tokens, use_graph, sync_every_step):
        B, P = prompt.shape
        if any(inference_tables(m.values) is None for m in self.model.memory_layers()):
            use_graph = False               # a staged table tier synchronises in every call: no capture
        if self.model.ngram is not None:
            use_graph = False               # Engram's conv and hash histories are new tensors every step
        for cache in self.caches:
            cache.extra.clear()             # no state of an earlier sequence
        if use_graph and not self._graphs_current():
            self._capture()
        logits = self.model(prompt, kv_caches=self.caches, pos0=0)
        self.hist[:, :P] = prompt
        self.start(logits[:, -1].argmax(-1), P)
        if use_graph and not sync_every_step:
            self.replay(new_tokens)
            return self.hist[:, P:P + new_tokens + 1].clone()
        for _ in range(new_tokens):
            if use_graph:
                self.graph.replay()
            else:
                self._step()
            if sync_every_step:
                torch.cuda.current_stream().synchronize()
        self.finish()
        return self.hist[:, P:P + new_tokens + 1].clone()
