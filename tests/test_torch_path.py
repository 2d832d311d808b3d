"""Pins oracle/torch_path.py (the reference's torch path restated on the CPU) with the reference's own
invariants (tests/test_pkm.py:16-37, 81-119): exact product-key search equals brute force over all n_keys^2
keys, cached decode equals a full forward, chunked prefill equals a full forward, causality."""
import torch

import oracle.pkm_oracle as O
import oracle.torch_path as TP
from smlm_hip.model import ModelConfig, Transformer


def tiny_sd(mem=True, seed=0):
    cfg = ModelConfig(vocab_size=128, d_model=32, n_layers=3, n_heads=4, ffn_hidden=64, max_seq_len=64,
                      mem_layers=[1] if mem else [], mem_n_keys=16, mem_heads=2, mem_knn=4, mem_k_dim=16)
    torch.manual_seed(seed)
    m = Transformer(cfg).double()
    with torch.no_grad():
        for n, b in m.named_buffers():
            if n.endswith("running_var"):
                b.uniform_(0.5, 2.0)
            elif n.endswith("running_mean"):
                b.normal_(0, 0.1)
    return {k: v.detach() for k, v in m.state_dict().items()}, cfg.to_dict()


def test_pkm_select_torch_equals_bruteforce():
    torch.manual_seed(1)
    N, H, NK, half, knn = 100, 3, 16, 8, 8
    q = torch.randn(N, H, 2 * half, dtype=torch.float64)
    keys = torch.rand(H, 2, NK, half, dtype=torch.float64) - 0.5
    s1 = torch.einsum("nhd,hkd->nhk", q[..., :half], keys[:, 0])
    s2 = torch.einsum("nhd,hkd->nhk", q[..., half:], keys[:, 1])
    sc, idx = TP.pkm_select_torch(s1, s2, knn)
    for h in range(H):
        full = torch.cat([keys[h, 0].repeat_interleave(NK, 0), keys[h, 1].repeat(NK, 1)], 1)
        bf, bi = (q[:, h] @ full.T).topk(knn, -1)
        torch.testing.assert_close(sc[:, h], bf, rtol=0, atol=1e-12)
        assert torch.equal(idx[:, h].sort(-1).values, bi.sort(-1).values)
    # and the numpy oracle agrees on the same (tie-free) scores
    _, oi, _ = O.pk_select(s1.float().numpy(), s2.float().numpy(), knn)
    assert torch.equal(torch.from_numpy(oi).sort(-1).values, idx.sort(-1).values)


def test_kv_cache_decode_matches_full_forward():
    sd, cfg = tiny_sd()
    x = torch.randint(0, 128, (1, 30), generator=torch.Generator().manual_seed(2))
    full = TP.lm_forward(sd, cfg, x)
    caches = [dict() for _ in range(cfg["n_layers"])]
    steps = [TP.lm_forward(sd, cfg, x[:, :10], caches, 0)]
    for t in range(10, 30):
        steps.append(TP.lm_forward(sd, cfg, x[:, t:t + 1], caches, t))
    torch.testing.assert_close(torch.cat(steps, 1), full)


def test_chunked_prefill_and_causality():
    sd, cfg = tiny_sd(seed=3)
    x = torch.randint(0, 128, (2, 30), generator=torch.Generator().manual_seed(3))
    full = TP.lm_forward(sd, cfg, x)
    caches = [dict() for _ in range(cfg["n_layers"])]
    chunks = [TP.lm_forward(sd, cfg, x[:, a:a + n], caches, a) for a, n in ((0, 10), (10, 5), (15, 1), (16, 14))]
    torch.testing.assert_close(torch.cat(chunks, 1), full)
    y = x.clone()
    y[:, 25:] = (y[:, 25:] + 1) % 128
    torch.testing.assert_close(TP.lm_forward(sd, cfg, y)[:, :25], full[:, :25])
    torch.testing.assert_close(TP.lm_forward(sd, cfg, x, last_only=True), full[:, -1:])


def test_greedy_decode_shapes():
    sd, cfg = tiny_sd(seed=4)
    out = TP.greedy_decode(sd, cfg, torch.randint(0, 128, (3, 5)), 7)
    assert out.shape == (3, 8) and out.dtype == torch.int64


def _complex_rope(x, pos0, theta):
    """RoPE written as complex rotation: dimension j < hd/2 and its partner j + hd/2 form z_j = x_j + i x_{j+hd/2},
    turned by the angle (pos0 + t) * theta^(-2j/hd) -- a formulation independent of the cos/sin cat form."""
    hd, T = x.shape[-1], x.shape[-2]
    j = torch.arange(hd // 2, dtype=torch.float64)
    ang = (pos0 + torch.arange(T, dtype=torch.float64))[:, None] * theta ** (-2.0 * j / hd)
    z = torch.complex(x[..., :hd // 2], x[..., hd // 2:]) * torch.polar(torch.ones_like(ang), ang)
    return torch.cat([z.real, z.imag], -1)


def test_rope_pairs_halves_and_turns_counterclockwise():
    """Known answers of smlm/model.py:63-78: the unit vector e_j (j < hd/2) at position p becomes
    cos(p w_j) e_j + sin(p w_j) e_{j+hd/2}, and e_{j+hd/2} becomes -sin(p w_j) e_j + cos(p w_j) e_{j+hd/2},
    w_j = theta^(-2j/hd).  An interleaved pairing (2j, 2j+1) or the opposite turn fails these."""
    import importlib.util
    import math
    import os
    from smlm_hip.model import RotaryEmbedding
    hd, theta, p = 8, 10000.0, 5
    eye = torch.eye(hd, dtype=torch.float64).view(1, 1, hd, hd).transpose(2, 3)     # row t of T=hd is e_t
    spec = importlib.util.spec_from_file_location(
        "gpu_attention_refs", os.path.join(os.path.dirname(__file__), "test_gpu_attention.py"))
    attn_tests = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(attn_tests)
    rope_mod = RotaryEmbedding(hd, 64, theta)
    for fn in (lambda x: TP.rope(x, p, theta),
               lambda x: attn_tests.rope_ref(x, rope_mod.cos, rope_mod.sin, p),
               lambda x: rope_mod(x.float(), p).double()):
        # every row of the batch at the same position p: feed the unit vectors as a batch of one-token sequences
        out = fn(eye.reshape(hd, 1, 1, hd)).reshape(hd, hd)
        for j in range(hd // 2):
            w = theta ** (-2.0 * j / hd)
            c, s = math.cos(p * w), math.sin(p * w)
            exp_lo = torch.zeros(hd, dtype=torch.float64)
            exp_lo[j], exp_lo[j + hd // 2] = c, s
            exp_hi = torch.zeros(hd, dtype=torch.float64)
            exp_hi[j], exp_hi[j + hd // 2] = -s, c
            assert torch.allclose(out[j], exp_lo, atol=1e-6), (j, out[j])
            assert torch.allclose(out[j + hd // 2], exp_hi, atol=1e-6), (j, out[j + hd // 2])
    x = torch.randn(2, 3, 7, 16, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    assert torch.allclose(TP.rope(x, 11, theta), _complex_rope(x, 11, theta), atol=1e-6)
