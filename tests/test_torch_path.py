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
