"""ProductKeyMemory and the LM entry points on the GPU, against the CPU oracles.

The lookup contract: scores within tolerance of fp64, selection bit-exact on the kernel's own scores,
outputs within 1e-5 (fp32) / 1e-2 relative (bf16) of the oracle's value bag on that selection; logits against
the reference's torch path restated on the CPU (oracle/torch_path.py).  Decode graphs replay bit-identically
to the eager path (tests/test_kernels.py:257-277); cached decode equals a full forward (tests/test_pkm.py:91-101).
"""
import numpy as np
import pytest
import torch

import oracle.pkm_oracle as O
import oracle.torch_path as TP
from smlm_hip import kernels as K
from smlm_hip.model import ModelConfig, Transformer
from smlm_hip.pkm import ProductKeyMemory

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(msg, flush=True)


def bits_of(t):
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def close(a, b, tol=1e-5):
    scale = max(1.0, float(np.abs(b).max()))
    np.testing.assert_allclose(a / scale, b / scale, rtol=tol, atol=tol)


@torch.no_grad()
def test_config0_layer_forward_fp32():
    """B-1M layer, fp32, 8x256 tokens, d=384, 4 heads x 512, 1024 sub-keys per half,
    top-32, 1,048,576 x 384 value table, no query norm, no swilu, seed 0."""
    note("config 0 layer forward")
    g = torch.Generator().manual_seed(0)
    N, d, H, kd, NK, knn = 2048, 384, 4, 512, 1024, 32
    x = torch.randn(N, d, generator=g)
    mem = ProductKeyMemory(d, d, n_keys=NK, heads=H, knn=knn, k_dim=kd, query_norm="none", swilu=False)
    mem.query_proj.weight.copy_(torch.randn(H * kd, d, generator=g) * 0.02)
    mem.query_proj.bias.zero_()
    mem.keys.copy_(torch.randn(H, 2, NK, kd // 2, generator=g) / 16)
    mem.values.weight.copy_(torch.randn(NK * NK, d, generator=g) * 0.02)
    mem = mem.to(DEV)
    mem.record = True
    xd = x.to(DEV)
    out = mem(xd)
    q = mem.query_proj(xd).view(N, H, kd)
    s1, s2 = K.pk_scores(q, mem.keys.detach())
    r1, r2 = O.subkey_scores(q.cpu().numpy(), mem.keys.cpu().numpy())
    mag = np.einsum("nhd,hkd->nhk", np.abs(q.cpu().numpy()[..., :kd // 2]).astype(np.float64),
                    np.abs(mem.keys.cpu().numpy()[:, 0]).astype(np.float64))
    assert np.all(np.abs(s1.cpu().numpy() - r1) <= 1e-5 * mag)
    close(s2.cpu().numpy(), r2)
    sc, idx, w = O.pk_select(s1.cpu().numpy(), s2.cpu().numpy(), knn)
    assert np.array_equal(mem.last_indices.cpu().numpy(), idx)
    assert np.array_equal(mem.last_scores.cpu().numpy(), sc)
    np.testing.assert_allclose(mem.last_weights.cpu().numpy(), w, rtol=0, atol=1e-6)
    table = mem.values.weight.cpu().numpy()
    ref = O.bag(idx.reshape(N, -1), w.reshape(N, -1), table, "f32")
    close(out.cpu().numpy(), ref)
    # the reference's torch path end to end (fp64 on the CPU): identical wherever its selection agrees
    sd = {k: v.double().cpu() for k, v in mem.state_dict().items()}
    tp = TP.pkm_forward(sd, "", x.double(), dict(heads=H, knn=knn, k_dim=kd, n_keys=NK, query_norm="none",
                                                 swilu=False)).numpy()
    same = np.array([set(TP.pkm_select_torch(*[torch.from_numpy(a[n:n + 1]).double() for a in (r1, r2)],
                                             knn)[1].reshape(-1).tolist()) == set(idx[n].reshape(-1).tolist())
                     for n in range(0, N, 64)])
    assert same.mean() >= 0.9
    rows = np.where(np.abs(out.cpu().numpy() - tp).max(1) <= 1e-5 * max(1.0, np.abs(tp).max()))[0]
    assert len(rows) >= 0.9 * N


@torch.no_grad()
def test_learned_score_scale_forward_fp32():
    """score_scale="learned" (smlm/pkm.py:60-62, 195-208): a positive per-head scale multiplies the selected scores
    before the softmax.  The selection is the kernels' (bit-exact against the oracle on their own scores), the
    weights are softmax(scale_h * scores) and the output is the value bag on them."""
    note("learned score scale forward")
    g = torch.Generator().manual_seed(3)
    N, d, H, kd, NK, knn = 256, 64, 3, 64, 128, 16
    mem = ProductKeyMemory(d, d, n_keys=NK, heads=H, knn=knn, k_dim=kd, query_norm="none", swilu=False,
                           score_scale="learned", score_scale_init=2.0)
    assert torch.allclose(mem.log_score_scale, torch.full((H,), float(np.log(2.0))))
    mem.query_proj.weight.copy_(torch.randn(H * kd, d, generator=g) * 0.1)
    mem.keys.copy_(torch.randn(H, 2, NK, kd // 2, generator=g) / 4)
    mem.values.weight.copy_(torch.randn(NK * NK, d, generator=g) * 0.02)
    scale = np.array([0.25, 1.0, 6.0])
    mem.log_score_scale.copy_(torch.from_numpy(np.log(scale)))
    mem = mem.to(DEV)
    mem.record = True
    x = torch.randn(N, d, generator=g).to(DEV)
    out = mem(x)
    q = mem.query_proj(x).view(N, H, kd)
    s1, s2 = K.pk_scores(q, mem.keys.detach())
    sc, idx, _ = O.pk_select(s1.cpu().numpy(), s2.cpu().numpy(), knn)
    assert np.array_equal(mem.last_indices.cpu().numpy(), idx)
    z = sc.astype(np.float64) * scale.reshape(1, H, 1)
    w = np.exp(z - z.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    np.testing.assert_allclose(mem.last_weights.cpu().numpy(), w, rtol=0, atol=1e-6)
    # the sharpest head's weights differ from the unscaled softmax: the scale is applied, not dropped
    w1 = np.exp(sc - sc.max(-1, keepdims=True))
    w1 /= w1.sum(-1, keepdims=True)
    assert np.abs(w[:, 2] - w1[:, 2]).max() > 1e-2
    ref = O.bag(idx.reshape(N, -1), w.reshape(N, -1).astype(np.float32), mem.values.weight.cpu().numpy(), "f32")
    close(out.cpu().numpy(), ref)


def _bf16_layer(N, seed, n_keys=1024, knn=32, d=384):
    g = torch.Generator().manual_seed(seed)
    mem = ProductKeyMemory(d, d, n_keys=n_keys, heads=4, knn=knn, k_dim=512)
    with torch.no_grad():
        for p in mem.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
        mem.keys.copy_(torch.randn(mem.keys.shape, generator=g) / 16)
        mem.query_norm.running_mean.copy_(torch.randn(4 * 512, generator=g) * 0.01)
        mem.query_norm.running_var.copy_(torch.rand(4 * 512, generator=g) * 0.001 + 0.0005)
        mem.query_norm.weight.fill_(1.0)
    mem = mem.to(DEV).eval()
    x = torch.randn(N, d, generator=g).to(DEV, torch.bfloat16)
    return mem, x


@pytest.mark.parametrize("kind", ["fp32", "bf16", "int8", "q4"])
@torch.no_grad()
def test_bf16_layer_with_bn_and_swilu(kind):
    """The decode-time memory layer (BatchNorm, swilu, bf16 autocast) on each inference table format."""
    note(f"bf16 layer {kind}")
    N = 64
    mem, x = _bf16_layer(N, 1)
    v = mem.values
    w32 = v.weight.detach()
    if kind == "fp32":
        v.infer_table, tn, scn, tk = None, w32.cpu().numpy(), None, "f32"
    elif kind == "bf16":
        v.infer_table = (w32.to(torch.bfloat16), None)
        tn, scn, tk = bits_of(v.infer_table[0]), None, "bf16"
    else:
        v.infer_table = (K.quantize_int8 if kind == "int8" else K.quantize_q4)(w32)
        tn, scn = v.infer_table[0].cpu().numpy(), v.infer_table[1].cpu().numpy()
        tk = "i8" if kind == "int8" else "q4"
    mem.record = True
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = mem(x)
        q = mem._query(x).to(torch.bfloat16).view(N, 4, 512)
        s1, s2 = K.pk_scores(q, mem.keys.detach().to(torch.bfloat16))
        pre = mem.swilu_proj(x).to(torch.bfloat16)
    sc, idx, w = O.pk_select(bits_of(s1), bits_of(s2), 32)
    assert np.array_equal(mem.last_indices.cpu().numpy(), idx)
    assert np.array_equal(bits_of(mem.last_scores), sc)
    bag = O.bag(idx.reshape(N, -1), w.reshape(N, -1), tn, tk, scn, pre=bits_of(pre), out_bf16=True)
    bag_t = torch.from_numpy(bag.view(np.int16)).view(torch.bfloat16).to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ref = mem.value_proj(bag_t).float().cpu().numpy()
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2 * np.abs(ref).max())


def tiny(seed=0, heads=2, v_dim=-1, dtype=torch.float32, d_model=32):
    cfg = ModelConfig(vocab_size=128, d_model=d_model, n_layers=4, n_heads=4, ffn_hidden=64, max_seq_len=64,
                      mem_layers=[0, 2, 3], mem_n_keys=16, mem_heads=heads, mem_knn=4, mem_k_dim=16,
                      mem_v_dim=v_dim, mem_share_values=True)
    torch.manual_seed(seed)
    return Transformer(cfg).to(DEV, dtype).eval()


@pytest.mark.parametrize("kind", ["fp32", "bf16", "q4", "int8"])
@torch.no_grad()
def test_decode_graph_bit_identical(kind):
    """Per-layer decode graphs give bit-identical logits to the eager kernels (tests/test_kernels.py:257-277)."""
    note(f"decode graph {kind}")
    m = tiny()
    m.set_memory_inference_table(kind)
    x = torch.randint(0, 128, (1, 8), generator=torch.Generator().manual_seed(2)).to(DEV)

    def decode():
        caches = [dict() for _ in range(m.cfg.n_layers)]
        outs = [m(x[:, :4], kv_caches=caches, pos0=0).float()]
        for i in range(4, 8):
            outs.append(m(x[:, i:i + 1], kv_caches=caches, pos0=i).float())
        return torch.cat(outs, 1)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        eager = decode()
        m.set_memory_decode_graphs(True)
        graph = decode()
        graph2 = decode()
        m.set_memory_decode_graphs(False)
    assert torch.equal(graph, eager) and torch.equal(graph2, eager)


@pytest.mark.parametrize("B", [1, 3])
@torch.no_grad()
def test_generate_whole_step_graph_matches_eager(B):
    """The captured whole decode step (static KV cache, fused attention kernel: head_dim 16) reproduces the eager
    static-cache loop token for token, on every replay."""
    note(f"generate B={B}")
    m = tiny(dtype=torch.bfloat16, d_model=64)
    prompt = torch.randint(0, 128, (B, 6), generator=torch.Generator().manual_seed(3)).to(DEV)
    eager = m.generate(prompt, 20, use_graph=False)
    graph = m.generate(prompt, 20, use_graph=True)
    graph2 = m.generate(prompt, 20, use_graph=True)
    assert torch.equal(graph, eager) and torch.equal(graph2, eager)


@torch.no_grad()
def test_static_cache_steps_match_dict_cache():
    """Single-token steps over the static cache (fused attention kernel, device-side position) give the logits of
    the reference's dict-cache path (torch.cat cache, smlm/model.py:94-98) on the same tokens.  The model has no
    memory layer here: the two attention paths round RoPE differently by a bf16 ulp, and a memory layer with
    knn = 4 turns such an ulp into a different selected row whenever two candidates are that close (the
    selection itself is checked against the oracle on its own scores elsewhere)."""
    from smlm_hip.model import StaticKVCache
    cfg = ModelConfig(vocab_size=128, d_model=64, n_layers=4, n_heads=4, ffn_hidden=64, max_seq_len=64)
    torch.manual_seed(0)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    x = torch.randint(0, 128, (3, 16), generator=torch.Generator().manual_seed(7)).to(DEV)
    dict_caches = [dict() for _ in range(m.cfg.n_layers)]
    hd = m.cfg.d_model // m.cfg.n_heads
    static = [StaticKVCache(3, m.cfg.n_heads, 32, hd, torch.bfloat16, DEV) for _ in range(m.cfg.n_layers)]
    a = [m(x[:, :6], kv_caches=dict_caches, pos0=0).float()]
    b = [m(x[:, :6], kv_caches=static, pos0=0).float()]
    for t in range(6, 16):
        a.append(m(x[:, t:t + 1], kv_caches=dict_caches, pos0=t).float())
        b.append(m(x[:, t:t + 1], kv_caches=static, pos0=torch.tensor(t, device=DEV)).float())
    a, b = torch.cat(a, 1), torch.cat(b, 1)
    assert float((a - b).abs().max() / a.abs().max()) < 2e-2


@torch.no_grad()
def test_kv_cache_decode_matches_full_forward():
    m = tiny()
    x = torch.randint(0, 128, (1, 30), generator=torch.Generator().manual_seed(4)).to(DEV)
    full = m(x)
    caches = [dict() for _ in range(m.cfg.n_layers)]
    steps = [m(x[:, :10], kv_caches=caches, pos0=0)]
    for t in range(10, 30):
        steps.append(m(x[:, t:t + 1], kv_caches=caches, pos0=t))
    torch.testing.assert_close(torch.cat(steps, 1), full, rtol=1e-4, atol=1e-4)


def _oracle_cfg(cfg):
    return cfg.to_dict()


@torch.no_grad()
def test_lm_logits_fp32_match_torch_path():
    """fp32 LM (memory layers on the kernels) against the reference's torch path in fp64 on the CPU."""
    m = tiny(seed=5)
    x = torch.randint(0, 128, (2, 24), generator=torch.Generator().manual_seed(5))
    got = m(x.to(DEV)).cpu()
    sd = {k: v.double().cpu() for k, v in m.state_dict().items()}
    ref = TP.lm_forward(sd, _oracle_cfg(m.cfg), x)
    torch.testing.assert_close(got.double(), ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()))


@torch.no_grad()
def test_lm_logits_bf16_within_1e2():
    """bf16 LM: the memory layer's selection is bit-exact against the oracle on the layer's own bf16 sub-key
    scores, and the logits are within 1e-2 of their scale of the fp32 torch path given that selection.
    (bf16 scores legitimately select other rows than fp32 scores wherever candidates lie within a bf16
    rounding step, so the logits are compared on one selection.)"""
    cfg = ModelConfig(vocab_size=512, d_model=128, n_layers=3, n_heads=2, ffn_hidden=256, max_seq_len=64,
                      mem_layers=[1], mem_n_keys=64, mem_heads=4, mem_knn=16, mem_k_dim=64)
    torch.manual_seed(6)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    x = torch.randint(0, 512, (2, 32), generator=torch.Generator().manual_seed(6))
    mem = m.layers[1].ffn
    mem.record = True
    seen = {}
    hook = mem.register_forward_hook(lambda mod, inp, out: seen.__setitem__("x", inp[0].detach().clone()))
    got = m(x.to(DEV)).float().cpu()
    hook.remove()
    q = mem._query(seen["x"].reshape(-1, cfg.d_model)).to(torch.bfloat16).view(-1, 4, 64)
    s1, s2 = K.pk_scores(q, mem.keys.detach())
    _, oi, ow = O.pk_select(bits_of(s1), bits_of(s2), 16)
    assert np.array_equal(mem.last_indices.cpu().numpy(), oi)
    np.testing.assert_allclose(mem.last_weights.cpu().numpy(), ow, rtol=0, atol=1e-6)
    sd = {k: v.float().cpu() for k, v in m.state_dict().items()}
    ref = TP.lm_forward(sd, cfg.to_dict(), x, selections={1: (mem.last_indices.cpu(), mem.last_weights.cpu())})
    err = (got - ref).abs().max() / ref.abs().max()
    assert float(err) < 1e-2, float(err)


@pytest.mark.parametrize("n_keys,knn", [(16, 8), (16, 16), (32, 5), (8, 1), (24, 4), (16, 5), (128, 100)])
@torch.no_grad()
def test_product_key_topk_equals_bruteforce(n_keys, knn):
    """tests/test_pkm.py:16-37 on the kernels, with the shapes the reference's torch path takes (non-power-of-two
    n_keys and knn, knn above 64): the product-key search returns the top-k of a brute-force search over all
    n_keys^2 full keys (fp64 on the host; the kernels score in fp32, so a row may differ at a near tie: 99% of the
    rows must be identical sets), and every returned score belongs to its index."""
    note(f"product-key search vs brute force n_keys={n_keys} knn={knn}")
    torch.manual_seed(0)
    mem = ProductKeyMemory(24, 24, n_keys=n_keys, heads=3, knn=knn, k_dim=16, impl="torch").to(DEV).eval()
    q = torch.randn(200, 3, 16, generator=torch.Generator().manual_seed(1)).to(DEV)
    scores, indices = mem.get_indices(q)
    assert scores.shape == (200, 3, knn) and indices.shape == (200, 3, knn)
    qd = q.double().cpu()
    for h in range(3):
        k1, k2 = mem.keys[h, 0].double().cpu(), mem.keys[h, 1].double().cpu()
        full = torch.cat([k1.repeat_interleave(n_keys, 0), k2.repeat(n_keys, 1)], 1)
        bf_scores, bf_idx = (qd[:, h] @ full.T).topk(knn, dim=-1)
        got = scores[:, h].double().cpu()
        torch.testing.assert_close(got, bf_scores, rtol=1e-5, atol=1e-5)
        same = (indices[:, h].cpu().sort(-1).values == bf_idx.sort(-1).values).all(-1)
        assert float(same.double().mean()) >= 0.99
        recomputed = (qd[:, h].unsqueeze(1) * full[indices[:, h].cpu()]).sum(-1)
        torch.testing.assert_close(got, recomputed, rtol=1e-5, atol=1e-5)


@torch.no_grad()
def test_generate_with_reference_torch_shapes():
    """A bf16 LM whose memory layer has n_keys = 24 and knn = 5 (shapes only the reference's torch path takes):
    the fused decode step selects bit-exactly against the oracle on its own sub-key scores, and the whole-step
    graphs give the eager loop's tokens."""
    cfg = ModelConfig(vocab_size=256, d_model=128, n_layers=2, n_heads=2, ffn_hidden=256, max_seq_len=64,
                      mem_layers=[1], mem_n_keys=24, mem_heads=4, mem_knn=5, mem_k_dim=64, mem_impl="torch")
    torch.manual_seed(4)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    m.set_memory_inference_table("bf16")
    prompt = torch.randint(0, 256, (3, 7), generator=torch.Generator().manual_seed(2)).to(DEV)
    note("generate n_keys=24 knn=5")
    eager = m.generate(prompt, 20, use_graph=False)
    graph = m.generate(prompt, 20, use_graph=True)
    assert torch.equal(eager, graph)
    dec = m._decoder(3, 28, DEV)
    assert dec.fused is not None
    rec = {}
    dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist, logits=True, record=rec)
    r = rec[1]
    rs, ri, rw = O.pk_select(bits_of(r["s1"]), bits_of(r["s2"]), 5)
    assert np.array_equal(r["indices"].cpu().numpy(), ri) and np.array_equal(bits_of(r["scores"]), rs)
    np.testing.assert_allclose(r["weights"].cpu().numpy(), rw, rtol=0, atol=1e-6)
