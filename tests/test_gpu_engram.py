"""Engram n-gram memory on the GPU (smlm_hip.engram): the hash kernel bit-exact against the oracle, the row gather
bit-exact against indexing, the module against the fp64 oracle (fp32 within 1e-5 of the output scale, bf16 within
2e-2), the model's cached / chunked decode against its full forward, and the row-sparse training path against fp64
autograd (1e-5)."""
import numpy as np
import pytest
import torch

import oracle.engram_oracle as E
from smlm_hip import kernels as K
from smlm_hip.engram import EngramMemory, NgramHash
from smlm_hip.model import ModelConfig, Transformer

pytestmark = pytest.mark.gpu
DEV = "cuda"
VOCAB = 1000


def note(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("orders,heads,rows,B,T", [((2, 3), 8, 524287, 4, 300), ((2, 3), 2, 101, 3, 1),
                                                   ((1, 2, 4), 3, 97, 2, 33)])
def test_hash_bit_exact(orders, heads, rows, B, T):
    note(f"engram hash orders={orders} heads={heads} rows={rows} B={B} T={T}")
    h = NgramHash(VOCAB, orders, heads, rows, seed=0, canon=torch.arange(VOCAB)).to(DEV)
    g = torch.Generator().manual_seed(T)
    c = torch.randint(0, h.pad + 1, (B, h.history + T), generator=g)
    got = h(c.to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, E.ngram_rows(c.numpy(), h.mult.cpu().numpy(), orders, heads, rows))
    big = torch.randint(2 ** 40, 2 ** 62, (1, h.history + 7), generator=g)   # wrap-around products
    np.testing.assert_array_equal(h(big.to(DEV)).cpu().numpy(),
                                  E.ngram_rows(big.numpy(), h.mult.cpu().numpy(), orders, heads, rows))


@pytest.mark.parametrize("dtype,D", [(torch.float32, 24), (torch.bfloat16, 24), (torch.float32, 5),
                                     (torch.bfloat16, 13), (torch.bfloat16, 8)])
def test_row_gather_bit_exact(dtype, D):
    note(f"row gather {dtype} D={D}")
    g = torch.Generator().manual_seed(D)
    table = torch.randn(777, D, generator=g).to(DEV, dtype)
    rows = torch.randint(0, 777, (5, 9, 16), generator=g).to(DEV)
    out = K.row_gather(rows, table)
    assert out.shape == (5, 9, 16, D) and torch.equal(out, table[rows])
    bad = torch.tensor([3, 777, -1], device=DEV)
    o2 = K.row_gather(bad, table).float().cpu()
    assert torch.equal(o2[0], table[3].float().cpu()) and torch.isnan(o2[1:]).all()


def _module_params(m):
    return {"values": m.values.weight, "w_k": m.w_k.weight, "w_v": m.w_v.weight, "h_norm": m.h_norm.weight,
            "k_norm": m.k_norm.weight, "v_norm": m.v_norm.weight, "conv": m.conv.weight}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@torch.no_grad()
def test_module_forward_against_fp64_oracle(dtype):
    note(f"engram module {dtype}")
    torch.manual_seed(1)
    m = EngramMemory(64, 16, 24, 53, conv_kernel=4, dilation=3).to(DEV)
    m.conv.weight.normal_(std=0.3)
    m = m.to(dtype)
    p = {k: v.detach().double().cpu() for k, v in _module_params(m).items()}
    g = torch.Generator().manual_seed(2)
    h = torch.randn(2, 21, 64, generator=g)
    rows = torch.randint(0, 53, (2, 21, 16), generator=g) + torch.arange(16) * 53
    ref, _ = E.engram_forward(p, h.to(dtype).double(), rows, 1e-5, 3)
    cache = {}
    got = torch.cat([m(h[:, a:a + n].to(DEV, dtype), rows[:, a:a + n].to(DEV), cache)
                     for a, n in ((0, 9), (9, 1), (10, 11))], 1)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    err = float((got.double().cpu() - ref).abs().max())
    assert err <= tol * float(ref.abs().max()), err


def _tiny(value_grad="row_sparse", seed=0, head_dim=24):
    cfg = ModelConfig(vocab_size=VOCAB, d_model=32, n_layers=4, n_heads=4, ffn_hidden=64, max_seq_len=64,
                      eng_layers=[0, 2], eng_heads=2, eng_head_dim=head_dim, eng_rows=101, eng_value_grad=value_grad)
    torch.manual_seed(seed)
    m = Transformer(cfg, ngram_canon=torch.arange(VOCAB))
    with torch.no_grad():
        for e in m.engram_layers():
            e.conv.weight.normal_(std=0.3)
    return m.to(DEV)


@torch.no_grad()
def test_model_cached_chunks_match_full_forward_and_causal():
    """tests/test_engram.py:58-78 on the GPU: cached chunks (hash history and conv past in the caches) give the
    full forward; changing later tokens leaves earlier logits alone."""
    note("engram model chunks")
    m = _tiny().eval()
    x = torch.randint(0, VOCAB, (2, 30), generator=torch.Generator().manual_seed(3)).to(DEV)
    full = m(x)
    caches = [dict() for _ in range(m.cfg.n_layers)]
    steps = [m(x[:, a:a + n], kv_caches=caches, pos0=a) for a, n in ((0, 7), (7, 1), (8, 1), (9, 12), (21, 9))]
    torch.testing.assert_close(torch.cat(steps, 1), full, rtol=1e-4, atol=1e-4)
    y = x.clone()
    y[:, 20:] = (y[:, 20:] + 1) % VOCAB
    torch.testing.assert_close(m(y)[:, :20], full[:, :20], rtol=0, atol=0)
    ids = m.generate(x[:, :9], 6)                           # eager steps (Engram decodes without graphs)
    assert ids.shape == (2, 7)
    cur = x[:, :9]
    for t in range(7):                                      # greedy tokens = argmax of full forwards
        nxt = m(cur)[:, -1].argmax(-1)
        assert torch.equal(nxt, ids[:, t])
        cur = torch.cat([cur, nxt[:, None]], 1)


def test_row_sparse_training_matches_fp64_autograd():
    """loss.backward() through the hash rows: the value tables' RowStore accumulators equal fp64 autograd of the
    oracle module (1e-5), touched flags are exactly the read rows, w_k's gradient too; value_grad="dense" gives
    the same table gradient as a dense .grad."""
    note("engram training")
    m = _tiny()
    e = m.engram_layers()[0]
    B, T = 2, 17
    g = torch.Generator().manual_seed(5)
    h = torch.randn(B, T, 32, generator=g)
    c = torch.randint(0, VOCAB, (B, 2 + T), generator=g)
    rows = m.ngram(c.to(DEV))
    G = torch.randn(B, T, 32, generator=g)
    (e(h.to(DEV), rows) * G.to(DEV)).sum().backward()
    p = {k: v.detach().double().cpu().requires_grad_(True) for k, v in _module_params(e).items()}
    y, _ = E.engram_forward(p, h.double(), rows.cpu(), 1e-5, 3)
    (y * G.double()).sum().backward()
    st = e.values.weight.row_store
    scale = float(p["values"].grad.abs().max())
    assert float((st.acc.double().cpu() - p["values"].grad).abs().max()) <= 1e-5 * scale
    read = torch.zeros(e.values.weight.shape[0], dtype=torch.bool)
    read[rows.reshape(-1).cpu()] = True
    assert torch.equal(st.touched.cpu(), read)
    assert e.values.weight.grad is None
    gk = float(p["w_k"].grad.abs().max())
    assert float((e.w_k.weight.grad.double().cpu() - p["w_k"].grad).abs().max()) <= 1e-5 * gk
    md = _tiny("dense")
    ed = md.engram_layers()[0]
    (ed(h.to(DEV), rows) * G.to(DEV)).sum().backward()
    assert float((ed.values.weight.grad.double().cpu() - p["values"].grad).abs().max()) <= 1e-5 * scale
