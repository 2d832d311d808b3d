"""The off-GPU value-table tiers (smlm_hip.offload) and the table files (smlm_hip.convert_table) on the GPU.

Every tier runs the same bag kernel as a table in HBM (smlm/offload.py:1-13: "every output is computed from the
same numbers in the same order"), so the bar is bit-exact equality with the in-HBM result: the zero-copy host
table (pinned RAM read over the host link), the staged tiers (compact device table with remapped indices), and
whole models loaded from rest.pt + table files.  The 4-bit files are checked against the oracle's quantisation.
"""
import numpy as np
import pytest
import torch

import oracle.pkm_oracle as O
from smlm_hip import kernels as K
from smlm_hip.convert_table import convert
from smlm_hip.model import ModelConfig, Transformer
from smlm_hip.offload import HostTable, MmapQ4Table, load_model

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(msg, flush=True)


def _table(kind, rows, D, g):
    w = torch.randn(rows, D, generator=g) * 0.05
    if kind == "f32":
        return w.to(DEV), None
    if kind == "bf16":
        return w.to(DEV, torch.bfloat16), None
    return (K.quantize_q4 if kind == "q4" else K.quantize_int8)(w.to(DEV))


def _lookups(N, Kl, rows, g):
    idx = torch.randint(0, rows, (N, Kl), generator=g)
    idx[0, :8] = 3                                       # repeated rows
    w = torch.softmax(torch.randn(N, Kl, generator=g), -1)
    return idx.to(DEV), w.to(DEV)


def _host(t):
    if t is None:
        return None
    out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    out.copy_(t)
    return out


@pytest.mark.parametrize("kind", ["f32", "bf16", "q4", "i8"])
def test_zero_copy_bag_matches_device_table(kind):
    note(f"zero-copy bag {kind}")
    g = torch.Generator().manual_seed(1)
    rows, D, N, Kl = 5000, 384, 64, 128
    table, scales = _table(kind, rows, D, g)
    idx, w = _lookups(N, Kl, rows, g)
    pre = torch.randn(N, D, generator=g).to(DEV, torch.bfloat16)
    ref = K.bag_infer(idx, w, table, scales, pre=pre, out_bf16=True)
    got = K.bag_infer(idx, w, _host(table), _host(scales), pre=pre, out_bf16=True)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    ref32 = K.bag_infer(idx, w, table, scales)
    assert torch.equal(K.bag_infer(idx, w, _host(table), _host(scales)), ref32)


def test_zero_copy_select_bag_and_graph_replays():
    """pk_select_bag reads a pinned host table like a device one, and a captured graph of it replays to the eager
    result every time (no synchronisation inside the call)."""
    note("zero-copy select_bag + graph")
    g = torch.Generator().manual_seed(2)
    N, H, NK, knn, D = 8, 4, 64, 16, 384
    table, scales = _table("q4", NK * NK, D, g)
    s1 = torch.randn(N, H, NK, generator=g).to(DEV, torch.bfloat16)
    s2 = torch.randn(N, H, NK, generator=g).to(DEV, torch.bfloat16)
    pre = torch.randn(N, D, generator=g).to(DEV, torch.bfloat16)
    ht, hs = _host(table), _host(scales)
    ref = K.pk_select_bag(s1, s2, knn, table, scales, pre=pre, out_bf16=True, record=True)
    got = K.pk_select_bag(s1, s2, knn, ht, hs, pre=pre, out_bf16=True, record=True)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        K.pk_select_bag(s1, s2, knn, ht, hs, pre=pre, out_bf16=True)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = K.pk_select_bag(s1, s2, knn, ht, hs, pre=pre, out_bf16=True)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref[0])


def test_pageable_host_table_is_refused():
    """A pageable CPU table never reaches a kernel: the wrapper refuses it, and so does the C ABI's check."""
    from smlm_hip import _lib
    g = torch.Generator().manual_seed(3)
    idx, w = _lookups(4, 8, 100, g)
    with pytest.raises(ValueError, match="pinned"):
        K.bag_infer(idx, w, torch.randn(100, 64))
    table = torch.randn(100, 64)
    with pytest.raises(_lib.SmlmError, match="not pinned"):
        _lib.host_device_pointer(table.data_ptr())
    with pytest.raises(_lib.SmlmError):
        _lib.host_device_pointer(torch.zeros(4, device=DEV).data_ptr())   # device memory is not host memory


@pytest.mark.parametrize("kind", ["bf16", "q4"])
def test_staged_host_table_matches_device(kind):
    note(f"staged host table {kind}")
    g = torch.Generator().manual_seed(4)
    rows, D, N, Kl = 3000, 256, 32, 64
    table, scales = _table(kind, rows, D, g)
    idx, w = _lookups(N, Kl, rows, g)
    pre = torch.randn(N, D, generator=g).to(DEV, torch.bfloat16)
    ref = K.bag_infer(idx, w, table, scales, pre=pre, out_bf16=True)
    t = HostTable(table.cpu(), scales.cpu() if scales is not None else None, staged=True)
    assert t.device_tables() is None and t.dim == D
    for _ in range(2):                                   # the second call reuses the staging buffers
        assert torch.equal(t.bag(idx, w, pre), ref)
    assert t.stats["calls"] == 2 and t.stats["unique_rows"] == 2 * len(torch.unique(idx))
    z = HostTable(table.cpu(), scales.cpu() if scales is not None else None)
    assert torch.equal(z.bag(idx, w, pre), ref)


def _lm_checkpoint(seed=3):
    cfg = ModelConfig(vocab_size=512, d_model=128, n_layers=3, n_heads=2, ffn_hidden=256, max_seq_len=64,
                      mem_layers=[2], mem_n_keys=64, mem_heads=4, mem_knn=16, mem_k_dim=64)
    torch.manual_seed(seed)
    m = Transformer(cfg).to(DEV, torch.bfloat16).eval()
    return cfg, m


def test_convert_q4_files_and_mmap_table(tmp_path):
    """values_q4.bin / scales_q4.bin equal the oracle's q4 encoding of the table (smlm/kernels.py:280-300), and
    MmapQ4Table (static + FIFO cache, the rest through the mapping) gives the in-HBM q4 bag bit for bit."""
    note("convert q4 + mmap table")
    cfg, m = _lm_checkpoint()
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    table = sd["layers.2.ffn.values.weight"].float()
    rows, D = table.shape
    hot = np.random.default_rng(0).integers(0, 50, rows)
    meta = convert({"model_config": cfg.to_dict(), "state_dict": sd}, str(tmp_path), chunk=1000, hot_counts=hot,
                   log=lambda *_: None)
    codes = np.fromfile(tmp_path / "values_q4.bin", dtype=np.uint8).reshape(rows, D // 2)
    sc = np.fromfile(tmp_path / "scales_q4.bin", dtype=np.float16)
    ref_codes, ref_scales = O.quantize_rows(table.numpy(), "q4")
    np.testing.assert_array_equal(codes, ref_codes)
    np.testing.assert_array_equal(sc.view(np.uint16), np.asarray(ref_scales, dtype=np.float16).view(np.uint16))
    assert meta["q4"] and "values_q4.bin" in meta["sha256"]
    dev_codes, dev_scales = torch.from_numpy(codes).to(DEV), torch.from_numpy(sc).to(DEV)
    t = MmapQ4Table(str(tmp_path / "values_q4.bin"), str(tmp_path / "scales_q4.bin"), rows, D,
                    hot_rows=np.load(tmp_path / "hot_rows.npy"), cache_rows=256, fifo_rows=512)
    g = torch.Generator().manual_seed(6)
    for call in range(3):
        idx, w = _lookups(16, 64, rows, g)
        pre = torch.randn(16, D, generator=g).to(DEV, torch.bfloat16)
        ref = K.bag_infer(idx, w, dev_codes, dev_scales, pre=pre, out_bf16=True)
        assert torch.equal(t.bag(idx, w, pre), ref), call
    assert t.stats["hits"] > 0 and t.stats["misses"] > 0
    t.close()


@torch.no_grad()
def test_load_model_on_each_tier_matches_the_in_hbm_model(tmp_path, monkeypatch):
    """rest.pt + table files -> load_model on (a) device q4 tensors, (b) the zero-copy host table, (c) the mmap
    table: the prompt logits equal the original model's with its in-HBM q4 table bit for bit; generate() on (a)
    and (b) (fused step, graphs) equals the original; (c) stages every call, so it decodes without graphs on the
    unfused step, and equals the original run on that same path."""
    note("load_model tiers")
    cfg, m = _lm_checkpoint()
    m.set_memory_inference_table("q4")
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    convert({"model_config": cfg.to_dict(), "state_dict": sd}, str(tmp_path), log=lambda *_: None)
    rows, D = sd["layers.2.ffn.values.weight"].shape
    codes = torch.from_numpy(np.fromfile(tmp_path / "values_q4.bin", dtype=np.uint8).reshape(rows, D // 2))
    sc = torch.from_numpy(np.fromfile(tmp_path / "scales_q4.bin", dtype=np.float16))
    prompt = torch.randint(0, cfg.vocab_size, (2, 11), generator=torch.Generator().manual_seed(7)).to(DEV)
    ref_logits = m(prompt)
    ref_tokens = m.generate(prompt, 12)
    rest = str(tmp_path / "rest.pt")
    mm = MmapQ4Table(str(tmp_path / "values_q4.bin"), str(tmp_path / "scales_q4.bin"), rows, D)
    tiers = {"device": (codes.to(DEV), sc.to(DEV)), "zero-copy": HostTable(codes, sc), "mmap": mm}
    for name, table in tiers.items():
        note(f"load_model tier {name}")
        lm = load_model(rest, table).to(torch.bfloat16)
        assert torch.equal(lm(prompt), ref_logits), name
        if name != "mmap":
            assert torch.equal(lm.generate(prompt, 12), ref_tokens), name
    from smlm_hip import model as model_mod
    monkeypatch.setattr(model_mod._FusedDecodeStep, "supported", staticmethod(lambda *a: False))
    m._decoders.clear()
    eager_ref = m.generate(prompt, 12, use_graph=False)
    staged = load_model(rest, mm).to(torch.bfloat16)
    assert torch.equal(staged.generate(prompt, 12), eager_ref)
    assert mm.stats["calls"] > 12
    mm.close()
