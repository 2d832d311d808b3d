"""Table files and the host side of the off-GPU table tiers (smlm_hip.convert_table, smlm_hip.offload), on the CPU:
the formats of scripts/convert_table.py:56-94 and the row cache of MmapQ4Table (smlm/offload.py:95-173).  The
4-bit files and every GPU read are checked in test_gpu_offload.py."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle.pkm_oracle as O
from smlm_hip import _lib
from smlm_hip.convert_table import convert, shared_table
from smlm_hip.model import ModelConfig, Transformer
from smlm_hip.offload import HostTable, MmapQ4Table


def tiny_checkpoint(share=True, seed=0):
    cfg = ModelConfig(vocab_size=128, d_model=64, n_layers=3, n_heads=2, ffn_hidden=128, max_seq_len=64,
                      mem_layers=[1, 2], mem_n_keys=16, mem_heads=2, mem_knn=4, mem_k_dim=32, mem_share_values=share)
    torch.manual_seed(seed)
    model = Transformer(cfg)
    return {"model_config": cfg.to_dict(), "state_dict": model.state_dict()}


def test_convert_writes_rest_bf16_hot_rows_and_meta(tmp_path):
    ck = tiny_checkpoint()
    keys, table = shared_table(ck["state_dict"])
    assert keys == ["layers.1.ffn.values.weight", "layers.2.ffn.values.weight"]
    rows, dim = table.shape
    counts = np.random.default_rng(0).integers(0, 5, rows)            # ties: the stable order keeps row order
    meta = convert(ck, str(tmp_path), chunk=100, q4=False, hot_counts=counts, log=lambda *_: None)
    rest = torch.load(tmp_path / "rest.pt", weights_only=True)
    assert rest["table_keys"] == keys and rest["table_shape"] == [rows, dim]
    assert rest["model_config"] == ck["model_config"]
    assert set(rest["state_dict"]) == set(ck["state_dict"]) - set(keys)
    for k, v in rest["state_dict"].items():
        assert torch.equal(v, ck["state_dict"][k])
    bits = np.fromfile(tmp_path / "values_bf16.bin", dtype=np.uint16).reshape(rows, dim)
    np.testing.assert_array_equal(bits, O.bf16_bits_rtne(table.numpy()))  # round to nearest even, row-major
    hot = np.load(tmp_path / "hot_rows.npy")
    expect = sorted(range(rows), key=lambda r: (-counts[r], r))       # most read first, ties by row id
    np.testing.assert_array_equal(hot, expect)
    on_disk = json.loads((tmp_path / "meta.json").read_text())
    assert on_disk == meta and meta["rows"] == rows and meta["dim"] == dim and meta["q4"] is None
    for name, digest in meta["sha256"].items():
        assert hashlib.sha256((tmp_path / name).read_bytes()).hexdigest() == digest
    assert set(meta["sha256"]) == {"rest.pt", "values_bf16.bin", "hot_rows.npy"}


def test_convert_refuses_unshared_tables(tmp_path):
    with pytest.raises(ValueError, match="shared"):
        convert(tiny_checkpoint(share=False), str(tmp_path), q4=False, log=lambda *_: None)


def _q4_files(tmp_path, rows=300, dim=8, seed=1):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, (rows, dim // 2), dtype=np.uint8)
    scales = rng.standard_normal(rows).astype(np.float16)
    codes.tofile(tmp_path / "values_q4.bin")
    scales.tofile(tmp_path / "scales_q4.bin")
    return codes, scales


def test_mmap_q4_table_fetch_static_and_fifo_cache(tmp_path):
    """fetch() returns the file's rows and scales whatever the cache holds: static hot rows, FIFO slots filled by
    misses (oldest evicted first), the rest from the mapping."""
    rows, dim = 300, 8
    codes, scales = _q4_files(tmp_path, rows, dim)
    hot = np.arange(rows)[::-1].copy()                                   # rows 299, 298, ... are "hot"
    t = MmapQ4Table(str(tmp_path / "values_q4.bin"), str(tmp_path / "scales_q4.bin"), rows, dim, hot_rows=hot,
                    cache_rows=20, fifo_rows=4, device="cpu")
    assert t.width == dim // 2 and t.q4
    calls = [np.array([1, 5, 290, 299]), np.array([5, 7, 9, 11, 13]), np.array([1, 5, 7, 285])]
    misses = []
    for want in calls:
        out = torch.empty(len(want), dim // 2, dtype=torch.uint8)
        out_s = torch.empty(len(want), dtype=torch.float16)
        before = t.stats["misses"]
        t.fetch(want, out, out_s)
        np.testing.assert_array_equal(out.numpy(), codes[want])
        np.testing.assert_array_equal(out_s.numpy(), scales[want])
        misses.append(t.stats["misses"] - before)
    # call 1: 1, 5 miss (290, 299 static); FIFO = {1, 5}.  call 2: 5 hits; 7, 9, 11, 13 miss and evict 1, 5 (FIFO of
    # 4 keeps the last 4 misses).  call 3: 1, 5 miss again, 7 hits (still in the FIFO), 285 static.
    assert misses == [2, 4, 2]
    assert t.stats["hits"] == 2 + 1 + 2
    assert t.stats["pages_requested"] > 0
    t.drop_os_cache()
    out = torch.empty(2, dim // 2, dtype=torch.uint8)
    t.fetch(np.array([0, 299]), out, torch.empty(2, dtype=torch.float16))
    np.testing.assert_array_equal(out.numpy(), codes[[0, 299]])
    t.close()


def test_mmap_q4_table_checks_file_sizes(tmp_path):
    _q4_files(tmp_path, 300, 8)
    with pytest.raises(ValueError, match="bytes"):
        MmapQ4Table(str(tmp_path / "values_q4.bin"), str(tmp_path / "scales_q4.bin"), 300, 16, device="cpu")
    with pytest.raises(ValueError, match="scales"):
        MmapQ4Table(str(tmp_path / "values_q4.bin"), str(tmp_path / "scales_q4.bin"), 299, 8, device="cpu")


def test_staged_host_table_fetch():
    table = torch.randn(50, 16)
    t = HostTable(table, staged=True, device="cpu")
    assert t.device_tables() is None and t.dim == 16 and not t.q4
    want = np.array([0, 7, 49])
    out = torch.empty(3, 16)
    t.fetch(want, out, None)
    assert torch.equal(out, table[want])


def test_host_table_pointer_argument_checks():
    """Refused before any HIP call (safe without a GPU)."""
    lib = _lib.lib()
    assert lib.smlm_host_table_pointer(None, None) == _lib.EINVAL
    assert "null" in _lib.last_error()
