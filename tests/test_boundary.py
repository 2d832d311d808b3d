"""The drop-in boundary, without a GPU: libsmlm_pkm.so loads, exports every function include/smlm_pkm.h
declares, and its argument checks return the documented status codes before anything is launched; the Python
host layer rejects unsupported shapes the way the reference does (tests/test_pkm.py:130-136)."""
import ctypes
import os
import re

import pytest
import torch

from smlm_hip import _lib
from smlm_hip.pkm import ProductKeyMemory

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "smlm_pkm.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(smlm_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert ctypes.cast(getattr(raw, name), ctypes.c_void_p).value


def test_version():
    assert _lib.version().startswith("smlm_pkm ") and "gfx950" in _lib.version()


def test_argument_checks_return_status_codes():
    """Invalid calls are refused before any HIP call (safe without a GPU)."""
    lib = _lib.lib()
    fake = 256                                           # never dereferenced: the checks fail first
    assert lib.smlm_pkm_bag(None, _lib.I64, fake, 1, 1, fake, _lib.F32, 1, 4, None, None, fake, _lib.F32,
                            None) == _lib.EINVAL
    assert "null" in _lib.last_error()
    assert lib.smlm_pkm_bag(fake, 99, fake, 1, 1, fake, _lib.F32, 1, 4, None, None, fake, _lib.F32,
                            None) == _lib.EINVAL
    assert lib.smlm_pkm_bag(fake, _lib.I64, fake, 1, 1, fake, _lib.I8, 1, 4, None, None, fake, _lib.F32,
                            None) == _lib.EINVAL                                 # i8 table without scales
    assert "scales" in _lib.last_error()
    assert lib.smlm_pkm_bag(fake, _lib.I64, fake, 1, 1, fake, _lib.Q4, 1, 5, fake, None, fake, _lib.F32,
                            None) == _lib.EINVAL                                 # odd D for q4
    assert lib.smlm_pkm_select(fake, fake, _lib.BF16, 1, 4, 1024, 129, fake, fake, fake, None) == _lib.EUNSUPPORTED
    assert "knn" in _lib.last_error()
    assert lib.smlm_pkm_select(fake, fake, _lib.BF16, 1, 4, 20, 32, fake, fake, fake, None) == _lib.EUNSUPPORTED
    assert lib.smlm_pkm_select(fake, fake, _lib.BF16, 1, 4, 131072, 32, fake, fake, fake, None) == _lib.EUNSUPPORTED
    assert lib.smlm_pkm_select(fake, fake, _lib.I8, 1, 4, 1024, 32, fake, fake, fake, None) == _lib.EINVAL
    assert lib.smlm_pkm_score(fake, 512, fake, _lib.BF16, 1, 1, 64, 12, fake, fake, None) == _lib.EUNSUPPORTED
    assert lib.smlm_pkm_score(fake, 100, fake, _lib.BF16, 1, 1, 64, 256, fake, fake, None) == _lib.EINVAL
    assert lib.smlm_pkm_score(fake + 2, 512, fake, _lib.BF16, 1, 1, 64, 256, fake, fake, None) == _lib.EINVAL
    assert "aligned" in _lib.last_error()
    assert lib.smlm_pkm_quantize(fake, _lib.F32, 4, 5, _lib.Q4, fake, fake, None) == _lib.EINVAL
    assert lib.smlm_pkm_quantize(fake, _lib.F32, 4, 8, _lib.BF16, fake, fake, None) == _lib.EINVAL
    # zero tokens is a valid no-op
    assert lib.smlm_pkm_select(fake, fake, _lib.BF16, 0, 4, 1024, 32, fake, fake, fake, None) == _lib.OK


def test_noalloc_lookup_validates_before_sizing():
    """smlm_pkm_lookup_noalloc checks every argument of its two steps before it computes the scratch size, so
    absurd head or key counts (whose N * H * NK product would overflow int64) are refused with a status code."""
    lib = _lib.lib()
    fake = 256
    args = dict(q_row_stride=1 << 20, half=256, knn=32, table_dtype=_lib.BF16, rows=1 << 20, D=384)

    def call(N, H, NK, **kw):
        a = dict(args, **kw)
        return lib.smlm_pkm_lookup_noalloc(fake, a["q_row_stride"], fake, _lib.BF16, N, H, NK, a["half"], a["knn"],
                                           fake, a["table_dtype"], a["rows"], a["D"], None, None, fake, _lib.F32,
                                           None)

    assert call(64, 1 << 30, 1 << 30) == _lib.EINVAL and "bad shape" in _lib.last_error()       # H > 32768
    assert call(64, 4, 0x7FFFFFFF) == _lib.EUNSUPPORTED and "NK" in _lib.last_error()            # NK > 65536
    assert call(64, 16, 1024) == _lib.EUNSUPPORTED and "H=16" in _lib.last_error()               # fused: H <= 8
    assert call(1024, 4, 1024) == _lib.EUNSUPPORTED and "scratch" in _lib.last_error()           # valid, too big
    assert call(1 << 40, 4, 1024) == _lib.EUNSUPPORTED and "scratch" in _lib.last_error()        # N alone
    assert call(-1, 4, 1024) == _lib.EINVAL
    assert call(0, 4, 1024) == _lib.OK                                                          # no-op, no HIP


def test_status_becomes_python_exception():
    with pytest.raises(_lib.SmlmError, match="status -1"):
        _lib.check(_lib.lib().smlm_pkm_quantize(None, _lib.F32, 1, 8, _lib.I8, None, None, None),
                   "smlm_pkm_quantize")


def test_shapes_of_the_reference_impls():
    """As the reference (smlm/pkm.py:49-53, tests/test_pkm.py:130-136): impl="triton" refuses non-power-of-two
    n_keys or knn at construction with a clear message, impl="torch" (and "hip") takes them; every impl is
    bounded by the kernels' limits, n_keys <= 65536 and knn <= 128."""
    for n_keys, knn in ((24, 4), (16, 5)):
        with pytest.raises(ValueError, match="powers of two"):
            ProductKeyMemory(32, 32, n_keys=n_keys, knn=knn, k_dim=16, impl="triton")
        for impl in ("torch", "hip"):
            m = ProductKeyMemory(32, 32, n_keys=n_keys, knn=knn, k_dim=16, impl=impl)
            assert m.keys.shape == (4, 2, n_keys, 8) and m.values.weight.shape == (n_keys ** 2, 32)
    for impl in ("hip", "torch", "triton"):
        ProductKeyMemory(32, 32, n_keys=256, knn=128, k_dim=16, impl=impl)
        with pytest.raises(ValueError, match="knn <= 128"):
            ProductKeyMemory(32, 32, n_keys=512, knn=256, k_dim=16, impl=impl)
    with pytest.raises(ValueError, match="k_dim must be even and knn <= n_keys"):
        ProductKeyMemory(32, 32, n_keys=8, knn=9, k_dim=16)


def test_impl_names_of_reference_configs():
    """A reference config's mem_impl ("torch", its default, or "triton") constructs the same module, kept in
    self.impl; any other name fails at construction."""
    a = ProductKeyMemory(32, 32, n_keys=16, knn=4, k_dim=16)
    for impl in ("torch", "triton"):
        m = ProductKeyMemory(32, 32, n_keys=16, knn=4, k_dim=16, impl=impl)
        assert m.impl == impl and set(m.state_dict()) == set(a.state_dict())
    with pytest.raises(ValueError, match="impl must be one of"):
        ProductKeyMemory(32, 32, n_keys=16, knn=4, k_dim=16, impl="cuda")
    from smlm_hip.model import ModelConfig, Transformer
    cfg = ModelConfig(vocab_size=64, d_model=32, n_layers=2, n_heads=2, ffn_hidden=64, max_seq_len=16,
                      mem_layers=[1], mem_n_keys=16, mem_heads=2, mem_knn=4, mem_k_dim=16, mem_impl="torch")
    assert Transformer(cfg).layers[1].ffn.impl == "torch"


def test_state_dict_keys_are_the_reference_names():
    m = ProductKeyMemory(24, 24, n_keys=16, heads=2, knn=4, k_dim=16)
    keys = set(m.state_dict())
    assert {"keys", "query_proj.weight", "query_proj.bias", "query_norm.weight", "query_norm.bias",
            "query_norm.running_mean", "query_norm.running_var", "values.weight", "swilu_proj.weight",
            "swilu_proj.bias", "value_proj.weight", "value_proj.bias"} <= keys


def test_kernels_refuse_cpu_tensors():
    from smlm_hip import kernels
    s = torch.zeros(1, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP"):
        kernels.pk_select(s, s, 8)


def test_linear_args_struct_layout_matches_header(tmp_path):
    """The ctypes mirror of struct smlm_linear_args has the C compiler's field offsets and size."""
    import subprocess
    fields = [f for f, _ in _lib.LinearArgs._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("{f} %zu\\n", offsetof(smlm_linear_args, {f}));\n' for f in fields)
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "smlm_pkm.h"\nint main(void) {\n' + body +
                   '  printf("sizeof %zu\\n", sizeof(smlm_linear_args));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{os.path.dirname(HEADER)}", str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    for f in fields:
        assert int(got[f]) == getattr(_lib.LinearArgs, f).offset, f
    assert int(got["sizeof"]) == ctypes.sizeof(_lib.LinearArgs)


def test_decode_linear_argument_checks():
    lib = _lib.lib()
    fake = 256
    assert lib.smlm_decode_linear(None, None) == _lib.EINVAL
    a = _lib.LinearArgs()
    a.prologue, a.epilogue, a.M, a.N, a.K = _lib.LIN_PLAIN, _lib.LIN_STORE, 4, 64, 384
    a.x, a.x_stride, a.w, a.n_split, a.out, a.out_stride = fake, 384, fake, 64, fake, 64
    a.N = 40                                              # not a multiple of 16
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.N, a.K = 64, 100                                    # K not a multiple of 32
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.K, a.x_stride, a.prologue, a.norm_w = 512, 512, _lib.LIN_RMSNORM, fake  # normalised rows too wide for LDS
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EUNSUPPORTED
    a.K, a.x_stride, a.prologue, a.epilogue = 384, 384, _lib.LIN_PLAIN, _lib.LIN_ARGMAX    # partial missing
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "partial" in _lib.last_error()
    a.epilogue, a.delta = _lib.LIN_STORE, fake            # delta without an RMSNorm prologue
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.delta, a.M = None, 0                                # zero rows: a valid no-op
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.OK
    assert lib.smlm_linear_argmax_blocks(32000) == 250 and lib.smlm_linear_argmax_blocks(129) == 2
    assert lib.smlm_argmax_finish(None, 1, 1, 1, fake, fake, None, 0, 0, 1, None) == _lib.EINVAL


def test_embed_argmax_prologue_argument_checks():
    """SMLM_LIN_EMBED_ARGMAX and pos_advance refuse bad arguments before any launch."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    a = _lib.LinearArgs()
    a.prologue, a.epilogue, a.M, a.N, a.K = _lib.LIN_EMBED_ARGMAX, _lib.LIN_STORE, 2, 64, 384
    a.w, a.norm_w, a.n_split, a.out, a.out_stride, a.emb, a.emb_rows = fake, fake, 64, fake, 64, fake, 100
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "tok_partial" in _lib.last_error()
    a.tok_partial, a.tok_blocks, a.tok_partial_stride = fake, 5, 5          # odd row stride
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "even" in _lib.last_error()
    a.tok_partial_stride = 4                                              # shorter than the blocks
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.tok_partial_stride, a.tok_partial = 6, ctypes.c_void_p(0x1008)      # keys not 16-byte aligned
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.tok_partial, a.hist, a.hist_len, a.hist_stride = fake, fake, 10, 10  # hist without pos
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "pos" in _lib.last_error()
    a.pos, a.M = fake, 0                                                  # valid; zero rows: a no-op
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.OK
    a.pos_advance = fake                                                  # pos_advance without ARGMAX
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "pos_advance" in _lib.last_error()
    a.epilogue, a.partial, a.partial_stride = _lib.LIN_ARGMAX, fake, 1   # ARGMAX with M = 0: nothing would advance
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "M >= 1" in _lib.last_error()


def test_prefill_attention_argument_checks():
    """smlm_prefill_attention refuses bad arguments before any launch, among them key / value rows that a 32-bit
    buffer offset from a (batch, head)'s first row cannot reach."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    st = (ctypes.c_int64 * 3)(6 * 4096 * 64, 4096 * 64, 64)            # (B, H, S, 64) contiguous
    args = [fake, st, fake, st, fake, st, fake, st]
    assert lib.smlm_prefill_attention(*args, 0, 6, 128, 4096, 64, None) == _lib.OK          # B = 0: a no-op
    assert lib.smlm_prefill_attention(*args, 0, 6, 128, 4096, 48, None) == _lib.EUNSUPPORTED  # head_dim
    assert lib.smlm_prefill_attention(*args, 0, 6, 5000, 4096, 64, None) == _lib.EINVAL       # S < T
    big = (ctypes.c_int64 * 3)(0, 0, 1 << 20)                            # 2^14 keys x 2 MB per row
    assert lib.smlm_prefill_attention(fake, st, fake, big, fake, st, fake, st, 0, 1, 1, 1 << 14, 64,
                                      None) == _lib.EUNSUPPORTED and "2 GB" in _lib.last_error()


def test_parts_prologue_and_attention_proj_argument_checks():
    """The RMSNORM_PARTS prologue and smlm_decode_attention_proj refuse bad arguments before any launch."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    a = _lib.LinearArgs()
    a.prologue, a.epilogue, a.M, a.N, a.K = _lib.LIN_RMSNORM_PARTS, _lib.LIN_STORE, 2, 64, 384
    a.x, a.x_stride, a.w, a.norm_w, a.n_split, a.out, a.out_stride = fake, 384, fake, fake, 64, fake, 64
    a.delta, a.delta_parts = None, 6                      # no parts
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.delta = fake
    for bad in (0, 9):                                    # 1..8 parts
        a.delta_parts = bad
        assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL and "parts" in _lib.last_error()
    a.delta_parts, a.epilogue, a.partial, a.partial_stride = 6, _lib.LIN_ARGMAX, fake, 1   # not with ARGMAX
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.EINVAL
    a.epilogue, a.M = _lib.LIN_STORE, 0                   # zero rows: a valid no-op
    assert lib.smlm_decode_linear(ctypes.byref(a), None) == _lib.OK
    # attention + wo: null wo / parts, short wo rows, misaligned wo
    args = [fake, 1152, fake, fake, _lib.F32, 16, fake, fake, fake, 2, 6, 64, 16]
    assert lib.smlm_decode_attention_proj(*args, None, 384, 384, fake, None) == _lib.EINVAL
    assert lib.smlm_decode_attention_proj(*args, fake, 384, 384, None, None) == _lib.EINVAL
    assert lib.smlm_decode_attention_proj(*args, fake, 200, 384, fake, None) == _lib.EINVAL
    assert lib.smlm_decode_attention_proj(*args, ctypes.c_void_p(0x1008), 384, 384, fake, None) == _lib.EINVAL
    args[9] = 0                                           # B = 0: a valid no-op
    assert lib.smlm_decode_attention_proj(*args, fake, 384, 384, fake, None) == _lib.OK


def test_bench_decode_roofline_accounting():
    """bench.py's decode floors on the config-3 model (meta tensors, nothing allocated): the bytes a step moves and
    its launch count, with and without wo folded into the attention launch."""
    import bench
    from smlm_hip.model import Transformer, _FusedDecodeStep
    cfg = bench.lm_config(4096, 400)
    with torch.device("meta"):
        m = Transformer(cfg)
    m = m.to(torch.bfloat16)
    C, L = 384, 6
    weights = 2 * (32000 * C + 5 * (3 * C * C + C * C + 2 * 1024 * C + 1024 * C)       # embedding / lm_head, dense
                   + 4 * C * C + 2048 * C + 2 * C * C + 4 * 2 * 4096 * 256            # block 3: attention, query,
                   + 2048 * 3 + 2 * C + (2 * L + 1) * C)                              # swilu, value, keys; biases,
    r = bench.decode_roofline(m, 64, 0.2, 100.0, 1.5, 1.8)                            # BatchNorm, norms
    assert r["weight_bytes"] == weights + 64 * C * 2
    assert r["value_row_bytes"] == 64 * 4 * 32 * C * 2
    assert r["kv_cache_bytes"] == L * 2 * 64 * 101 * C * 2
    assert r["launches_per_step"] == 5 * 5 + 7 + 1 and r["bound"] == "launch"   # dense, memory block, head
    assert abs(r["launch_floor_ms"] - r["launches_per_step"] * 1.5e-3) < 1e-12
    assert abs(r["hbm_floor_ms"] - r["hbm_bytes_per_step"] / 8e12 * 1e3) < 1e-12
    assert _FusedDecodeStep.proj_max_batch >= 1
    assert bench.decode_roofline(m, 1, 0.15, 100.0, 1.5, 1.8)["launches_per_step"] == 4 * 5 + 6 + 1   # wo folded


def test_bench_reads_counter_traffic_only_for_the_measured_sources(tmp_path):
    """bench.py takes the gather's HBM traffic from the committed rocprofv3 summary only while the summary names the
    sha256 of the gather sources it runs with; another hash, or none, leaves the traffic unmeasured."""
    import bench
    good = bench.read_traffic()
    assert not good["stale"] and good["uniform"] > 3.4e9 and good["zipf"] > 1e9
    text = open(os.path.join(os.path.dirname(HEADER), "..", "profiles", "gather_config4_pmc.txt")).read()
    stale = tmp_path / "stale.txt"
    stale.write_text(text.replace(bench.gather_sources_sha256(), "0" * 64))
    r = bench.read_traffic(str(stale))
    assert r["stale"] and r["uniform"] is None and r["zipf"] is None
    none = tmp_path / "none.txt"
    none.write_text("\n".join(line for line in text.splitlines() if not line.startswith("gather_sources_sha256")))
    assert bench.read_traffic(str(none))["stale"]
