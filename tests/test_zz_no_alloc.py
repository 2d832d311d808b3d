"""smlm_pkm_lookup_noalloc -- the decode lookup with its sub-key scores in a static device array, for callers that
cannot allocate -- called through the C ABI against the same lookup on caller buffers (smlm_pkm_score into s1, s2,
then smlm_pkm_select_bag): the outputs must be identical (the same kernels run on the same scores), on two calls in
a row with the second one smaller, for bf16 and fp32 scores and a bf16 and an int8 table.  Requests beyond the
array are refused before anything is launched."""
import pytest
import torch

from smlm_hip import _lib
from smlm_hip import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, NK, HALF, KNN, D = 4, 1024, 256, 32, 384


def note(msg):
    print(msg, flush=True)


def lookup_noalloc(q, keys, table, scales, pre, out):
    N = q.shape[0]
    kind, d = K._table_kind(table, scales, "lookup_noalloc")
    return _lib.lib().smlm_pkm_lookup_noalloc(
        q.data_ptr(), H * 2 * HALF, keys.data_ptr(), _lib.BF16 if q.dtype == torch.bfloat16 else _lib.F32, N, H, NK,
        HALF, KNN, table.data_ptr(), kind, table.shape[0], d, scales.data_ptr() if scales is not None else None,
        pre.data_ptr() if pre is not None else None, out.data_ptr(),
        _lib.BF16 if out.dtype == torch.bfloat16 else _lib.F32, torch.cuda.current_stream().cuda_stream)


def with_buffers(q, keys, table, scales, pre, out_bf16):
    s1, s2 = K.pk_scores(q, keys)
    return K.pk_select_bag(s1, s2, KNN, table, scales, pre=pre, out_bf16=out_bf16)


@pytest.fixture(scope="module")
def tables():
    g = torch.Generator(device=DEV).manual_seed(0)
    bf = torch.empty(NK * NK, D, device=DEV).normal_(0.0, 0.02, generator=g).to(torch.bfloat16)
    codes, scales = K.quantize_int8(bf)
    return {"bf16": (bf, None), "int8": (codes, scales)}


@pytest.mark.parametrize("table_kind", ["bf16", "int8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@torch.no_grad()
def test_noalloc_lookup_matches_buffered_lookup(tables, table_kind, dtype):
    table, scales = tables[table_kind]
    g = torch.Generator(device=DEV).manual_seed(1)
    keys = (torch.randn(H, 2, NK, HALF, generator=g, device=DEV) / 16).to(dtype)
    for call, N in enumerate((64, 5)):
        note(f"lookup_noalloc {dtype} scores, {table_kind} table, call {call + 1}: N={N}")
        q = torch.randn(N, H, 2 * HALF, generator=g, device=DEV).to(dtype)
        pre = torch.randn(N, D, generator=g, device=DEV).to(torch.bfloat16)
        for out_bf16, p in ((False, None), (True, pre)):
            out = torch.full((N, D), float("nan"), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=DEV)
            _lib.check(lookup_noalloc(q, keys, table, scales, p, out), "smlm_pkm_lookup_noalloc")
            ref = with_buffers(q, keys, table, scales, p, out_bf16)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"call {call + 1} (N={N}, out_bf16={out_bf16}) differs"


@torch.no_grad()
def test_noalloc_lookup_refuses_more_than_the_array(tables):
    table, _ = tables["bf16"]
    N = 1024                                          # 2 x 1024 x 4 x 1024 bf16 scores = 16 MiB > 8 MiB
    q = torch.zeros(N, H, 2 * HALF, dtype=torch.bfloat16, device=DEV)
    keys = torch.zeros(H, 2, NK, HALF, dtype=torch.bfloat16, device=DEV)
    out = torch.full((N, D), 7.0, device=DEV)
    rc = lookup_noalloc(q, keys, table, None, None, out)
    assert rc == _lib.EUNSUPPORTED and "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call must not launch anything"


@torch.no_grad()
def test_noalloc_lookup_refuses_absurd_shapes_before_sizing(tables):
    """Head and key counts whose N * H * NK product would overflow int64 are refused by the argument checks of the
    two steps, which run before the scratch size is computed; nothing is launched."""
    table, _ = tables["bf16"]
    q = torch.zeros(4, H, 2 * HALF, dtype=torch.bfloat16, device=DEV)
    out = torch.full((4, D), 7.0, device=DEV)
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for h, nk, code in ((1 << 30, 1 << 30, _lib.EINVAL), (H, 0x7FFFFFFF, _lib.EUNSUPPORTED)):
        note(f"lookup_noalloc refused shape: H={h} NK={nk}")
        rc = lib.smlm_pkm_lookup_noalloc(q.data_ptr(), 1 << 20, q.data_ptr(), _lib.BF16, 4, h, nk, HALF, KNN,
                                         table.data_ptr(), _lib.BF16, table.shape[0], D, None, None, out.data_ptr(),
                                         _lib.F32, stream)
        assert rc == code, _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call must not launch anything"
