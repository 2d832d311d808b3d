"""LazyRowAdam's argument checks (the cases of the reference's tests/test_lowmem_values.py:153-183), which run before
any kernel, so on the CPU."""
import pytest
import torch

from smlm_hip.sparse_values import LazyRowAdam, OptimizerSet, RowStore, row_store, row_sparse_tables


@pytest.mark.parametrize("mode", ["fp32", "bf16", "int8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float64])
def test_states_require_fp32_parameters(mode, dtype):
    with pytest.raises(ValueError, match="fp32"):
        LazyRowAdam([torch.nn.Parameter(torch.zeros(4, 7, dtype=dtype))], lr=0.01, state_dtype=mode)


def test_invalid_state_dtype_fails_loudly():
    with pytest.raises(ValueError, match="state_dtype"):
        LazyRowAdam([torch.nn.Parameter(torch.zeros(4, 7))], lr=0.01, state_dtype="fp16")


@pytest.mark.parametrize("mode", ["fp32", "bf16", "int8"])
@pytest.mark.parametrize("options", [{"lr": float("nan")}, {"eps": float("nan")}, {"lr": -0.1}, {"eps": -0.1},
                                     {"betas": (0.9, 1.0)}])
def test_adam_hyperparameter_validation(mode, options):
    with pytest.raises(ValueError):
        LazyRowAdam([torch.nn.Parameter(torch.zeros(4, 7))], state_dtype=mode, **dict({"lr": 0.01}, **options))


@pytest.mark.parametrize("mode", ["fp32", "bf16", "int8"])
@pytest.mark.parametrize("shape", [(5,), (2, 3, 4), (2, 0)])
def test_states_require_nonempty_matrix_width(mode, shape):
    with pytest.raises(ValueError, match="contiguous fp32 tables"):
        LazyRowAdam([torch.nn.Parameter(torch.zeros(shape))], lr=0.01, state_dtype=mode)


@pytest.mark.parametrize("mode", ["fp32", "bf16", "int8"])
def test_states_require_contiguous_tables(mode):
    table = torch.nn.Parameter(torch.zeros(7, 11).t())
    with pytest.raises(ValueError, match="contiguous fp32 tables"):
        LazyRowAdam([table], lr=0.01, state_dtype=mode)


def test_impl_names():
    """The reference's impl names construct the same optimizer; other names fail."""
    for impl in ("hip", "triton", "torch"):
        assert LazyRowAdam([torch.nn.Parameter(torch.zeros(4, 7))], lr=0.01, impl=impl).impl == impl
    with pytest.raises(ValueError, match="impl must be one of"):
        LazyRowAdam([torch.nn.Parameter(torch.zeros(4, 7))], lr=0.01, impl="cuda")


def test_row_store_follows_its_table_and_state_dict_checks():
    table = torch.nn.Parameter(torch.zeros(6, 4))
    st = row_store(table)
    assert isinstance(st, RowStore) and row_store(table) is st
    assert st.acc.shape == (6, 4) and st.acc.dtype == torch.float32 and st.touched.dtype == torch.bool
    st.acc[2] = 1.0
    st.touched[2] = True
    st.grad_scale = 0.5
    st.reset(torch.tensor([2]))
    assert not st.acc.any() and not st.touched.any() and st.grad_scale == 1.0
    opt = LazyRowAdam([table], lr=0.01, state_dtype="int8")
    sd = opt.state_dict()
    assert sd["format"] == "smlm.lazy_row_adam.v1" and sd["shapes"] == [[6, 4]]
    with pytest.raises(ValueError, match="int8"):
        LazyRowAdam([table], lr=0.01, state_dtype="bf16").load_state_dict(sd)
    other = LazyRowAdam([torch.nn.Parameter(torch.zeros(5, 4))], lr=0.01, state_dtype="int8")
    with pytest.raises(ValueError, match="shapes"):
        other.load_state_dict(sd)
    with pytest.raises(ValueError, match="smlm.optimizer_set.v1"):
        OptimizerSet(opt).load_state_dict({"format": "something else"})
    assert row_sparse_tables(torch.nn.Linear(2, 2)) == []
