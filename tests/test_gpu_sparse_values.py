"""Row-sparse table training on the kernels, the behaviour the reference's tests/test_sparse_values.py and
tests/test_lowmem_values.py check: row-sparse gradients equal dense ones through three memory layers sharing one
table over two micro-batches; rows that were not read keep their values and every state tensor bit for bit; the
first lazy step equals torch Adam on the read rows; an empty step changes nothing but the step count; the state
takes the budgeted bytes per row; int8 moments keep a positive second moment; frozen tables stay untouched."""
import pytest
import torch

from smlm_hip.model import ModelConfig, Transformer
from smlm_hip.sparse_values import LazyRowAdam, OptimizerSet, clip_row_sparse, row_sparse_tables, row_store

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(msg, flush=True)


def tiny(value_grad, seed=0):
    cfg = ModelConfig(vocab_size=128, d_model=32, n_layers=4, n_heads=4, ffn_hidden=64, max_seq_len=64,
                      mem_layers=[0, 2, 3], mem_n_keys=16, mem_heads=2, mem_knn=4, mem_k_dim=16,
                      mem_share_values=True, mem_value_grad=value_grad)
    torch.manual_seed(seed)
    return Transformer(cfg).to(DEV)


def table_of(m):
    return m.memory_layers()[0].values.weight


def backward_twice(m):
    """Two micro-batches through three memory layers sharing one table; returns the rows read."""
    g = torch.Generator(device=DEV).manual_seed(1)
    read = set()
    for _ in range(2):
        for x in m.memory_layers():
            x.record = True
        idx = torch.randint(0, 128, (2, 12), generator=g, device=DEV)
        _, loss = m(idx[:, :-1], idx[:, 1:])
        (loss / 2).backward()
        for x in m.memory_layers():
            read |= set(x.last_indices.reshape(-1).tolist())
    return read


def test_row_sparse_gradients_equal_dense():
    note("row-sparse vs dense gradients")
    dense, sparse = tiny("dense"), tiny("row_sparse")
    sparse.load_state_dict(dense.state_dict())
    assert backward_twice(dense) == backward_twice(sparse)
    st = row_store(table_of(sparse))
    assert table_of(sparse).grad is None
    torch.testing.assert_close(st.acc, table_of(dense).grad, rtol=1e-4, atol=1e-7)
    for (n, pd), ps in zip(dense.named_parameters(), sparse.parameters()):
        if pd is table_of(dense):
            continue
        torch.testing.assert_close(ps.grad, pd.grad, rtol=1e-4, atol=1e-6, msg=n)
    # the clip norm over the accumulated rows equals the dense table gradient's norm
    total = clip_row_sparse([table_of(sparse)], 1e-3)
    torch.testing.assert_close(total, table_of(dense).grad.norm(), rtol=1e-5, atol=0)
    assert float(st.grad_scale) == pytest.approx(min(1.0, 1e-3 / (float(total) + 1e-6)))


def test_touched_rows_are_the_rows_read():
    m = tiny("row_sparse")
    read = backward_twice(m)
    assert set(torch.nonzero(row_store(table_of(m)).touched).squeeze(1).tolist()) == read


def test_unread_rows_unchanged_values_and_state():
    note("unread rows over three steps")
    m = tiny("row_sparse")
    table = table_of(m)
    rest = [p for p in m.parameters() if p is not table]
    lazy = LazyRowAdam(row_sparse_tables(m), lr=2.4e-2)
    opt = OptimizerSet(torch.optim.AdamW(rest, lr=1e-2, weight_decay=0.1), lazy)
    assert row_sparse_tables(m) == [table]
    for step in range(3):
        before = table.detach().clone()
        st_before = {k: v.clone() for k, v in lazy.state[table].items()} if lazy.state[table] else None
        read = backward_twice(m)
        rows = torch.tensor(sorted(read), device=DEV)
        unread = torch.ones(table.shape[0], dtype=torch.bool, device=DEV)
        unread[rows] = False
        clip_row_sparse([table], 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        after = table.detach()
        assert torch.equal(after[unread], before[unread])
        assert not torch.equal(after[rows], before[rows])
        st = lazy.state[table]
        if st_before is not None:
            assert torch.equal(st["exp_avg"][unread], st_before["exp_avg"][unread])
            assert torch.equal(st["exp_avg_sq"][unread], st_before["exp_avg_sq"][unread])
        else:
            assert torch.count_nonzero(st["exp_avg"][unread]) == 0
        assert int(st["step"]) == step + 1
        assert not row_store(table).touched.any()
        assert torch.count_nonzero(row_store(table).acc) == 0


def test_lazy_adam_first_step_equals_adam_on_read_rows():
    torch.manual_seed(0)
    table = torch.nn.Parameter(torch.randn(50, 8, device=DEV))
    ref = torch.nn.Parameter(table.detach().clone())
    grad = torch.zeros_like(table)
    rows = torch.tensor([3, 7, 7, 20, 41], device=DEV)
    grad.index_add_(0, rows, torch.randn(5, 8, device=DEV))
    st = row_store(table)
    st.acc.copy_(grad)
    st.touched[rows] = True
    LazyRowAdam([table], lr=0.01, betas=(0.9, 0.95), eps=1e-8).step()
    ref.grad = grad
    torch.optim.Adam([ref], lr=0.01, betas=(0.9, 0.95), eps=1e-8, foreach=False).step()
    touched = torch.unique(rows)
    torch.testing.assert_close(table.detach()[touched], ref.detach()[touched], rtol=1e-6, atol=1e-7)
    mask = torch.ones(50, dtype=torch.bool, device=DEV)
    mask[touched] = False
    assert torch.equal(table.detach()[mask], ref.detach()[mask])


def apply_gradient(table, opt, rows, gradient, scale=1.0):
    st = row_store(table)
    st.acc.index_add_(0, rows, gradient)
    st.touched[rows] = True
    st.grad_scale = scale
    opt.step()


def same_bits(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("mode", ["fp32", "bf16", "int8"])
def test_unread_rows_preserve_every_state_tensor(mode):
    note(f"unread rows keep state {mode}")
    g = torch.Generator().manual_seed(71)
    table = torch.nn.Parameter(torch.randn(19, 13, generator=g).to(DEV))
    opt = LazyRowAdam([table], lr=0.01, state_dtype=mode)
    for step, visited in enumerate([list(range(19)), [1, 5, 8], [2, 9], [1, 5, 18]]):
        rows = torch.tensor(visited, device=DEV)
        before = table.detach().clone()
        prev = {k: v.clone() for k, v in opt.state[table].items() if k != "step"} if opt.state[table] else {}
        apply_gradient(table, opt, rows, torch.randn(len(visited), 13, generator=g).to(DEV),
                       torch.tensor(0.25, device=DEV))
        unread = torch.ones(19, dtype=torch.bool, device=DEV)
        unread[rows] = False
        assert same_bits(table.detach()[unread], before[unread])
        for k, v in prev.items():
            assert same_bits(opt.state[table][k][unread], v[unread]), k
        assert int(opt.state[table]["step"]) == step + 1
        assert table.grad is None and not row_store(table).touched.any()
        assert torch.count_nonzero(row_store(table).acc) == 0 and row_store(table).grad_scale == 1.0


@pytest.mark.parametrize("mode", ["fp32", "bf16", "int8"])
def test_empty_step_changes_nothing_but_the_step(mode):
    table = torch.nn.Parameter(torch.ones(7, 11, device=DEV))
    opt = LazyRowAdam([table], lr=0.01, state_dtype=mode)
    opt.step()
    assert int(opt.state[table]["step"]) == 1 and torch.equal(table.detach(), torch.ones(7, 11, device=DEV))
    apply_gradient(table, opt, torch.tensor([3], device=DEV), torch.ones(1, 11, device=DEV))
    before = table.detach().clone()
    prev = {k: v.clone() for k, v in opt.state[table].items() if k != "step"}
    opt.step()
    assert same_bits(before, table.detach())
    for k, v in prev.items():
        assert same_bits(v, opt.state[table][k]), k
    assert int(opt.state[table]["step"]) == 3


@pytest.mark.parametrize("mode,bytes_per_row", [("fp32", 8 * 64), ("bf16", 4 * 64), ("int8", 2 * 64 + 8)])
def test_state_storage_matches_budget(mode, bytes_per_row):
    rows = 300
    table = torch.nn.Parameter(torch.zeros(rows, 64, device=DEV))
    opt = LazyRowAdam([table], lr=0.01, state_dtype=mode)
    apply_gradient(table, opt, torch.tensor([0], device=DEV), torch.zeros(1, 64, device=DEV))
    st = opt.state[table]
    assert sum(v.numel() * v.element_size() for k, v in st.items() if k != "step") == rows * bytes_per_row
    expected = {"fp32": (torch.float32, torch.float32), "bf16": (torch.bfloat16, torch.bfloat16),
                "int8": (torch.int8, torch.uint8)}[mode]
    assert (st["exp_avg"].dtype, st["exp_avg_sq"].dtype) == expected


def test_int8_cancellation_retains_small_positive_variance():
    tables = {m: torch.nn.Parameter(torch.zeros(1, 2, device=DEV)) for m in ("fp32", "int8")}
    opts = {m: LazyRowAdam([t], lr=0.003, state_dtype=m) for m, t in tables.items()}
    for values in ([1000.0, 0.0], [-900.0, 1.0], [0.0, 0.0]):
        for m, t in tables.items():
            apply_gradient(t, opts[m], torch.tensor([0], device=DEV), torch.tensor([values], device=DEV))
    assert opts["int8"].state[tables["int8"]]["exp_avg_sq"][0, 1] > 0
    assert torch.isfinite(tables["int8"]).all()
    torch.testing.assert_close(tables["int8"][:, 1], tables["fp32"][:, 1], rtol=0.05, atol=1e-6)


def test_int8_positive_variance_never_rounds_to_zero():
    table = torch.nn.Parameter(torch.zeros(1, 3, device=DEV))
    opt = LazyRowAdam([table], lr=0.003, state_dtype="int8")
    apply_gradient(table, opt, torch.tensor([0], device=DEV), torch.tensor([[1e6, 1e-6, 0.0]], device=DEV))
    v = opt.state[table]["exp_avg_sq"]
    assert v[0, 0] == 255 and v[0, 1] == 1 and v[0, 2] == 0


def test_eval_path_and_frozen_table():
    """No-grad forwards need no row store; a frozen table keeps its values and gets no accumulator while the
    rest trains; with everything else frozen the table alone trains."""
    note("eval path and frozen table")
    m = tiny("row_sparse").eval()
    x = torch.randint(0, 128, (1, 20), generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.no_grad():
        out = m(x)
    d = tiny("dense").eval()
    d.load_state_dict(m.state_dict())
    with torch.no_grad():
        torch.testing.assert_close(out, d(x), rtol=1e-5, atol=1e-6)
    assert not hasattr(table_of(m), "row_store")
    assert row_sparse_tables(m) == [table_of(m)] and row_sparse_tables(d) == []
    for frozen in ("table", "rest"):
        m = tiny("row_sparse")
        table = table_of(m)
        for p in m.parameters():
            p.requires_grad_((p is not table) if frozen == "table" else (p is table))
        before = {n: p.detach().clone() for n, p in m.named_parameters()}
        trainable = [p for p in m.parameters() if p.requires_grad and p is not table]
        opts = [torch.optim.AdamW(trainable, lr=1e-2)] if trainable else []
        if table.requires_grad:
            opts.append(LazyRowAdam([table], lr=1e-2))
        backward_twice(m)
        OptimizerSet(*opts).step()
        changed = {n for n, p in m.named_parameters() if not torch.equal(p.detach(), before[n])}
        if frozen == "table":
            assert "layers.0.ffn.values.weight" not in changed and not hasattr(table, "row_store")
            assert any("query_proj" in n for n in changed)
        else:
            assert changed == {"layers.0.ffn.values.weight"}
