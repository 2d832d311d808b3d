"""Parity at the BASELINE configurations themselves (the shapes bench.py measures), not scaled-down models.

  c1  the 21M LM (d 384, 6 layers, 6 heads, vocab 32000) with the B-1M memory at layer 3, 512-token prompt, bs 1
  c3  the same LM with the B-16M memory (4096^2 x 384 bf16, 12.9 GB), 128-token prompts, bs 1 and 64
  c2  the B-4M sub-key scoring kernel at its bench shape (16,384 tokens x 4 heads x 2048 sub-keys of 256), and
      one 8 x 2048 prefill forward of the LM with the B-4M memory
  c4  the full 16,777,216 x 384 int8 table (byte offsets past 2^32) read by the gather

Decode (c1, c3): the prompt pass runs with the memory layer recording its selection, then several fused decode
steps record theirs (sub-key scores, selected scores, rows, weights).  Each step's selection must be bit-exact
against the oracle on the step's own scores (oracle/pkm_oracle.py, smlm/kernels.py:128-177), and its logits within
1e-2 of their scale of the reference torch path (oracle/torch_path.py: smlm/model.py:63-118, 156-163, 266-293 in
fp32 on the CPU) run on the same tokens with the same selections -- the KV-cache decode equality of
tests/test_pkm.py:91-119, with the einsum scores taken from the kernel (their bits are not reproducible across
backends).  The whole-step graph then replays the same steps from the same state and must produce the same tokens.
Only the table rows the selections use are pulled to the host (as tests/test_kernels.py:323-360 does for its
large table).
"""
import numpy as np
import pytest
import torch

import oracle.pkm_oracle as O
import oracle.torch_path as TP
import query_check as QC

pytestmark = pytest.mark.gpu
DEV = "cuda"
MEM_LAYER = 3


def note(msg):
    print(msg, flush=True)


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def build_lm(n_keys, max_seq_len, seed=0):
    """The LM of configs 1-3 with every matrix, the sub-keys and the value table drawn from N(0, 0.02), in bf16
    (bench.py builds the same model), and the memory layer's BatchNorm given statistics and affine parameters away
    from the identity (so that its query check can tell the columns apart)."""
    from smlm_hip.model import ModelConfig, Transformer
    cfg = ModelConfig(vocab_size=32000, d_model=384, n_layers=6, n_heads=6, ffn_hidden=1024,
                      max_seq_len=max_seq_len, mem_layers=[MEM_LAYER], mem_n_keys=n_keys, mem_heads=4, mem_knn=32,
                      mem_k_dim=512)
    torch.manual_seed(seed)
    with torch.device(DEV):
        model = Transformer(cfg)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() >= 2 or name.endswith("keys"):
                p.normal_(0.0, 0.02)
    model = model.to(torch.bfloat16).eval()
    QC.randomize_batchnorm(model.layers[MEM_LAYER].ffn.query_norm, seed + 100)
    torch.cuda.empty_cache()
    model.set_memory_inference_table("bf16")
    return model


def compact_rows(table, idx_list):
    """Rows of `table` (device) used by the index tensors of idx_list, as an fp32 host table, and the indices
    remapped into it."""
    allidx = torch.cat([i.reshape(-1) for i in idx_list])
    used, inv = torch.unique(allidx, return_inverse=True)
    sub = table.index_select(0, used).float().cpu()
    out, a = [], 0
    for i in idx_list:
        out.append(inv[a:a + i.numel()].view(i.shape).cpu())
        a += i.numel()
    return sub, out


def host_weights(model):
    return {k: v.float().cpu() for k, v in model.state_dict().items() if not k.endswith("values.weight")}


def check_selection(s1, s2, sc, idx, w, knn):
    rs, ri, rw = O.pk_select(bits(s1), bits(s2), knn)
    assert np.array_equal(idx.cpu().numpy(), ri), "selected rows differ from the oracle"
    assert np.array_equal(bits(sc), rs), "selected scores differ from the oracle"
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=0, atol=1e-6)


@torch.no_grad()
def decode_parity(model, B, P, steps, seed):
    from smlm_hip.model import _StepDecoder
    cfg = model.cfg
    mem = model.layers[MEM_LAYER].ffn
    dec = model._decoder(B, P + steps + 1, DEV)
    assert dec.fused is not None, "the fused decode step must cover the config"
    dec._capture()                               # before the prompt pass: its warm-up steps write cache slots 0, 1
    prompt = torch.randint(0, cfg.vocab_size, (B, P), generator=torch.Generator().manual_seed(seed)).to(DEV)
    mem.record = True
    logits = model(prompt, kv_caches=dec.caches, pos0=0)
    mem.record = False
    sel_prompt = (mem.last_indices.clone(), mem.last_weights.clone())
    first = logits[:, -1].argmax(-1)
    dec.hist[:, :P] = prompt
    dec.hist[:, P] = first
    dec.tok.copy_(first.view(B, 1))
    dec.pos.fill_(P)
    got_logits, toks, sels = [], [], []
    for t in range(steps):
        rec = {}
        toks.append(dec.tok.clone().cpu())
        lg = dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist, logits=True, record=rec)
        r = rec[MEM_LAYER]
        s1, s2, sc, idx, w = r["s1"], r["s2"], r["scores"], r["indices"], r["weights"]
        QC.check_decode_step_query(model, MEM_LAYER, r)
        check_selection(s1, s2, sc, idx, w, cfg.mem_knn)
        got_logits.append(lg.float().cpu())
        sels.append((idx.clone(), w.clone()))
        dec.fused.run(dec.tok, dec.pos, dec.caches, dec.hist)
        assert int(dec.pos) == P + t + 1
    eager = dec.hist[:, P:P + steps + 1].clone()
    note(f"  B={B} P={P}: {steps} fused steps, queries and scores within bounds, selections bit-exact; checking "
         f"logits on the host")

    # the reference torch path on the same tokens with the same selections
    sub, remapped = compact_rows(mem.values.weight, [sel_prompt[0]] + [s[0] for s in sels])
    sd = host_weights(model)
    cd = cfg.to_dict()
    caches = [dict() for _ in range(cfg.n_layers)]
    TP.lm_forward(sd, cd, prompt.cpu(), caches, 0, tables={MEM_LAYER: sub}, last_only=True,
                  selections={MEM_LAYER: (remapped[0], sel_prompt[1].cpu())})
    worst = 0.0
    for t in range(steps):
        ref = TP.lm_forward(sd, cd, toks[t], caches, P + t, tables={MEM_LAYER: sub},
                            selections={MEM_LAYER: (remapped[t + 1], sels[t][1].cpu())})[:, -1]
        err = float((got_logits[t] - ref).abs().max() / ref.abs().max())
        assert err < 1e-2, f"step {t}: logits off by {err:.3e} of their scale"
        worst = max(worst, err)
    note(f"  logits within {worst:.2e} of their scale ({sub.shape[0]} distinct rows pulled)")

    # the whole-step graphs from the same state give the same tokens (runs of 8 steps, then single steps)
    dec.hist[:, P + 1:] = -1
    dec.start(first, P)
    dec.replay(steps)
    torch.cuda.synchronize()
    assert 8 in _StepDecoder.run_lengths
    assert torch.equal(dec.hist[:, P:P + steps + 1], eager), "graph replays differ from the eager steps"


@pytest.mark.parametrize("B", [1, 64])
def test_config3_decode_b16m(B):
    """Config 3: B-16M (16,777,216 x 384 bf16), 128-token prompts, 9 decode steps (a graph run of 8 + 1)."""
    note(f"config 3 decode B={B}: building the LM with the B-16M table")
    model = build_lm(4096, 160)
    decode_parity(model, B, 128, 9, seed=B)
    del model
    torch.cuda.empty_cache()


def test_config1_decode_b1m():
    """Config 1: B-1M (1,048,576 x 384 bf16), a 512-token prompt, batch 1, 9 decode steps."""
    note("config 1 decode: building the LM with the B-1M table")
    model = build_lm(1024, 544)
    decode_parity(model, 1, 512, 9, seed=11)
    del model
    torch.cuda.empty_cache()


# --------------------------------------------------------------------------------------------- config 2
@torch.no_grad()
def test_config2_scoring_and_selection_at_bench_shape():
    """pk_scores at (16,384 tokens, 4 heads, 2048 sub-keys, half 256) -- the launch bench.py times for config 2
    -- within one bf16 ulp of fp64 on 96 sampled tokens (every head, both halves, all 2048 sub-keys), and the
    selection of the full launch bit-exact against the oracle on those tokens' rows."""
    from smlm_hip import kernels as K
    N, H, NK, half = 16384, 4, 2048, 256
    note(f"config 2 scoring N={N} H={H} NK={NK} half={half}")
    g = torch.Generator().manual_seed(21)
    q = torch.randn(N, H, 2 * half, generator=g).to(torch.bfloat16)
    keys = (torch.randn(H, 2, NK, half, generator=g) / 16).to(torch.bfloat16)
    s1, s2 = K.pk_scores(q.to(DEV), keys.to(DEV))
    sc, idx, w = K.pk_select(s1, s2, 32)
    rows = torch.cat([torch.arange(0, 32), torch.arange(N // 2 - 16, N // 2 + 16), torch.arange(N - 32, N)])
    rows = torch.cat([rows, torch.randint(0, N, (32,), generator=g)])
    qs = q[rows].float().numpy()
    kf = keys.float().numpy()
    r1, r2 = O.subkey_scores(qs, kf)
    mag1 = np.einsum("nhd,hkd->nhk", np.abs(qs[..., :half]).astype(np.float64), np.abs(kf[:, 0]).astype(np.float64))
    mag2 = np.einsum("nhd,hkd->nhk", np.abs(qs[..., half:]).astype(np.float64), np.abs(kf[:, 1]).astype(np.float64))
    rd = rows.to(DEV)
    for got, ref, mag in ((s1, r1, mag1), (s2, r2, mag2)):
        gv = got.index_select(0, rd).float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(gv - ref) <= 2 ** -7 * np.abs(ref) + 1e-5 * mag)
    check_selection(s1.index_select(0, rd), s2.index_select(0, rd), sc.index_select(0, rd),
                    idx.index_select(0, rd), w.index_select(0, rd), 32)


@torch.no_grad()
def test_config2_prefill_forward_b4m():
    """Config 2: one forward of the LM with the B-4M memory over 8 x 2048 uniform prompt tokens (no cache).  The
    memory layer's lookup for every token is recorded; on 256 of them its query (from the layer's input through
    query_proj and the BatchNorm) and its sub-key scores are recomputed on the host and the selection is checked
    bit-exact against the oracle; the reference torch path given the selection must give the same logits within
    1e-2 of their scale at 64 positions of every sequence."""
    cfg_keys, B, T = 2048, 8, 2048
    note("config 2 prefill: building the LM with the B-4M table")
    model = build_lm(cfg_keys, T)
    mem = model.layers[MEM_LAYER].ffn
    prompt = torch.randint(0, 32000, (B, T), generator=torch.Generator().manual_seed(31)).to(DEV)
    mem.record = True
    logits = model(prompt)
    mem.record = False
    idx, w = mem.last_indices.clone(), mem.last_weights.clone()
    assert idx.shape == (B * T, 4, 32)
    rows = torch.cat([torch.arange(0, 64), torch.arange(B * T - 64, B * T),
                      torch.randint(0, B * T, (128,), generator=torch.Generator().manual_seed(32))]).to(DEV)
    QC.check_layer_query(mem, rows)
    check_selection(mem.last_lookup["s1"].index_select(0, rows), mem.last_lookup["s2"].index_select(0, rows),
                    mem.last_scores.index_select(0, rows), idx.index_select(0, rows), w.index_select(0, rows), 32)
    mem.last_lookup = None
    note("  prompt-pass query, scores and selection of 256 tokens pinned")
    pos = torch.cat([torch.arange(0, 16), torch.arange(T - 48, T)])
    got = logits[:, pos.to(DEV)].float().cpu()
    del logits
    sub, (ridx,) = compact_rows(mem.values.weight, [idx])
    note(f"  host check over {sub.shape[0]} distinct rows")
    sd = host_weights(model)
    ref = TP.lm_forward(sd, model.cfg.to_dict(), prompt.cpu(), tables={MEM_LAYER: sub},
                        selections={MEM_LAYER: (ridx, w.cpu())}, positions=pos)
    err = float((got - ref).abs().max() / ref.abs().max())
    note(f"  prefill logits within {err:.2e} of their scale")
    assert err < 1e-2, f"prefill logits off by {err:.3e} of their scale"
    del model
    torch.cuda.empty_cache()


@torch.no_grad()
def test_forward_graphed_equals_eager():
    """Transformer.forward_graphed (the prompt pass captured once per shape and replayed) gives the eager forward's
    logits bit for bit: the configs' LM with a small memory table, two prompts of one shape replayed in turn with
    eager forwards between the replays, and a second shape (its own graph)."""
    note("forward_graphed: configs LM, NK 256")
    model = build_lm(256, 512)
    g = torch.Generator().manual_seed(5)
    p1, p2 = (torch.randint(0, 32000, (2, 300), generator=g).to(DEV) for _ in range(2))
    p3 = torch.randint(0, 32000, (3, 100), generator=g).to(DEV)
    e1, e2, e3 = model(p1), model(p2), model(p3)
    for prompt, eager in ((p1, e1), (p2, e2), (p1, e1), (p3, e3), (p2, e2)):
        got = model.forward_graphed(prompt).clone()
        model(p3)                                       # eager work between the replays
        assert np.array_equal(bits(got), bits(eager))
    assert len(model._fwd_graphs) == 2
    model.set_memory_inference_table("bf16")             # a table switch drops the graphs
    assert len(model._fwd_graphs) == 0
    del model
    torch.cuda.empty_cache()


@torch.no_grad()
def test_graphs_follow_parameter_changes():
    """A captured graph reads the tensors and derived copies (cast sub-keys, BatchNorm affine, the concatenated
    query | swilu weights) of its capture.  After the memory layer's BatchNorm statistics and sub-keys are written
    in place, forward_graphed and the whole-step decode graphs must give what the eager forward and eager steps
    give with the new values (they are captured again), on replays with eager work between them."""
    note("graphs after parameter changes: configs LM, NK 256")
    model = build_lm(256, 512)
    mem = model.layers[MEM_LAYER].ffn
    g = torch.Generator().manual_seed(6)
    prompt = torch.randint(0, 32000, (2, 100), generator=g).to(DEV)
    gen_prompt = torch.randint(0, 32000, (2, 20), generator=g).to(DEV)
    before = model.forward_graphed(prompt).clone()
    assert np.array_equal(bits(before), bits(model(prompt)))
    gen_before = model.generate(gen_prompt, 40, use_graph=True)
    assert torch.equal(gen_before, model.generate(gen_prompt, 40, use_graph=False))
    for change in ("batchnorm", "keys"):
        if change == "batchnorm":
            mem.query_norm.running_var.mul_(3.0)
            mem.query_norm.running_mean.add_(0.2)
        else:
            mem.keys.mul_(-1.0)
        for rep in range(2):
            got = model.forward_graphed(prompt).clone()
            eager = model(prompt)
            assert np.array_equal(bits(got), bits(eager)), f"forward_graphed after the {change} change, replay {rep}"
        assert not np.array_equal(bits(got), bits(before)), f"the {change} change must change the logits"
        gen_graph = model.generate(gen_prompt, 40, use_graph=True)
        gen_eager = model.generate(gen_prompt, 40, use_graph=False)
        assert torch.equal(gen_graph, gen_eager), f"decode graphs after the {change} change"
    del model
    torch.cuda.empty_cache()


@torch.no_grad()
def test_lazy_capture_in_replay_keeps_the_prompt_state():
    """replay() on a decoder without graphs captures them first; the capture's warm-up steps write position 0 and
    1 of the KV caches, the token, the position, the history and the argmax keys, and must put them back, so a
    prompt prefilled and started before the first replay decodes as eager steps from the same state do."""
    note("lazy capture in replay: configs LM, NK 256")
    model = build_lm(256, 512)
    B, P, n = 2, 30, 40
    prompt = torch.randint(0, 32000, (B, P), generator=torch.Generator().manual_seed(8)).to(DEV)
    out = []
    for graphs in (False, True):
        model._decoders.clear()
        dec = model._decoder(B, P + n + 1, DEV)
        assert dec.graph is None
        logits = model(prompt, kv_caches=dec.caches, pos0=0)
        dec.hist[:, :P] = prompt
        dec.start(logits[:, -1].argmax(-1), P)
        if graphs:
            dec.replay(n)
            assert dec.graph is not None
        else:
            dec.steps(n)
        out.append(dec.hist[:, P:P + n + 1].clone())
    assert torch.equal(out[0], out[1]), "the lazily captured replay differs from the eager steps"
    del model
    torch.cuda.empty_cache()


# --------------------------------------------------------------------------------------------- config 4
@torch.no_grad()
def test_config4_full_int8_table_gather():
    """Config 4's table at full size: 16,777,216 x 384 int8 codes (6.44 GB) + fp16 row scales, quantised on the
    GPU from N(0, 0.02).  2,048 tokens x 128 lookups: Zipf(1.1) ranks through a seeded row permutation, plus
    forced rows above 11,184,810 (row x 384 past 2^32 bytes) and the last row.  The fp32 output must match the
    oracle's fp64 bag of the same rows within 1e-5 of the output scale, and the quantisation of the pulled rows
    must be bit-exact against the oracle on their bf16-free fp32 sources (regenerated from the same seed)."""
    from smlm_hip import kernels as K
    rows, D, N, Kl = 4096 * 4096, 384, 2048, 128
    note("config 4: quantising the full 16.8M-row int8 table")
    g = torch.Generator(device=DEV).manual_seed(0)
    codes = torch.empty(rows, D, dtype=torch.int8, device=DEV)
    scales = torch.empty(rows, dtype=torch.float16, device=DEV)
    chunk = 1 << 21
    for a in range(0, rows, chunk):
        src = torch.empty(chunk, D, device=DEV).normal_(0.0, 0.02, generator=g)
        c, s = K.quantize_int8(src)
        codes[a:a + chunk] = c
        scales[a:a + chunk] = s
        if a == rows - chunk:                          # the last chunk: keep its fp32 source for the check below
            last_src = src[-4096:].cpu().numpy()
        del src, c, s
    rng = np.random.default_rng(41)
    p = 1.0 / np.arange(1, rows + 1, dtype=np.float64) ** 1.1
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    ranks = np.minimum(np.searchsorted(cdf, rng.random((N, Kl))), rows - 1)
    idx = rng.permutation(rows)[ranks]
    idx[:, 0] = rows - 1
    idx[:, 1] = rng.integers(11_184_811, rows, N)
    idx[:, 2] = rng.integers(rows - 4096, rows, N)
    assert (idx.astype(np.int64) * D >= 2 ** 32).mean() > 0.3
    w = np.concatenate([O.softmax_f32(rng.standard_normal((N, 32)).astype(np.float32)) for _ in range(4)], 1)
    ti = torch.from_numpy(idx).to(DEV)
    out = K.bag_infer(ti, torch.from_numpy(w).to(DEV), codes, scales).cpu().numpy()
    used = np.unique(idx)
    ud = torch.from_numpy(used).to(DEV)
    sub_codes = codes.index_select(0, ud).cpu().numpy()
    sub_scales = scales.index_select(0, ud).cpu().numpy()
    ref = O.bag(np.searchsorted(used, idx), w, sub_codes, "i8", sub_scales)
    err = np.abs(out - ref).max() / np.abs(ref).max()
    note(f"  {used.size} distinct rows, max row {used.max()}, error {err:.2e} of the output scale")
    assert err <= 1e-5, f"int8 gather off by {err:.3e} of the output scale"
    rc, rs = O.quantize_rows(last_src, "i8")
    assert np.array_equal(codes[-4096:].cpu().numpy(), rc)
    assert np.array_equal(scales[-4096:].cpu().numpy().view(np.uint16), rs.view(np.uint16))
    del codes, scales
    torch.cuda.empty_cache()
