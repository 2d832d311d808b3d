"""Benchmark of the product-key-memory lookup on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--phases ...]

Prints ONE JSON line, whatever a phase raises (a failed phase is recorded under "phase_errors").  Metric
"decode tok/s (B-16M, bs1/bs64); PKM lookup tok/s + value-gather HBM GB/s".  Phases, in the
order they run (the headline ones first):
  decode         value: config 3 decode tok/s at batch 64 -- the 21M LM (d=384, 6 layers, vocab 32000) with the
                 B-16M memory (4096^2 = 16,777,216 x 384 bf16 values, 12.9 GB) replacing layer 3's FFN,
                 128-token prompts (prefilled once, untimed), then 256 greedy tokens.  A step is one such
                 256-token generation (8 replays of the captured 32-step whole-step HIP graph); W untimed and K
                 timed generations, each bracketed by synchronisations (the loop of smlm/train.py:283-301).
                 value = 64 * 256 * K / time.  The same at batch 1, and each token step against its floors
                 (decode_roofline: HBM bytes / 8 TB/s; kernel count x the chained-launch time).
  gather         config 4: int8 row-quantised B-16M table, 65,536 tokens x 128 Zipf(1.1) lookups, fp32 out
                 (3,439,329,280 algorithmic bytes per call), and the uniform-index control of the same shapes.
                 roofline: the control's algorithmic GB/s (= its physical traffic: no row repeats in cache) over
                 HBM peak, from HIP events on the launch stream; roofline.zipf: the Zipf call's algorithmic rate
                 and its physical rate from the committed rocprofv3 counters (profiles/gather_config4_pmc.txt, used
                 only while it names the sha256 of the gather's present sources).  The box's own ceilings beside
                 them (csrc/bench/ceiling.hip): sequential read / write / copy and random 384-byte row reads.
  cpu            cpu_baseline: the reference's torch path (oracle/torch_path.py) on the host cores, config 3 at
                 batch 64 (and 1), a bounded sample of the 256 steps; config 4 on the host (chunked int8 gather and
                 dequantise + embedding_bag) over 2,048 tokens; config 2 over one 2048-token prompt.
  config1        config 1: the LM with the B-1M memory (1024^2 rows), 512-token prompt, 256 greedy tokens, bs 1.
  config0        config 0: the B-1M PKM layer forward alone in fp32 over 8 x 256 tokens, GPU and host CPU.
  prefill        config 2: the LM with the B-4M memory (2048^2 rows) forward over 8 x 2048 prompt tokens (no
                 cache), tokens / median forward time; the prompt-pass attention kernel alone at that shape.
  lookup         config 2 PKM lookup (B-4M, 8 x 2048 tokens): scoring, then selection + bag as one launch (and
                 the selection and the bag as separate launches);
                 roofline_score: the scoring against the bf16 MFMA peak.
  offload        config 3 decode with the B-16M table as q4 in HBM, q4 / bf16 in pinned host RAM (zero-copy,
                 graphs), and bs1 from a q4 file through mmap (staged, no graphs).
  train          the training side at the reference's training shape (4,096 tokens x 128 lookups, B-1M fp32).
  engram         the Engram n-gram hash, row gather and row-sparse backward over 8 x 2048 tokens x 16 lookups.
All inputs are seeded synthetic data; weights are random N(0, 0.02).
"""
import argparse
import json
import os
import sys
import tempfile
import time
import traceback

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "sparse-memory-lm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def lm_config(n_keys, max_seq_len):
    from smlm_hip.model import ModelConfig
    return ModelConfig(vocab_size=32000, d_model=384, n_layers=6, n_heads=6, ffn_hidden=1024,
                       max_seq_len=max_seq_len, mem_layers=[3], mem_n_keys=n_keys, mem_heads=4, mem_knn=32,
                       mem_k_dim=512)


def build_lm(cfg, dev, seed=0):
    """The LM with every weight matrix, the sub-keys and the value table drawn from N(0, 0.02), in bf16 on the
    GPU (norm weights 1, BatchNorm at its initial statistics)."""
    import torch
    from smlm_hip.model import Transformer
    torch.manual_seed(seed)
    with torch.device(dev):
        model = Transformer(cfg)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() >= 2 or name.endswith("keys"):
                p.normal_(0.0, 0.02)
    model = model.to(torch.bfloat16).eval()
    torch.cuda.empty_cache()
    model.set_memory_inference_table("bf16")
    return model


GEN_TOKENS = 256          # new tokens per generation in configs 1 and 3


def time_generations(model, B, reps, warmup, dev, prompt_len=128, new_tokens=GEN_TOKENS, seed=1):
    """The decode loop of smlm/train.py:283-301 at batch B: prefill B uniform prompts of prompt_len tokens once
    (untimed), then `warmup` untimed and `reps` timed generations of `new_tokens` greedy tokens each, every one
    starting from the prompt's first sampled token and bracketed by synchronisations.  A generation is
    new_tokens / 32 replays of the captured 32-step graph (_StepDecoder.run_lengths; each step reads and advances its
    position and token on the device).  Greedy decoding is deterministic, so every repetition must produce the
    same tokens; that is checked.  Returns (tok/s, ms per generation, ms per token step)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    P = prompt_len
    prompt = torch.randint(0, model.cfg.vocab_size, (B, P), generator=g, device=dev)
    with torch.no_grad():
        dec = model._decoder(B, P + new_tokens + 1, dev)
        dec._capture()
        logits = model(prompt, kv_caches=dec.caches, pos0=0)
        first = logits[:, -1].argmax(-1)
        dec.hist[:, :P] = prompt

        def start():
            dec.start(first, P)

        for _ in range(warmup):
            start()
            dec.replay(new_tokens)
        torch.cuda.synchronize(dev)
        ref = dec.hist[:, P:P + new_tokens + 1].clone()
        total = 0.0
        for _ in range(reps):
            start()
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            dec.replay(new_tokens)
            torch.cuda.synchronize(dev)
            total += time.perf_counter() - t0
        if warmup and not torch.equal(ref, dec.hist[:, P:P + new_tokens + 1]):
            raise RuntimeError("greedy generations differ between repetitions")
    ms_gen = 1000.0 * total / reps
    return B * new_tokens * reps / total, ms_gen, ms_gen / new_tokens


def chained_launch_us(dev, numel=384, kernels=264, replays=40):
    """Device time per kernel of a HIP graph of `kernels` back-to-back elementwise kernels, each reading the `numel`
    fp32 values its predecessor wrote (in-place adds): 384 values are one workgroup, the floor every kernel of a
    captured decode step pays whatever its work; 262,144 values spread one kernel over the whole chip.
    264 = 8 decode steps of 33 kernels (the graph length does not change the per-kernel floor)."""
    import torch
    x = torch.zeros(numel, dtype=torch.float32, device=dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(3):
            x.add_(1.0)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(kernels):
            x.add_(1.0)
    return 1000.0 * event_time_ms(graph.replay, replays) / kernels


def decode_roofline(model, B, ms_per_step, mean_pos, launch_us, wide_launch_us):
    """The two floors of one fused decode step against its measured time.
    HBM: the bytes a step must move — every weight matrix once (the tied embedding once as lm_head, plus B embedding
    rows), every memory layer's sub-keys, the B x heads x knn value rows (bf16 table), the K and V cache rows of
    positions 0..pos-1 read and row pos written per layer — over 8 TB/s.
    Launch: the step's kernel count (5 per dense block, 7 per memory block, 1 for the head — the token is picked in
    the next step's first launch; one fewer per block where the attention launch does wo as well) x the
    one-workgroup chained-kernel time of chained_launch_us."""
    from smlm_hip.model import _FusedDecodeStep
    cfg = model.cfg
    C = cfg.d_model
    w = 0
    for name, p in model.named_parameters():
        if name.endswith("values.weight"):
            continue
        w += p.numel() * p.element_size()
    w += B * C * 2                                                      # embedding rows of the step's tokens
    n_mem = len(cfg.mem_layers)
    values = n_mem * B * cfg.mem_heads * cfg.mem_knn * C * 2
    kv = cfg.n_layers * 2 * B * (mean_pos + 1) * C * 2                  # read rows < pos, write row pos
    total = w + values + kv
    hbm_ms = total / (HBM_PEAK_GBS * 1e9) * 1e3
    fold = B <= _FusedDecodeStep.proj_max_batch and cfg.n_heads <= 8
    launches = (4 if fold else 5) * (cfg.n_layers - n_mem) + (6 if fold else 7) * n_mem + 1
    launch_ms = launches * launch_us / 1e3
    return {"bound": "launch" if launch_ms >= hbm_ms else "hbm", "ms_per_step": ms_per_step,
            "hbm_bytes_per_step": total, "weight_bytes": w, "value_row_bytes": values, "kv_cache_bytes": kv,
            "mean_position": mean_pos, "hbm_floor_ms": hbm_ms, "hbm_frac": hbm_ms / ms_per_step,
            "launches_per_step": launches, "chained_launch_us": launch_us,
            "chained_launch_us_chip_wide": wide_launch_us, "launch_floor_ms": launch_ms,
            "launch_frac": launch_ms / ms_per_step}


def time_prefill(model, B, T, reps, dev, seed=3, graphed=False):
    """Config 2 prefill: the LM forward (no cache) over B uniform prompts of T tokens; median wall time of `reps`
    forwards after 2 warm-ups, each synchronised.  graphed: Transformer.forward_graphed (the same kernels, the
    pass captured once and replayed; the capture happens in the warm-ups)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    prompt = torch.randint(0, model.cfg.vocab_size, (B, T), generator=g, device=dev)
    fwd = model.forward_graphed if graphed else model
    times = []
    with torch.no_grad():
        for i in range(2 + reps):
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            fwd(prompt)
            torch.cuda.synchronize(dev)
            if i >= 2:
                times.append(time.perf_counter() - t0)
    if graphed:
        model.drop_graphs()
    times.sort()
    ms = 1000.0 * times[len(times) // 2]
    return B * T / ms * 1e3, ms


def event_time_ms(fn, reps, warm=3):
    """Average device time of fn() in ms, from HIP events recorded on torch's current stream (the stream the
    kernels are launched on)."""
    import torch
    for _ in range(warm):
        fn()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def zipf_rows(n, rows, s, g, dev):
    """n draws of Zipf(s) ranks over [0, rows) by inverse CDF, mapped through a seeded row permutation."""
    import torch
    cdf = torch.cumsum(torch.arange(1, rows + 1, device=dev, dtype=torch.float64).pow_(-s), 0)
    cdf /= cdf[-1].clone()
    u = torch.rand(n, generator=g, device=dev, dtype=torch.float64)
    ranks = torch.searchsorted(cdf, u).clamp_(max=rows - 1)
    del cdf, u
    perm = torch.randperm(rows, generator=g, device=dev)
    return perm[ranks]


def prefill_attention_kernel(dev, reps):
    """The prompt-pass attention kernel alone at the config-2 shape (8 x 2048 tokens, 6 heads of 64): causal flops
    (q k^T and p v over the T (T + 1) / 2 visible pairs) / HIP-event time against the bf16 MFMA peak."""
    import torch
    from smlm_hip import kernels as K
    B, H, T, hd = 8, 6, 2048, 64
    g = torch.Generator(device=dev).manual_seed(4)
    q, k, v = (torch.randn(B, H, T, hd, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    out = torch.empty(B, T, H, hd, dtype=torch.bfloat16, device=dev)
    ms = event_time_ms(lambda: K.prefill_attention(q, k, v, out=out), reps)
    flops = 4.0 * B * H * hd * T * (T + 1) / 2
    del q, k, v, out
    return {"shape": f"B={B} H={H} T={T} head_dim={hd}, causal", "ms": ms, "TFLOPs": flops / ms / 1e9,
            "mfma_frac": flops / ms / 1e9 / BF16_MFMA_PEAK_TFLOPS}


def gather_stress(dev, reps, cpu_tokens=0):
    """Config 4: int8 B-16M table (per-row fp16 scales), 65,536 x 128 Zipf(1.1) lookups, fp32 out; plus the
    uniform-index control (same shapes, physical traffic = algorithmic).  With cpu_tokens, the host-CPU forms of
    cpu_gather_c4 over that many of the Zipf tokens."""
    import torch
    from smlm_hip import kernels as K
    rows, D, N, Kl = 4096 * 4096, 384, 65536, 128
    g = torch.Generator(device=dev).manual_seed(0)
    codes = torch.empty(rows, D, dtype=torch.int8, device=dev)
    scales = torch.empty(rows, dtype=torch.float16, device=dev)
    chunk = 1 << 21
    for a in range(0, rows, chunk):
        src = torch.empty(min(chunk, rows - a), D, device=dev).normal_(0.0, 0.02, generator=g)
        c, s = K.quantize_int8(src)
        codes[a:a + len(src)] = c
        scales[a:a + len(src)] = s
        del src, c, s
    idx = zipf_rows(N * Kl, rows, 1.1, g, dev).view(N, Kl)
    w = torch.softmax(torch.randn(N, 4, 32, generator=g, device=dev), -1).view(N, Kl)
    uni = torch.randint(0, rows, (N, Kl), generator=g, device=dev)
    alg_bytes = N * Kl * (D + 2 + 8 + 4) + N * D * 4          # 3,439,329,280
    ms_zipf = event_time_ms(lambda: K.bag_infer(idx, w, codes, scales), reps)
    ms_uni = event_time_ms(lambda: K.bag_infer(uni, w, codes, scales), reps)
    out = None
    res = {"tokens": N, "lookups_per_token": Kl, "table": "16,777,216 x 384 int8 + fp16 row scales",
           "alg_bytes_per_call": alg_bytes, "ms_zipf": ms_zipf, "ms_uniform": ms_uni,
           "alg_GBps_zipf": alg_bytes / ms_zipf / 1e6, "alg_GBps_uniform": alg_bytes / ms_uni / 1e6}
    res["ceilings"] = memory_ceilings(dev, max(5, reps // 2), codes, codes, uni)
    log(f"memory ceilings: " + ", ".join(f"{k} {v['GBps']:.0f} GB/s" for k, v in res["ceilings"].items()))
    if cpu_tokens:
        out = K.bag_infer(idx, w, codes, scales)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        res["cpu"] = cpu_gather_c4(codes, scales, idx, w, out, cpu_tokens)
        log(f"gather config 4 on the host: {res['cpu']} ({time.perf_counter() - t0:.1f} s)")
    del codes, scales, idx, w, uni, out
    torch.cuda.empty_cache()
    return res


def _bench_lib():
    import ctypes
    from smlm_hip import build as hip_build
    lib = ctypes.CDLL(hip_build.BENCH_LIB_PATH)
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.smlm_bench_stream.argtypes = [ci, vp, vp, i64, ci, vp, vp]
    lib.smlm_bench_random_rows.argtypes = [vp, i64, vp, i64, ci, ci, vp, vp]
    return lib


def memory_ceilings(dev, reps, read_buf, rows_table, rows_idx):
    """The box's own memory ceilings, from kernels that only move bytes (csrc/bench/ceiling.hip):
      read / write / copy  sequential 16-byte accesses over buffers far larger than the 256 MB of caches: read over
                           `read_buf` (the config-4 int8 table, 6.44 GB), write and copy over 2 GiB buffers; best of
                           four grid sizes; GB/s = bytes read + written / HIP-event time;
      random rows          whole rows of `rows_table` at the indices `rows_idx` (the uniform-index control of config
                           4: 8,388,608 lookups of 384-byte int8 rows), no arithmetic, no output; best of the launch
                           shapes (row slots per workgroup x rows in flight per thread); GB/s counts the row bytes
                           and the 8-byte indices."""
    import ctypes
    import torch
    lib = _bench_lib()
    vp = ctypes.c_void_p
    sink = torch.zeros(4, dtype=torch.int32, device=dev)

    def stream():
        return vp(torch.cuda.current_stream(dev).cuda_stream)

    def run_stream(op, src, dst, nbytes, grid):
        rc = lib.smlm_bench_stream(op, vp(src), vp(dst), nbytes, grid, vp(sink.data_ptr()), stream())
        if rc != 0:
            raise RuntimeError(f"smlm_bench_stream({op}): {rc}")

    out = {}
    read_bytes = read_buf.numel() * read_buf.element_size() // (1 << 20) * (1 << 20)
    big = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    big2 = torch.empty_like(big)
    for op, name, src, dst, nbytes, moved in (
            (0, "read", read_buf.data_ptr(), 0, read_bytes, read_bytes),
            (1, "write", 0, big.data_ptr(), big.numel(), big.numel()),
            (2, "copy", big.data_ptr(), big2.data_ptr(), big.numel(), 2 * big.numel())):
        best = None
        for grid in (1024, 2048, 4096, 8192):
            ms = event_time_ms(lambda: run_stream(op, src, dst, nbytes, grid), reps)
            if best is None or ms < best[0]:
                best = (ms, grid)
        out[name] = {"bytes": moved, "ms": best[0], "grid": best[1], "GBps": moved / best[0] / 1e6}
    del big, big2
    n = rows_idx.numel()
    rows, row_bytes = rows_table.shape[0], rows_table.shape[1] * rows_table.element_size()
    shapes = {}
    for sh in range(lib.smlm_bench_random_row_shapes()):
        code = lib.smlm_bench_random_row_shape(sh)

        def run(sh=sh):
            rc = lib.smlm_bench_random_rows(vp(rows_idx.data_ptr()), n, vp(rows_table.data_ptr()), rows, row_bytes,
                                            sh, vp(sink.data_ptr()), stream())
            if rc != 0:
                raise RuntimeError(f"smlm_bench_random_rows(shape {sh}): {rc}")
        ms = event_time_ms(run, reps)
        shapes[f"slots{code // 1000}_rows{code % 1000}"] = {"ms": ms, "GBps": n * (row_bytes + 8) / ms / 1e6}
    best = min(shapes, key=lambda k: shapes[k]["ms"])
    out["random_rows"] = {"lookups": n, "row_bytes": row_bytes, "bytes": n * (row_bytes + 8),
                          "best_shape": best, "ms": shapes[best]["ms"], "GBps": shapes[best]["GBps"],
                          "shapes": shapes}
    if int(sink.abs().sum()):
        raise RuntimeError("ceiling kernels: the never-taken store was taken")
    return out


def cpu_lookup_c2(q, keys, table, pre, idx_gpu, tokens, reps=3):
    """Config 2's lookup on the host cores over its first `tokens` tokens (all 16,384 by default, in chunks of
    2,048): the reference's torch path from the query
    on (smlm/pkm.py:117-148, 205-223: the two sub-key einsums, topk per half, top-k over the knn^2 Cartesian sums,
    softmax, the weighted bag of the bf16 rows, times silu of the swilu input), in fp32 on the same query, sub-keys
    and bf16 table (oracle/torch_path.py's functions); median of `reps` timed runs after one untimed.  The selected
    rows are compared with the GPU's (the fp32 einsum and the kernels' bf16 scores may order near-ties
    differently)."""
    import torch
    import torch.nn.functional as F
    import oracle.torch_path as TP
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    t0 = time.perf_counter()
    qh = q[:tokens].float().cpu()
    kh = keys.float().cpu()
    th = table.cpu()
    ph = pre[:tokens].float().cpu()
    copy_s = time.perf_counter() - t0
    N, H, kd = qh.shape
    half = kd // 2

    def run(chunk=2048):                 # token chunks bound the gathered rows' host memory
        outs, idxs = [], []
        for a in range(0, N, chunk):
            qc = qh[a:a + chunk]
            n = qc.shape[0]
            s1 = torch.einsum("nhd,hkd->nhk", qc[..., :half], kh[:, 0])
            s2 = torch.einsum("nhd,hkd->nhk", qc[..., half:], kh[:, 1])
            sc, idx = TP.pkm_select_torch(s1, s2, 32)
            w = torch.softmax(sc, -1)
            rows = F.embedding(idx.view(n, -1), th).float()
            out = torch.einsum("nj,njd->nd", w.view(n, -1), rows)
            outs.append((out * F.silu(ph[a:a + chunk])).to(torch.bfloat16))
            idxs.append(idx)
        return torch.cat(outs), torch.cat(idxs)

    with torch.no_grad():
        run()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            _, idx = run()
            ts.append(time.perf_counter() - t)
        # the check (untimed): the bf16 model's scores are the einsums rounded to bf16, as the kernels round them
        b1 = torch.einsum("nhd,hkd->nhk", qh[..., :half], kh[:, 0]).bfloat16().float()
        b2 = torch.einsum("nhd,hkd->nhk", qh[..., half:], kh[:, 1]).bfloat16().float()
        bsc, bidx = TP.pkm_select_torch(b1, b2, 32)
        g = idx_gpu[:tokens].cpu()
        NK = b1.shape[-1]
        # the bf16 model's candidate rule (smlm/kernels.py:200-211, the kernels' rule): the (i+1)(j+1) <= knn pairs of
        # the two halves' top 32, each scored bf16(v1 + v2); the top-32 VALUES of that are tie-independent
        a1, a2 = b1.topk(32, -1).values, b2.topk(32, -1).values
        r = torch.arange(32)
        keep = ((r[:, None] + 1) * (r[None, :] + 1) <= 32).reshape(-1)
        cand = (a1.unsqueeze(-1) + a2.unsqueeze(-2)).bfloat16().float().flatten(-2)[..., keep]
        bsc = cand.topk(32, -1).values
        gsc = (b1.gather(-1, g // NK) + b2.gather(-1, g % NK)).bfloat16().float()   # the GPU selection, same rule
    ts.sort()
    dt = ts[len(ts) // 2]
    same = float((bidx.sort(-1).values == g.sort(-1).values).all(-1).double().mean())
    same_scores = float((bsc.sort(-1).values == gsc.sort(-1).values).all(-1).double().mean())
    return {"value": tokens / dt, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{tokens} of the 16,384 tokens: query -> scores -> selection -> softmax -> bag "
                      f"(x silu) in fp32 on the bf16 table, median of {reps} ({dt:.3f} s each; host copies "
                      f"{copy_s:.1f} s untimed), reference torch path restated in oracle/torch_path.py",
            "rows_with_the_gpu_selection_frac": same,
            "rows_with_the_gpu_top_scores_frac": same_scores,
            "rows_check": "per (token, head) row, on the bf16-rounded einsum scores: rows_with_the_gpu_selection_frac "
                          "= the torch path's top-32 index set (fp32 candidate sums) equals the GPU's; "
                          "rows_with_the_gpu_top_scores_frac = the GPU's 32 rows have the same multiset of bf16(v1 + "
                          "v2) scores as the top 32 of the pruned candidates by that rule (the bf16 model's; "
                          "independent of how ties are broken, which torch.topk does arbitrarily and the kernels by "
                          "index)"}


def lookup_prefill(dev, reps, cpu_tokens=0):
    """Config 2 PKM lookup: 8 x 2048 tokens, 4 heads x 2 halves x 2048 sub-keys of 256, top-32, 4M x 384 bf16
    table; the scoring, the selection and the bag kernels timed separately with HIP events, and the fused
    selection + bag launch the memory layer runs (pk_select_bag): tok_s = tokens / (scoring + fused launch).  With cpu_tokens, the torch path
    on the host cores over that many of the tokens (cpu_lookup_c2)."""
    import torch
    from smlm_hip import kernels as K
    N, H, kd, NK, D = 8 * 2048, 4, 512, 2048, 384
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(N, H, kd, generator=g, device=dev).to(torch.bfloat16)
    keys = (torch.randn(H, 2, NK, kd // 2, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    table = torch.empty(NK * NK, D, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=g)
    pre = torch.randn(N, D, generator=g, device=dev).to(torch.bfloat16)
    s1, s2 = K.pk_scores(q, keys)
    sc, idx, w = K.pk_select(s1, s2, 32)
    ms_score = event_time_ms(lambda: K.pk_scores(q, keys), reps)
    ms_select = event_time_ms(lambda: K.pk_select(s1, s2, 32), reps)
    ms_bag = event_time_ms(lambda: K.bag_infer(idx.view(N, -1), w.view(N, -1), table, pre=pre, out_bf16=True),
                           reps)
    ms_select_bag = event_time_ms(lambda: K.pk_select_bag(s1, s2, 32, table, None, pre=pre, out_bf16=True), reps)
    flops = 2.0 * N * H * 2 * NK * (kd // 2)
    total = ms_score + ms_select_bag
    res = {"tokens": N, "ms_score": ms_score, "ms_select": ms_select, "ms_bag": ms_bag,
           "ms_select_bag": ms_select_bag, "tok_s": N / total * 1e3,
           "tok_s_separate_launches": N / (ms_score + ms_select + ms_bag) * 1e3, "score_TFLOPs": flops / ms_score / 1e9,
           "score_write_GBps": 2 * N * H * NK * 2 / ms_score / 1e6,
           "bag_alg_GBps": N * 128 * (2 * D + 12) / ms_bag / 1e6}
    if cpu_tokens:
        res["cpu_baseline"] = cpu_lookup_c2(q, keys, table, pre, idx, cpu_tokens)
        log(f"cpu baseline config 2 lookup: {res['cpu_baseline']}")
    del q, keys, table, pre, s1, s2, sc, idx, w
    torch.cuda.empty_cache()
    return res


def time_decode_eager(model, B, steps, dev, seed=1, prompt_len=128):
    """Decode steps run one by one without graphs (tables that stage every call synchronise inside the step)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    P = prompt_len
    prompt = torch.randint(0, model.cfg.vocab_size, (B, P), generator=g, device=dev)
    with torch.no_grad():
        dec = model._decoder(B, P + steps + 3, dev)
        logits = model(prompt, kv_caches=dec.caches, pos0=0)
        dec.hist[:, :P] = prompt
        dec.start(logits[:, -1].argmax(-1), P)
        dec.steps(2)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        dec.steps(steps)
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0
    return B * steps / dt, 1000.0 * dt / steps


def offload_tiers(model, dev, reps, staged_steps=32):
    """Config 3 (B-16M) decode with the value table in each tier of smlm_hip.offload: q4 in HBM, q4 and bf16 in
    pinned host RAM read by the kernels over the host link (zero-copy, whole-step graphs), and bs1 from a q4 file
    through mmap (staged: one synchronisation and host fetch per memory-layer call, no graphs); plus the
    zero-copy q4 gather's host-link bandwidth (4,096 tokens x 128 uniform lookups)."""
    import tempfile
    import torch
    from smlm_hip import kernels as K
    from smlm_hip.offload import HostTable, MmapQ4Table
    mem = model.memory_layers()
    bf16_table = mem[0].values.infer_table
    res = {}

    def use(table, name, graphs=True):
        for m in mem:
            m.values.infer_table = table
            m._graph = None
        model._decoders.clear()
        for B in (1, 64):
            if not graphs and B > 1:
                continue
            if graphs:
                tok_s, _, ms = time_generations(model, B, 1, 1, dev)
            else:
                tok_s, ms = time_decode_eager(model, B, staged_steps, dev)
            res[f"{name}_bs{B}"] = {"tok_s": tok_s, "ms_per_step": ms}
            log(f"offload {name} bs{B}: {tok_s:.1f} tok/s ({ms:.3f} ms/step)")

    codes, scales = K.quantize_q4(mem[0].values.weight.detach())
    use((codes, scales), "q4_hbm")
    t0 = time.perf_counter()
    host_q4 = HostTable(codes.cpu(), scales.cpu())
    res["q4_host_pin_s"] = time.perf_counter() - t0
    use(host_q4, "q4_host_zero_copy")
    g = torch.Generator(device=dev).manual_seed(9)
    N, Kl = 4096, 128
    idx = torch.randint(0, codes.shape[0], (N, Kl), generator=g, device=dev)
    w = torch.softmax(torch.randn(N, Kl, generator=g, device=dev), -1)
    ms = event_time_ms(lambda: K.bag_infer(idx, w, host_q4.table, host_q4.scales), reps)
    alg = N * Kl * (codes.shape[1] + 2)
    res["q4_host_gather"] = {"tokens": N, "lookups_per_token": Kl, "ms": ms, "row_bytes_GBps": alg / ms / 1e6}
    log(f"offload zero-copy q4 gather: {res['q4_host_gather']}")
    del idx, w
    with tempfile.TemporaryDirectory() as d:
        codes.cpu().numpy().tofile(os.path.join(d, "values_q4.bin"))
        scales.cpu().numpy().tofile(os.path.join(d, "scales_q4.bin"))
        rows, D = codes.shape[0], codes.shape[1] * 2
        mm = MmapQ4Table(os.path.join(d, "values_q4.bin"), os.path.join(d, "scales_q4.bin"), rows, D)
        use(mm, "q4_mmap_staged", graphs=False)
        res["q4_mmap_staged_stats"] = dict(mm.stats)
        mm.close()
    del host_q4
    t0 = time.perf_counter()
    host_bf16 = HostTable(bf16_table[0].cpu())
    res["bf16_host_pin_s"] = time.perf_counter() - t0
    use(host_bf16, "bf16_host_zero_copy")
    del host_bf16
    for m in mem:
        m.values.infer_table = bf16_table
        m._graph = None
    model._decoders.clear()
    del codes, scales
    torch.cuda.empty_cache()
    return res


def engram_cpu_baseline(ng, c, res):
    """The reference's path of the Engram lookup on the host cores over the whole workload: the n-gram hash
    (oracle/engram_oracle.ngram_rows, the int64 arithmetic of smlm/engram.py:60-73), the fp32 row gather (index_select
    into the 16 x 524,287 x 24 table) and the row-sparse backward with unit weights (oracle/torch_path.bag_backward_rows,
    the torch branch of smlm/sparse_values.py:66-104 at K = 1).  Medians of 3, each beside the GPU's time."""
    import torch
    import oracle.engram_oracle as EO
    import oracle.torch_path as TP
    cc, mult = c.cpu().numpy(), ng.mult.cpu().numpy()
    g = torch.Generator().manual_seed(11)
    table = torch.randn(ng.n_lookups * ng.rows, 24, generator=g) * 0.2
    acc = torch.zeros_like(table)
    touched = torch.zeros(table.shape[0], dtype=torch.bool)

    def median_s(fn):
        t = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return sorted(t)[1]

    rows = torch.from_numpy(EO.ngram_rows(cc, mult, ng.orders, ng.heads, ng.rows)).reshape(-1)
    M = rows.numel()
    grad = torch.randn(M, 24, generator=g)
    ones = torch.ones(M, 1)
    t_hash = median_s(lambda: EO.ngram_rows(cc, mult, ng.orders, ng.heads, ng.rows))
    t_gather = median_s(lambda: table.index_select(0, rows))
    t_back = median_s(lambda: TP.bag_backward_rows(grad, rows.view(-1, 1), ones, table, acc, touched))
    out = {}
    for name, t, gpu_ms in (("hash", t_hash, res["ms_hash"]), ("gather_fp32", t_gather, res["gather_fp32"]["ms"]),
                            ("backward_fp32", t_back, res["backward_fp32"]["ms"])):
        out[name] = {"value": M / t, "unit": "lookups/s", "cores": torch.get_num_threads(), "kind": "port",
                     "gpu_value": M / gpu_ms * 1e3, "sample": f"the whole workload, {M:,} lookups ({t * 1e3:.2f} ms; "
                                                            f"the GPU {gpu_ms:.4f} ms)"}
    return out


def engram_lookup(dev, reps, cpu=False):
    """The Engram row lookup at the reference's default shape (orders 2 and 3, 8 heads each = 16 lookups per token,
    524,287 rows per head, head_dim 24) over 8 x 2048 tokens: the hash kernel, the row gather (fp32 and bf16
    tables) and the row-sparse backward (weight 1 per lookup) into an fp32 accumulator."""
    import torch
    from smlm_hip import kernels as K
    from smlm_hip.engram import NgramHash
    B, T, vocab = 8, 2048, 50304
    ng = NgramHash(vocab, (2, 3), 8, 524287, seed=0, canon=torch.arange(vocab)).to(dev)
    g = torch.Generator(device=dev).manual_seed(11)
    c = torch.randint(0, ng.pad, (B, ng.history + T), generator=g, device=dev)
    rows = ng(c)
    M = rows.numel()
    res = {"tokens": B * T, "lookups_per_token": ng.n_lookups, "ms_hash": event_time_ms(lambda: ng(c), reps)}
    res["hash_alg_GBps"] = (B * (ng.history + T) * 8 + M * 8) / res["ms_hash"] / 1e6
    for dt, name in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        table = (torch.randn(ng.n_lookups * ng.rows, 24, generator=g, device=dev) * 0.2).to(dt)
        ms = event_time_ms(lambda: K.row_gather(rows, table), reps)
        alg = M * (8 + 2 * 24 * table.element_size())
        res[f"gather_{name}"] = {"ms": ms, "alg_GBps": alg / ms / 1e6}
        if dt == torch.float32:
            acc = torch.zeros_like(table)
            touched = torch.zeros(table.shape[0], dtype=torch.bool, device=dev)
            grad = torch.randn(M, 24, generator=g, device=dev)
            flat, ones = rows.reshape(-1, 1), torch.ones(M, 1, device=dev)
            # the form EngramMemory's backward uses: unit weights, no weight gradient, no table read
            ms_b = event_time_ms(lambda: K.bag_backward_rows(grad, flat, None, table, acc, touched, ordered=False,
                                                             weight_grad=False), reps)
            # the general atomic bag backward on the same lookups (weights of 1 read, weight gradient computed)
            ms_w = event_time_ms(lambda: K.bag_backward_rows(grad, flat, ones, table, acc, touched, ordered=False),
                                 reps)
            distinct = int(torch.unique(flat).numel())
            alg_b = M * 8 + M * 24 * 4 + distinct * (2 * 24 * 4 + 1)
            res["backward_fp32"] = {"ms": ms_b, "distinct_rows": distinct, "alg_bytes": alg_b,
                                    "alg_GBps": alg_b / ms_b / 1e6, "ms_with_weight_grad": ms_w}
            del acc, touched, grad
        del table
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = engram_cpu_baseline(ng, c, res)
    return res


def layer_config0(dev, reps, cpu_reps=3):
    """Config 0: the B-1M PKM layer forward alone in fp32 (8 x 256 tokens of N(0,1) hidden states, d 384, query
    384 -> 4 heads x 512, sub-keys N(0, 1/256) of 1024 x 256 per half, top-32 twice, softmax, 1,048,576 x 384 fp32
    values N(0, 0.02), no query norm, no swilu, seed 0): median synchronised forward time on the GPU, and the
    reference's torch path (oracle/torch_path.py) on the host cores for the same layer and inputs."""
    import torch
    import oracle.torch_path as TP
    from smlm_hip.pkm import ProductKeyMemory
    g = torch.Generator().manual_seed(0)
    N, d, H, kd, NK, knn = 2048, 384, 4, 512, 1024, 32
    x = torch.randn(N, d, generator=g)
    mem = ProductKeyMemory(d, d, n_keys=NK, heads=H, knn=knn, k_dim=kd, query_norm="none", swilu=False)
    with torch.no_grad():
        mem.query_proj.weight.copy_(torch.randn(H * kd, d, generator=g) * 0.02)
        mem.query_proj.bias.zero_()
        mem.keys.copy_(torch.randn(H, 2, NK, kd // 2, generator=g) / 16)
        mem.values.weight.copy_(torch.randn(NK * NK, d, generator=g) * 0.02)
    sd = {k: v.detach().clone() for k, v in mem.state_dict().items()}
    mem = mem.to(dev).eval()
    xd = x.to(dev)
    times = []
    with torch.no_grad():
        for i in range(3 + reps):
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            mem(xd)
            torch.cuda.synchronize(dev)
            if i >= 3:
                times.append(time.perf_counter() - t0)
    times.sort()
    ms = 1000.0 * times[len(times) // 2]
    mcfg = {"heads": H, "knn": knn, "k_dim": kd, "n_keys": NK, "query_norm": "none", "swilu": False}
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cpu = []
    with torch.no_grad():
        for _ in range(cpu_reps):
            t0 = time.perf_counter()
            TP.pkm_forward(sd, "", x, mcfg)
            cpu.append(time.perf_counter() - t0)
    cpu.sort()
    cpu_ms = 1000.0 * cpu[len(cpu) // 2]
    del mem, xd
    torch.cuda.empty_cache()
    return {"tokens": N, "ms": ms, "tok_s": N / ms * 1e3, "cpu_ms": cpu_ms, "cpu_tok_s": N / cpu_ms * 1e3,
            "cpu_cores": torch.get_num_threads(), "cpu_kind": "port (reference torch path)"}


def event_time_each_ms(prep, fn, reps):
    """Average device time of fn() in ms over `reps` calls, each bracketed by its own HIP events so that prep()
    (state reset between calls) stays outside the timed intervals."""
    import torch
    prep()
    fn()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    for a, b in pairs:
        prep()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) / reps


def train_cpu_baseline(res):
    """The reference's torch path of the training side on the host cores (oracle/torch_path.py: the torch branch of
    the row-sparse bag backward, smlm/sparse_values.py:66-104, and the fp32 torch path of LazyRowAdam, 271-306) at
    train_kernels' B-1M shape, on a bounded sample: the bag backward over 512 of the micro-batch's 4,096 tokens (all
    128 uniform lookups each; median of 3), the lazy Adam as the reference steps it, one dense torch.optim.Adam step
    over the whole 1,048,576 x 384 table with the rows a 32,768-token step reads touched (the first step, which
    creates the moments, untimed; mean of the next 2), and the selection backward (PKSelect.backward, smlm/kernels.py:
    253-266) on 2,048 of config 2's tokens (median of 3).  Each figure sits beside the GPU's in the same unit."""
    import torch
    import oracle.torch_path as TP
    rows, D, Kl, n = 1 << 20, 384, 128, 512
    g = torch.Generator().manual_seed(5)
    table = torch.empty(rows, D).normal_(0.0, 0.02, generator=g)
    acc = torch.zeros(rows, D)
    touched = torch.zeros(rows, dtype=torch.bool)
    idx = torch.randint(0, rows, (n, Kl), generator=g)
    gout = torch.randn(n, D, generator=g)
    w = torch.softmax(torch.randn(n, 4, 32, generator=g), -1).view(n, Kl)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        TP.bag_backward_rows(gout, idx, w, table, acc, touched)
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[1]
    gpu_ms = res["bag_backward_uniform"]["ms"]
    out = {"bag_backward": {"value": n * Kl / dt, "unit": "lookups/s", "cores": torch.get_num_threads(),
                            "kind": "port", "gpu_value": 4096 * Kl / gpu_ms * 1e3,
                            "sample": f"512 tokens x 128 uniform lookups into the 1,048,576 x 384 fp32 table "
                                      f"({dt * 1e3:.1f} ms; the GPU's 4,096-token micro-batch {gpu_ms:.3f} ms)"}}
    del idx, gout, w
    mask = torch.zeros(rows, dtype=torch.bool)
    mask[torch.randint(0, rows, (8 * 4096 * Kl,), generator=g)] = True
    hot = int(mask.sum())
    param = torch.nn.Parameter(table)
    adam = torch.optim.Adam([param], lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    times = []
    for _ in range(3):
        acc.fill_(1e-3)
        touched.copy_(mask)
        t0 = time.perf_counter()
        TP.lazy_adam_fp32_step(param, adam, acc, touched)
        times.append(time.perf_counter() - t0)
    dt = sum(times[1:]) / 2
    gpu_ms = res["lazy_adam_fp32"]["ms"]
    out["lazy_adam_fp32"] = {"value": hot / dt, "unit": "touched rows/s", "cores": torch.get_num_threads(),
                             "kind": "port", "gpu_value": hot / gpu_ms * 1e3,
                             "sample": f"the whole step: {hot:,} of 1,048,576 rows touched ({dt * 1e3:.0f} ms per "
                                       f"step; the GPU's {gpu_ms:.3f} ms)"}
    del param, adam, table, acc, touched, mask
    # the selection backward at config 2's shape on 2,048 of its 16,384 tokens (PKSelect.backward's torch ops)
    n, H, NK, knn = 2048, 4, 2048, 32
    idx = torch.randint(0, NK * NK, (n, H, knn), generator=g)
    wsel = torch.softmax(torch.randn(n, H, knn, generator=g), -1)
    gs = torch.randn(n, H, knn, generator=g).to(torch.bfloat16)
    gwv = torch.randn(n, H, knn, generator=g)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        TP.select_backward(idx, wsel, gs, gwv, NK, torch.bfloat16)
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[1]
    gpu_ms = res["select_backward_config2"]["ms"]
    out["select_backward_config2"] = {"value": n / dt, "unit": "tok/s", "cores": torch.get_num_threads(),
                                      "kind": "port", "gpu_value": 16384 / gpu_ms * 1e3,
                                      "sample": f"2,048 of the 16,384 tokens ({dt * 1e3:.1f} ms; the GPU's 16,384 "
                                                f"{gpu_ms:.3f} ms)"}
    return out


def train_kernels(dev, reps, cpu=False):
    """The training side of the lookup at the reference's training shape (one micro-batch = 4 x 1024 tokens, 4
    heads x top-32 = 128 lookups per token, B-1M fp32 value table 1,048,576 x 384): the row-sparse bag backward on
    uniform and Zipf(1.1) indices (the ordered form, and the atomic form as ms_atomic), the lazy row Adam (fp32 / bf16 / int8 moments) on the rows a 32,768-token step
    (8 micro-batches) reads, and the selection backward at config 2 (8 x 2048 tokens, NK 2048, bf16 scores).
    Algorithmic bytes are the least any implementation moves: every distinct row read or written once."""
    import torch
    from smlm_hip import kernels as K
    rows, D, N, Kl = 1 << 20, 384, 4096, 128
    g = torch.Generator(device=dev).manual_seed(5)
    table = torch.empty(rows, D, device=dev).normal_(0.0, 0.02, generator=g)
    acc = torch.zeros(rows, D, device=dev)
    touched = torch.zeros(rows, dtype=torch.bool, device=dev)
    gout = torch.randn(N, D, generator=g, device=dev)
    w = torch.softmax(torch.randn(N, 4, 32, generator=g, device=dev), -1).view(N, Kl)
    res = {"shape": "4,096 tokens x 128 lookups, table 1,048,576 x 384 fp32 (B-1M)"}
    for name, idx in (("uniform", torch.randint(0, rows, (N, Kl), generator=g, device=dev)),
                      ("zipf", zipf_rows(N * Kl, rows, 1.1, g, dev).view(N, Kl))):
        distinct = int(torch.unique(idx).numel())
        alg = N * Kl * (8 + 4 + 4) + N * D * 4 + distinct * (3 * D * 4 + 1)
        ms = event_time_ms(lambda: K.bag_backward_rows(gout, idx, w, table, acc, touched), reps)
        ms_atomic = event_time_ms(lambda: K.bag_backward_rows(gout, idx, w, table, acc, touched, ordered=False),
                                  reps)
        res[f"bag_backward_{name}"] = {"ms": ms, "distinct_rows": distinct, "alg_bytes": alg,
                                       "alg_GBps": alg / ms / 1e6, "ms_atomic": ms_atomic}
    del acc, gout, w
    # rows read by a 32,768-token step: 8 micro-batches of uniform lookups
    mask = torch.zeros(rows, dtype=torch.bool, device=dev)
    mask[torch.randint(0, rows, (8 * N * Kl,), generator=g, device=dev)] = True
    hot = int(mask.sum())
    acc = torch.randn(rows, D, generator=g, device=dev) * 1e-3
    per_row = {"fp32": 8 * D * 4, "bf16": D * (8 + 4 + 4 + 8), "int8": D * (8 + 2 + 2 + 8) + 16}
    for sd in ("fp32", "bf16", "int8"):
        if sd == "fp32":
            m, v = torch.zeros_like(table), torch.zeros_like(table)
            step = lambda: K.lazy_adam_step(table, m, v, acc, touched, 1.0, 1, 1e-3, 0.9, 0.95, 1e-8)
        elif sd == "bf16":
            m = torch.zeros(rows, D, dtype=torch.bfloat16, device=dev)
            v = torch.zeros_like(m)
            step = lambda: K.lazy_adam_step_lowmem(table, m, v, acc, touched, 1.0, 1, 1e-3, 0.9, 0.95, 1e-8, "bf16")
        else:
            m = torch.zeros(rows, D, dtype=torch.int8, device=dev)
            v = torch.zeros(rows, D, dtype=torch.uint8, device=dev)
            ms_, vs_ = torch.zeros(rows, device=dev), torch.zeros(rows, device=dev)
            step = lambda: K.lazy_adam_step_lowmem(table, m, v, acc, touched, 1.0, 1, 1e-3, 0.9, 0.95, 1e-8, "int8",
                                                   ms_, vs_)
        ms = event_time_each_ms(lambda: touched.copy_(mask), step, reps)
        alg = rows + hot * (per_row[sd] + 1)
        res[f"lazy_adam_{sd}"] = {"ms": ms, "touched_rows": hot, "alg_bytes": alg, "alg_GBps": alg / ms / 1e6}
        del m, v
    del table, acc, touched, mask
    torch.cuda.empty_cache()
    Ns, H, NK, knn = 8 * 2048, 4, 2048, 32
    s1 = torch.randn(Ns, H, NK, generator=g, device=dev).to(torch.bfloat16)
    s2 = torch.randn(Ns, H, NK, generator=g, device=dev).to(torch.bfloat16)
    _, idx, wsel = K.pk_select(s1, s2, knn)
    del s1, s2
    gs = torch.randn(Ns, H, knn, generator=g, device=dev).to(torch.bfloat16)
    gw = torch.randn(Ns, H, knn, generator=g, device=dev)
    ms = event_time_ms(lambda: K.pk_select_backward(idx, wsel, gs, gw, NK, torch.bfloat16), reps)
    alg = Ns * H * knn * (8 + 4 + 2 + 4) + 2 * Ns * H * NK * 2
    res["select_backward_config2"] = {"ms": ms, "alg_bytes": alg, "alg_GBps": alg / ms / 1e6}
    del idx, wsel, gs, gw
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = train_cpu_baseline(res)
    return res


def cpu_info():
    """Host CPU description for the CPU baselines: model name (lscpu), core counts and torch's thread count."""
    import subprocess
    import torch
    name = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                name = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if name is None and os.path.exists("/proc/cpuinfo"):
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    return {"model_name": name, "cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads()}


def cpu_decode(sd, cfg, B, max_steps, budget_s, prompt_len=128):
    """The reference's torch path (oracle/torch_path.py) on the host cores: B prompts of prompt_len uniform ids,
    prefill (untimed), then greedy decode steps of the loop of smlm/train.py:283-301, timed until `budget_s`
    seconds or `max_steps` steps (the config's 256 new tokens at most)."""
    import torch
    import oracle.torch_path as TP
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg["vocab_size"], (B, prompt_len), generator=g)
    with torch.no_grad():
        caches = [dict() for _ in range(cfg["n_layers"])]
        t0 = time.perf_counter()
        nxt = TP.lm_forward(sd, cfg, prompt, caches, 0, last_only=True).argmax(-1)
        t_prefill = time.perf_counter() - t0
        steps = 0
        t0 = time.perf_counter()
        while steps < max_steps and (steps < 2 or time.perf_counter() - t0 < budget_s):
            nxt = TP.lm_forward(sd, cfg, nxt, caches, prompt_len + steps).argmax(-1)
            steps += 1
        dt = time.perf_counter() - t0
    return {"value": B * steps / dt, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"batch {B}: {prompt_len}-token prompt prefill ({t_prefill:.1f} s, untimed), then {steps} "
                      f"of the {GEN_TOKENS} greedy steps timed ({dt:.1f} s), reference torch path restated in "
                      f"oracle/torch_path.py (fp32 weights, bf16 table read by row gather)"}


def host_state(model):
    """The model's weights on the host for the CPU path: fp32, except the value tables, which stay bf16."""
    sd = {}
    for k, v in model.state_dict().items():
        sd[k] = v.cpu() if k.endswith("values.weight") else v.float().cpu()
    return sd


def cpu_gather_c4(codes, scales, idx, w, out_gpu, tokens, reps=3):
    """Config 4 on the host cores over the first `tokens` tokens of the same lookups (the reference has no int8
    gather; its CPU-side forms, as BASELINE.md plans them):
      chunked   table_i8[idx].float() * (w * scale[idx])[..., None] summed over the 128 lookups, 256 tokens a chunk
      dequant   the table dequantised once to fp32 (untimed), then F.embedding_bag(mode="sum",
                per_sample_weights) -- the reference's bag_forward path on a dequantised inference table
                (smlm/pkm.py:138-148, scripts/quantize_table_eval.py:55-61); only when host RAM allows 26 GB more.
    Both are checked against the GPU output rows of the same tokens.  Rates are algorithmic bytes (52,480 per
    token) per second."""
    import torch
    import torch.nn.functional as F
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    t0 = time.perf_counter()
    codes_h, scales_h = codes.cpu(), scales.cpu()
    idx_h, w_h = idx[:tokens].cpu(), w[:tokens].cpu()
    ref = out_gpu[:tokens].cpu()
    copy_s = time.perf_counter() - t0
    per_tok = idx.shape[1] * (codes.shape[1] + 2 + 8 + 4) + codes.shape[1] * 4

    def chunked():
        out = torch.empty(tokens, codes.shape[1])
        for a in range(0, tokens, 256):
            i = idx_h[a:a + 256]
            wr = w_h[a:a + 256] * scales_h[i].float()
            out[a:a + 256] = (codes_h[i].float() * wr[..., None]).sum(1)
        return out

    def median_s(fn):
        fn()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            o = fn()
            ts.append(time.perf_counter() - t)
        ts.sort()
        return ts[len(ts) // 2], o

    s1, o1 = median_s(chunked)
    res = {"tokens": tokens, "host_copy_s": copy_s, "alg_bytes_per_token": per_tok,
           "chunked": {"ms": 1000 * s1, "alg_GBps": tokens * per_tok / s1 / 1e9,
                       "tok_s": tokens / s1,
                       "max_abs_diff_vs_gpu": float((o1 - ref).abs().max())}}
    try:
        import psutil
        avail = psutil.virtual_memory().available
    except ImportError:
        avail = 0
    rows = codes.shape[0]
    if avail > rows * codes.shape[1] * 4 * 1.5:
        t0 = time.perf_counter()
        table = torch.empty(rows, codes.shape[1])
        for a in range(0, rows, 1 << 20):
            table[a:a + (1 << 20)] = codes_h[a:a + (1 << 20)].float() * scales_h[a:a + (1 << 20), None].float()
        deq_s = time.perf_counter() - t0
        s2, o2 = median_s(lambda: F.embedding_bag(idx_h, table, per_sample_weights=w_h, mode="sum"))
        res["dequant_embedding_bag"] = {"ms": 1000 * s2, "alg_GBps": tokens * per_tok / s2 / 1e9,
                                        "tok_s": tokens / s2, "dequantise_s_untimed": deq_s,
                                        "max_abs_diff_vs_gpu": float((o2 - ref).abs().max())}
        del table
    else:
        res["dequant_embedding_bag"] = f"skipped: {avail / 2**30:.0f} GiB of host RAM available"
    res.update(cpu_info())
    del codes_h, scales_h
    return res


def cpu_prefill_c2(model, tokens=2048):
    """Config 2 on the host cores: the reference torch path's LM forward (oracle/torch_path.py) over ONE of the
    8 prompts of 2048 tokens (a bounded sample), tok/s."""
    import torch
    import oracle.torch_path as TP
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    sd = host_state(model)
    cfg = model.cfg.to_dict()
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, cfg["vocab_size"], (1, tokens), generator=g)
    with torch.no_grad():
        TP.lm_forward(sd, cfg, prompt[:, :64])
        t0 = time.perf_counter()
        TP.lm_forward(sd, cfg, prompt, last_only=True)
        dt = time.perf_counter() - t0
    del sd
    return {"value": tokens / dt, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"1 of the 8 prompts: LM forward over {tokens} tokens ({dt:.1f} s), reference torch path"}


GATHER_SOURCES = ("sparse-memory-lm_amd/csrc/pkm_bag.hip", "sparse-memory-lm_amd/csrc/pkm_bag_dev.h")


def gather_sources_sha256():
    """sha256 over the sources of the config-4 gather kernel: ties a committed counter summary to the code it
    measured."""
    import hashlib
    h = hashlib.sha256()
    for f in GATHER_SOURCES:
        with open(os.path.join(REPO, f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def read_traffic(path=None):
    """HBM bytes per launch of the config-4 gather (uniform control, Zipf) from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy kernel).  The summary names the sha256 of the
    gather's sources it was measured on; when that is absent or differs from the sources here, the counters
    belong to other code and the traffic is None (with "stale": True)."""
    path = path or os.path.join(REPO, "profiles", "gather_config4_pmc.txt")
    out = {"uniform": None, "zipf": None, "stale": True}
    if not os.path.exists(path):
        return out
    vals, sha = {}, None
    for line in open(path):
        if line.startswith("gather_sources_sha256:"):
            sha = line.split(":", 1)[1].strip()
        for k in ("uniform", "zipf"):
            if line.startswith(f"traffic_bytes_per_launch_{k}:"):
                vals[k] = float(line.split(":", 1)[1])
    if sha is not None and sha == gather_sources_sha256():
        out.update(vals, stale=False)
    return out


def calibration_copy(dev, nbytes=1 << 30):
    """A plain device copy of known size (reads and writes nbytes): the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters in the PMC runs."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


HEADLINE_PHASES = "decode,gather,cpu,config1,config0,prefill,lookup"
OPTIONAL_PHASES = "offload,train,engram"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5,
                    help=f"timed generations of {GEN_TOKENS} greedy tokens per decode measurement")
    ap.add_argument("--warmup", type=int, default=2, help="untimed generations before them")
    ap.add_argument("--reps", type=int, default=20, help="timed launches per kernel measurement")
    ap.add_argument("--prefill-reps", type=int, default=5, help="timed forwards of the config-2 prefill")
    ap.add_argument("--cpu-steps", type=int, default=GEN_TOKENS, help="most CPU-baseline decode steps")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU-baseline decode timing budget")
    ap.add_argument("--cpu-gather-tokens", type=int, default=2048, help="config-4 tokens timed on the host")
    ap.add_argument("--cpu-lookup-tokens", type=int, default=16384, help="config-2 lookup tokens timed on the host")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--phases", default=HEADLINE_PHASES + "," + OPTIONAL_PHASES,
                    help="subset of " + HEADLINE_PHASES + "," + OPTIONAL_PHASES + ",calibrate (profiling runs); "
                         "the JSON line is complete only with the default")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)
    phases = set(args.phases.split(","))
    if args.no_cpu:
        phases.discard("cpu")

    import torch
    from smlm_hip import _lib
    dev = torch.device("cuda:0")
    log(f"{_lib.version()} on {torch.cuda.get_device_name(dev)}")
    R = {}                  # phase -> result
    errors = {}             # phase -> error text (the line is printed whatever a phase raises)

    def phase(name, fn, when=True):
        if name not in phases or not when:
            return None
        t0 = time.perf_counter()
        try:
            R[name] = fn()
        except Exception as e:                                  # noqa: BLE001 -- recorded in the line
            traceback.print_exc()
            errors[name] = f"{type(e).__name__}: {e}"
            R[name] = None
        torch.cuda.empty_cache()
        log(f"phase {name}: {time.perf_counter() - t0:.1f} s")
        return R[name]

    line = {
        "metric": "decode tok/s (B-16M, bs1/bs64); PKM lookup tok/s + value-gather HBM GB/s",
        "value": None, "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded uniform prompt ids, random N(0,0.02) weights; Zipf(1.1) gather indices",
        "config": {"workload": f"config 3: 21M LM (d384, 6 layers, vocab 32000) + B-16M PKM at layer 3 "
                               f"(16,777,216 x 384 bf16 values), batch 64, 128-token prompts, then {GEN_TOKENS} "
                               f"greedy tokens; a step is one such generation (whole-step hipGraph replays)",
                   "global_batch": 64, "prompt_len": 128, "new_tokens": GEN_TOKENS},
    }
    try:
        if "calibrate" in phases:
            calibration_copy(dev)
            log("calibration copy of 1 GiB done")
        model = None
        if phases & {"decode", "cpu", "offload"}:
            t0 = time.perf_counter()
            model = build_lm(lm_config(4096, 512), dev)
            log(f"B-16M LM built in {time.perf_counter() - t0:.1f} s")

        def decode():
            out = {}
            for B in (64, 1):
                tok_s, ms_gen, ms_tok = time_generations(model, B, args.steps, args.warmup, dev)
                out[f"bs{B}"] = {"tok_s": tok_s, "ms_per_generation": ms_gen, "ms_per_token_step": ms_tok}
                log(f"decode config 3 bs{B}: {tok_s:.1f} tok/s ({ms_tok:.4f} ms per token step, "
                    f"{ms_gen:.2f} ms per {GEN_TOKENS}-token generation)")
            launch_us, wide_us = chained_launch_us(dev), chained_launch_us(dev, numel=1 << 18)
            mean_pos = 128 + (GEN_TOKENS - 1) / 2.0
            for B in (64, 1):
                out[f"bs{B}"]["roofline"] = decode_roofline(model, B, out[f"bs{B}"]["ms_per_token_step"], mean_pos,
                                                            launch_us, wide_us)
            return out

        dec = phase("decode", decode)
        if dec is not None:
            line["value"] = dec["bs64"]["tok_s"]
            line["ms_per_step"] = dec["bs64"]["ms_per_generation"]
            line["ms_per_token_step"] = dec["bs64"]["ms_per_token_step"]
            line["decode_bs1_tok_s"] = dec["bs1"]["tok_s"]
            line["decode_bs1_ms_per_token_step"] = dec["bs1"]["ms_per_token_step"]
            line["decode_roofline"] = {k: v["roofline"] for k, v in dec.items()}

        ga = phase("gather", lambda: gather_stress(dev, args.reps,
                                                   cpu_tokens=args.cpu_gather_tokens if "cpu" in phases else 0))
        line["gather_config4"] = ga
        if ga is not None:
            traffic = read_traffic()
            tz = traffic["zipf"]
            ce = ga["ceilings"]
            read_c, rows_c = ce["read"]["GBps"], ce["random_rows"]["GBps"]
            line["hbm_read_ceiling_GBps"] = read_c
            line["random_row_ceiling_GBps"] = rows_c
            line["roofline"] = {
                "kernel": "bag_rows_kernel<int8> (config-4 shapes, uniform-index control)", "bound": "hbm",
                "achieved": ga["alg_GBps_uniform"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": ga["alg_GBps_uniform"] / HBM_PEAK_GBS, "traffic": traffic["uniform"],
                "traffic_stale": traffic["stale"],
                "alg_bytes_per_launch": ga["alg_bytes_per_call"], "ms_per_launch": ga["ms_uniform"],
                "frac_of_read_ceiling": ga["alg_GBps_uniform"] / read_c,
                "frac_of_random_row_ceiling": ga["alg_GBps_uniform"] / rows_c,
                "time_vs_random_row_ceiling": ce["random_rows"]["ms"] / ga["ms_uniform"],
                "zipf": {"ms_per_launch": ga["ms_zipf"], "alg_GBps": ga["alg_GBps_zipf"], "traffic": tz,
                         "physical_GBps": tz / ga["ms_zipf"] / 1e6 if tz else None,
                         "physical_frac": tz / ga["ms_zipf"] / 1e6 / HBM_PEAK_GBS if tz else None,
                         "physical_frac_of_read_ceiling": tz / ga["ms_zipf"] / 1e6 / read_c if tz else None}}

        def cpu():
            sd = host_state(model)
            cfg = model.cfg.to_dict()
            t0 = time.perf_counter()
            out = {"bs64": cpu_decode(sd, cfg, 64, args.cpu_steps, args.cpu_seconds)}
            log(f"cpu baseline config 3 bs64: {out['bs64']} ({time.perf_counter() - t0:.1f} s)")
            out["bs1"] = cpu_decode(sd, cfg, 1, args.cpu_steps, args.cpu_seconds / 2)
            log(f"cpu baseline config 3 bs1: {out['bs1']}")
            del sd
            return out

        cb = phase("cpu", cpu, when=model is not None)
        if cb is not None:
            info = cpu_info()
            line["cpu_baseline"] = dict(cb["bs64"], **info)
            line["cpu_baseline"]["sample"] = "config 3 decode, " + cb["bs64"]["sample"]
            line["cpu_baseline_bs1"] = dict(cb["bs1"], **info)
            if ga is not None and "cpu" in ga:
                line["cpu_baseline_gather_config4"] = ga["cpu"]

        def config1():
            m1 = build_lm(lm_config(1024, 1024), dev)
            tok_s, ms_gen, ms_tok = time_generations(m1, 1, args.steps, args.warmup, dev, prompt_len=512)
            out = {"tok_s": tok_s, "ms_per_generation": ms_gen, "ms_per_token_step": ms_tok, "batch": 1,
                   "prompt_len": 512, "new_tokens": GEN_TOKENS, "table": "1,048,576 x 384 bf16 (B-1M)"}
            if "cpu" in phases:
                sd = host_state(m1)
                out["cpu_baseline"] = dict(cpu_decode(sd, m1.cfg.to_dict(), 1, args.cpu_steps, args.cpu_seconds / 2,
                                                      prompt_len=512), **cpu_info())
                log(f"cpu baseline config 1: {out['cpu_baseline']}")
                del sd
            del m1
            return out

        line["decode_config1_bs1"] = phase("config1", config1)
        line["layer_config0"] = phase("config0", lambda: layer_config0(dev, args.reps))

        def prefill():
            m2 = build_lm(lm_config(2048, 2048), dev)
            import torch.cuda.tunable as tunable
            # PyTorch's TunableOp: the dense GEMMs (hipBLASLt / rocBLAS candidates) timed per shape at first use,
            # in the warm-up forwards, before the graph capture
            tunable.enable(True)
            tunable.tuning_enable(True)
            tunable.set_filename(os.path.join(tempfile.gettempdir(), f"smlm_tunableop_{os.getpid()}.csv"))
            tok_e, ms_e = time_prefill(m2, 8, 2048, args.prefill_reps, dev)
            tok_s, ms = time_prefill(m2, 8, 2048, args.prefill_reps, dev, graphed=True)
            tunable.enable(False)
            out = {"tok_s": tok_s, "ms_per_forward": ms, "graphed": True, "tunableop": True, "eager_tok_s": tok_e,
                   "eager_ms_per_forward": ms_e, "batch": 8, "seq_len": 2048,
                   "table": "4,194,304 x 384 bf16 (B-4M)", "attention": prefill_attention_kernel(dev, args.reps)}
            log(f"prefill config 2 (B-4M, 8 x 2048): {tok_s:.0f} tok/s ({ms:.2f} ms per forward, graph replay; "
                f"eager {tok_e:.0f} tok/s, {ms_e:.2f} ms)")
            if "cpu" in phases:
                out["cpu_baseline"] = cpu_prefill_c2(m2)
                log(f"cpu baseline config 2: {out['cpu_baseline']}")
            del m2
            return out

        line["prefill_config2"] = phase("prefill", prefill)
        line["pkm_lookup_config2"] = phase("lookup", lambda: lookup_prefill(
            dev, args.reps, cpu_tokens=args.cpu_lookup_tokens if "cpu" in phases else 0))
        if R.get("lookup"):
            lk = R["lookup"]
            line["roofline_score"] = {
                "kernel": "config-2 sub-key scoring", "bound": "mfma", "achieved": lk["score_TFLOPs"],
                "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": lk["score_TFLOPs"] / BF16_MFMA_PEAK_TFLOPS}
        line["offload_config3"] = phase("offload", lambda: offload_tiers(model, dev, args.reps),
                                        when=model is not None)
        tr = phase("train", lambda: train_kernels(dev, args.reps, cpu="cpu" in phases))
        if tr is not None:
            for v in tr.values():
                if isinstance(v, dict) and "alg_GBps" in v:
                    v["hbm_frac"] = v["alg_GBps"] / HBM_PEAK_GBS
        line["train_kernels"] = tr
        line["engram_lookup"] = phase("engram", lambda: engram_lookup(dev, args.reps, cpu="cpu" in phases))
    finally:
        if errors:
            line["phase_errors"] = errors
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
