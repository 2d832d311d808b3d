"""Split a memory-model checkpoint into the small rest and the value table as flat files, in the formats of
scripts/convert_table.py (its lines 56-94), for smlm_hip.offload:

    python -m smlm_hip.convert_table --ckpt runs/B-16M/model.pt --out tables/B-16M

  rest.pt           {"model_config", "state_dict" (every weight except the table), "table_keys", "table_shape"}
  values_bf16.bin   the table in bf16, row-major (rows x dim x 2 bytes), rounded to nearest even
  values_q4.bin     the table in 4 bit, row-major (rows x dim/2 bytes): per row d = fp16(signed max-abs / -8),
                    code = clamp(round(w / d), -8, 7) + 8, byte i = column i (low nibble) | column i + dim/2 (high)
  scales_q4.bin     the fp16 d of every row (rows x 2 bytes)
  hot_rows.npy      row ids by training reads, most read first (from mem_access_train.npy beside the checkpoint)
  meta.json         shapes, the q4 format, the sha256 of every file

The checkpoint ({"model_config", "state_dict"}, the model.pt of train.py) is memory-mapped and the table is
processed in chunks of rows.  The 4-bit codes come from the gfx950 quantisation kernel (smlm_pkm_quantize), so a
GPU is needed unless q4=False.
"""
import argparse
import hashlib
import json
import os
import time

import numpy as np
import torch

from . import kernels

Q4_FORMAT = ("per row d = fp16(max-abs value with sign / -8), code = clamp(round(w/d),-8,7)+8, low nibble = dims "
             "0..dim/2-1, high nibble = dims dim/2..dim-1")


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 24), b""):
            h.update(block)
    return h.hexdigest()


def shared_table(state_dict):
    """(keys, tensor) of the value table: every "...values.weight" entry, which must all be one tensor."""
    keys = [k for k in state_dict if k.endswith("values.weight")]
    if not keys:
        raise ValueError("the checkpoint has no memory value table (no '...values.weight' entry)")
    table = state_dict[keys[0]]
    ptr = table.untyped_storage().data_ptr()
    if any(state_dict[k].untyped_storage().data_ptr() != ptr or state_dict[k].shape != table.shape for k in keys):
        raise ValueError("expected one value table shared by every memory layer")
    return keys, table


def convert(ckpt, out, chunk=1 << 20, q4=True, device="cuda", hot_counts=None, log=print):
    """Write the files above into directory `out`.  ckpt: a model.pt path or its loaded dict.  hot_counts: per-row
    training reads (default: mem_access_train.npy next to a ckpt path, if present).  Returns the meta dict."""
    t0 = time.time()
    os.makedirs(out, exist_ok=True)
    source = os.path.abspath(ckpt) if isinstance(ckpt, str) else None
    if source is not None:
        ck = torch.load(ckpt, mmap=True, map_location="cpu", weights_only=True)
        if hot_counts is None:
            acc = os.path.join(os.path.dirname(source), "mem_access_train.npy")
            if os.path.exists(acc):
                hot_counts = np.load(acc)
    else:
        ck = ckpt
    sd = ck["state_dict"]
    keys, table = shared_table(sd)
    rows, dim = table.shape
    if q4 and dim % 2:
        raise ValueError(f"q4 needs an even table width, got {dim}")
    rest = {k: v.clone() for k, v in sd.items() if k not in keys}
    torch.save({"model_config": ck["model_config"], "state_dict": rest, "table_keys": keys,
                "table_shape": [rows, dim]}, os.path.join(out, "rest.pt"))
    log(f"rest.pt: {sum(v.numel() for v in rest.values()) / 1e6:.1f} M parameters; table {rows} x {dim}")
    files = {"values_bf16.bin": open(os.path.join(out, "values_bf16.bin"), "wb")}
    if q4:
        files["values_q4.bin"] = open(os.path.join(out, "values_q4.bin"), "wb")
        files["scales_q4.bin"] = open(os.path.join(out, "scales_q4.bin"), "wb")
    try:
        for a in range(0, rows, chunk):
            w = table[a:a + chunk]
            files["values_bf16.bin"].write(w.to(torch.bfloat16).view(torch.int16).numpy().tobytes())
            if q4:
                packed, scales = kernels.quantize_q4(w.to(device=device, dtype=torch.float32))
                files["values_q4.bin"].write(packed.cpu().numpy().tobytes())
                files["scales_q4.bin"].write(scales.view(torch.int16).cpu().numpy().tobytes())
    finally:
        for f in files.values():
            f.close()
    if hot_counts is not None:
        counts = np.asarray(hot_counts)
        if counts.shape != (rows,):
            raise ValueError(f"hot_counts must have one entry per row ({rows}), got {counts.shape}")
        np.save(os.path.join(out, "hot_rows.npy"), np.argsort(-counts, kind="stable").astype(np.int64))
    meta = {"source": source, "rows": int(rows), "dim": int(dim), "table_keys": keys,
            "q4": Q4_FORMAT if q4 else None, "seconds": round(time.time() - t0, 1),
            "sha256": {n: _sha256(os.path.join(out, n)) for n in sorted(os.listdir(out))
                       if n.endswith((".bin", ".pt", ".npy"))}}
    with open(os.path.join(out, "meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    return meta


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--ckpt", required=True)
    ap.add_argument("--out", required=True)
    ap.add_argument("--chunk", type=int, default=1 << 20)
    ap.add_argument("--no-q4", action="store_true", help="write rest.pt and values_bf16.bin only (no GPU needed)")
    args = ap.parse_args()
    meta = convert(args.ckpt, args.out, args.chunk, q4=not args.no_q4)
    print(json.dumps(meta, indent=1))


if __name__ == "__main__":
    main()
