"""Build the gfx950 C-ABI library libsmlm_pkm.so from csrc/*.hip with hipcc (no torch extension machinery).

    python -m smlm_hip.build            (from sparse-memory-lm_amd/)

Every .hip file is compiled to an object in sparse-memory-lm_amd/_build/ (in parallel), then linked into
smlm_hip/libsmlm_pkm.so next to this file, where smlm_hip._lib loads it.  The memory-ceiling kernels of bench.py
(csrc/bench/*.hip: sequential read / write / copy and random-row reads) go into a separate smlm_hip/libsmlm_bench.so,
so the lookup library holds only the product.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                       # sparse-memory-lm_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_NAME = "libsmlm_pkm.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
BENCH_LIB_PATH = os.path.join(PKG_DIR, "libsmlm_bench.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # no packed-fp32 (v_pk_*_f32) instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: otherwise the compiler keeps them in AGPRs and copies them back and
    # forth around every epilogue / softmax (v_accvgpr_read / write; ~23k of them across the decode linears)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
]


def sources(folder=CSRC):
    return sorted(os.path.join(folder, f) for f in os.listdir(folder) if f.endswith(".hip"))


def _compile(src):
    sub = os.path.relpath(os.path.dirname(src), CSRC).replace(os.sep, "_").strip("._")
    obj = os.path.join(BUILD_DIR, (sub + "_" if sub else "") + os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that warning is harmless
    err = "\n".join(line for line in r.stderr.splitlines() if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _link(objs, path):
    tmp = path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, path)


def build(verbose=True):
    """Compile every csrc/*.hip for gfx950 and link libsmlm_pkm.so, and csrc/bench/*.hip into libsmlm_bench.so.
    Always rebuilds."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs, bench_srcs = sources(), sources(os.path.join(CSRC, "bench"))
    with ThreadPoolExecutor(max_workers=min(8, len(srcs) + len(bench_srcs))) as ex:
        objs = list(ex.map(_compile, srcs + bench_srcs))
    _link(objs[:len(srcs)], LIB_PATH)
    _link(objs[len(srcs):], BENCH_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources and {BENCH_LIB_PATH} from {len(bench_srcs)}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
