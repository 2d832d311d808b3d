"""ctypes binding of the C ABI in include/smlm_pkm.h (libsmlm_pkm.so, built by smlm_hip.build).

torch is imported first on purpose: torch's ROCm wheel ships its own libamdhip64.so.7, and loading it before
libsmlm_pkm.so makes the library bind to that same HIP runtime, so the stream handles torch hands out are
valid in our launches.  There is no fallback: if the library is missing, every op raises.
"""
import ctypes
import os

import torch  # noqa: F401  (see module docstring)

LIB_NAME = "libsmlm_pkm.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# smlm_dtype / smlm_status values of include/smlm_pkm.h
F32, BF16, F16, I8, Q4, I32, I64 = range(7)
OK, EINVAL, EUNSUPPORTED, EHIP = 0, -1, -2, -3

_p, _i, _i64, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

# smlm_linear_prologue / smlm_linear_epilogue
LIN_PLAIN, LIN_RMSNORM, LIN_EMBED_RMSNORM, LIN_RMSNORM_PARTS, LIN_EMBED_ARGMAX = range(5)
LIN_STORE, LIN_SWIGLU, LIN_ARGMAX = range(3)


class LinearArgs(ctypes.Structure):
    """struct smlm_linear_args of include/smlm_pkm.h, field for field."""
    _fields_ = [
        ("prologue", _i), ("epilogue", _i), ("M", _i64), ("N", _i), ("K", _i),
        ("x", _p), ("x_stride", _i64), ("delta", _p), ("tok", _p), ("emb", _p), ("emb_rows", _i64),
        ("norm_w", _p), ("eps", ctypes.c_float), ("x_out", _p), ("w", _p), ("bias", _p), ("scale", _p),
        ("shift", _p), ("n_affine", _i), ("n_split", _i), ("out", _p), ("out_stride", _i64), ("out2", _p),
        ("out2_stride", _i64), ("partial", _p), ("partial_stride", _i64), ("delta_parts", _i),
        ("tok_partial", _p), ("tok_partial_stride", _i64), ("tok_blocks", _i), ("tok_out", _p), ("hist", _p),
        ("hist_stride", _i64), ("hist_len", _i64), ("pos", _p), ("pos_advance", _p),
    ]

# name -> (restype, argtypes); every function declared in include/smlm_pkm.h
EXPORTS = {
    "smlm_pkm_version": (ctypes.c_char_p, []),
    "smlm_pkm_last_error": (ctypes.c_char_p, []),
    "smlm_host_table_pointer": (_i, [_p, ctypes.POINTER(ctypes.c_void_p)]),
    "smlm_pkm_score": (_i, [_p, _i64, _p, _i, _i64, _i, _i, _i, _p, _p, _p]),
    "smlm_pkm_select": (_i, [_p, _p, _i, _i64, _i, _i, _i, _p, _p, _p, _p]),
    "smlm_pkm_bag": (_i, [_p, _i, _p, _i64, _i, _p, _i, _i64, _i, _p, _p, _p, _i, _p]),
    "smlm_pkm_select_bag": (_i, [_p, _p, _i, _i64, _i, _i, _i, _p, _i, _i64, _i, _p, _p, _p, _i, _p, _p, _p, _p]),
    "smlm_pkm_lookup_noalloc": (_i, [_p, _i64, _p, _i, _i64, _i, _i, _i, _i, _p, _i, _i64, _i, _p, _p, _p, _i,
                                     _p]),
    "smlm_pkm_quantize": (_i, [_p, _i, _i64, _i, _i, _p, _p, _p]),
    "smlm_decode_attention": (_i, [_p, _i64, _p, _p, _i, _i, _p, _p, _p, _i64, _i, _i, _i, _p, _p]),
    "smlm_decode_attention_proj": (_i, [_p, _i64, _p, _p, _i, _i, _p, _p, _p, _i64, _i, _i, _i, _p, _i64, _i, _p,
                                        _p]),
    "smlm_swiglu": (_i, [_p, _i64, _p, _i64, _i, _p]),
    "smlm_linear_swiglu": (_i, [_p, _i64, _p, _i64, _i64, _i, _i, _p, _i64, _p]),
    "smlm_prompt_linear": (_i, [_p, _i64, _p, _i64, _p, _p, _p, _i64, _i, _i, _p, _i64, _p]),
    "smlm_greedy_argmax": (_i, [_p, _i64, _i64, _i, _p, _p, _p, _i64, _i64, _p]),
    "smlm_add_rmsnorm": (_i, [_p, _p, _p, ctypes.c_float, _i64, _i, _p, _p, _p]),
    "smlm_affine_bf16": (_i, [_p, _i64, _p, _p, _i64, _i, _p, _i64, _p]),
    "smlm_rope_qkv": (_i, [_p, _i64, _p, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i, _p]),
    "smlm_prefill_attention": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i, _i, _p]),
    "smlm_linear_argmax_blocks": (_i, [_i]),
    "smlm_decode_linear": (_i, [ctypes.POINTER(LinearArgs), _p]),
    "smlm_argmax_finish": (_i, [_p, _i64, _i, _i64, _p, _p, _p, _i64, _i64, _i, _p]),
    "smlm_pkm_select_backward": (_i, [_p, _p, _p, _p, _i, _i64, _i, _i, _i, _p, _p, _p]),
    "smlm_bag_backward_rows": (_i, [_p, _p, _p, _i64, _i, _p, _i, _i64, _i, _p, _p, _p, _p]),
    "smlm_bag_backward_sorted_workspace": (_i, [_i64, _i, _i64, _i, _p]),
    "smlm_bag_backward_sorted": (_i, [_p, _p, _p, _i64, _i, _p, _i, _i64, _i, _p, _p, _p, _p, _sz, _p]),
    "smlm_lazy_adam": (_i, [_p, _p, _p, _p, _p, _i, _p, _p, _p, _i64, _i, _f, _f, _f, _f, _f, _f, _f, _p]),
    "smlm_engram_hash": (_i, [_p, _i64, _i64, _i64, _p, _p, _i, _i, _i, _i64, _p, _p]),
    "smlm_row_gather": (_i, [_p, _i64, _p, _i, _i64, _i, _p, _p]),
}
ADAM_F32, ADAM_BF16, ADAM_INT8 = 0, 1, 2

_lib = None


class SmlmError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, what, code, message):
        super().__init__(f"{what} failed with status {code}: {message}")
        self.code = code


def lib():
    """The loaded library (loaded once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `python -m smlm_hip.build` in sparse-memory-lm_amd/ "
                               "or __graft_entry__.build()); the HIP kernels have no fallback")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def version():
    return lib().smlm_pkm_version().decode()


def last_error():
    return lib().smlm_pkm_last_error().decode()


def check(rc, what):
    if rc != OK:
        raise SmlmError(what, rc, last_error())


def stream_handle(device):
    """hipStream_t (as int) of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def host_device_pointer(host_ptr):
    """Device address of pinned host memory (smlm_host_table_pointer); raises SmlmError for anything else."""
    out = ctypes.c_void_p()
    check(lib().smlm_host_table_pointer(host_ptr, ctypes.byref(out)), "smlm_host_table_pointer")
    return out.value
