"""ctypes binding of libmicro_engram_amd.so (the C-ABI declared in include/micro_engram.h).

The library is the only compute path of this package: if it is missing, every op raises
instead of falling back to anything else.
"""
import ctypes
import os
import threading

from ._build import LIB_PATH

c_i32, c_i64, c_ptr, c_size = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
c_int, c_float, c_double = ctypes.c_int, ctypes.c_float, ctypes.c_double

# element type codes (include/micro_engram.h)
ME_I32, ME_I64, ME_F32, ME_BF16, ME_U8 = 1, 2, 3, 4, 5
ME_GATE_SCALAR, ME_GATE_SCALAR_SQRT = 0, 1
ME_MAX_TABLES, ME_MAX_ORDER = 64, 8

_HASH_COMMON = [c_ptr, c_i64, c_ptr, c_i32, c_i32, c_ptr, c_ptr, c_i64]  # canon..pad_id
# name -> argtypes; every function returns int (ME_OK or a negative error code)
SIGNATURES = {
    "me_hash_ngrams": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_int, c_i64, *_HASH_COMMON, c_ptr, c_ptr],
    "me_hash_prev": [c_ptr, c_int, c_i64, c_i64, c_i64, *_HASH_COMMON, c_ptr, c_ptr],
    "me_gather": [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_ptr, c_i32, c_int, c_ptr, c_ptr],
    "me_hash_gather": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_int, c_i64, *_HASH_COMMON,
                       c_ptr, c_i32, c_int, c_ptr, c_ptr, c_ptr],
    "me_hash_prev_gather": [c_ptr, c_int, c_i64, c_i64, c_i64, *_HASH_COMMON,
                            c_ptr, c_i32, c_int, c_ptr, c_ptr, c_ptr],
    "me_gate_workspace_size": [c_i64, c_i64, ctypes.POINTER(c_size)],
    "me_gate_residual": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_int,
                         c_ptr, c_ptr, c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_size,
                         c_ptr],
    "me_gate_residual_noalloc": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_int,
                                 c_ptr, c_ptr, c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "me_kv_proj": [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_int, c_ptr, c_ptr],
    "me_gate_rows": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_int, c_ptr, c_ptr, c_int,
                     c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "me_gate_rows_backward_workspace_size": [c_i64, c_i64, ctypes.POINTER(c_size)],
    "me_gate_rows_backward": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_int, c_ptr, c_ptr,
                              c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
                              c_ptr, c_size, c_ptr],
    "me_gate_backward_workspace_size": [c_i64, c_i64, ctypes.POINTER(c_size)],
    "me_gate_backward": [c_ptr, c_int, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_int,
                         c_ptr, c_ptr, c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
                         c_ptr, c_ptr, c_ptr, c_size, c_ptr],
    "me_linear_grads": [c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
                        c_ptr],
    "me_dedup_workspace_size": [c_i64, ctypes.POINTER(c_size)],
    "me_dedup": [c_ptr, c_i64, c_i64, c_ptr, c_int, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
                 c_size, c_ptr],
    "me_dedup_plan_size": [c_i64, ctypes.POINTER(c_size)],
    "me_dedup_keys": [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_size, c_ptr, c_size, c_ptr],
    "me_dedup_table_bounds": [c_ptr, c_i64, c_ptr, c_ptr, c_i32, c_ptr, c_ptr, c_ptr],
    "me_dedup_tables_workspace_size": [c_i64, c_i32, c_ptr, ctypes.POINTER(c_size)],
    "me_dedup_tables": [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_size,
                        c_ptr, c_size, c_ptr],
    "me_dedup_sums": [c_ptr, c_size, c_i64, c_ptr, c_ptr, c_int, c_i32, c_ptr, c_ptr],
    "me_sumsq": [c_ptr, c_i64, c_ptr, c_int, c_ptr, c_size, c_ptr],
    "me_sparse_adam": [c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_int, c_ptr, c_ptr, c_ptr, c_i32, c_int,
                       c_int, c_int, c_int, c_double, c_double, c_double, c_double, c_double,
                       c_int, ctypes.c_uint64, c_ptr],
    "me_clip_scale": [c_ptr, c_int, c_i64, c_ptr, c_double, c_ptr],
    "me_stochastic_bf16": [c_ptr, c_i64, c_ptr, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                           c_ptr],
    "me_fill_engram_ids": [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_int, c_ptr, c_int, c_ptr, c_int,
                           c_ptr, c_int, c_ptr, c_int, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                           c_ptr, c_int, c_i32, c_ptr, c_ptr],
    "me_mask_media": [c_ptr, c_int, c_i64, c_i64, c_i64, c_ptr, c_int, c_i32, c_ptr, c_ptr, c_ptr],
}

_lock = threading.Lock()
_lib = None


class EngramLibError(RuntimeError):
    """A call into the HIP library returned an error status."""


def lib_path():
    return os.environ.get("MICRO_ENGRAM_AMD_LIB") or LIB_PATH


def load():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(
                    f"[micro_engram] {path} is missing: build the HIP library first "
                    "(python -m micro_engram_fork_amd._build). There is no fallback path.")
            lib = ctypes.CDLL(path)
            lib.me_last_error.restype = ctypes.c_char_p
            lib.me_last_error.argtypes = []
            lib.me_version.restype = c_int
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = c_int
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name, *args):
    """Calls entry point `name`; raises EngramLibError with the library's message on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.me_last_error().decode(errors="replace")
        raise EngramLibError(f"[micro_engram] {name} failed ({status}): {msg}")


def exported_symbols():
    """Names of the entry points this binding declares, plus the two utility calls."""
    return ["me_last_error", "me_version", *SIGNATURES]


def i32_array(values):
    return (c_i32 * len(values))(*values)


def i64_array(values):
    return (c_i64 * len(values))(*values)


def ptr_array(values):
    return (c_ptr * len(values))(*values)
