"""ctypes binding of libfe_paged.so, the C ABI declared in include/flexengine_amd.h and
include/flexengine_amd_model.h.

There is no fallback: if the library is missing, or no ROCm GPU is present when
a kernel is called, the call raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

# FE_PAGED_LIB may point at another build of the same library (e.g. a tuning
# variant); by default the in-tree build next to this file is used.
LIB_PATH = Path(os.environ.get("FE_PAGED_LIB", Path(__file__).resolve().parent / "libfe_paged.so"))

FE_OK = 0
FE_ERR_INVALID_ARGUMENT = -1
FE_ERR_UNSUPPORTED = -2
FE_ERR_WORKSPACE = -3
FE_ERR_SCRATCH_LIMIT = -4
# FE_PAGED_DECODE_NOALLOC_SCRATCH_BYTES of include/flexengine_amd.h
NOALLOC_SCRATCH_BYTES = 16 << 20

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/flexengine_amd.h
SIGNATURES: dict[str, tuple] = {
    "fe_version": (_i, []),
    "fe_error_string": (ctypes.c_char_p, [_i]),
    "fe_write_kv": (_i, [_p, _p, _i64, _p, _p, _i, _p, _p, _i, _i, _i, _i, _p]),
    "fe_write_kv_ragged": (_i, [_p, _p, _i64, _p, _p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _i, _p]),
    "fe_gather_tables": (_i, [_p, _i, _p, _i, _p, _i, _i, _i, _p, _i, _p]),
    "fe_write_kv_decode": (_i, [_p, _p, _i64, _p, _p, _i, _p, _i, _p, _i, _i, _i, _i, _p]),
    "fe_gather_kv": (_i, [_p, _p, _i, _p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p]),
    "fe_paged_decode_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
    "fe_paged_decode": (_i, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i, _p, _i, _p, _p, _sz,
                             _i, _i, _i, _i, _i, _f, _i, _p]),
    "fe_paged_decode_plan_size": (_sz, [_i, _i, _i, _i]),
    "fe_paged_decode_plan": (_i, [_p, _i, _p, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "fe_paged_decode_planned": (_i, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i, _p, _i, _p, _p, _sz,
                                     _i, _i, _i, _i, _i, _f, _i, _p, _sz, _p]),
    "fe_paged_decode_noalloc": (_i, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i, _p, _i, _p,
                                     _i, _i, _i, _i, _i, _f, _i, _p]),
    "fe_paged_decode_shared_prefix_workspace_size": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "fe_paged_decode_shared_prefix": (_i, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i, _p, _i, _p,
                                           _p, _p, _i, _p, _sz, _i, _i, _i, _i, _i, _f, _i, _p]),
    "fe_paged_decode_shared_prefix_bf16": (_i, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i, _p, _i,
                                                _p, _p, _p, _i, _p, _sz, _i, _i, _i, _i, _i, _f,
                                                _i, _p]),
    "fe_paged_decode_shared_prefix_f32": (_i, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i, _p, _i,
                                               _p, _p, _p, _i, _p, _sz, _i, _i, _i, _i, _i, _f,
                                               _i, _p]),
    "fe_lse_merge": (_i, [_p, _p, _i, _i, _i, _p, _p, _p]),
    "fe_lse_merge_bf16": (_i, [_p, _p, _i, _i, _i, _p, _p, _p]),
    "fe_prefill_paged": (_i, [_p, _p, _p, _p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _i,
                              _f, _p, _sz, _p]),
    "fe_prefill_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
}
SIGNATURES["fe_prefill_plan_size"] = (_sz, [_i, _i, _i, _i])
SIGNATURES["fe_prefill_plan"] = (_i, [_p, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p])
SIGNATURES["fe_prefill_paged_planned"] = (
    _i, SIGNATURES["fe_prefill_paged"][1][:-1] + [_p, _sz, _p])
# the bf16 forms take the fp16 entry points' arguments
for _name in ("fe_paged_decode", "fe_paged_decode_planned", "fe_prefill_paged",
              "fe_prefill_paged_planned"):
    SIGNATURES[_name + "_bf16"] = SIGNATURES[_name]
# and so do the fp32 forms
for _name in ("fe_write_kv", "fe_write_kv_decode", "fe_write_kv_ragged", "fe_gather_kv",
              "fe_paged_decode", "fe_prefill_paged"):
    SIGNATURES[_name + "_f32"] = SIGNATURES[_name]
SIGNATURES |= {
    # include/flexengine_amd_model.h
    "fe_rmsnorm": (_i, [_p, _i, _p, _p, _p, _p, _i, _i, _f, _p]),
    "fe_rope_qkv": (_i, [_p, _i64, _i, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "fe_silu_mul": (_i, [_p, _i64, _i, _p, _i, _i, _p]),
    "fe_gemm_skinny_splits": (_i, [_i, _i]),
    "fe_gemm_skinny": (_i, [_p, _i, _i, _p, _i, _p, _i, _p]),
    "fe_gemm_fused_workspace_size": (_sz, [_i, _i, _i]),
    "fe_gemm_rows64_workspace_size": (_sz, [_i, _i, _i]),
    "fe_gemm_f16": (_i, [_p, _p, _i, _p, _f, _i, _i, _p, _i, _p, _p, _p, _sz, _p]),
    "fe_gemm_resid": (_i, [_p, _i, _i, _p, _i, _p, _p, _p, _p, _sz, _p]),
    "fe_gemm_rows64": (_i, [_p, _i, _i, _p, _i, _p, _p, _p, _sz, _p]),
    "fe_gemm_resid_rmsnorm": (_i, [_p, _i, _i, _p, _i, _p, _p, _p, _p, _f, _p, _p, _sz, _p]),
    "fe_gemm_silu": (_i, [_p, _p, _i, _p, _f, _i, _i, _p, _i, _p, _p, _sz, _p]),
    "fe_gemm_rope": (_i, [_p, _p, _i, _p, _f, _i, _i, _p, _p, _p, _p, _i, _i, _i, _p, _p, _p,
                          _p, _sz, _p]),
}

_LIB: ctypes.CDLL | None = None
_LOCK = threading.Lock()


class FlexEngineAMDError(RuntimeError):
    """A nonzero return code from libfe_paged.so."""

    def __init__(self, func: str, code: int, text: str):
        super().__init__(f"{func} failed with code {code}: {text}")
        self.code = code


def load() -> ctypes.CDLL:
    """Loads libfe_paged.so once and declares every C-ABI signature."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m flexengine_amd.build` "
                    "(hipcc for gfx950) before using the HIP paged-attention kernels"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _LIB = lib
    return _LIB


def error_string(code: int) -> str:
    return load().fe_error_string(int(code)).decode()


def check(func: str, code: int) -> None:
    if code != FE_OK:
        raise FlexEngineAMDError(func, code, error_string(code))


def call(name: str, *args) -> None:
    """Calls an int-returning entry point and raises on a nonzero code."""
    check(name, getattr(load(), name)(*args))
