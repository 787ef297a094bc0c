"""ctypes binding of libssm_hip.so (include/ssm_hip.h).

The library is the product path: there is no CPU fallback. If the shared object is missing
the import of this module still succeeds, but `lib()` raises `BackendUnavailable`, so every
GPU operation fails loudly.

torch (when installed) is imported before the library is loaded: torch's HIP libraries name
the runtime as "libamdhip64.so" while libssm_hip.so names "libamdhip64.so.7"; loading torch
first makes both resolve to one runtime instance, so torch device pointers are valid here.
"""
from __future__ import annotations

import ctypes as C
import os

try:  # see module docstring
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - the Node host does not use torch
    torch = None

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libssm_hip.so")

SSM_OK = 0
SSM_ERR_INVALID_ARG = 1
SSM_ERR_GPU_UNAVAILABLE = 2
SSM_ERR_CHECKPOINT_INVALID = 3
SSM_ERR_DESTROYED = 4
SSM_ERR_HIP = 5
SSM_ERR_OUT_OF_MEMORY = 6
SSM_ERR_UNSUPPORTED = 7

SSM_F32 = 0
SSM_BF16 = 1

SSM_LAYER_MAMBA1 = 1
SSM_LAYER_MAMBA2 = 2
SSM_LAYER_MAMBA3 = 3
SSM_LAYER_ATTENTION = 4
LAYER_CODES = {"mamba1": SSM_LAYER_MAMBA1, "mamba2": SSM_LAYER_MAMBA2,
               "mamba3": SSM_LAYER_MAMBA3, "attention": SSM_LAYER_ATTENTION}


class BackendUnavailable(RuntimeError):
    """libssm_hip.so is not built / cannot be loaded."""


class SsmError(RuntimeError):
    """A non-zero ssm_status. `.status` is the numeric code, `.code` the reference's string
    (SessionErrorCode, src/session/errors.ts:5-13)."""

    def __init__(self, status: int, message: str, code: str):
        super().__init__(message)
        self.status = status
        self.code = code


class ssm_config(C.Structure):
    _fields_ = [("vocab_size", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int),
                ("d_state", C.c_int), ("d_conv", C.c_int), ("expand", C.c_int),
                ("n_heads", C.c_int), ("n_groups", C.c_int), ("chunk_len", C.c_int),
                ("mimo_group", C.c_int), ("eos_id", C.c_int), ("dt_rank", C.c_int),
                ("norm_eps", C.c_float), ("layer_types", C.POINTER(C.c_int))]


_vp = C.c_void_p
_fp = C.c_void_p   # device float* passed as integers / c_void_p
_l = C.c_long
_i = C.c_int
_f = C.c_float
_d = C.c_double
_sz = C.c_size_t

# name -> (restype, argtypes). Keep in the order of include/ssm_hip.h.
PROTOTYPES = {
    "ssm_last_error": (C.c_char_p, []),
    "ssm_status_name": (C.c_char_p, [_i]),
    "ssm_abi_version": (_i, []),
    "ssm_set_fault_injection": (_i, [C.c_char_p]),
    "ssm_ctx_create": (_i, [_i, C.POINTER(_vp)]),
    "ssm_ctx_destroy": (_i, [_vp]),
    "ssm_ctx_set_stream": (_i, [_vp, _vp]),
    "ssm_ctx_stream": (_vp, [_vp]),
    "ssm_ctx_synchronize": (_i, [_vp]),
    "ssm_ctx_profile": (_i, [_vp, _i]),
    "ssm_ctx_profile_report": (_i, [_vp, C.c_char_p, _sz]),
    "ssm_ctx_info": (_i, [_vp, C.c_char_p, _i, C.POINTER(_i), C.POINTER(_sz)]),
    "ssm_malloc": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "ssm_free": (_i, [_vp, _vp]),
    "ssm_memcpy_h2d": (_i, [_vp, _vp, _vp, _sz]),
    "ssm_memcpy_d2h": (_i, [_vp, _vp, _vp, _sz]),
    "ssm_causal_conv1d": (_i, [_fp, _l, _fp, _fp, _fp, _l, _i, _i, _i, _i, _i, _fp, _fp, _vp]),
    "ssm_conv1d_update": (_i, [_fp, _l, _fp, _fp, _fp, _l, _fp, _i, _i, _i, _i, _vp]),
    "ssm_selective_scan_workspace": (_sz, [_i, _i, _i, _i]),
    "ssm_selective_scan": (_i, [_fp, _l, _fp, _l, _fp, _i, _fp, _fp, _l, _fp, _l, _fp, _fp, _l,
                                _fp, _l, _i, _i, _i, _i, _fp, _fp, _vp, _sz, _vp]),
    "ssm_m1_state_update": (_i, [_fp, _l, _fp, _l, _fp, _i, _fp, _fp, _l, _fp, _l, _fp, _fp,
                                 _l, _fp, _l, _fp, _i, _i, _i, _vp]),
    "ssm_ssd_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "ssm_ssd_chunk_scan": (_i, [_i, _vp, _l, _fp, _l, _fp, _i, _f, _f, _fp, _vp, _l, _vp, _l,
                                _fp, _fp, _l, _i, _i, _i, _i, _i, _i, _fp, _fp, _vp, _sz, _vp]),
    "ssm_m2_state_update": (_i, [_fp, _l, _fp, _l, _fp, _i, _f, _f, _fp, _fp, _l, _fp, _l, _fp,
                                 _fp, _l, _fp, _l, _fp, _i, _i, _i, _i, _i, _vp]),
    "ssm_rmsnorm": (_i, [_fp, _l, _fp, _fp, _l, _i, _i, _f, _vp]),
    "ssm_gated_rmsnorm": (_i, [_fp, _l, _fp, _l, _fp, _fp, _l, _i, _i, _i, _f, _vp]),
    "ssm_linear_rows_workspace": (_sz, [_i, _i, _i]),
    "ssm_linear_rows": (_i, [_i, _fp, _l, _fp, _l, _fp, _fp, _fp, _l, _i, _i, _i, _f, _f, _vp, _sz,
                             _vp]),
    "ssm_linear": (_i, [_fp, _l, _fp, _l, _fp, _fp, _l, _i, _i, _i, _f, _vp]),
    "ssm_m1_xproj_dt": (_i, [_fp, _l, _fp, _fp, _fp, _l, _fp, _l, _i, _i, _i, _i, _vp]),
    "ssm_argmax": (_i, [_fp, _l, _i, _i, _vp, _vp]),
    "ssm_sample_workspace": (_sz, [_i, _i]),
    "ssm_sample": (_i, [_fp, _l, _i, _i, _d, _i, _d, _vp, _vp, _vp, _sz, _vp]),
    "ssm_sample_noalloc": (_i, [_fp, _l, _i, _i, _d, _i, _d, _vp, _vp, _vp]),
    "ssm_model_create": (_i, [_vp, C.POINTER(ssm_config), C.c_uint64, C.POINTER(_vp)]),
    "ssm_model_destroy": (_i, [_vp]),
    "ssm_model_config": (_i, [_vp, C.POINTER(ssm_config)]),
    "ssm_model_load_weights": (_i, [_vp, _vp, _sz]),
    "ssm_model_export_weights": (_i, [_vp, _i, _vp, _sz, C.POINTER(_sz)]),
    "ssm_forward": (_i, [_vp, _vp, _i, _i, _vp]),
    "ssm_forward_device": (_i, [_vp, _vp, _i, _i, _vp]),
    "ssm_mixer_forward_device": (_i, [_vp, _i, _vp, _vp, _i, _i]),
    "ssm_mixer_forward_device_bf16": (_i, [_vp, _i, _vp, _vp, _i, _i]),
    "ssm_state_create": (_i, [_vp, _i, C.POINTER(_vp)]),
    "ssm_state_destroy": (_i, [_vp]),
    "ssm_state_reset": (_i, [_vp]),
    "ssm_state_floats": (_sz, [_vp]),
    "ssm_state_read": (_i, [_vp, _vp]),
    "ssm_state_write": (_i, [_vp, _vp]),
    "ssm_state_layer": (_i, [_vp, _i, C.POINTER(_vp), C.POINTER(_vp)]),
    "ssm_prefill": (_i, [_vp, _vp, _vp, _i, _vp, _vp]),
    "ssm_decode_step": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "ssm_decode_step_device": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "ssm_generate_greedy": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "ssm_generate_sample": (_i, [_vp, _vp, _vp, _i, _i, _d, _i, _d, _vp, _vp]),
}

_lib = None


def lib():
    """The loaded library (raises BackendUnavailable when it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise BackendUnavailable(
                f"{LIB_PATH} is not built; run `python -m ssmjs_amd.build` (hipcc, gfx950)")
        try:
            L = C.CDLL(LIB_PATH)
        except OSError as e:
            raise BackendUnavailable(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, what: str = "") -> None:
    """Raise SsmError for a non-zero status, with the library's thread-local message."""
    if status != SSM_OK:
        L = lib()
        msg = (L.ssm_last_error() or b"").decode(errors="replace")
        code = (L.ssm_status_name(status) or b"UNKNOWN").decode()
        raise SsmError(status, f"{what}: {msg}" if what else msg, code)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
