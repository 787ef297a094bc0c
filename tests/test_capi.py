"""CPU checks of the C ABI boundary: libssm_hip.so loads, exports every symbol that
include/ssm_hip.h declares, and reports a missing device as GPU_UNAVAILABLE (the reference's
'GPU_UNAVAILABLE' SessionErrorCode, src/session/session.ts:262-270). No compute calls."""
import ctypes as C
import os
import re

import pytest

from ssmjs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "ssm_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ssm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_symbols() == sorted(_lib.PROTOTYPES), "ctypes prototypes drift from header"


def test_library_exports_every_symbol():
    L = _lib.lib()
    missing = [s for s in header_symbols() if not hasattr(L, s)]
    assert not missing, missing
    assert L.ssm_abi_version() == 1


def test_status_names_map_to_reference_codes():
    L = _lib.lib()
    assert L.ssm_status_name(_lib.SSM_ERR_GPU_UNAVAILABLE) == b"GPU_UNAVAILABLE"
    assert L.ssm_status_name(_lib.SSM_ERR_CHECKPOINT_INVALID) == b"CHECKPOINT_INVALID"
    assert L.ssm_status_name(_lib.SSM_ERR_DESTROYED) == b"SESSION_DESTROYED"
    assert L.ssm_status_name(_lib.SSM_ERR_HIP) == b"UNKNOWN"


def test_forced_no_device_is_gpu_unavailable(monkeypatch):
    monkeypatch.setenv("SSM_HIP_FAULT", "nodevice")
    h = C.c_void_p()
    st = _lib.lib().ssm_ctx_create(0, C.byref(h))
    assert st == _lib.SSM_ERR_GPU_UNAVAILABLE
    assert b"no HIP device" in _lib.lib().ssm_last_error()


def test_null_arguments_are_rejected():
    L = _lib.lib()
    assert L.ssm_causal_conv1d(None, 0, None, None, None, 0, 1, 1, 1, 4, 1, None, None,
                               None) == _lib.SSM_ERR_INVALID_ARG
    assert L.ssm_model_destroy(None) == _lib.SSM_OK
    with pytest.raises(_lib.SsmError) as e:
        _lib.call("ssm_ctx_synchronize", None)
    assert e.value.code == "UNKNOWN"
