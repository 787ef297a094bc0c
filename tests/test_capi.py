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


def test_fault_injection_hook_overrides_environment(monkeypatch):
    """ssm_set_fault_injection pins the injected kind against the environment until it is
    called with NULL; unknown kinds are refused."""
    L = _lib.lib()
    monkeypatch.delenv("SSM_HIP_FAULT", raising=False)
    h = C.c_void_p()
    try:
        assert L.ssm_set_fault_injection(b"nodevice") == _lib.SSM_OK
        assert L.ssm_ctx_create(0, C.byref(h)) == _lib.SSM_ERR_GPU_UNAVAILABLE
        assert b"injected fault: nodevice" in L.ssm_last_error()
        assert L.ssm_set_fault_injection(b"no-such-kind") == _lib.SSM_ERR_INVALID_ARG
        # pinned: the environment variable no longer decides
        monkeypatch.setenv("SSM_HIP_FAULT", "")
        assert L.ssm_ctx_create(0, C.byref(h)) == _lib.SSM_ERR_GPU_UNAVAILABLE
        assert b"injected fault: nodevice" in L.ssm_last_error()
    finally:
        assert L.ssm_set_fault_injection(None) == _lib.SSM_OK
    # released: ssm_ctx_create reads the environment again
    monkeypatch.setenv("SSM_HIP_FAULT", "nodevice")
    assert L.ssm_ctx_create(0, C.byref(h)) == _lib.SSM_ERR_GPU_UNAVAILABLE
    assert b"injected fault: nodevice" in L.ssm_last_error()


def test_null_arguments_are_rejected():
    L = _lib.lib()
    assert L.ssm_causal_conv1d(None, 0, None, None, None, 0, 1, 1, 1, 4, 1, None, None,
                               None) == _lib.SSM_ERR_INVALID_ARG
    assert L.ssm_model_destroy(None) == _lib.SSM_OK
    with pytest.raises(_lib.SsmError) as e:
        _lib.call("ssm_ctx_synchronize", None)
    assert e.value.code == "UNKNOWN"


def _scan_call(L, B, Lq, D, N, ld, ws=None, ws_bytes=0):
    """ssm_selective_scan with placeholder (never dereferenced) pointers: every call here is
    refused by the host-side checks before anything is launched."""
    p = 1 << 20
    return L.ssm_selective_scan(p, ld, p, ld, None, 1, p, p, ld, p, ld, None, None, 0, p, ld,
                                B, Lq, D, N, None, None, ws, ws_bytes, None)


def test_scan_workspace_query_matches_the_plan():
    """The scan's plan depends on (B, D, N) and on whether L is at most 256 (short sequences
    take the single pass whatever their width), not on strides, so the workspace query and
    the launch agree: a single-pass shape needs no workspace even where a whole sequence
    spans more than 2 GiB of rows, and a chunked shape asks for exactly what the query
    says."""
    L = _lib.lib()
    # single pass (B*D*N/64 >= 1024 waves): (2, 140000, 2048, 16) with a 4096-float stride
    # spans 2.3 GB per sequence; before, the launch fell back to the chunked passes here
    # while the query said 0
    assert L.ssm_selective_scan_workspace(2, 140000, 2048, 16) == 0
    assert L.ssm_selective_scan_workspace(4, 2048, 1536, 16) == 0
    # one sequence of 512 channels: single pass up to 256 steps, chunked beyond
    assert L.ssm_selective_scan_workspace(1, 256, 512, 16) == 0
    assert L.ssm_selective_scan_workspace(1, 257, 512, 16) > 0
    # chunked (one sequence of 512 channels): the launch without it names the query's size
    need = L.ssm_selective_scan_workspace(1, 4096, 512, 16)
    assert need > 0
    assert _scan_call(L, 1, 4096, 512, 16, 512) == _lib.SSM_ERR_INVALID_ARG
    assert f"workspace of {need} bytes".encode() in L.ssm_last_error()
    assert _scan_call(L, 1, 4096, 512, 16, 512, ws=1 << 20, ws_bytes=need - 4) == \
        _lib.SSM_ERR_INVALID_ARG
    # a stride whose 128-row block does not fit 32-bit offsets is refused, not overflowed
    assert _scan_call(L, 2, 140000, 2048, 16, 1 << 23) == _lib.SSM_ERR_INVALID_ARG
    assert b"too large for 32-bit block offsets" in L.ssm_last_error()
