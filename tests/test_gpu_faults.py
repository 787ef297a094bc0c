"""Failure handling forced from the host (SSM_HIP_FAULT), as SURVEY's auxiliary plan asks:
every kernel still runs normally; the library reports the injected failure through the error
contract of the reference (src/session/session.ts:262-270,393-401; errors.ts:5-13), and the
same device and model work again once the fault is cleared.
  alloc   every device allocation fails -> SSM_ERR_OUT_OF_MEMORY ('UNKNOWN' to the session,
          which wraps model construction failures as 'UNKNOWN', session.ts:359-362)
  launch  every launch check reports a failure -> SSM_ERR_HIP ('UNKNOWN')
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from oracle import oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from ssmjs_amd import backend
    d = backend.Device(0)
    yield d
    d.destroy()


CFG = {"vocabSize": 64, "dModel": 64, "numLayers": 2, "dState": 16, "dConv": 4, "expand": 2,
       "nHeads": 2, "layers": [{"type": "mamba1"}, {"type": "mamba2"}]}


def test_alloc_failure_then_recovery(device, monkeypatch):
    case("SSM_HIP_FAULT=alloc")
    from ssmjs_amd import _lib, backend
    monkeypatch.setenv("SSM_HIP_FAULT", "alloc")
    with pytest.raises(_lib.SsmError) as e:
        backend.Model(device, CFG, seed=1)
    assert e.value.status == 6 and e.value.code == "UNKNOWN"   # SSM_ERR_OUT_OF_MEMORY
    monkeypatch.delenv("SSM_HIP_FAULT")
    m = backend.Model(device, CFG, seed=1)
    # a workspace that has to grow under the fault fails the call, not the model
    monkeypatch.setenv("SSM_HIP_FAULT", "alloc")
    ids = np.arange(40, dtype=np.uint32).reshape(2, 20) % 64
    with pytest.raises(_lib.SsmError) as e:
        m.forward(ids)
    assert e.value.status == 6
    monkeypatch.delenv("SSM_HIP_FAULT")
    out = m.forward(ids)
    ref = O.Model(m.export_weights()).forward(ids)
    assert np.abs(out - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    m.destroy()


def test_launch_failure_then_recovery(device, monkeypatch):
    case("SSM_HIP_FAULT=launch")
    from ssmjs_amd import _lib, backend
    m = backend.Model(device, CFG, seed=2)
    ids = np.arange(30, dtype=np.uint32).reshape(1, 30) % 64
    monkeypatch.setenv("SSM_HIP_FAULT", "launch")
    with pytest.raises(_lib.SsmError) as e:
        m.forward(ids)
    assert e.value.status == 5 and e.value.code == "UNKNOWN"   # SSM_ERR_HIP
    assert "injected" in str(e.value)
    st = m.new_state(1)
    with pytest.raises(_lib.SsmError):
        st.prefill(ids)
    monkeypatch.delenv("SSM_HIP_FAULT")
    device.synchronize()
    out = m.forward(ids)
    ref = O.Model(m.export_weights()).forward(ids)
    assert np.abs(out - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    st.destroy()
    m.destroy()


def test_session_create_reports_model_failure(monkeypatch):
    """MambaSession.create with every allocation failing: the device opens (no allocation), the
    model construction fails and the session raises SessionError('UNKNOWN') as session.ts
    does for a throwing HybridMambaModel constructor."""
    case("MambaSession.create under SSM_HIP_FAULT=alloc")
    from ssmjs_amd import ByteTokenizer, MambaSession, SessionError
    monkeypatch.setenv("SSM_HIP_FAULT", "alloc")
    with pytest.raises(SessionError) as e:
        MambaSession.create({"tokenizer": ByteTokenizer(256), "mambaVersion": "mamba1",
                             "modelSize": "nano"})
    assert e.value.code == "UNKNOWN"
