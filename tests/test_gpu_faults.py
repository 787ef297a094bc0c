"""Failure handling forced from the host (ssm_set_fault_injection), as SURVEY's auxiliary plan asks:
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


@pytest.fixture
def inject():
    """Sets the library's injected fault for one test and always clears it afterwards."""
    from ssmjs_amd import _lib

    def set_kind(kind):
        _lib.call("ssm_set_fault_injection", None if kind is None else kind.encode())
    yield set_kind
    set_kind(None)


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


def test_alloc_failure_then_recovery(device, inject):
    case("injected fault: alloc")
    from ssmjs_amd import _lib, backend
    inject("alloc")
    with pytest.raises(_lib.SsmError) as e:
        backend.Model(device, CFG, seed=1)
    assert e.value.status == 6 and e.value.code == "UNKNOWN"   # SSM_ERR_OUT_OF_MEMORY
    inject(None)
    m = backend.Model(device, CFG, seed=1)
    # a workspace that has to grow under the fault fails the call, not the model
    inject("alloc")
    ids = np.arange(40, dtype=np.uint32).reshape(2, 20) % 64
    with pytest.raises(_lib.SsmError) as e:
        m.forward(ids)
    assert e.value.status == 6
    inject(None)
    out = m.forward(ids)
    ref = O.Model(m.export_weights()).forward(ids)
    assert np.abs(out - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    m.destroy()


def test_launch_failure_then_recovery(device, inject):
    case("injected fault: launch")
    from ssmjs_amd import _lib, backend
    m = backend.Model(device, CFG, seed=2)
    ids = np.arange(30, dtype=np.uint32).reshape(1, 30) % 64
    inject("launch")
    with pytest.raises(_lib.SsmError) as e:
        m.forward(ids)
    assert e.value.status == 5 and e.value.code == "UNKNOWN"   # SSM_ERR_HIP
    assert "injected" in str(e.value)
    st = m.new_state(1)
    with pytest.raises(_lib.SsmError):
        st.prefill(ids)
    inject(None)
    device.synchronize()
    out = m.forward(ids)
    ref = O.Model(m.export_weights()).forward(ids)
    assert np.abs(out - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    st.destroy()
    m.destroy()


def test_session_create_reports_model_failure(inject):
    """MambaSession.create with every allocation failing: the device opens (no allocation), the
    model construction fails and the session raises SessionError('UNKNOWN') as session.ts
    does for a throwing HybridMambaModel constructor."""
    case("MambaSession.create under an injected alloc fault")
    from ssmjs_amd import ByteTokenizer, MambaSession, SessionError
    inject("alloc")
    with pytest.raises(SessionError) as e:
        MambaSession.create({"tokenizer": ByteTokenizer(256), "mambaVersion": "mamba1",
                             "modelSize": "nano"})
    assert e.value.code == "UNKNOWN"
