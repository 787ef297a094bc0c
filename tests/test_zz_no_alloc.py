"""ssm_sample_noalloc (the allocation-free sampler: static device scratch, no hipMalloc) against
ssm_sample with a caller workspace, through the C ABI: the picked indices must be identical
(index work is bit-exact), on two calls in a row, the second smaller than the first, so that
stale scratch contents from the first call cannot leak into the second. A call beyond the
static scratch is refused with SSM_ERR_UNSUPPORTED before anything is launched."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _pick(noalloc, logits, u, T, K, P):
    from ssmjs_amd import _lib
    rows, n = logits.shape
    out = torch.full((rows,), 0xFFFFFFFF, dtype=torch.int64, device="cuda").to(torch.int32)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        _lib.call("ssm_sample_noalloc", logits.data_ptr(), logits.stride(0), rows, n, float(T),
                  int(K), float(P), u.data_ptr(), out.data_ptr(), stream)
    else:
        wsb = _lib.lib().ssm_sample_workspace(rows, n)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        _lib.call("ssm_sample", logits.data_ptr(), logits.stride(0), rows, n, float(T), int(K),
                  float(P), u.data_ptr(), out.data_ptr(), ws.data_ptr(), wsb, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32).copy()


@pytest.mark.parametrize("T,K,P", [(0.8, 50, 0.9), (1.0, 1, 0.9), (1.3, 1024, 1.0)])
def test_noalloc_sampler_matches_workspace_sampler(T, K, P):
    from ssmjs_amd import backend
    dev = backend.Device(0)   # ssm_ctx_create resolves the scratch address on this device
    r = np.random.default_rng(91)
    for rows, n in ((64, 32000), (3, 700)):   # second call smaller than the first
        case(f"noalloc sampler rows={rows} n={n} T={T} topK={K} topP={P}")
        lg = (3.0 * r.standard_normal((rows, n))).astype(np.float32)
        lg[0, :8] = lg[0].max()                    # a plateau of equal maxima in row 0
        logits = torch.from_numpy(lg).cuda()
        u = torch.from_numpy(r.random(rows)).cuda()
        want = _pick(False, logits, u, T, K, P)
        got = _pick(True, logits, u, T, K, P)
        np.testing.assert_array_equal(got, want)
        assert (got < n).all()
    dev.destroy()


def test_noalloc_sampler_refuses_beyond_scratch():
    case("noalloc sampler beyond the static scratch")
    from ssmjs_amd import _lib
    rows, n = 64, 262144    # 64 MiB of keys: beyond the 32 MiB scratch
    logits = torch.zeros(1, dtype=torch.float32, device="cuda")   # never read
    u = torch.zeros(1, dtype=torch.float64, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.SsmError) as e:
        _lib.call("ssm_sample_noalloc", logits.data_ptr(), n, rows, n, 0.8, 50, 0.9,
                  u.data_ptr(), out.data_ptr(), None)
    assert "scratch" in str(e.value)
