"""GPU parity at BASELINE.json's full sizes. The whole problem runs on the GPU in one call
and every output element and final state is compared with the CPU oracle (the C oracle's
sequential recurrence, OpenMP over sequences: about half a second per configuration on 16
cores); one property that holds at any size is checked on the whole output as well.

- SSD, config 3 (B=8 L=4096 H=64 P=64 N=128, fp32 inputs): all 512 (batch, head) sequences
  and their final states against the oracle, per element; the sequence run as two halves,
  the second seeded with the first half's final state, gives the same y and final state as
  one run (the chunk recurrence carried across launches).
- SSD, config 3 with bf16 inputs: all sequences and final states.
- SSD, config 5 (B=1 L=65536 H=32, bf16 inputs; the segmented path: state-only pass, combine,
  full pass): all 32 heads and their final states.
- Mamba-1 scan, config 2 (B=4 L=2048 D=1536 N=16, the single-pass kernel): all channels of
  every sequence and their final states, per element.

Tolerances as in test_gpu_kernels.py: fp32 per element |gpu - oracle| <= 1e-4 |oracle| +
1e-5 max|oracle|; bf16 inputs max|gpu - oracle| / max(1, max|oracle|) <= 2e-2, the oracle
getting the same bf16-rounded inputs as float32.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from oracle import oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu

F32_TOL, F32_FLOOR, BF16_TOL = 1e-4, 1e-5, 2e-2


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from ssmjs_amd import kernels  # noqa: F401


def K():
    from ssmjs_amd import kernels
    return kernels


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def _rows(a):
    """Leading-axis slices of at most 2**24 elements (bounded float64 temporaries)."""
    a = np.asarray(a)
    if a.ndim == 0 or a.size <= (1 << 24):
        return [a]
    step = max(1, (1 << 24) // max(1, a.size // a.shape[0]))
    return [a[i:i + step] for i in range(0, a.shape[0], step)]


def check_f32(got, ref, what):
    assert np.shape(got) == np.shape(ref), f"{what}: shape {np.shape(got)} vs {np.shape(ref)}"
    scale = float(np.abs(ref).max())
    ratio = 0.0
    for g, r_ in zip(_rows(got), _rows(ref)):
        g, r_ = g.astype(np.float64), r_.astype(np.float64)
        assert np.isfinite(g).all(), f"{what}: non-finite values"
        bound = F32_TOL * np.abs(r_) + F32_FLOOR * scale
        ratio = max(ratio, float((np.abs(g - r_) / bound).max()))
    print(f"  {what}: worst |err| / bound {ratio:.3f}", flush=True)
    assert ratio <= 1.0, f"{what}: an element exceeds 1e-4 relative + 1e-5 of max ({ratio:.2f}x)"


def check_bf16(got, ref, what):
    assert np.shape(got) == np.shape(ref), f"{what}: shape {np.shape(got)} vs {np.shape(ref)}"
    err = 0.0
    for g, r_ in zip(_rows(got), _rows(ref)):
        g, r_ = g.astype(np.float64), r_.astype(np.float64)
        assert np.isfinite(g).all(), f"{what}: non-finite values"
        err = max(err, float(np.abs(g - r_).max()))
    e = err / max(1.0, float(np.abs(ref).max()))
    print(f"  {what}: err {e:.2e}", flush=True)
    assert e <= BF16_TOL, f"{what}: {e:.2e} beyond {BF16_TOL}"


def bf16_round(a):
    return torch.from_numpy(a).to(torch.bfloat16).float().numpy()


def ssd_inputs(r, B, L, H, P, N, bc_scale):
    """Config 3's distributions: x, B, C ~ N(0,1) (B, C times bc_scale), dt = N(0,1) - 3 before
    the softplus, A ~ -U(1,16)."""
    x = r.standard_normal((B, L, H, P), dtype=np.float32)
    dt = (r.standard_normal((B, L, H), dtype=np.float32) - 3.0).astype(np.float32)
    A = -r.uniform(1.0, 16.0, H).astype(np.float32)
    Bm = (bc_scale * r.standard_normal((B, L, 1, N), dtype=np.float32)).astype(np.float32)
    Cm = (bc_scale * r.standard_normal((B, L, 1, N), dtype=np.float32)).astype(np.float32)
    Dk = r.standard_normal(H).astype(np.float32)
    return x, dt, A, Bm, Cm, Dk


def oracle_all(x, dt, A, Bm, Cm, Dk):
    """The oracle on every (batch, head) sequence over its full length (one group)."""
    return O.ssd(x, dt, A, Bm, Cm, Dk, return_state=True)


def test_ssd_config3_full_size_f32():
    B, L, H, P, N = 8, 4096, 64, 64, 128
    case(f"ssd full size cfg3 f32 B={B} L={L} H={H}")
    r = np.random.default_rng(3003)
    x, dt, A, Bm, Cm, Dk = ssd_inputs(r, B, L, H, P, N, 1.0)
    tx, tdt, tA, tB, tC, tD = dev(x), dev(dt), dev(A), dev(Bm), dev(Cm), dev(Dk)
    hT = torch.zeros(B, H, P, N, device="cuda")
    y = K().ssd_chunk_scan(tx, tdt, tA, tB, tC, tD, None, True, hT=hT)
    yh, hTh = host(y), host(hT)
    ry, rh = oracle_all(x, dt, A, Bm, Cm, Dk)
    check_f32(yh, ry, "y (all 512 sequences)")
    check_f32(hTh, rh, "final states (all 512)")
    del ry, rh
    # two halves, the second seeded with the first half's final state
    Lh = L // 2
    hm = torch.zeros(B, H, P, N, device="cuda")
    y1 = K().ssd_chunk_scan(tx[:, :Lh].contiguous(), tdt[:, :Lh].contiguous(), tA,
                            tB[:, :Lh].contiguous(), tC[:, :Lh].contiguous(), tD, None, True,
                            hT=hm)
    h2 = torch.zeros(B, H, P, N, device="cuda")
    y2 = K().ssd_chunk_scan(tx[:, Lh:].contiguous(), tdt[:, Lh:].contiguous(), tA,
                            tB[:, Lh:].contiguous(), tC[:, Lh:].contiguous(), tD, None, True,
                            h0=hm, hT=h2)
    check_f32(np.concatenate([host(y1), host(y2)], axis=1), yh, "y from two halves")
    check_f32(host(h2), hTh, "final state from two halves")


def test_ssd_config3_full_size_bf16():
    B, L, H, P, N = 8, 4096, 64, 64, 128
    case(f"ssd full size cfg3 bf16 B={B} L={L} H={H}")
    r = np.random.default_rng(3103)
    x, dt, A, Bm, Cm, Dk = ssd_inputs(r, B, L, H, P, N, 1.0)
    x, Bm, Cm = bf16_round(x), bf16_round(Bm), bf16_round(Cm)
    hT = torch.zeros(B, H, P, N, device="cuda")
    y = K().ssd_chunk_scan(dev(x, torch.bfloat16), dev(dt), dev(A), dev(Bm, torch.bfloat16),
                           dev(Cm, torch.bfloat16), dev(Dk), None, True, hT=hT)
    yh, hTh = host(y), host(hT)
    ry, rh = oracle_all(x, dt, A, Bm, Cm, Dk)
    check_bf16(yh, ry, "y (all 512 sequences)")
    check_bf16(hTh, rh, "final states (all 512)")


def test_ssd_config5_full_size_bf16():
    B, L, H, P, N = 1, 65536, 32, 64, 128
    case(f"ssd full size cfg5 bf16 B={B} L={L} H={H}")
    r = np.random.default_rng(5005)
    x, dt, A, Bm, Cm, Dk = ssd_inputs(r, B, L, H, P, N, 128 ** -0.25)
    x, Bm, Cm = bf16_round(x), bf16_round(Bm), bf16_round(Cm)
    hT = torch.zeros(B, H, P, N, device="cuda")
    y = K().ssd_chunk_scan(dev(x, torch.bfloat16), dev(dt), dev(A), dev(Bm, torch.bfloat16),
                           dev(Cm, torch.bfloat16), dev(Dk), None, True, hT=hT)
    yh, hTh = host(y), host(hT)
    ry, rh = oracle_all(x, dt, A, Bm, Cm, Dk)
    check_bf16(yh, ry, "y (all 32 heads)")
    check_bf16(hTh, rh, "final states (all 32 heads)")


def test_scan_config2_full_size():
    B, L, D, N = 4, 2048, 1536, 16
    case(f"selective scan full size cfg2 B={B} L={L} D={D} N={N}")
    r = np.random.default_rng(2002)
    u = r.standard_normal((B, L, D), dtype=np.float32)
    z = r.standard_normal((B, L, D), dtype=np.float32)
    dt = (0.5 * r.standard_normal((B, L, D), dtype=np.float32) - 1.0).astype(np.float32)
    Bm = r.standard_normal((B, L, N), dtype=np.float32)
    Cm = r.standard_normal((B, L, N), dtype=np.float32)
    A = -np.exp(r.uniform(0.0, np.log(16.0), (D, N))).astype(np.float32)
    Dk = r.standard_normal(D).astype(np.float32)
    hT = torch.zeros(B, D, N, device="cuda")
    y = K().selective_scan(dev(u), dev(dt), dev(A), dev(Bm), dev(Cm), dev(Dk), dev(z), hT=hT)
    yh, hTh = host(y), host(hT)
    ry, rh = O.selective_scan(u, dt, A, Bm, Cm, Dk, z, return_state=True)
    check_f32(yh, ry, "y (all channels and sequences)")
    check_f32(hTh, rh, "final states (all channels)")
