"""Kernel-level entry points of libssm_hip.so on torch device tensors.

torch supplies device memory and the current HIP stream only; every computation runs in
the HIP kernels of libssm_hip.so. All tensors must live on a HIP device; a CPU tensor is an
error (there is no CPU path).

Shapes (row-major):
  causal_conv1d    x (B,L,C) [row stride may exceed C], w (C,K) -> y (B,L,C)
  selective_scan   u, dt, z (B,L,D); B, C (B,L,N); A (D,N); state (B,D,N)
  ssd_chunk_scan   x (B,L,H,P); dt (B,L,H); B, C (B,L,G,N); A (H); state (B,H,P,N)
"""
from __future__ import annotations

import torch

from . import _lib
from .backend import sample_supported  # noqa: F401  (re-export)

_NULL = None


def _p(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("ssmjs_amd kernels need HIP device tensors (no CPU path)")
    return t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _rows(t, width):
    """Row stride (elements between consecutive time steps) of a (..., width) view whose
    last dim is contiguous and whose leading dims flatten to rows."""
    if t.stride(-1) != 1:
        raise ValueError("last dimension must be contiguous")
    return t.stride(-2) if t.dim() >= 2 else width


def _f32(t):
    if t is not None and t.dtype != torch.float32:
        raise TypeError(f"expected float32, got {t.dtype}")
    return t


def causal_conv1d(x, w, bias=None, silu=True, state_in=None, state_out=None, out=None):
    B, L, Cc = x.shape
    K = w.shape[1]
    _f32(x)
    y = out if out is not None else torch.empty(B, L, Cc, device=x.device, dtype=torch.float32)
    if x.stride(2) != 1 or (L > 1 and x.stride(0) != L * x.stride(1)):
        raise ValueError("x must be a row-strided (B,L,C) view")
    ldx = x.stride(1)
    _lib.call("ssm_causal_conv1d", _p(x), ldx, _p(w.contiguous()), _p(bias), _p(y), y.stride(1),
              B, L, Cc, K, int(silu), _p(state_in), _p(state_out), _stream())
    return y


def conv1d_update(x, w, bias, state, silu=True, out=None):
    B, Cc = x.shape
    y = out if out is not None else torch.empty(B, Cc, device=x.device, dtype=torch.float32)
    _lib.call("ssm_conv1d_update", _p(x), x.stride(0), _p(w.contiguous()), _p(bias), _p(y),
              y.stride(0), _p(state), B, Cc, w.shape[1], int(silu), _stream())
    return y


def selective_scan(u, dt, A, Bm, Cm, D=None, z=None, dt_bias=None, softplus=True, h0=None,
                   hT=None, out=None):
    B, L, Dd = u.shape
    N = A.shape[1]
    y = out if out is not None else torch.empty(B, L, Dd, device=u.device, dtype=torch.float32)
    nbytes = _lib.lib().ssm_selective_scan_workspace(B, L, Dd, N)
    ws = torch.empty(max(nbytes, 4), device=u.device, dtype=torch.uint8)
    for t in (u, dt, Bm, Cm, z):
        if t is not None and t.dim() == 3 and t.shape[1] > 1 and t.stride(0) != t.shape[1] * t.stride(1):
            raise ValueError("row-strided (B,L,X) views only")
    _lib.call("ssm_selective_scan", _p(u), u.stride(1), _p(dt), dt.stride(1), _p(dt_bias),
              int(softplus), _p(A.contiguous()), _p(Bm), Bm.stride(1), _p(Cm), Cm.stride(1),
              _p(D), _p(z), z.stride(1) if z is not None else 0, _p(y), y.stride(1), B, L, Dd, N,
              _p(h0), _p(hT), _p(ws), ws.numel(), _stream())
    return y


def m1_state_update(x, dt, A, Bm, Cm, D, z, dt_bias, h, softplus=True, out=None):
    B, Dd = x.shape
    N = A.shape[1]
    y = out if out is not None else torch.empty(B, Dd, device=x.device, dtype=torch.float32)
    _lib.call("ssm_m1_state_update", _p(x), x.stride(0), _p(dt), dt.stride(0), _p(dt_bias),
              int(softplus), _p(A.contiguous()), _p(Bm), Bm.stride(0), _p(Cm), Cm.stride(0),
              _p(D), _p(z), z.stride(0) if z is not None else 0, _p(y), y.stride(0), _p(h), B, Dd,
              N, _stream())
    return y


def ssd_workspace(B, L, H, P, G, N, device):
    n = _lib.lib().ssm_ssd_workspace(B, L, H, P, G, N)
    return torch.empty(max(n, 4), device=device, dtype=torch.uint8)


def ssd_chunk_scan(x, dt, A, Bm, Cm, D=None, dt_bias=None, softplus=True, dt_min=0.0,
                   dt_max=float("inf"), h0=None, hT=None, out=None, workspace=None):
    """x (B,L,H,P), Bm/Cm (B,L,G,N) in float32 or bfloat16 (same dtype); y is float32."""
    B, L, H, P = x.shape
    G, N = Bm.shape[2], Bm.shape[3]
    if x.dtype == torch.float32:
        dtype = _lib.SSM_F32
    elif x.dtype == torch.bfloat16:
        dtype = _lib.SSM_BF16
    else:
        raise TypeError("x must be float32 or bfloat16")
    if Bm.dtype != x.dtype or Cm.dtype != x.dtype:
        raise TypeError("x, B and C must share a dtype")
    y = out if out is not None else torch.empty(B, L, H, P, device=x.device, dtype=torch.float32)
    ws = workspace if workspace is not None else ssd_workspace(B, L, H, P, G, N, x.device)
    ldx = x.stride(1)
    _lib.call("ssm_ssd_chunk_scan", dtype, _p(x), ldx, _p(dt), dt.stride(1), _p(dt_bias),
              int(softplus), float(dt_min), float(dt_max), _p(A), _p(Bm), Bm.stride(1), _p(Cm),
              Cm.stride(1), _p(D), _p(y), y.stride(1), B, L, H, P, G, N, _p(h0), _p(hT), _p(ws),
              ws.numel(), _stream())
    return y


def m2_state_update(x, dt, A, Bm, Cm, D, dt_bias, h, z=None, softplus=True, dt_min=0.0,
                    dt_max=float("inf"), out=None):
    """x (B,H,P); dt (B,H); Bm, Cm (B,G,N); h (B,H,P,N) updated in place."""
    B, H, P = x.shape
    G, N = Bm.shape[1], Bm.shape[2]
    y = out if out is not None else torch.empty(B, H, P, device=x.device, dtype=torch.float32)
    _lib.call("ssm_m2_state_update", _p(x), x.stride(0), _p(dt), dt.stride(0), _p(dt_bias),
              int(softplus), float(dt_min), float(dt_max), _p(A), _p(Bm), Bm.stride(0), _p(Cm),
              Cm.stride(0), _p(D), _p(z), z.stride(0) if z is not None else 0, _p(y), y.stride(0),
              _p(h), B, H, P, G, N, _stream())
    return y


def rmsnorm(x, w, eps=1e-5, out=None):
    M, n = x.shape
    y = out if out is not None else torch.empty_like(x)
    _lib.call("ssm_rmsnorm", _p(x), x.stride(0), _p(w), _p(y), y.stride(0), M, n, float(eps),
              _stream())
    return y


def argmax(x, out=None):
    """Row-wise greedy pick (ssm_argmax): lowest index among equal maxima, NaN never wins."""
    rows, n = x.shape
    o = out if out is not None else torch.empty(rows, dtype=torch.int32, device=x.device)
    _lib.call("ssm_argmax", _p(x), x.stride(0), rows, n, _p(o), _stream())
    return o


def sample_workspace(rows, n, device):
    """Workspace for sample (ssm_sample_workspace bytes)."""
    return torch.empty(max(1, _lib.lib().ssm_sample_workspace(rows, n)), dtype=torch.uint8,
                       device=device)


def sample(x, u, temperature=1.0, topK=50, topP=0.9, out=None, workspace=None):
    """sampleToken per row on the device (ssm_sample, src/session/streaming.ts:53-97).

    x: (rows, n) fp32 logits; u: (rows,) float64 draws in [0, 1) (Math.random()). Returns
    (rows,) int32 picks. Raises for n > 262144 or min(topK, n) > 1024."""
    rows, n = x.shape
    assert u.dtype == torch.float64 and u.numel() == rows and u.is_contiguous()
    o = out if out is not None else torch.empty(rows, dtype=torch.int32, device=x.device)
    ws = workspace if workspace is not None else sample_workspace(rows, n, x.device)
    _lib.call("ssm_sample", _p(x), x.stride(0), rows, n, float(temperature), int(topK),
              float(topP), _p(u), _p(o), _p(ws), ws.numel(), _stream())
    return o


def linear_rows_workspace(M, N, K, device):
    """Split-K workspace for linear_rows (None when the shape never splits)."""
    n = _lib.lib().ssm_linear_rows_workspace(M, N, K)
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def linear_rows(x, W, mode=0, g=None, z=None, eps=1e-5, out=None, beta=0.0, workspace=None):
    """y = beta*y + s * p(x) W^T for M <= 64 rows (ssm_linear_rows): mode 0 plain, 1 RMSNorm
    (weight g), 2 gated RMSNorm (z, weight g). `workspace` (linear_rows_workspace) lets the
    kernel split K; without it the kernel runs unsplit."""
    M, K = x.shape
    N = W.shape[0]
    y = out if out is not None else torch.zeros(M, N, device=x.device, dtype=torch.float32)
    ws = _p(workspace) if workspace is not None else None
    nws = workspace.numel() if workspace is not None else 0
    _lib.call("ssm_linear_rows", mode, _p(x), x.stride(0), _p(z) if z is not None else None,
              z.stride(0) if z is not None else 0, _p(g) if g is not None else None, _p(W),
              _p(y), y.stride(0), M, N, K, float(beta), float(eps), ws, nws, _stream())
    return y


def linear(x, W, bias=None, out=None, beta=0.0):
    """y = beta*y + x W^T (+ bias) for any number of rows (ssm_linear, fp32 matrix cores)."""
    M, K = x.shape
    N = W.shape[0]
    y = out if out is not None else torch.zeros(M, N, device=x.device, dtype=torch.float32)
    _lib.call("ssm_linear", _p(x), x.stride(0), _p(W), W.stride(0),
              _p(bias) if bias is not None else None, _p(y), y.stride(0), M, N, K, float(beta),
              _stream())
    return y


def m1_xproj_dt(x, Wx, Wdt, d_state):
    """Mamba-1 x_proj then dt_proj in one pass (ssm_m1_xproj_dt): returns (dbl, dt) with
    dbl = x Wx^T (T, R + 2N) and dt = dbl[:, :R] Wdt^T (T, D)."""
    T, D = x.shape
    R = Wdt.shape[1]
    dbl = torch.empty(T, R + 2 * d_state, device=x.device, dtype=torch.float32)
    dt = torch.empty(T, D, device=x.device, dtype=torch.float32)
    _lib.call("ssm_m1_xproj_dt", _p(x), x.stride(0), _p(Wx), _p(Wdt), _p(dbl), dbl.stride(0),
              _p(dt), dt.stride(0), T, D, R, d_state, _stream())
    return dbl, dt


def gated_rmsnorm(x, z, w, groups=1, eps=1e-5, out=None):
    M, n = x.shape
    y = out if out is not None else torch.empty_like(x)
    _lib.call("ssm_gated_rmsnorm", _p(x), x.stride(0), _p(z), z.stride(0), _p(w), _p(y),
              y.stride(0), M, n, groups, float(eps), _stream())
    return y
