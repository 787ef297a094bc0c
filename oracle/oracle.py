"""ctypes wrapper over oracle/libssm_oracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement in ssm_oracle.c is the checker for the HIP path. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the
product package (ssmjs_amd) never does.

Every function takes numpy float32 arrays and returns numpy arrays. Shapes follow the
canonical Mamba layouts (row-major, last index fastest):
  conv1d       x (B,L,C) -> y (B,L,C);  w (C,K)
  selective    u, dt, z (B,L,D); Bm, Cm (B,L,N); A (D,N); state (B,D,N)
  ssd          x, z (B,L,H,P); dt (B,L,H); Bm, Cm (B,L,G,N); A (H); state (B,H,P,N)
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# SSM_ORACLE_LIB selects another build of the same source (the sanitizer build of
# tests/test_sanitizers.py)
_LIB_PATH = os.environ.get("SSM_ORACLE_LIB") or os.path.join(_HERE, "libssm_oracle.so")
_lib = None

_fp = C.POINTER(C.c_float)
_u32p = C.POINTER(C.c_uint32)


def build() -> None:
    """Compile libssm_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    L.orc_causal_conv1d.argtypes = [_fp, C.c_long, _fp, _fp, _fp, C.c_long, C.c_int, C.c_int,
                                    C.c_int, C.c_int, C.c_int, _fp, _fp]
    L.orc_selective_scan.argtypes = [_fp, C.c_long, _fp, C.c_long, _fp, C.c_int, _fp, _fp,
                                     C.c_long, _fp, C.c_long, _fp, _fp, C.c_long, _fp, C.c_long,
                                     C.c_int, C.c_int, C.c_int, C.c_int, _fp, _fp]
    ssd = [_fp, C.c_long, _fp, C.c_long, _fp, C.c_int, C.c_float, C.c_float, _fp, _fp, C.c_long,
           _fp, C.c_long, _fp, _fp, C.c_long, _fp, C.c_long, C.c_int, C.c_int, C.c_int, C.c_int,
           C.c_int, C.c_int]
    L.orc_ssd_sequential.argtypes = ssd + [_fp, _fp]
    L.orc_ssd_chunked.argtypes = ssd + [C.c_int, _fp, _fp]
    L.orc_conv_update.argtypes = [_fp, _fp, _fp, _fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int]
    L.orc_m1_state_update.argtypes = [_fp, _fp, _fp, C.c_int, _fp, _fp, _fp, _fp, _fp, _fp, _fp,
                                      C.c_int, C.c_int, C.c_int]
    L.orc_m2_state_update.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float, C.c_float, _fp, _fp, _fp,
                                      _fp, _fp, _fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int]
    L.orc_linear.argtypes = [_fp, C.c_long, _fp, _fp, _fp, C.c_long, C.c_int, C.c_int, C.c_int,
                             C.c_int]
    L.orc_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_int, C.c_float]
    L.orc_sample_token.argtypes = [_fp, C.c_int, C.c_double, C.c_int, C.c_double, C.c_double]
    L.orc_sample_token.restype = C.c_int
    L.orc_gated_rmsnorm.argtypes = [_fp, C.c_long, _fp, C.c_long, _fp, _fp, C.c_long, C.c_int,
                                    C.c_int, C.c_int, C.c_float]
    L.orc_model_open.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p, C.c_int]
    L.orc_model_open.restype = C.c_void_p
    L.orc_model_close.argtypes = [C.c_void_p]
    L.orc_model_vocab.argtypes = [C.c_void_p]
    L.orc_model_forward.argtypes = [C.c_void_p, _u32p, C.c_int, C.c_int, _fp]
    L.orc_mixer_forward.argtypes = [C.c_void_p, C.c_int, _fp, C.c_int, C.c_int, _fp]
    L.orc_state_new.argtypes = [C.c_void_p, C.c_int]
    L.orc_state_new.restype = C.c_void_p
    L.orc_state_free.argtypes = [C.c_void_p]
    L.orc_model_prefill.argtypes = [C.c_void_p, C.c_void_p, _u32p, C.c_int, _fp]
    L.orc_model_decode.argtypes = [C.c_void_p, C.c_void_p, _u32p, _fp]
    L.orc_state_floats.argtypes = [C.c_void_p]
    L.orc_state_floats.restype = C.c_size_t
    L.orc_state_read.argtypes = [C.c_void_p, C.c_void_p, _fp]
    L.orc_state_write.argtypes = [C.c_void_p, C.c_void_p, _fp]
    L.orc_num_threads.restype = C.c_int


def num_threads() -> int:
    """Threads of the oracle's OpenMP loops (OMP_NUM_THREADS, else every host core)."""
    return int(lib().orc_num_threads())


def _f(a):
    """float32 C-contiguous view pointer (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "oracle wants contiguous float32"
    return a.ctypes.data_as(_fp)


def _c32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def causal_conv1d(x, w, bias=None, silu=True, state_in=None, return_state=False):
    x, w, bias, state_in = map(_c32, (x, w, bias, state_in))
    B, L, Cc = x.shape
    K = w.shape[1]
    y = np.empty_like(x)
    st = np.empty((B, Cc, K - 1), np.float32) if return_state else None
    lib().orc_causal_conv1d(_f(x), Cc, _f(w), _f(bias), _f(y), Cc, B, L, Cc, K, int(silu),
                            _f(state_in), _f(st))
    return (y, st) if return_state else y


def selective_scan(u, dt, A, Bm, Cm, D=None, z=None, dt_bias=None, softplus=True, h0=None,
                   return_state=False):
    u, dt, A, Bm, Cm, D, z, dt_bias, h0 = map(_c32, (u, dt, A, Bm, Cm, D, z, dt_bias, h0))
    B, L, Dd = u.shape
    N = A.shape[1]
    y = np.empty_like(u)
    hT = np.empty((B, Dd, N), np.float32) if return_state else None
    lib().orc_selective_scan(_f(u), Dd, _f(dt), Dd, _f(dt_bias), int(softplus), _f(A), _f(Bm), N,
                             _f(Cm), N, _f(D), _f(z), Dd, _f(y), Dd, B, L, Dd, N, _f(h0), _f(hT))
    return (y, hT) if return_state else y


def _ssd_args(x, dt, A, Bm, Cm, D, z, dt_bias, h0):
    x, dt, A, Bm, Cm, D, z, dt_bias, h0 = map(_c32, (x, dt, A, Bm, Cm, D, z, dt_bias, h0))
    return x, dt, A, Bm, Cm, D, z, dt_bias, h0


def ssd(x, dt, A, Bm, Cm, D=None, z=None, dt_bias=None, softplus=True, dt_min=0.0,
        dt_max=float("inf"), h0=None, return_state=False, chunk=None):
    """Mamba-2 SSD. chunk=None runs the sequential recurrence, else the chunked algorithm."""
    x, dt, A, Bm, Cm, D, z, dt_bias, h0 = _ssd_args(x, dt, A, Bm, Cm, D, z, dt_bias, h0)
    B, L, H, P = x.shape
    G, N = Bm.shape[2], Bm.shape[3]
    y = np.empty_like(x)
    hT = np.empty((B, H, P, N), np.float32) if return_state else None
    args = [_f(x), H * P, _f(dt), H, _f(dt_bias), int(softplus), dt_min, dt_max, _f(A), _f(Bm),
            G * N, _f(Cm), G * N, _f(D), _f(z), H * P, _f(y), H * P, B, L, H, P, G, N]
    if chunk is None:
        lib().orc_ssd_sequential(*args, _f(h0), _f(hT))
    else:
        lib().orc_ssd_chunked(*args, int(chunk), _f(h0), _f(hT))
    return (y, hT) if return_state else y


def conv_update(x, w, bias, state, silu=True):
    """One token; returns (y, new_state) without modifying the inputs."""
    x, w, bias = map(_c32, (x, w, bias))
    st = np.array(state, dtype=np.float32, copy=True, order="C")
    B, Cc = x.shape
    y = np.empty_like(x)
    lib().orc_conv_update(_f(x), _f(w), _f(bias), _f(y), _f(st), B, Cc, w.shape[1], int(silu))
    return y, st


def m1_state_update(x, dt, A, Bm, Cm, D, z, dt_bias, h, softplus=True):
    x, dt, A, Bm, Cm, D, z, dt_bias = map(_c32, (x, dt, A, Bm, Cm, D, z, dt_bias))
    hh = np.array(h, dtype=np.float32, copy=True, order="C")
    B, Dd = x.shape
    y = np.empty_like(x)
    lib().orc_m1_state_update(_f(x), _f(dt), _f(dt_bias), int(softplus), _f(A), _f(Bm), _f(Cm),
                              _f(D), _f(z), _f(y), _f(hh), B, Dd, A.shape[1])
    return y, hh


def m2_state_update(x, dt, A, Bm, Cm, D, dt_bias, h, z=None, softplus=True, dt_min=0.0,
                    dt_max=float("inf")):
    x, dt, A, Bm, Cm, D, z, dt_bias = map(_c32, (x, dt, A, Bm, Cm, D, z, dt_bias))
    hh = np.array(h, dtype=np.float32, copy=True, order="C")
    B, H, P = x.shape
    G, N = Bm.shape[1], Bm.shape[2]
    y = np.empty_like(x)
    lib().orc_m2_state_update(_f(x), _f(dt), _f(dt_bias), int(softplus), dt_min, dt_max, _f(A),
                              _f(Bm), _f(Cm), _f(D), _f(z), _f(y), _f(hh), B, H, P, G, N)
    return y, hh


def linear(x, W, bias=None):
    x, W, bias = map(_c32, (x, W, bias))
    M, K = x.shape
    y = np.empty((M, W.shape[0]), np.float32)
    lib().orc_linear(_f(x), K, _f(W), _f(bias), _f(y), W.shape[0], M, K, W.shape[0], 0)
    return y


def sample_token(logits, temperature, topK, topP, u) -> int:
    """sampleToken (src/session/streaming.ts:53-97) on one row with Math.random() = u."""
    lg = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    r = lib().orc_sample_token(_f(lg), lg.size, float(temperature), int(topK), float(topP),
                               float(u))
    if r < 0:
        raise ValueError("sample_token: needs n >= 1 and topK >= 1")
    return r


def rmsnorm(x, w, eps=1e-5):
    x, w = map(_c32, (x, w))
    y = np.empty_like(x)
    lib().orc_rmsnorm(_f(x), _f(w), _f(y), x.shape[0], x.shape[1], eps)
    return y


def gated_rmsnorm(x, z, w, groups=1, eps=1e-5):
    x, z, w = map(_c32, (x, z, w))
    y = np.empty_like(x)
    M, n = x.shape
    lib().orc_gated_rmsnorm(_f(x), n, _f(z), n, _f(w), _f(y), n, M, n, groups, eps)
    return y


class Model:
    """A checkpoint image (bytes in the ssmjs_amd "SSMW" format) opened by the oracle."""

    def __init__(self, blob: bytes):
        self._blob = C.create_string_buffer(bytes(blob), len(blob))
        err = C.create_string_buffer(256)
        self._h = lib().orc_model_open(C.cast(self._blob, C.c_void_p), len(blob), err, 256)
        if not self._h:
            raise ValueError("oracle rejected checkpoint: " + err.value.decode())
        self.vocab = lib().orc_model_vocab(self._h)

    def close(self):
        if self._h:
            lib().orc_model_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        B, L = ids.shape
        out = np.empty((B, L, self.vocab), np.float32)
        lib().orc_model_forward(self._h, ids.ctypes.data_as(_u32p), B, L, _f(out))
        return out

    def mixer(self, layer, x):
        """Mixer of `layer` (no norm / residual) on hidden states x (B, L, d)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        B, L, _ = x.shape
        out = np.empty_like(x)
        lib().orc_mixer_forward(self._h, layer, _f(x), B, L, _f(out))
        return out

    def new_state(self, B):
        return _State(self, B)


class _State:
    def __init__(self, model: Model, B: int):
        self.m = model
        self.B = B
        self._h = lib().orc_state_new(model._h, B)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_state_free(self._h)
            self._h = None

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        assert ids.shape[0] == self.B
        out = np.empty((self.B, self.m.vocab), np.float32)
        lib().orc_model_prefill(self.m._h, self._h, ids.ctypes.data_as(_u32p), ids.shape[1],
                                _f(out))
        return out

    def decode(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(self.B)
        out = np.empty((self.B, self.m.vocab), np.float32)
        lib().orc_model_decode(self.m._h, self._h, ids.ctypes.data_as(_u32p), _f(out))
        return out

    def read(self):
        out = np.empty(lib().orc_state_floats(self._h), np.float32)
        lib().orc_state_read(self.m._h, self._h, _f(out))
        return out

    def write(self, img):
        img = np.ascontiguousarray(img, dtype=np.float32)
        assert img.size == lib().orc_state_floats(self._h)
        lib().orc_state_write(self.m._h, self._h, _f(img))


def greedy(model: Model, prompt, n_new: int, eos_id: int = -1):
    """Greedy continuation of prompt (B, Lp): prefill then recurrent decode; argmax with the
    lowest index on ties (the topK=1 case of sampleToken, src/session/streaming.ts:74-75).
    Returns (ids (B, n_new), margins (B, n_new)) where margin = top1 - top2 logit."""
    prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
    B = prompt.shape[0]
    st = model.new_state(B)
    logits = st.prefill(prompt)
    ids = np.zeros((B, n_new), np.uint32)
    margins = np.zeros((B, n_new), np.float64)
    for s in range(n_new):
        nxt = np.argmax(logits, axis=1)
        srt = np.sort(logits, axis=1)
        margins[:, s] = srt[:, -1].astype(np.float64) - srt[:, -2]
        ids[:, s] = nxt
        if s + 1 < n_new:
            logits = st.decode(nxt.astype(np.uint32))
    return ids, margins
