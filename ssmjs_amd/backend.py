"""Object wrappers over the model-level C ABI of libssm_hip.so (host buffers, numpy).

Device   -- a HIP device context (initWebGPU / adapter.requestDevice, session.ts:263,274;
            destroy() is device.destroy(), session.ts:592)
Model    -- device weights of one HybridMambaModel (session.ts:359)
State    -- recurrent ssm + conv state of B sequences
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


def sample_supported(n: int, topK: int) -> bool:
    """Whether the device sampler (ssm_sample / ssm_generate_sample) takes a row of n logits
    with this topK: n <= 262144 and min(topK, n) <= 1024."""
    return 1 <= n <= 262144 and topK >= 1 and min(topK, n) <= 1024


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Device:
    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        _lib.call("ssm_ctx_create", ordinal, C.byref(h))
        self._h = h
        self.ordinal = ordinal
        arch = C.create_string_buffer(64)
        cus, mem = C.c_int(), C.c_size_t()
        _lib.call("ssm_ctx_info", self._h, arch, 64, C.byref(cus), C.byref(mem))
        self.arch = arch.value.decode()
        self.compute_units = cus.value
        self.total_memory = mem.value
        self.destroyed = False

    @property
    def handle(self):
        return self._h

    def set_stream(self, stream_ptr):
        """Route all library work to an existing hipStream_t (int pointer) or back (None)."""
        _lib.call("ssm_ctx_set_stream", self._h, C.c_void_p(stream_ptr) if stream_ptr else None)

    def synchronize(self):
        _lib.call("ssm_ctx_synchronize", self._h)

    def profile(self, enable: bool = True):
        """Opt-in per-stage HIP-event timing of model-level calls."""
        _lib.call("ssm_ctx_profile", self._h, int(enable))

    def profile_report(self) -> dict:
        """{stage: (launches, total_ms)} since the last report; clears the record."""
        buf = C.create_string_buffer(1 << 16)
        _lib.call("ssm_ctx_profile_report", self._h, buf, len(buf))
        out = {}
        for line in buf.value.decode().splitlines():
            name, n, ms = line.split()
            out[name] = (int(n), float(ms))
        return out

    def destroy(self):
        if not self.destroyed:
            _lib.call("ssm_ctx_destroy", self._h)
            self.destroyed = True


def make_config(cfg: dict) -> _lib.ssm_config:
    """ssm_config from a HybridMambaModelConfig-shaped dict (camelCase keys as in
    src/session/presets.ts:107-120; `layers` is a list of {'type': ...})."""
    layers = cfg.get("layers") or [{"type": "mamba1"}] * cfg["numLayers"]
    codes = (C.c_int * max(1, len(layers)))(*[_lib.LAYER_CODES.get(l["type"], 0) for l in layers])
    c = _lib.ssm_config(
        vocab_size=cfg["vocabSize"], d_model=cfg["dModel"], n_layers=cfg["numLayers"],
        d_state=cfg["dState"], d_conv=cfg["dConv"], expand=cfg["expand"],
        n_heads=cfg["nHeads"], n_groups=cfg.get("nGroups", 1), chunk_len=cfg.get("chunkLen", 256),
        mimo_group=cfg.get("mimoGroup", 1), eos_id=cfg.get("eosId", -1),
        dt_rank=cfg.get("dtRank", 0), norm_eps=cfg.get("normEps", 0.0),
        layer_types=C.cast(codes, C.POINTER(C.c_int)))
    c._codes = codes  # keep the array alive with the struct
    return c


class Model:
    def __init__(self, device: Device, cfg: dict, seed: int = 0):
        self.device = device
        self.config = dict(cfg)
        h = C.c_void_p()
        c = make_config(cfg)
        _lib.call("ssm_model_create", device.handle, C.byref(c), C.c_uint64(seed), C.byref(h))
        self._h = h
        out = _lib.ssm_config()
        _lib.call("ssm_model_config", self._h, C.byref(out))
        self.vocab = out.vocab_size
        self.config["dtRank"] = out.dt_rank
        self.config["normEps"] = out.norm_eps

    @property
    def handle(self):
        return self._h

    def destroy(self):
        if self._h:
            _lib.call("ssm_model_destroy", self._h)
            self._h = None

    def load_weights(self, blob: bytes):
        buf = (C.c_char * len(blob)).from_buffer_copy(blob)
        _lib.call("ssm_model_load_weights", self._h, buf, len(blob))

    def export_weights(self, f16: bool = False) -> bytes:
        n = C.c_size_t()
        _lib.call("ssm_model_export_weights", self._h, int(f16), None, 0, C.byref(n))
        buf = C.create_string_buffer(n.value)
        _lib.call("ssm_model_export_weights", self._h, int(f16), buf, n.value, C.byref(n))
        return buf.raw[: n.value]

    def forward(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        if ids.ndim == 1:
            ids = ids[None]
        B, L = ids.shape
        out = np.empty((B, L, self.vocab), np.float32)
        _lib.call("ssm_forward", self._h, _ptr(ids), B, L, _ptr(out))
        return out

    def new_state(self, B: int) -> "State":
        return State(self, B)


class State:
    def __init__(self, model: Model, B: int):
        self.model = model
        self.B = B
        h = C.c_void_p()
        _lib.call("ssm_state_create", model.handle, B, C.byref(h))
        self._h = h

    def destroy(self):
        if self._h:
            _lib.call("ssm_state_destroy", self._h)
            self._h = None

    def reset(self):
        _lib.call("ssm_state_reset", self._h)

    def read(self) -> np.ndarray:
        out = np.empty(_lib.lib().ssm_state_floats(self._h), np.float32)
        _lib.call("ssm_state_read", self._h, _ptr(out))
        return out

    def write(self, img):
        img = np.ascontiguousarray(img, dtype=np.float32)
        if img.size != _lib.lib().ssm_state_floats(self._h):
            raise ValueError("state image size mismatch")
        _lib.call("ssm_state_write", self._h, _ptr(img))

    def layer_ptrs(self, layer: int):
        a, b = C.c_void_p(), C.c_void_p()
        _lib.call("ssm_state_layer", self._h, layer, C.byref(a), C.byref(b))
        return a.value, b.value

    def prefill(self, ids, want_logits=True):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        if ids.ndim == 1:
            ids = ids[None]
        assert ids.shape[0] == self.B
        lg = np.empty((self.B, self.model.vocab), np.float32) if want_logits else None
        am = np.empty(self.B, np.uint32)
        _lib.call("ssm_prefill", self.model.handle, self._h, _ptr(ids), ids.shape[1], _ptr(lg),
                  _ptr(am))
        return lg, am

    def decode(self, ids, want_logits=True):
        ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(self.B)
        lg = np.empty((self.B, self.model.vocab), np.float32) if want_logits else None
        am = np.empty(self.B, np.uint32)
        _lib.call("ssm_decode_step", self.model.handle, self._h, _ptr(ids), _ptr(lg), _ptr(am))
        return lg, am

    def generate_greedy(self, prompt, n_new: int) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        if prompt.ndim == 1:
            prompt = prompt[None]
        out = np.empty((self.B, n_new), np.uint32)
        _lib.call("ssm_generate_greedy", self.model.handle, self._h, _ptr(prompt),
                  prompt.shape[1], n_new, _ptr(out))
        return out

    def generate_sample(self, prompt, n_new: int, temperature: float, topK: int, topP: float,
                        u) -> np.ndarray:
        """ssm_generate_sample: u (n_new, B) float64 draws, token k of row b uses u[k, b]."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        if prompt.ndim == 1:
            prompt = prompt[None]
        u = np.ascontiguousarray(u, dtype=np.float64).reshape(n_new, self.B)
        out = np.empty((self.B, n_new), np.uint32)
        _lib.call("ssm_generate_sample", self.model.handle, self._h, _ptr(prompt),
                  prompt.shape[1], n_new, float(temperature), int(topK), float(topP), _ptr(u),
                  _ptr(out))
        return out
