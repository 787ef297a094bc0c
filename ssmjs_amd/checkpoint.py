"""Checkpoint image format ("SSMW") for HybridMambaModel weights.

The reference stores weights as the opaque ArrayBuffer produced by
`model.exportWeights()` (src/session/session.ts:518) and consumed by
`model.loadWeights(buf)` (src/session/session.ts:394,575); its checks are "bad magic,
version, or size mismatch" (src/session/errors.ts:9). That byte format lives in the absent
MambaCode.js package, so this module defines the build's own format, with the same three
checks, and the C library (ssm_model_load_weights / ssm_model_export_weights) reads and
writes exactly these bytes.

Layout, little-endian:
  0  char[4] "SSMW"          4  u32 version (1)      8  u32 dtype (0 = f32, 1 = f16)
  12 u32 header_bytes        16 u64 payload_bytes
  24 i32 vocab  28 i32 d_model  32 i32 n_layers  36 i32 d_state  40 i32 d_conv
  44 i32 expand 48 i32 n_heads  52 i32 n_groups  56 i32 dt_rank  60 f32 norm_eps
  64 i32 chunk_len  68 i32 eos_id  72 i32 mimo_group  76 u32 reserved
  80 u8 layer_type[n_layers] (1 = mamba1, 2 = mamba2), zero padded to a multiple of 16
  header_bytes: tensors, row-major, in the order of `tensor_specs`.
The LM head is tied to the embedding table.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"SSMW"
VERSION = 1
LAYER_CODES = {"mamba1": 1, "mamba2": 2}
LAYER_NAMES = {v: k for k, v in LAYER_CODES.items()}


@dataclass
class ModelDims:
    vocab: int
    d_model: int
    n_layers: int
    d_state: int
    d_conv: int
    expand: int
    n_heads: int
    n_groups: int
    layers: list = field(default_factory=list)     # list of "mamba1" / "mamba2"
    dt_rank: int = 0
    norm_eps: float = 1e-5
    chunk_len: int = 256
    eos_id: int = -1
    mimo_group: int = 1

    def __post_init__(self):
        if not self.dt_rank:
            self.dt_rank = math.ceil(self.d_model / 16)
        if not self.layers:
            self.layers = ["mamba1"] * self.n_layers

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def head_dim(self) -> int:
        return self.d_inner // self.n_heads


def tensor_specs(dims: ModelDims):
    """[(name, shape)] in payload order."""
    d, D, N, K, R = dims.d_model, dims.d_inner, dims.d_state, dims.d_conv, dims.dt_rank
    H, G = dims.n_heads, dims.n_groups
    specs = [("embedding", (dims.vocab, d))]
    for i, t in enumerate(dims.layers):
        p = f"layers.{i}."
        specs.append((p + "norm", (d,)))
        if t == "mamba1":
            specs += [(p + "in_proj", (2 * D, d)), (p + "conv_w", (D, K)), (p + "conv_b", (D,)),
                      (p + "x_proj", (R + 2 * N, D)), (p + "dt_proj_w", (D, R)),
                      (p + "dt_proj_b", (D,)), (p + "A_log", (D, N)), (p + "D", (D,)),
                      (p + "out_proj", (d, D))]
        elif t == "mamba2":
            cd = D + 2 * G * N
            specs += [(p + "in_proj", (2 * D + 2 * G * N + H, d)), (p + "conv_w", (cd, K)),
                      (p + "conv_b", (cd,)), (p + "dt_bias", (H,)), (p + "A_log", (H,)),
                      (p + "D", (H,)), (p + "gnorm", (D,)), (p + "out_proj", (d, D))]
        else:
            raise ValueError(f"layer type {t!r} is not supported by this backend")
    specs.append(("norm_f", (d,)))
    return specs


def header_bytes(n_layers: int) -> int:
    return 80 + ((n_layers + 15) // 16) * 16


def pack(dims: ModelDims, tensors: dict, dtype: str = "f32") -> bytes:
    """Serialize named tensors into an SSMW image."""
    if dtype not in ("f32", "f16"):
        raise ValueError("dtype must be f32 or f16")
    npdt = np.float32 if dtype == "f32" else np.float16
    parts = []
    for name, shape in tensor_specs(dims):
        a = np.asarray(tensors[name], dtype=np.float32)
        if a.shape != tuple(shape):
            raise ValueError(f"{name}: shape {a.shape} != {shape}")
        parts.append(np.ascontiguousarray(a, dtype=npdt).tobytes())
    payload = b"".join(parts)
    hb = header_bytes(dims.n_layers)
    head = bytearray(hb)
    struct.pack_into("<4sIIIQ", head, 0, MAGIC, VERSION, 0 if dtype == "f32" else 1, hb,
                     len(payload))
    struct.pack_into("<9if", head, 24, dims.vocab, dims.d_model, dims.n_layers, dims.d_state,
                     dims.d_conv, dims.expand, dims.n_heads, dims.n_groups, dims.dt_rank,
                     dims.norm_eps)
    struct.pack_into("<iiiI", head, 64, dims.chunk_len, dims.eos_id, dims.mimo_group, 0)
    for i, t in enumerate(dims.layers):
        head[80 + i] = LAYER_CODES[t]
    return bytes(head) + payload


def unpack(blob: bytes):
    """Parse an SSMW image -> (ModelDims, {name: float32 array}). Raises ValueError with the
    reason (bad magic / version / size) on a malformed image."""
    if len(blob) < 80 or blob[:4] != MAGIC:
        raise ValueError("bad magic")
    _, version, dt, hb, nbytes = struct.unpack_from("<4sIIIQ", blob, 0)
    if version != VERSION:
        raise ValueError(f"unsupported version {version}")
    if dt not in (0, 1):
        raise ValueError(f"unsupported dtype code {dt}")
    f = struct.unpack_from("<9if", blob, 24)
    chunk, eos, mimo, _ = struct.unpack_from("<iiiI", blob, 64)
    n_layers = f[2]
    if n_layers < 0 or hb != header_bytes(n_layers) or hb + nbytes != len(blob):
        raise ValueError("size mismatch")
    layers = []
    for i in range(n_layers):
        code = blob[80 + i]
        if code not in LAYER_NAMES:
            raise ValueError(f"bad layer type code {code}")
        layers.append(LAYER_NAMES[code])
    dims = ModelDims(vocab=f[0], d_model=f[1], n_layers=n_layers, d_state=f[3], d_conv=f[4],
                     expand=f[5], n_heads=f[6], n_groups=f[7], dt_rank=f[8], norm_eps=f[9],
                     chunk_len=chunk, eos_id=eos, mimo_group=mimo, layers=layers)
    npdt = np.float32 if dt == 0 else np.float16
    esz = 4 if dt == 0 else 2
    specs = tensor_specs(dims)
    total = sum(int(np.prod(s)) for _, s in specs)
    if total * esz != nbytes:
        raise ValueError("size mismatch")
    out, off = {}, hb
    for name, shape in specs:
        n = int(np.prod(shape))
        out[name] = np.frombuffer(blob, npdt, n, off).astype(np.float32).reshape(shape)
        off += n * esz
    return dims, out
