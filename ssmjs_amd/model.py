"""MambaCode.js-compatible model objects on the MI355X backend.

The reference's session layer uses these members of @seanhogg/mambacode.js (absent from the
reference; its call sites are listed in include/ssm_hip.h):
  initWebGPU({powerPreference}) -> {device}          src/session/session.ts:274-277
  adapter.requestDevice() / device.destroy()          session.ts:263,592
  new HybridMambaModel(device, config)                session.ts:359
    .config.{vocabSize, eosId}                        streaming.ts:24
    .forward(ids: Uint32Array, batch, seqLen) -> {logits: Float32Array(batch*seqLen*V)}
                                                      streaming.ts:31-35
    .generate(ids, maxNewTokens, {temperature, topK, topP}) -> prompt + continuation ids
                                                      session.ts:421-425
    .loadWeights(buffer) / .exportWeights()           session.ts:394,518,575
  new MambaTrainer(model, tokenizer).evaluate(text) -> perplexity   session.ts:506
Every numeric path runs in libssm_hip.so; there is no CPU fallback.
"""
from __future__ import annotations

import math
import random

import numpy as np

from . import _lib, backend, checkpoint
from .streaming import MIN_TEMPERATURE, sample_token


class HipDevice:
    """The device object MambaSession holds (GPUDevice stand-in): only destroy() is used by
    the session layer (session.ts:592)."""

    def __init__(self, ordinal: int = 0):
        self._dev = backend.Device(ordinal)
        self.arch = self._dev.arch
        self.compute_units = self._dev.compute_units

    @property
    def backend(self) -> backend.Device:
        return self._dev

    def destroy(self):
        self._dev.destroy()


class HipAdapter:
    """GPUAdapter stand-in for MambaSessionOptions.gpuAdapter (session.ts:113,260-271)."""

    def __init__(self, ordinal: int = 0):
        self.ordinal = ordinal

    def requestDevice(self) -> HipDevice:
        return HipDevice(self.ordinal)


def init_webgpu(options: dict | None = None) -> dict:
    """initWebGPU({powerPreference}) -> {device} (session.ts:274-277). powerPreference has no
    meaning on one MI355X and is ignored."""
    return {"device": HipDevice(0)}


initWebGPU = init_webgpu


class HybridMambaModel:
    def __init__(self, device: HipDevice, config: dict, seed: int = 0):
        self.device = device
        self.config = dict(config)
        self._m = backend.Model(device.backend, self.config, seed=seed)
        self.config["dtRank"] = self._m.config["dtRank"]

    @property
    def native(self) -> backend.Model:
        return self._m

    # -- forward: full re-prefill, logits for every position (streaming.ts:31-41)
    def forward(self, ids, batch: int, seq_len: int) -> dict:
        a = np.ascontiguousarray(ids, dtype=np.uint32).reshape(batch, seq_len)
        logits = self._m.forward(a)
        return {"logits": logits.reshape(-1)}

    # -- generate: recurrent decode (prefill once, one state update per token)
    def generate(self, prompt_ids, max_new_tokens: int = 200, sampling: dict | None = None,
                 rng=None) -> list:
        s = sampling or {}
        temperature = s.get("temperature", 1.0)
        topK = s.get("topK", 50)
        topP = s.get("topP", 0.9)
        ids = [int(i) for i in prompt_ids]
        if max_new_tokens <= 0:
            return ids
        if not ids:
            raise ValueError("generate: empty prompt")
        eos = self.config.get("eosId", -1)
        st = self._m.new_state(1)
        try:
            if backend.sample_supported(self.config["vocabSize"], topK):
                # sampleToken on the device (topK = 1 included: its pick is the lowest index
                # among f32 exps equal to the largest, which an argmax of the logits misses
                # when two exps round alike). The draws are taken from rng up front, one per
                # step in the reference's order (streaming.ts:91), so the tokens up to eos
                # are those of the host loop below with the same rng; rng is then advanced
                # max_new_tokens times even when eos comes earlier.
                draw = rng or random.random
                u = np.array([draw() for _ in range(max_new_tokens)], np.float64)
                out = st.generate_sample(np.array([ids], np.uint32), max_new_tokens,
                                         temperature, topK, topP, u[:, None])[0].tolist()
            elif topK == 1:
                # vocabularies beyond the device sampler: device argmax of the logits (lowest
                # index among equal maxima)
                out = st.generate_greedy(np.array([ids], np.uint32), max_new_tokens)[0].tolist()
            else:
                out = None
            if out is not None:
                for t in out:
                    ids.append(int(t))
                    if t == eos:
                        break
                return ids
            logits, _ = st.prefill(np.array([ids], np.uint32))
            for step in range(max_new_tokens):
                nxt = sample_token(logits[0], temperature, topK, topP, rng)
                ids.append(nxt)
                if nxt == eos or step + 1 == max_new_tokens:
                    break
                logits, _ = st.decode(np.array([nxt], np.uint32))
            return ids
        finally:
            st.destroy()

    def loadWeights(self, buffer) -> None:
        """Validates magic / version / dims / size (src/session/errors.ts:9) and uploads."""
        blob = bytes(buffer)
        dims, _ = checkpoint.unpack(blob)   # raises ValueError with the reason
        self._m.load_weights(blob)

    def exportWeights(self, f16: bool = False) -> bytes:
        return self._m.export_weights(f16=f16)

    def destroy(self):
        self._m.destroy()


class MambaTrainer:
    """Only evaluate() is on the forward path (session.ts:504-507); train() drives backward
    and an optimizer, which this backend does not implement."""

    def __init__(self, model: HybridMambaModel, tokenizer):
        self.model = model
        self.tokenizer = tokenizer

    def evaluate(self, text: str) -> float:
        """Perplexity = exp(mean next-token cross-entropy) of the encoded text under one
        forward pass (positions 0..n-2 predict tokens 1..n-1)."""
        ids = list(self.tokenizer.encode(text))
        if len(ids) < 2:
            return float("inf")
        V = self.model.config["vocabSize"]
        logits = self.model.forward(np.asarray(ids, np.uint32), 1, len(ids))["logits"]
        lg = logits.reshape(len(ids), V)[:-1].astype(np.float64)
        tgt = np.asarray(ids[1:])
        m = lg.max(axis=1)
        lse = m + np.log(np.exp(lg - m[:, None]).sum(axis=1))
        nll = lse - lg[np.arange(len(tgt)), tgt]
        return float(math.exp(nll.mean()))

    def train(self, *args, **kwargs):
        raise NotImplementedError("training (MambaSession.adapt) is not part of the MI355X "
                                  "forward-path backend")


__all__ = ["HipDevice", "HipAdapter", "init_webgpu", "initWebGPU", "HybridMambaModel",
           "MambaTrainer", "MIN_TEMPERATURE"]
