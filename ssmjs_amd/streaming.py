"""Token streaming and sampling (restates src/session/streaming.ts:17-97).

token_stream re-runs model.forward over the whole sequence every step, exactly as the
reference's tokenStream does (streaming.ts:30-41); HybridMambaModel.generate is the
recurrent path. sample_token reproduces sampleToken step for step: temperature scaling in
double stored as float32, a numerically stable softmax whose exponentials are computed in
double and stored as float32 and summed in index order, a stable descending sort of the
exponentials, top-K, the nucleus cut at the first
cumulative probability >= topP, and an inverse-CDF draw. With topK = 1 the draw cannot
change the result, so greedy decoding is deterministic.
"""
from __future__ import annotations

import math
import random as _random

import numpy as np

MIN_TEMPERATURE = 1e-7   # streaming.ts:11


def sample_token(logits, temperature: float = 1.0, topK: int = 50, topP: float = 0.9,
                 rng=None) -> int:
    """src/session/streaming.ts:53-97. `rng()` returns a float in [0, 1) (Math.random)."""
    lg = np.asarray(logits, dtype=np.float32)
    n = lg.shape[0]
    # JS numbers are doubles: the division is in double, the Float32Array store rounds
    scaled = (lg.astype(np.float64) / max(temperature, MIN_TEMPERATURE)).astype(np.float32)
    max_l = float(scaled.max()) if n else -math.inf
    exps = np.exp(scaled.astype(np.float64) - max_l).astype(np.float32)
    # sumE += exps[i] in index order (a cumulative sum is sequential; np.sum is pairwise)
    sum_e = float(np.cumsum(exps.astype(np.float64))[-1]) if n else 0.0
    # Array.prototype.sort is stable: equal exps keep ascending index order
    order = np.argsort(-exps.astype(np.float64), kind="stable")
    top = order[: max(int(topK), 0)]
    nucleus = []
    cum = 0.0
    for idx in top:
        cum += float(exps[idx]) / sum_e
        nucleus.append(int(idx))
        if cum >= topP:
            break
    if not nucleus:
        # topK <= 0: the reference indexes nucleus[-1] of an empty array (undefined)
        raise ValueError("sampleToken: topK must be at least 1")
    nsum = 0.0
    for idx in nucleus:
        nsum += float(exps[idx])
    threshold = (rng or _random.random)() * nsum
    acc = 0.0
    for idx in nucleus:
        acc += float(exps[idx])
        if acc >= threshold:
            return idx
    return nucleus[-1]


def token_stream(model, prompt_ids, max_new_tokens: int, sampling: dict | None = None,
                 rng=None):
    """src/session/streaming.ts:17-49: yields one id per step; stops after eosId."""
    s = sampling or {}
    temperature = s.get("temperature", 1.0)
    topK = s.get("topK", 50)
    topP = s.get("topP", 0.9)
    V = model.config["vocabSize"]
    eos = model.config.get("eosId", -1)
    ids = list(prompt_ids)
    for _ in range(max_new_tokens):
        out = model.forward(np.asarray(ids, dtype=np.uint32), 1, len(ids))
        logits = out["logits"]
        last = logits[(len(ids) - 1) * V: len(ids) * V]
        nxt = sample_token(last, temperature, topK, topP, rng)
        ids.append(nxt)
        yield nxt
        if nxt == eos:
            break


sampleToken = sample_token
tokenStream = token_stream
