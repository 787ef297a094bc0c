"""CPU tests of the host-side mirror of the reference's session API: config resolution
(src/session/presets.ts), sampling and streaming (src/session/streaming.ts), and the error
contract of MambaSession / SSMRuntime (src/session/session.ts, src/runtime/SSMRuntime.ts).
Like the reference's own jest suites, the GPU is never faked for numerics; fake objects stand
in only for the injected adapter and for a model in the host-only streaming loop."""
import math

import numpy as np
import pytest

from ssmjs_amd import (MODEL_PRESETS, SSM, ByteTokenizer, MambaSession, SessionError, SSMError,
                       SSMRuntime, resolveLayerSchedule, resolveModelConfig, sampleToken,
                       tokenStream)

# ---------------------------------------------------------------- presets.ts


def test_presets_table_is_the_references():
    # src/session/presets.ts:14-19
    assert MODEL_PRESETS["nano"] == {"dModel": 128, "numLayers": 4, "dState": 16, "dConv": 4,
                                     "expand": 2, "nHeads": 4}
    assert MODEL_PRESETS["small"]["dModel"] == 256 and MODEL_PRESETS["small"]["numLayers"] == 6
    assert MODEL_PRESETS["medium"]["dModel"] == 512 and MODEL_PRESETS["medium"]["nHeads"] == 8
    assert MODEL_PRESETS["large"] == {"dModel": 768, "numLayers": 12, "dState": 16, "dConv": 4,
                                      "expand": 2, "nHeads": 12}


def test_default_is_nano_with_field_defaults():
    cfg = resolveModelConfig({}, 1000)
    assert cfg == {"vocabSize": 1000, "dModel": 128, "numLayers": 4, "dState": 16, "dConv": 4,
                   "expand": 2, "nHeads": 4, "nGroups": 1, "chunkLen": 256, "mimoGroup": 1,
                   "eosId": -1, "layers": [{"type": "mamba1"}] * 4}


def test_model_config_applies_only_for_custom():
    over = {"dModel": 1024, "numLayers": 24, "nHeads": 32, "dState": 128}
    assert resolveModelConfig({"modelSize": "small", "modelConfig": over}, 10)["dModel"] == 256
    cfg = resolveModelConfig({"modelSize": "custom", "modelConfig": over,
                              "mambaVersion": "mamba2"}, 32000)
    assert (cfg["dModel"], cfg["numLayers"], cfg["nHeads"], cfg["dState"]) == (1024, 24, 32, 128)
    assert cfg["layers"] == [{"type": "mamba2"}] * 24 and cfg["vocabSize"] == 32000
    # a custom config falls back to the nano preset for fields it leaves out
    assert resolveModelConfig({"modelSize": "custom", "modelConfig": {"dModel": 64}}, 5)["numLayers"] == 4


def test_unknown_preset_falls_back_to_nano():
    assert resolveModelConfig({"modelSize": "huge"}, 7)["dModel"] == 128


def test_heads_must_divide_dmodel():
    with pytest.raises(ValueError, match=r"dModel \(100\) must be divisible by nHeads \(3\)"):
        resolveModelConfig({"modelSize": "custom", "modelConfig": {"dModel": 100, "nHeads": 3}}, 5)


def test_layer_schedules():
    j = resolveLayerSchedule("jamba", 8, "mamba1")
    assert [l["type"] for l in j] == ["mamba2"] * 3 + ["attention"] + ["mamba2"] * 3 + ["attention"]
    z = resolveLayerSchedule("zamba", 12, "mamba1")
    assert [i for i, l in enumerate(z) if l["type"] == "attention"] == [5, 11]
    assert all(l["type"] == "mamba3" for i, l in enumerate(z) if i not in (5, 11))
    explicit = [{"type": "mamba2"}, {"type": "mamba1"}]
    assert resolveLayerSchedule(explicit, 2, "mamba1") is explicit
    assert resolveModelConfig({"layerSchedule": "jamba"}, 3)["layers"][3] == {"type": "attention"}


# ---------------------------------------------------------------- streaming.ts


def test_greedy_is_argmax_with_lowest_index_on_ties():
    lg = np.array([0.1, 3.0, -2.0, 3.0, 1.0], np.float32)
    for r in (0.0, 0.5, 0.999999):
        assert sampleToken(lg, temperature=0.8, topK=1, topP=0.9, rng=lambda: r) == 1


def test_nucleus_membership_and_order():
    lg = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    # topP 0.7: nucleus = [0, 1] (0.5 < 0.7, 0.8 >= 0.7)
    assert sampleToken(lg, temperature=1.0, topK=50, topP=0.7, rng=lambda: 0.0) == 0
    assert sampleToken(lg, temperature=1.0, topK=50, topP=0.7, rng=lambda: 0.99) == 1
    # topK 3, topP 1: the draw can reach the third token but never the fourth
    assert sampleToken(lg, temperature=1.0, topK=3, topP=1.0, rng=lambda: 0.999) == 2


def test_sampling_distribution_matches_renormalised_nucleus():
    lg = np.array([2.0, 1.5, 1.0, 0.0, -1.0], np.float32)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    r = np.random.default_rng(0)
    draws = [sampleToken(lg, 1.0, 3, 1.0, rng=lambda: r.random()) for _ in range(20000)]
    freq = np.bincount(draws, minlength=5) / len(draws)
    q = np.zeros(5)
    q[:3] = p[:3] / p[:3].sum()
    assert freq[3] == 0 and freq[4] == 0
    assert np.abs(freq - q).max() < 0.02


def test_temperature_floor():
    lg = np.array([1.0, 1.0 + 1e-3], np.float32)
    # temperature 0 clamps to 1e-7 (streaming.ts:11,61): effectively greedy
    assert sampleToken(lg, temperature=0.0, topK=50, topP=0.9, rng=lambda: 0.99) == 1


class _FakeModel:
    """Host-only stand-in: logits favour (last id + 1) mod V. Used to check the loop's
    slicing of the last row and the EOS stop (streaming.ts:38-47)."""

    def __init__(self, V, eos):
        self.config = {"vocabSize": V, "eosId": eos}
        self.calls = []

    def forward(self, ids, batch, seq_len):
        self.calls.append(list(ids))
        V = self.config["vocabSize"]
        lg = np.zeros((seq_len, V), np.float32)
        for t, i in enumerate(ids):
            lg[t, (int(i) + 1) % V] = 5.0
        return {"logits": lg.reshape(-1)}


def test_token_stream_reprefills_and_stops_at_eos():
    m = _FakeModel(V=10, eos=7)
    out = list(tokenStream(m, [3], 20, {"topK": 1}))
    assert out == [4, 5, 6, 7]
    assert m.calls[-1] == [3, 4, 5, 6]         # full sequence each step


# ---------------------------------------------------------------- errors / session


def test_error_codes():
    e = SessionError("CHECKPOINT_INVALID", "bad", cause=ValueError("x"))
    assert e.code == "CHECKPOINT_INVALID" and e.name == "SessionError" and str(e) == "bad"
    assert SSMError("RUNTIME_DESTROYED", "x").code == "RUNTIME_DESTROYED"
    with pytest.raises(ValueError):
        SessionError("NOPE", "x")


class _BadAdapter:
    def requestDevice(self):
        raise RuntimeError("adapter exploded")


class _FakeDevice:
    destroyed = False

    def destroy(self):
        self.destroyed = True


class _FakeAdapter:
    def __init__(self):
        self.dev = _FakeDevice()

    def requestDevice(self):
        return self.dev


def test_injected_adapter_failure_is_gpu_unavailable():
    with pytest.raises(SessionError) as e:
        MambaSession.create({"gpuAdapter": _BadAdapter(), "tokenizer": ByteTokenizer()})
    assert e.value.code == "GPU_UNAVAILABLE"
    assert "adapter exploded" in str(e.value)


def test_no_device_is_gpu_unavailable(monkeypatch):
    monkeypatch.setenv("SSM_HIP_FAULT", "nodevice")
    for fallback in (False, True):
        with pytest.raises(SessionError) as e:
            MambaSession.create({"tokenizer": ByteTokenizer(), "allowCpuFallback": fallback})
        assert e.value.code == "GPU_UNAVAILABLE"


def test_missing_tokenizer_is_tokenizer_load_failed():
    a = _FakeAdapter()
    stages = []
    with pytest.raises(SessionError) as e:
        MambaSession.create({"gpuAdapter": a}, {"onProgress": stages.append})
    assert e.value.code == "TOKENIZER_LOAD_FAILED"
    assert a.dev.destroyed
    assert [s["stage"] for s in stages] == ["gpu", "gpu", "tokenizer"]


def test_runtime_rejects_bridges_and_guards_destroy():
    with pytest.raises(SSMError):
        SSM.create({"session": {}, "bridge": object()})

    class _S:
        destroyed = False

        def destroy(self):
            self.destroyed = True

        def complete(self, *a, **k):
            return "x"

    rt = SSMRuntime(_S())
    assert rt.generate("hi") == "x"
    rt.destroy()
    assert rt.destroyed
    with pytest.raises(SSMError) as e:
        rt.generate("hi")
    assert e.value.code == "RUNTIME_DESTROYED"
    assert rt.getRoutingAuditLog() == [] and rt.bridge is None


def test_byte_tokenizer_roundtrip():
    t = ByteTokenizer(300)
    assert t.decode(t.encode("héllo")) == "héllo" and t.vocabSize == 300
    assert math.isfinite(len(t.encode("")))
