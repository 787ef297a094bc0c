"""The Node-API binding (ssmjs_amd/napi): the module the reference's TypeScript host loads in
place of MambaCode.js (src/session/session.ts:10-18). CPU tests check that the addon loads
under Node and maps a missing device to GPU_UNAVAILABLE (session.ts:262-270); the GPU test
drives initWebGPU -> HybridMambaModel -> loadWeights / generate / forward / evaluate /
exportWeights / destroy from Node and checks the results against the CPU oracle."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "ssmjs_amd", "napi", "ssm_napi.node")
NODE = shutil.which("node")

needs_addon = pytest.mark.skipif(NODE is None or not os.path.exists(ADDON),
                                 reason="node or the built addon is absent")


def _node(code, env=None, timeout=120):
    return subprocess.run([NODE, "-e", code], capture_output=True, text=True, cwd=ROOT,
                          env=env, timeout=timeout)


@needs_addon
def test_addon_exports_the_binding():
    r = _node("const a = require('./ssmjs_amd/napi/ssm_napi.node');"
              "const m = require('./ssmjs_amd/napi');"
              "console.log(JSON.stringify({a: Object.keys(a), m: Object.keys(m), v: a.version()}))")
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert set(out["a"]) >= {"ctxCreate", "ctxDestroy", "modelCreate", "modelDestroy", "loadWeights",
                             "exportWeights", "forward", "stateCreate", "prefill", "decodeStep",
                             "generateGreedy"}
    assert set(out["m"]) >= {"initWebGPU", "HybridMambaModel", "MambaTrainer", "sampleToken"}
    assert out["v"] >= 1


@needs_addon
def test_no_device_rejects_with_gpu_unavailable():
    env = dict(os.environ, SSM_HIP_FAULT="nodevice")
    r = _node("require('./ssmjs_amd/napi').initWebGPU({}).then(() => console.log('OK'),"
              " (e) => console.log(e.code))", env=env)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "GPU_UNAVAILABLE"


@needs_addon
def test_js_sample_token_matches_python():
    from ssmjs_amd import sampleToken
    lg = [0.1, 3.0, -2.0, 3.0, 1.0, 2.5]
    cases = [(0.8, 1, 0.9, 0.3), (1.0, 50, 0.7, 0.0), (1.0, 50, 0.7, 0.99), (1.0, 3, 1.0, 0.999),
             (0.0, 50, 0.9, 0.99)]
    code = ("const m = require('./ssmjs_amd/napi'); const lg = Float32Array.from(%s);"
            "console.log(JSON.stringify(%s.map(c => m.sampleToken(lg, c[0], c[1], c[2], () => c[3]))))"
            % (json.dumps(lg), json.dumps(cases)))
    r = _node(code)
    assert r.returncode == 0, r.stderr
    js = json.loads(r.stdout)
    py = [sampleToken(np.array(lg, np.float32), t, k, p, rng=lambda r_=r_: r_) for t, k, p, r_ in cases]
    assert js == py


@needs_addon
def test_js_sample_token_matches_python_random():
    """Random logits and temperatures that float32 cannot hold (the division happens in JS
    doubles): the Python restatement picks what the JS sampleToken picks."""
    from ssmjs_amd import sampleToken
    r = np.random.default_rng(5)
    lgs = [(3.0 * r.standard_normal(700)).astype(np.float32).tolist() for _ in range(4)]
    cases = [(0.7, 50, 0.9), (1.3, 200, 0.95), (0.8, 50, 0.9), (0.33, 7, 0.5)]
    us = r.random(6).tolist()
    code = ("const m = require('./ssmjs_amd/napi'); const L = %s; const C = %s; const U = %s;"
            "const out = []; for (const l of L) { const lg = Float32Array.from(l);"
            " for (const c of C) for (const u of U) out.push(m.sampleToken(lg, c[0], c[1], c[2], () => u)); }"
            "console.log(JSON.stringify(out))" % (json.dumps(lgs), json.dumps(cases), json.dumps(us)))
    res = _node(code)
    assert res.returncode == 0, res.stderr
    js = json.loads(res.stdout)
    py = [sampleToken(np.array(l, np.float32), t, k, p, rng=lambda u_=u_: u_)
          for l in lgs for t, k, p in cases for u_ in us]
    assert js == py


@pytest.mark.gpu
@needs_addon
def test_node_session_path_matches_oracle(tmp_path):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("[case] node: initWebGPU -> HybridMambaModel -> generate/forward/evaluate", flush=True)
    from oracle import oracle as O
    from ssmjs_amd import backend, checkpoint
    cfg = {"vocabSize": 256, "dModel": 128, "numLayers": 2, "dState": 64, "dConv": 4, "expand": 2,
           "nHeads": 2, "nGroups": 1, "layers": [{"type": "mamba2"}, {"type": "mamba1"}]}
    d = backend.Device(0)
    m = backend.Model(d, cfg, seed=21)
    dims, T = checkpoint.unpack(m.export_weights())
    m.destroy()
    d.destroy()
    T["embedding"] = T["embedding"] * 40.0          # wide top-1 margins for bit-exact greedy
    blob = checkpoint.pack(dims, T)
    ck, cj = tmp_path / "w.ssmw", tmp_path / "cfg.json"
    ck.write_bytes(blob)
    cj.write_text(json.dumps(cfg))
    prompt = list(b"Mamba on MI355X")
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "napi_check.js"), str(ck), str(cj),
                        ",".join(map(str, prompt)), "16"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    om = O.Model(blob)
    ids, margins = O.greedy(om, np.array([prompt], np.uint32), 16)
    assert margins.min() > 1e-3
    assert out["generated"] == prompt + ids[0].tolist()
    # sampled generation (device sampler behind generate) == the host loop over the same
    # device logits with the oracle's sampleToken and the same draws
    draws = [0.1, 0.7, 0.35, 0.9, 0.5]
    d = backend.Device(0)
    m = backend.Model(d, cfg, seed=0)
    m.load_weights(blob)
    st = m.new_state(1)
    want = list(prompt)
    lg, _ = st.prefill(np.array([prompt], np.uint32))
    for k in range(8):
        want.append(O.sample_token(lg[0], 1.3, 5, 0.9, draws[k % 5]))
        if k + 1 < 8:
            lg, _ = st.decode(np.array([want[-1]], np.uint32))
    st.destroy()
    m.destroy()
    d.destroy()
    assert out["sampled"] == want
    ref = om.forward(np.array([prompt], np.uint32))[0]
    lg = np.array(out["logits"], np.float32).reshape(len(prompt), 256)
    assert np.abs(lg - ref).max() / np.abs(ref).max() <= 1e-4
    assert out["badCode"] == "CHECKPOINT_INVALID"
    assert out["destroyedCode"] == "SESSION_DESTROYED"
    assert out["exportedBytes"] == len(blob)
    text = list(b"hello mamba")
    lgt = om.forward(np.array([text], np.uint32))[0, :-1].astype(np.float64)
    mx = lgt.max(1)
    lse = mx + np.log(np.exp(lgt - mx[:, None]).sum(1))
    nll = float((lse - lgt[np.arange(len(lgt)), text[1:]]).mean())
    # mean NLL moves by at most twice the logits' error (1e-4 of their range)
    assert abs(np.log(out["ppl"]) - nll) <= 2e-4 * np.abs(lgt).max()
    sys.stdout.flush()


@pytest.mark.gpu
@needs_addon
def test_node_two_models_one_device(tmp_path):
    """Two HybridMambaModels on one initWebGPU device driven with Promise.all (their calls
    run on libuv pool threads at the same time, serialised by the library's context lock):
    each model's greedy ids and logits match the oracle. Then device.destroy() while a
    generate is in flight: the generate either completes or rejects with SESSION_DESTROYED,
    the process does not crash, and later calls reject with SESSION_DESTROYED (the reference
    keeps one model per session and device, session.ts:359,589-592)."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("[case] node: two models on one device, destroy while pending", flush=True)
    from oracle import oracle as O
    from ssmjs_amd import backend, checkpoint
    cfgs = [{"vocabSize": 256, "dModel": 128, "numLayers": 2, "dState": 64, "dConv": 4,
             "expand": 2, "nHeads": 2, "nGroups": 1, "layers": [{"type": "mamba2"}] * 2},
            {"vocabSize": 256, "dModel": 96, "numLayers": 3, "dState": 16, "dConv": 4,
             "expand": 2, "nHeads": 2, "layers": [{"type": "mamba1"}] * 3}]
    blobs, args = [], []
    d = backend.Device(0)
    for i, cfg in enumerate(cfgs):
        m = backend.Model(d, cfg, seed=31 + i)
        dims, T = checkpoint.unpack(m.export_weights())
        m.destroy()
        T["embedding"] = T["embedding"] * 40.0
        blob = checkpoint.pack(dims, T)
        blobs.append(blob)
        ck, cj = tmp_path / f"w{i}.ssmw", tmp_path / f"cfg{i}.json"
        ck.write_bytes(blob)
        cj.write_text(json.dumps(cfg))
        args += [str(ck), str(cj)]
    d.destroy()
    prompt = list(b"two models")
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "napi_concurrent.js"), *args,
                        ",".join(map(str, prompt)), "12"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    for key, fkey, blob in (("genA", "fwdA", blobs[0]), ("genB", "fwdB", blobs[1])):
        om = O.Model(blob)
        ids, margins = O.greedy(om, np.array([prompt], np.uint32), 12)
        assert margins.min() > 1e-3
        assert out[key] == prompt + ids[0].tolist()
        ref = om.forward(np.array([prompt], np.uint32))[0]
        lg = np.array(out[fkey], np.float32).reshape(len(prompt), 256)
        assert np.abs(lg - ref).max() / np.abs(ref).max() <= 1e-4
    assert out["genA2"] == out["genA"]
    assert out["during"]["ok"] or out["during"]["code"] == "SESSION_DESTROYED", out["during"]
    if out["during"]["ok"]:
        assert out["during"]["len"] == len(prompt) + 400
    assert out["after"] == "SESSION_DESTROYED"
