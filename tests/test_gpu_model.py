"""GPU parity of the model-level C ABI (forward / prefill / decode / greedy generate) against
the CPU oracle and the HF golden fixtures, plus its error contract.

Logits and states are compared per element (1e-4 relative plus a floor of 1e-5 of the
tensor's largest magnitude). Greedy ids are compared bit-exactly. The models used for greedy runs scale the embedding so
that the oracle's top-1/top-2 logit margin stays far above the fp32 summation-order noise;
each test asserts that minimum margin, so a pass is not luck on near-ties.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from oracle import oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
# per element: |gpu - oracle| <= RTOL |oracle| + ATOL_FRAC max|oracle| (north_star: max rel
# err <= 1e-4 fp32; the floor is the fp32 rounding of the model's K-term sums)
RTOL = 1e-4
ATOL_FRAC = 1e-5


@pytest.fixture(scope="module")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from ssmjs_amd import backend
    d = backend.Device(0)
    yield d
    d.destroy()


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def close(got, ref, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    scale = float(np.abs(ref).max())
    ratio = float((np.abs(got - ref) / (RTOL * np.abs(ref) + ATOL_FRAC * scale)).max())
    print(f"  {what}: worst |err|/bound {ratio:.3f}", flush=True)
    assert ratio <= 1.0, f"{what}: beyond {RTOL} |ref| + {ATOL_FRAC} max|ref|"


def cfg_of(dims):
    return {"vocabSize": dims.vocab, "dModel": dims.d_model, "numLayers": dims.n_layers,
            "dState": dims.d_state, "dConv": dims.d_conv, "expand": dims.expand,
            "nHeads": dims.n_heads, "nGroups": dims.n_groups, "dtRank": dims.dt_rank,
            "layers": [{"type": t} for t in dims.layers]}


@pytest.mark.parametrize("kind", ["mamba1", "mamba2"])
def test_hf_fixture_logits(device, golden, kind):
    case(f"hf fixture {kind}")
    from ssmjs_amd import backend, checkpoint
    g = golden[f"hf_model_{kind}"]
    blob = g["blob"].tobytes()
    dims, _ = checkpoint.unpack(blob)
    m = backend.Model(device, cfg_of(dims))
    m.load_weights(blob)
    out = m.forward(g["ids"])
    close(out, g["logits"], "logits")
    close(out, O.Model(blob).forward(g["ids"]), "logits")
    m.destroy()


def _model(device, layers, d=128, N=16, H=4, V=512, seed=7, emb_scale=40.0, dt_rank=None):
    """Random-init GPU model; embedding scaled up for wide greedy margins. Returns (model, blob)."""
    from ssmjs_amd import backend, checkpoint
    cfg = {"vocabSize": V, "dModel": d, "numLayers": len(layers), "dState": N, "dConv": 4,
           "expand": 2, "nHeads": H, "nGroups": 1, "layers": [{"type": t} for t in layers]}
    if dt_rank is not None:
        cfg["dtRank"] = dt_rank
    m = backend.Model(device, cfg, seed=seed)
    dims, T = checkpoint.unpack(m.export_weights())
    T["embedding"] = T["embedding"] * emb_scale
    blob = checkpoint.pack(dims, T)
    m.load_weights(blob)
    return m, blob


@pytest.mark.parametrize("layers,N,H", [(["mamba1", "mamba1"], 16, 4),
                                        (["mamba2", "mamba2"], 128, 4),
                                        (["mamba1", "mamba2"], 64, 4)])
def test_forward_matches_oracle(device, layers, N, H):
    case(f"forward {layers} N={N}")
    m, blob = _model(device, layers, N=N, H=H)
    ids = np.random.default_rng(1).integers(0, 512, (2, 150)).astype(np.uint32)
    out = m.forward(ids)
    ref = O.Model(blob).forward(ids)
    close(out, ref, "logits")
    m.destroy()


@pytest.mark.parametrize("layers,N,H,R", [(["mamba1", "mamba1"], 16, 4, None),
                                          (["mamba1", "mamba1"], 16, 4, 6),
                                          (["mamba2", "mamba2"], 128, 4, None),
                                          (["mamba2", "mamba2"], 128, 32, None),
                                          (["mamba1", "mamba2", "mamba1"], 64, 4, None)])
def test_prefill_decode_state_matches_oracle(device, layers, N, H, R):
    """H = 32 gives head dim 8, less than one workgroup's block of state rows in the one-token
    update (the guarded variant of the fused step's state update). The Mamba-1 layers take
    the fused one-token step except with dt_rank 6 (not a multiple of 4: the separate
    launches); the mixed stack hands the next layer's norm operand across layer types."""
    case(f"prefill/decode state {layers} N={N} H={H} dt_rank={R}")
    m, blob = _model(device, layers, N=N, H=H, dt_rank=R)
    om = O.Model(blob)
    ids = np.random.default_rng(2).integers(0, 512, (3, 40)).astype(np.uint32)
    st = m.new_state(3)
    ost = om.new_state(3)
    lg, _ = st.prefill(ids[:, :33])
    close(lg, ost.prefill(ids[:, :33]), "logits")
    close(st.read(), ost.read(), "state")
    for t in range(33, 40):
        lg, _ = st.decode(ids[:, t])
        close(lg, ost.decode(ids[:, t]), "logits")
    close(st.read(), ost.read(), "state")
    st.destroy()
    m.destroy()


@pytest.mark.parametrize("layers,N,H", [(["mamba1", "mamba1"], 16, 4),
                                        (["mamba2", "mamba2"], 128, 4),
                                        (["mamba1", "mamba2"], 64, 4)])
@pytest.mark.parametrize("B,L", [(1, 16), (2, 32), (4, 9)])
def test_short_prefill_matches_oracle(device, layers, N, H, B, L):
    """Prompts of at most 64 tokens: every product of the mixers on the few-row kernel (the
    gated norm in its prologue for Mamba-2), the LM head on the B last positions; then a
    forward of the same B x L tokens (the LM head on all of them, no greedy picks) and two
    decode steps from the prefilled state."""
    case(f"short prefill {layers} N={N} B={B} L={L}")
    m, blob = _model(device, layers, N=N, H=H)
    om = O.Model(blob)
    ids = np.random.default_rng(11 + B * L).integers(0, 512, (B, L + 2)).astype(np.uint32)
    close(m.forward(ids[:, :L]), om.forward(ids[:, :L]), "forward logits")
    st = m.new_state(B)
    ost = om.new_state(B)
    lg, am = st.prefill(ids[:, :L])
    ref = ost.prefill(ids[:, :L])
    close(lg, ref, "prefill logits")
    close(st.read(), ost.read(), "state")
    for t in range(L, L + 2):
        lg, _ = st.decode(ids[:, t])
        close(lg, ost.decode(ids[:, t]), "decode logits")
    close(st.read(), ost.read(), "state after decode")
    st.destroy()
    m.destroy()


@pytest.mark.parametrize("layers,N,H", [(["mamba1", "mamba1"], 16, 16),
                                        (["mamba2", "mamba2"], 128, 16)])
@pytest.mark.parametrize("B,L", [(1, 300), (3, 200)])
def test_split_k_prefill_matches_oracle(device, layers, N, H, B, L):
    """Prompts of a few hundred tokens on a wide model (d_model 512): the own GEMM's tiles
    leave CUs idle, so its products split K over workgroups (partials added in slice order
    by the finishing kernel, the residual add and the gated norm's row scale there); the
    Mamba-1 x_proj / dt_proj as two products. The prefill's logits and state."""
    case(f"split-K prefill {layers} d=512 N={N} B={B} L={L}")
    m, blob = _model(device, layers, d=512, N=N, H=H)
    om = O.Model(blob)
    ids = np.random.default_rng(5 + L).integers(0, 512, (B, L)).astype(np.uint32)
    st = m.new_state(B)
    ost = om.new_state(B)
    lg, _ = st.prefill(ids)
    close(lg, ost.prefill(ids), "prefill logits")
    close(st.read(), ost.read(), "state")
    st.destroy()
    m.destroy()


@pytest.mark.parametrize("layers,N", [(["mamba1"] * 4, 16), (["mamba2"] * 2, 128)])
def test_greedy_ids_bit_exact(device, layers, N):
    case(f"greedy {layers}")
    m, blob = _model(device, layers, N=N)
    prompt = np.random.default_rng(3).integers(0, 512, (4, 12)).astype(np.uint32)
    st = m.new_state(4)
    got = st.generate_greedy(prompt, 24)
    ref, margins = O.greedy(O.Model(blob), prompt, 24)
    print(f"  min top1-top2 margin {margins.min():.3e}")
    assert margins.min() > 1e-3, "model too close to a tie for a bit-exact check"
    np.testing.assert_array_equal(got, ref)
    st.destroy()
    m.destroy()


@pytest.mark.parametrize("B", [4, 40])
def test_greedy_exact_ties_pick_lowest_index(device, B):
    """Every embedding row is +v or -v, so every logit of a row is one of two values, tied
    across the whole vocabulary: the one-token LM head's per-block picks and their merge must
    give the lowest index of the larger value, as the oracle's greedy pick does. +v rows start
    at 130, past the first 128-column block; B = 40 spans three row tiles."""
    case(f"greedy exact ties, {B} sequences")
    from ssmjs_amd import backend, checkpoint
    V = 1024
    cfg = {"vocabSize": V, "dModel": 128, "numLayers": 2, "dState": 16, "dConv": 4,
           "expand": 2, "nHeads": 4, "nGroups": 1, "layers": [{"type": "mamba1"}] * 2}
    m = backend.Model(device, cfg, seed=11)
    dims, T = checkpoint.unpack(m.export_weights())
    v = T["embedding"][0] * 40.0
    plus = (np.arange(V) % 3 == 1) & (np.arange(V) >= 130)
    T["embedding"] = np.where(plus[:, None], v[None, :], -v[None, :]).astype(np.float32)
    blob = checkpoint.pack(dims, T)
    m.load_weights(blob)
    om = O.Model(blob)
    prompt = np.random.default_rng(5).integers(0, V, (B, 6)).astype(np.uint32)
    st = m.new_state(B)
    ost = om.new_state(B)
    st.prefill(prompt)
    ost.prefill(prompt)
    ids = prompt[:, -1]
    for _ in range(4):
        lg, got = st.decode(ids)
        ref = ost.decode(ids)
        close(lg, ref, "logits")
        top = ref.max(axis=1, keepdims=True)
        want = np.argmax(ref == top, axis=1)     # lowest index among the maxima
        assert len(np.unique(ref[0])) == 2, "logits are not two tied values"
        np.testing.assert_array_equal(got, want)
        ids = want.astype(np.uint32)
    st.destroy()
    m.destroy()


@pytest.mark.parametrize("V,B", [(1000, 20), (300, 64)])
def test_decode_logits_ragged_vocab(device, V, B):
    """One-token steps through the own LM head with a vocabulary that is not a whole number of
    16-column tiles or 128-column workgroup blocks, and row counts that leave padding rows in
    the last 16-row tile: logits and greedy picks against the oracle."""
    case(f"decode logits V={V} B={B}")
    from ssmjs_amd import backend, checkpoint
    cfg = {"vocabSize": V, "dModel": 128, "numLayers": 2, "dState": 64, "dConv": 4,
           "expand": 2, "nHeads": 4, "nGroups": 1,
           "layers": [{"type": "mamba2"}, {"type": "mamba1"}]}
    m = backend.Model(device, cfg, seed=13)
    dims, T = checkpoint.unpack(m.export_weights())
    T["embedding"] = T["embedding"] * 40.0
    blob = checkpoint.pack(dims, T)
    m.load_weights(blob)
    om = O.Model(blob)
    ids = np.random.default_rng(9).integers(0, V, (B, 5)).astype(np.uint32)
    st, ost = m.new_state(B), om.new_state(B)
    st.prefill(ids[:, :3])
    ost.prefill(ids[:, :3])
    for t in range(3, 5):
        lg, am = st.decode(ids[:, t])
        ref = ost.decode(ids[:, t])
        close(lg, ref, "logits")
        top2 = np.sort(ref, axis=1)[:, -2:]
        ok = (top2[:, 1] - top2[:, 0]) > 1e-4 * np.abs(ref).max()
        np.testing.assert_array_equal(am[ok], np.argmax(ref, axis=1)[ok])
    st.destroy()
    m.destroy()


def test_decode_graph_replay_matches_eager(device, monkeypatch):
    """Repeated one-token steps replay a captured HIP graph (from the second step with the same
    buffers on). Every replayed step must give the same bits as eager launches from the same
    state, also after another state with a larger batch has moved the shared workspaces (the
    graph is then captured again)."""
    case("decode graph replay vs eager")
    m, _ = _model(device, ["mamba2", "mamba1", "mamba2"], N=64)
    r = np.random.default_rng(7)
    ids = r.integers(0, 512, (2, 10)).astype(np.uint32)
    tmp = m.new_state(2)
    img = (0.1 * r.standard_normal(tmp.read().size)).astype(np.float32)
    tmp.destroy()
    runs = {}
    for mode in ("eager", "graph"):
        monkeypatch.setenv("SSM_DECODE_GRAPH", "0" if mode == "eager" else "1")
        st = m.new_state(2)
        st.write(img)
        out = []
        for t in range(10):
            if t == 5:
                big = m.new_state(6)   # larger batch: the shared workspaces grow
                big.decode(r.integers(0, 512, 6))
                big.destroy()
            lg, am = st.decode(ids[:, t])
            out.append((lg.copy(), am.copy(), st.read()))
        runs[mode] = out
        st.destroy()
    for t, (a, b) in enumerate(zip(runs["eager"], runs["graph"])):
        for x, y in zip(a, b):
            assert np.array_equal(x, y), f"step {t} differs"
    m.destroy()


@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_decode_rejects_out_of_range_id(device, monkeypatch, mode):
    """A token id at or past the vocabulary in a one-token step (whose embedding gather also
    writes the first fused layer's norm operand) is reported as INVALID_ARG, eagerly and from
    a replayed graph; the flag does not stick, so the next valid step succeeds and matches a
    model that never saw the bad id from the same state."""
    case(f"decode out-of-range id ({mode})")
    from ssmjs_amd import _lib
    monkeypatch.setenv("SSM_DECODE_GRAPH", "0" if mode == "eager" else "1")
    m, _ = _model(device, ["mamba2", "mamba1"], N=64)
    V = m.vocab
    r = np.random.default_rng(11)
    st = m.new_state(3)
    for _ in range(2):   # from the second step on, graph mode replays a captured step
        st.decode(r.integers(0, V, 3))
    with pytest.raises(_lib.SsmError) as e:
        st.decode(np.array([1, V, 2], np.uint32))
    assert e.value.status == 1 and "out of range" in str(e.value)
    img = st.read()
    good = r.integers(0, V, 3)
    lg, am = st.decode(good)
    ref = m.new_state(3)
    ref.write(img)
    lg_ref, am_ref = ref.decode(good)
    assert np.array_equal(lg, lg_ref) and np.array_equal(am, am_ref)
    ref.destroy()
    st.destroy()
    m.destroy()


def test_greedy_equals_reprefill(device):
    """generate() (recurrent) == tokenStream semantics (full re-prefill each step,
    src/session/streaming.ts:30-45) for topK = 1."""
    case("greedy vs re-prefill")
    m, _ = _model(device, ["mamba2", "mamba1"], N=64)
    ids = [5, 17, 99]
    st = m.new_state(1)
    fast = st.generate_greedy(np.array([ids], np.uint32), 8)[0].tolist()
    slow = list(ids)
    for _ in range(8):
        lg = m.forward(np.array([slow], np.uint32))[0, -1]
        slow.append(int(np.argmax(lg)))
    assert fast == slow[len(ids):]
    m.destroy()


def test_checkpoint_errors(device):
    case("checkpoint errors")
    from ssmjs_amd import _lib
    m, blob = _model(device, ["mamba1"])
    with pytest.raises(_lib.SsmError) as e:
        m.load_weights(b"XXXX" + blob[4:])
    assert e.value.code == "CHECKPOINT_INVALID"
    with pytest.raises(_lib.SsmError) as e:
        m.load_weights(blob[:-8])
    assert e.value.code == "CHECKPOINT_INVALID"
    f16 = m.export_weights(f16=True)
    m.load_weights(f16)            # f16 images load (values rounded to half)
    m.load_weights(blob)
    with pytest.raises(_lib.SsmError):
        m.forward(np.array([[600]], np.uint32))   # id >= vocab
    h = m.handle
    m.destroy()
    ids = np.zeros((1, 1), np.uint32)
    out = np.zeros((1, 1, 512), np.float32)
    with pytest.raises(_lib.SsmError) as e:
        _lib.call("ssm_forward", h, ids.ctypes.data, 1, 1, out.ctypes.data)
    assert e.value.code == "SESSION_DESTROYED"


def test_unsupported_layer_types(device):
    case("unsupported layers")
    from ssmjs_amd import _lib, backend
    for t in ("attention", "mamba3"):
        cfg = {"vocabSize": 10, "dModel": 16, "numLayers": 1, "dState": 8, "dConv": 4,
               "expand": 2, "nHeads": 4, "layers": [{"type": t}]}
        with pytest.raises(_lib.SsmError):
            backend.Model(device, cfg)


@pytest.mark.parametrize("T,topK,topP", [(0.8, 50, 0.9), (1.3, 1024, 1.0), (0.8, 1, 0.9),
                                         (1.0, 3, 0.5)])
def test_sampled_generation_matches_oracle_sampler(device, T, topK, topP):
    """ssm_generate_sample (prefill, then per token one recurrent step and sampleToken on the
    device) picks, row by row, what the oracle's sampleToken (streaming.ts:53-97) picks on
    the same device logits with the same draws."""
    case(f"generate_sample T={T} topK={topK} topP={topP}")
    m, _ = _model(device, ["mamba2", "mamba1"], N=64, emb_scale=4.0)
    r = np.random.default_rng(21)
    B, Lp, n_new = 3, 9, 16
    prompt = r.integers(0, 512, (B, Lp)).astype(np.uint32)
    u = r.random((n_new, B))
    u[0, 0], u[1, 1] = 0.0, 0.9999999999
    st = m.new_state(B)
    got = st.generate_sample(prompt, n_new, T, topK, topP, u)
    st.destroy()
    st = m.new_state(B)
    lg, _ = st.prefill(prompt)
    want = np.zeros((B, n_new), np.uint32)
    for k in range(n_new):
        for b in range(B):
            want[b, k] = O.sample_token(lg[b], T, topK, topP, u[k, b])
        if k + 1 < n_new:
            lg, _ = st.decode(want[:, k])
    st.destroy()
    print(f"  distinct picks {len(np.unique(want))}")
    np.testing.assert_array_equal(got, want)
    m.destroy()


def test_model_generate_sampled_equals_host_loop(device):
    """HybridMambaModel.generate (device sampler) == the host loop of streaming.ts:17-49
    (prefill, decode, host sampleToken) with the same seeded draws, up to eos."""
    case("HybridMambaModel.generate sampled vs host loop")
    import random as _random
    from ssmjs_amd import model as M
    from ssmjs_amd.streaming import sample_token
    dev_ = M.HipDevice(0)
    cfg = {"vocabSize": 300, "dModel": 128, "numLayers": 2, "dState": 32, "dConv": 4,
           "expand": 2, "nHeads": 4, "layers": [{"type": "mamba2"}, {"type": "mamba1"}],
           "eosId": 7}
    hm = M.HybridMambaModel(dev_, cfg, seed=5)
    sampling = {"temperature": 0.8, "topK": 50, "topP": 0.9}
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    got = hm.generate(prompt, 40, sampling, rng=_random.Random(1234).random)
    rng = _random.Random(1234).random
    st = hm.native.new_state(1)
    ids = list(prompt)
    lg, _ = st.prefill(np.array([ids], np.uint32))
    for k in range(40):
        nxt = sample_token(lg[0], 0.8, 50, 0.9, rng)
        ids.append(nxt)
        if nxt == 7 or k + 1 == 40:
            break
        lg, _ = st.decode(np.array([nxt], np.uint32))
    st.destroy()
    assert got == ids
    hm.destroy()
    dev_.destroy()
