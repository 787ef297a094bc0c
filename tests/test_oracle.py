"""Pins the CPU oracle (oracle/ssm_oracle.c) before it is trusted as the HIP path's checker.

Each oracle function is checked against (a) the golden vectors written by
tests/golden/make_golden.py from HF transformers' independent torch implementation of the
same published math, and (b) closed forms, invariants and cross-checks between oracle
functions written with different code (chunked vs sequential SSD, SSD vs Mamba-1 scan,
one-token updates vs L=1 prefill), chosen so that a dropped term, a sign or an index slip
fails at least one of them.
"""
import numpy as np
import pytest

from oracle import oracle as O

RTOL = 1e-4


def close(a, b, rtol=RTOL, atol=1e-5):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = max(1.0, float(np.abs(b).max()))
    err = float(np.abs(a - b).max()) / scale
    assert err <= max(rtol, atol), f"max scaled err {err:.3e}"


rng = np.random.default_rng(7)


def rn(*s, sc=1.0):
    return (rng.standard_normal(s) * sc).astype(np.float32)


# ---------------------------------------------------------------- golden (HF) vectors

def test_conv_matches_hf(golden):
    g = golden["hf_kernels"]
    close(O.causal_conv1d(g["conv_x"], g["conv_w"], g["conv_b"]), g["conv_y"])


def test_conv_update_matches_hf(golden):
    g = golden["hf_kernels"]
    y, st = O.conv_update(g["convu_x"], g["conv_w"], g["conv_b"], g["convu_state"])
    close(y, g["convu_y"])
    close(st, g["convu_state_out"])


def test_selective_scan_matches_hf(golden):
    g = golden["hf_kernels"]
    y, hT = O.selective_scan(g["scan_u"], g["scan_dt"], g["scan_A"], g["scan_B"], g["scan_C"],
                             g["scan_D"], g["scan_z"], g["scan_dtb"], True, return_state=True)
    close(y, g["scan_y"])
    close(hT, g["scan_hT"])


def test_m1_state_update_matches_hf(golden):
    g = golden["hf_kernels"]
    y, h = O.m1_state_update(g["m1u_x"], g["m1u_dt"], g["scan_A"], g["m1u_B"], g["m1u_C"],
                             g["scan_D"], g["m1u_z"], g["scan_dtb"], g["m1u_h0"])
    close(y, g["m1u_y"])
    close(h, g["m1u_h"])


@pytest.mark.parametrize("chunk", [None, 8, 5])
def test_ssd_matches_hf(golden, chunk):
    g = golden["hf_kernels"]
    y, hT = O.ssd(g["ssd_x"], g["ssd_dt"], g["ssd_A"], g["ssd_B"], g["ssd_C"], g["ssd_D"],
                  dt_bias=g["ssd_dtb"], h0=g["ssd_h0"], return_state=True, chunk=chunk)
    close(y, g["ssd_y"])
    close(hT, g["ssd_hT"])


def test_m2_state_update_matches_hf(golden):
    g = golden["hf_kernels"]
    y, h = O.m2_state_update(g["m2u_x"], g["m2u_dt"], g["ssd_A"], g["m2u_B"], g["m2u_C"],
                             g["ssd_D"], g["ssd_dtb"], g["ssd_h0"], z=g["m2u_z"])
    close(y, g["m2u_y"])
    close(h, g["m2u_h"])


def test_gated_rmsnorm_matches_hf(golden):
    g = golden["hf_kernels"]
    close(O.gated_rmsnorm(g["gn_x"], g["gn_z"], g["gn_w"]), g["gn_y"])


@pytest.mark.parametrize("kind", ["mamba1", "mamba2"])
def test_model_forward_matches_hf(golden, kind):
    g = golden[f"hf_model_{kind}"]
    m = O.Model(g["blob"].tobytes())
    close(m.forward(g["ids"]), g["logits"], rtol=2e-4)


# ---------------------------------------------------------------- closed forms / brute force

def test_conv_k1_is_pointwise():
    x, w, b = rn(2, 5, 3), rn(3, 1), rn(3)
    v = x * w[:, 0] + b
    close(O.causal_conv1d(x, w, b), v / (1 + np.exp(-v)))


def test_conv_impulse_returns_weights():
    K, Cc = 4, 3
    x = np.zeros((1, 6, Cc), np.float32)
    x[0, 1, :] = 1.0
    w = rn(Cc, K)
    y = O.causal_conv1d(x, w, None, silu=False)
    # impulse at t=1 reaches y[t] through tap k = K-1-(t-1)
    for t in range(1, 1 + K):
        close(y[0, t], w[:, K - 1 - (t - 1)])
    close(y[0, 0], np.zeros(Cc))


def test_conv_streaming_equals_prefill():
    B, L, Cc, K = 2, 9, 4, 4
    x, w, b = rn(B, L, Cc), rn(Cc, K), rn(Cc)
    full, st_full = O.causal_conv1d(x, w, b, return_state=True)
    st = np.zeros((B, Cc, K - 1), np.float32)
    for t in range(L):
        y, st = O.conv_update(x[:, t], w, b, st)
        close(y, full[:, t])
    close(st, st_full)
    # split prefill with a carried state
    a, sa = O.causal_conv1d(x[:, :4], w, b, return_state=True)
    c = O.causal_conv1d(x[:, 4:], w, b, state_in=sa)
    close(np.concatenate([a, c], 1), full)


def test_scan_zero_input_keeps_skip():
    B, L, D, N = 1, 7, 3, 4
    u, z = rn(B, L, D), rn(B, L, D)
    A = -np.abs(rn(D, N)) - 0.1
    y = O.selective_scan(u, rn(B, L, D), A, np.zeros((B, L, N), np.float32), rn(B, L, N),
                         np.full(D, 0.7, np.float32), z)
    close(y, 0.7 * u * z / (1 + np.exp(-z)))


def test_scan_geometric_closed_form():
    # constant delta, u = B = C = 1, no softplus: h_t = sum_{s<=t} e^{dA s} * delta
    L, d, a = 9, 0.3, -0.8
    u = np.ones((1, L, 1), np.float32)
    y = O.selective_scan(u, np.full((1, L, 1), d, np.float32), np.array([[a]], np.float32),
                         np.ones((1, L, 1), np.float32), np.ones((1, L, 1), np.float32),
                         softplus=False)
    q = np.exp(d * a)
    ref = np.array([d * (1 - q ** (t + 1)) / (1 - q) for t in range(L)])
    close(y[0, :, 0], ref)


def test_scan_state_passing():
    B, L, D, N = 2, 12, 3, 5
    args = dict(A=-np.exp(rn(D, N, sc=0.3)), D=rn(D), dt_bias=rn(D, sc=0.1))
    u, dt, z, Bm, Cm = rn(B, L, D), rn(B, L, D), rn(B, L, D), rn(B, L, N), rn(B, L, N)
    y, hT = O.selective_scan(u, dt, Bm=Bm, Cm=Cm, z=z, return_state=True, **args)
    y1, h1 = O.selective_scan(u[:, :5], dt[:, :5], Bm=Bm[:, :5], Cm=Cm[:, :5], z=z[:, :5],
                              return_state=True, **args)
    y2, h2 = O.selective_scan(u[:, 5:], dt[:, 5:], Bm=Bm[:, 5:], Cm=Cm[:, 5:], z=z[:, 5:],
                              h0=h1, return_state=True, **args)
    close(np.concatenate([y1, y2], 1), y)
    close(h2, hT)


@pytest.mark.parametrize("Q", [1, 3, 16, 64])
def test_ssd_chunked_equals_sequential(Q):
    B, L, H, P, G, N = 2, 19, 4, 3, 2, 5
    x, dt, Bm, Cm, z = rn(B, L, H, P), rn(B, L, H), rn(B, L, G, N), rn(B, L, G, N), rn(B, L, H, P)
    A = -np.exp(rn(H, sc=0.5))
    h0 = rn(B, H, P, N, sc=0.2)
    Dh, db = rn(H), rn(H)
    ys, hs = O.ssd(x, dt, A, Bm, Cm, Dh, z=z, dt_bias=db, h0=h0, return_state=True)
    yc, hc = O.ssd(x, dt, A, Bm, Cm, Dh, z=z, dt_bias=db, h0=h0, return_state=True, chunk=Q)
    close(yc, ys)
    close(hc, hs)


def test_ssd_equals_mamba1_scan_with_tied_params():
    # one head of SSD == Mamba-1 scan over P channels with A[d,n] = A_h, shared delta/B/C
    B, L, P, N = 1, 10, 3, 4
    x, dt, Bm, Cm = rn(B, L, 1, P), rn(B, L, 1), rn(B, L, 1, N), rn(B, L, 1, N)
    A = np.array([-0.7], np.float32)
    y = O.ssd(x, dt, A, Bm, Cm, np.array([0.5], np.float32), dt_bias=np.array([0.1], np.float32))
    y1 = O.selective_scan(x[:, :, 0, :], np.repeat(dt, P, 2), np.full((P, N), -0.7, np.float32),
                          Bm[:, :, 0], Cm[:, :, 0], np.full(P, 0.5, np.float32),
                          dt_bias=np.full(P, 0.1, np.float32))
    close(y[:, :, 0, :], y1)


def test_ssd_dt_limits_clamp():
    B, L, H, P, G, N = 1, 6, 2, 2, 1, 3
    x, dt, Bm, Cm = rn(B, L, H, P), rn(B, L, H) * 3, rn(B, L, G, N), rn(B, L, G, N)
    A = np.array([-1.0, -2.0], np.float32)
    y = O.ssd(x, dt, A, Bm, Cm, dt_min=0.2, dt_max=0.2)
    # all deltas equal 0.2 -> compare against softplus-free input of 0.2
    y2 = O.ssd(x, np.full_like(dt, 0.2), A, Bm, Cm, softplus=False)
    close(y, y2)


def test_m1_update_equals_L1_scan():
    B, D, N = 2, 4, 3
    h0 = rn(B, D, N)
    x, dt, z, Bm, Cm = rn(B, D), rn(B, D), rn(B, D), rn(B, N), rn(B, N)
    A, Dk, db = -np.exp(rn(D, N, sc=0.3)), rn(D), rn(D)
    y, h = O.m1_state_update(x, dt, A, Bm, Cm, Dk, z, db, h0)
    y1, h1 = O.selective_scan(x[:, None], dt[:, None], A, Bm[:, None], Cm[:, None], Dk,
                              z[:, None], db, h0=h0, return_state=True)
    close(y, y1[:, 0])
    close(h, h1)


def test_m2_update_equals_L1_ssd():
    B, H, P, G, N = 2, 4, 3, 2, 5
    h0 = rn(B, H, P, N)
    x, dt, Bm, Cm = rn(B, H, P), rn(B, H), rn(B, G, N), rn(B, G, N)
    A, Dk, db = -np.exp(rn(H, sc=0.3)), rn(H), rn(H)
    y, h = O.m2_state_update(x, dt, A, Bm, Cm, Dk, db, h0)
    y1, h1 = O.ssd(x[:, None], dt[:, None], A, Bm[:, None], Cm[:, None], Dk, dt_bias=db, h0=h0,
                   return_state=True)
    close(y, y1[:, 0])
    close(h, h1)


def test_rmsnorm_unit_rows():
    x = rn(3, 8)
    y = O.rmsnorm(x, np.ones(8, np.float32), eps=0.0)
    close(np.sqrt((y.astype(np.float64) ** 2).mean(1)), np.ones(3))
    close(O.rmsnorm(2.5 * x, np.ones(8, np.float32), eps=0.0), y)


def test_linear_brute_force():
    x, W, b = rn(4, 6), rn(5, 6), rn(5)
    close(O.linear(x, W, b), x.astype(np.float64) @ W.T.astype(np.float64) + b)


@pytest.mark.parametrize("kind", ["mamba1", "mamba2"])
def test_model_prefill_decode_equals_forward(golden, kind):
    g = golden[f"hf_model_{kind}"]
    m = O.Model(g["blob"].tobytes())
    ids = g["ids"]
    full = m.forward(ids)
    st = m.new_state(ids.shape[0])
    close(st.prefill(ids[:, :5]), full[:, 4])
    for t in range(5, ids.shape[1]):
        close(st.decode(ids[:, t]), full[:, t])


def test_model_rejects_bad_images(golden):
    blob = bytearray(golden["hf_model_mamba1"]["blob"].tobytes())
    with pytest.raises(ValueError, match="magic"):
        O.Model(b"XXXX" + bytes(blob[4:]))
    with pytest.raises(ValueError, match="size"):
        O.Model(bytes(blob[:-4]))
    bad = bytearray(blob)
    bad[4] = 9
    with pytest.raises(ValueError, match="version"):
        O.Model(bytes(bad))


# ---------------------------------------------------------------- sampleToken restatement
# orc_sample_token follows src/session/streaming.ts:53-97. It is pinned by answers the
# reference's arithmetic fixes (stable sort, nucleus cut, draw order), by the exact-tie rule
# of the f32 exps, and by agreement with the independent numpy restatement in
# ssmjs_amd/streaming.py on rows with many ties.

def test_sample_token_known_answers():
    lg = np.array([0.1, 3.0, -2.0, 3.0, 1.0], np.float32)
    for u in (0.0, 0.5, 0.999999):                 # topK 1: first of the stable sort
        assert O.sample_token(lg, 0.8, 1, 0.9, u) == 1
    p = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    assert O.sample_token(p, 1.0, 50, 0.7, 0.0) == 0      # nucleus [0, 1]
    assert O.sample_token(p, 1.0, 50, 0.7, 0.99) == 1
    assert O.sample_token(p, 1.0, 3, 1.0, 0.999) == 2     # topK 3 never reaches index 3
    assert O.sample_token(p, 1.0, 50, 0.0, 0.999) == 0    # topP 0: nucleus = top entry
    assert O.sample_token(p, 1.0, 99, 1.0, 0.999) == 3    # topK > n: every index
    assert O.sample_token(np.zeros(7, np.float32), 1.0, 50, 1.0, 0.999) == 6
    with pytest.raises(ValueError):
        O.sample_token(p, 1.0, 0, 0.9, 0.5)


def test_sample_token_ties_of_rounded_exps():
    """Two logits whose exps round to the same f32 tie, and the lower index wins even when
    its logit is smaller: exp(-7.45e-9) rounds to 1.0f."""
    a = np.float32(0.1)
    b = np.nextafter(a, np.float32(1.0))
    assert b > a
    assert O.sample_token(np.array([a, b], np.float32), 1.0, 1, 0.9, 0.5) == 0
    assert O.sample_token(np.array([b, a], np.float32), 1.0, 1, 0.9, 0.5) == 0
    # far enough apart, the larger logit wins whatever its index
    c = np.float32(0.1 + 1e-6)
    assert O.sample_token(np.array([a, c], np.float32), 1.0, 1, 0.9, 0.5) == 1
    # temperature rounding: adjacent logits whose quotients by 5 collide in f32 tie as well
    # (ulp 1.19e-7 over 5 is below the quotient's ulp of 2.98e-8)
    x = np.float32(1.9)
    for _ in range(64):
        y = np.nextafter(x, np.float32(2.0))
        if np.float32(np.float64(x) / 5.0) == np.float32(np.float64(y) / 5.0):
            break
        x = y
    assert np.float32(np.float64(x) / 5.0) == np.float32(np.float64(y) / 5.0)
    assert O.sample_token(np.array([x, y], np.float32), 5.0, 1, 0.9, 0.5) == 0
    assert O.sample_token(np.array([y, x], np.float32), 5.0, 1, 0.9, 0.5) == 0


def test_sample_token_temperature_floor():
    lg = np.array([0.0, 1e-6, -1e-6], np.float32)
    # T <= 1e-7 acts as 1e-7: scaled gaps of 10 make the top entry take the whole nucleus
    for T in (0.0, -1.0, 1e-9):
        assert O.sample_token(lg, T, 50, 0.9, 0.999) == 1


def test_sample_token_draw_is_renormalised_nucleus():
    """Over a uniform grid of draws the picks follow e_k / (nucleus sum): the CDF walk."""
    lg = np.log(np.array([0.4, 0.25, 0.2, 0.1, 0.05], np.float32))
    M = 2000
    counts = np.zeros(5)
    for j in range(M):
        counts[O.sample_token(lg, 1.0, 4, 0.8, (j + 0.5) / M)] += 1
    e = np.exp(lg.astype(np.float64) - lg.max())
    nucleus = e[:3]                                   # 0.4 + 0.25 + 0.2 >= 0.8
    want = np.zeros(5)
    want[:3] = nucleus / nucleus.sum()
    assert np.abs(counts / M - want).max() <= 1.0 / M + 1e-12


@pytest.mark.parametrize("n", [1, 2, 700, 5000])
def test_sample_token_agrees_with_host_restatement(n):
    from ssmjs_amd.streaming import sample_token as host_sample
    r = np.random.default_rng(900 + n)
    for trial in range(12):
        if trial % 3 == 0:
            lg = r.integers(-3, 3, n).astype(np.float32) * 0.5   # heavy ties
        else:
            lg = (r.standard_normal(n) * (0.05 if trial % 3 == 1 else 3.0)).astype(np.float32)
        if trial % 4 == 3 and n > 1:
            lg[r.random(n) < 0.3] = -np.inf     # masked tokens: e = 0
            lg[0] = 0.5
        T = [1.0, 0.8, 2.5, 1e-9][trial % 4]
        K = [1, 2, 50, n, n + 5, 1024][trial % 6]
        P = [0.9, 1.0, 0.5, 0.0][(trial // 2) % 4]
        for u in (0.0, 0.3, float(r.random()), 0.9999999):
            assert O.sample_token(lg, T, K, P, u) == host_sample(lg, T, K, P, rng=lambda: u)
