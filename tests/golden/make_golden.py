"""Writes the golden vectors in tests/golden/*.npz (run here, never on the GPU box).

The reference has no golden vectors for the SSM path: its arithmetic lives in the absent
@seanhogg/mambacode.js package. These vectors come from an independent third-party
implementation of the same published math that happens to be installed in this container:
HF transformers 5.15.0, pure-torch fallbacks in transformers/models/mamba/modeling_mamba.py
(causal_conv1d_fn, causal_conv1d_update, mamba_selective_scan, mamba_selective_state_update)
and transformers/models/mamba2/modeling_mamba2.py (mamba2_chunk_scan,
mamba2_selective_state_update, MambaRMSNormGated), plus tiny random-init MambaForCausalLM /
Mamba2ForCausalLM models built from a config (no download). They pin the CPU oracle in
oracle/ssm_oracle.c; the oracle in turn is the checker for the HIP kernels.

Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from ssmjs_amd import checkpoint as ckpt  # noqa: E402


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def n(x):
    return x.detach().cpu().numpy().astype(np.float32)


def kernels(seed=1001):
    from transformers.models.mamba import modeling_mamba as hm
    from transformers.models.mamba2 import modeling_mamba2 as hm2

    r = np.random.default_rng(seed)
    f = lambda *s, sc=1.0: (r.standard_normal(s) * sc).astype(np.float32)  # noqa: E731
    out = {}

    # conv1d + SiLU, prefill: HF layout is (B, C, L)
    B, L, C, K = 2, 11, 6, 4
    x = f(B, L, C)
    w = r.uniform(-0.5, 0.5, (C, K)).astype(np.float32)
    b = f(C, sc=0.1)
    y = hm.causal_conv1d_fn(t(x.transpose(0, 2, 1)), t(w), t(b), activation="silu")
    out.update(conv_x=x, conv_w=w, conv_b=b, conv_y=n(y).transpose(0, 2, 1))

    # conv update (decode): state (B, C, K-1)
    st = f(B, C, K - 1)
    xs = f(B, C)
    st_t = t(st.copy())
    ys = hm.causal_conv1d_update(t(xs[:, :, None]), st_t, t(w), t(b), activation="silu")
    out.update(convu_x=xs, convu_state=st, convu_y=n(ys)[:, :, 0], convu_state_out=n(st_t))

    # Mamba-1 selective scan: HF layout u, dt, z (B, D, L); B, C (B, N, L)
    B, L, D, N = 2, 13, 5, 4
    u, z = f(B, L, D), f(B, L, D)
    dt = (f(B, L, D) * 0.5 - 1.0).astype(np.float32)
    A = -np.exp(f(D, N, sc=0.5))
    Bm, Cm = f(B, L, N), f(B, L, N)
    Dsk = f(D)
    dtb = f(D, sc=0.1)
    with torch.no_grad():
        ys, hT = hm.mamba_selective_scan(
            t(u.transpose(0, 2, 1)), t(dt.transpose(0, 2, 1)), t(A), t(Bm.transpose(0, 2, 1)),
            t(Cm.transpose(0, 2, 1)), D=t(Dsk), z=t(z.transpose(0, 2, 1)), delta_bias=t(dtb),
            delta_softplus=True, return_last_state=True, use_associative_scan=False)
    out.update(scan_u=u, scan_dt=dt, scan_A=A, scan_B=Bm, scan_C=Cm, scan_D=Dsk, scan_z=z,
               scan_dtb=dtb, scan_y=n(ys).transpose(0, 2, 1), scan_hT=n(hT))

    # Mamba-1 one-token state update
    h0 = f(B, D, N, sc=0.3)
    x1, dt1, z1 = f(B, D), f(B, D) * 0.5 - 1.0, f(B, D)
    B1, C1 = f(B, N), f(B, N)
    h_t = t(h0.copy())
    with torch.no_grad():
        y1 = hm.mamba_selective_state_update(h_t, t(x1), t(dt1.astype(np.float32)), t(A), t(B1),
                                             t(C1), D=t(Dsk), dt_bias=t(dtb), dt_softplus=True,
                                             z=t(z1))
    out.update(m1u_h0=h0, m1u_x=x1, m1u_dt=dt1.astype(np.float32), m1u_z=z1, m1u_B=B1, m1u_C=C1,
               m1u_y=n(y1), m1u_h=n(h_t))

    # Mamba-2 SSD (chunked), L not a multiple of the chunk, with initial states
    B, L, H, P, G, N, Q = 2, 37, 4, 3, 2, 5, 8
    x = f(B, L, H, P)
    dt = (f(B, L, H) - 1.0).astype(np.float32)
    A = -np.exp(f(H, sc=0.5))
    Bm, Cm = f(B, L, G, N), f(B, L, G, N)
    Dsk, dtb = f(H), f(H, sc=0.1)
    hs0 = f(B, H, P, N, sc=0.3)
    with torch.no_grad():
        y2, hT2 = hm2.mamba2_chunk_scan(t(x), t(dt), t(A), t(Bm), t(Cm), Q, D=t(Dsk),
                                        dt_bias=t(dtb), initial_states=t(hs0), dt_softplus=True,
                                        return_final_states=True)
    out.update(ssd_x=x, ssd_dt=dt, ssd_A=A, ssd_B=Bm, ssd_C=Cm, ssd_D=Dsk, ssd_dtb=dtb,
               ssd_h0=hs0, ssd_Q=np.int32(Q), ssd_y=n(y2), ssd_hT=n(hT2))

    # Mamba-2 one-token state update: HF expects per-(h,p) expanded dt, A, dt_bias, D
    x1 = f(B, H, P)
    dt1 = (f(B, H) - 1.0).astype(np.float32)
    B1, C1 = f(B, G, N), f(B, G, N)
    z1 = f(B, H, P)
    h_t = t(hs0.copy())
    with torch.no_grad():
        y1 = hm2.mamba2_selective_state_update(
            h_t, t(x1), t(np.repeat(dt1[:, :, None], P, 2)),
            t(np.broadcast_to(A[:, None, None], (H, P, N)).copy()), t(B1), t(C1),
            D=t(np.repeat(Dsk[:, None], P, 1)), dt_bias=t(np.repeat(dtb[:, None], P, 1)),
            dt_softplus=True, z=t(z1))
    out.update(m2u_x=x1, m2u_dt=dt1, m2u_B=B1, m2u_C=C1, m2u_z=z1, m2u_y=n(y1), m2u_h=n(h_t))

    # gated RMSNorm (group = whole row), norm after gate
    M, Dn = 3, 10
    xg, zg, wg = f(M, Dn), f(M, Dn), f(Dn, sc=0.5) + 1.0
    norm = hm2.MambaRMSNormGated(Dn, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(t(wg))
        yg = norm(t(xg), t(zg))
    out.update(gn_x=xg, gn_z=zg, gn_w=wg, gn_y=n(yg))
    return out


def hf_model_fixture(kind, seed):
    """Tiny random-init HF causal LM -> (SSMW image, ids, logits)."""
    torch.manual_seed(seed)
    V, d, nl, L, Bsz = 64, 32, 2, 12, 2
    if kind == "mamba1":
        from transformers import MambaConfig, MambaForCausalLM
        cfg = MambaConfig(vocab_size=V, hidden_size=d, state_size=8, num_hidden_layers=nl,
                          expand=2, conv_kernel=4, time_step_rank=4, tie_word_embeddings=True,
                          use_mambapy=False, use_associative_scan=False)
        m = MambaForCausalLM(cfg).eval()
        dims = ckpt.ModelDims(vocab=V, d_model=d, n_layers=nl, d_state=8, d_conv=4, expand=2,
                              n_heads=4, n_groups=1, dt_rank=4, layers=["mamba1"] * nl)
        T = {"embedding": n(m.backbone.embeddings.weight), "norm_f": n(m.backbone.norm_f.weight)}
        for i, blk in enumerate(m.backbone.layers):
            mx, p = blk.mixer, f"layers.{i}."
            T[p + "norm"] = n(blk.norm.weight)
            T[p + "in_proj"] = n(mx.in_proj.weight)
            T[p + "conv_w"] = n(mx.conv1d.weight)[:, 0, :]
            T[p + "conv_b"] = n(mx.conv1d.bias)
            T[p + "x_proj"] = n(mx.x_proj.weight)
            T[p + "dt_proj_w"] = n(mx.dt_proj.weight)
            T[p + "dt_proj_b"] = n(mx.dt_proj.bias)
            T[p + "A_log"] = n(mx.A_log)
            T[p + "D"] = n(mx.D)
            T[p + "out_proj"] = n(mx.out_proj.weight)
    else:
        from transformers import Mamba2Config, Mamba2ForCausalLM
        H, P, N = 4, 16, 16
        cfg = Mamba2Config(vocab_size=V, hidden_size=d, num_heads=H, head_dim=P, state_size=N,
                           num_hidden_layers=nl, expand=2, n_groups=1, conv_kernel=4,
                           chunk_size=8, tie_word_embeddings=True)
        m = Mamba2ForCausalLM(cfg).eval()
        # random-init HF zeroes nothing we need; perturb D and norms so they matter
        with torch.no_grad():
            for blk in m.backbone.layers:
                blk.mixer.D.uniform_(0.5, 1.5)
                blk.mixer.norm.weight.uniform_(0.5, 1.5)
                blk.norm.weight.uniform_(0.5, 1.5)
        dims = ckpt.ModelDims(vocab=V, d_model=d, n_layers=nl, d_state=N, d_conv=4, expand=2,
                              n_heads=H, n_groups=1, layers=["mamba2"] * nl, chunk_len=8)
        T = {"embedding": n(m.backbone.embeddings.weight), "norm_f": n(m.backbone.norm_f.weight)}
        for i, blk in enumerate(m.backbone.layers):
            mx, p = blk.mixer, f"layers.{i}."
            T[p + "norm"] = n(blk.norm.weight)
            T[p + "in_proj"] = n(mx.in_proj.weight)
            T[p + "conv_w"] = n(mx.conv1d.weight)[:, 0, :]
            T[p + "conv_b"] = n(mx.conv1d.bias)
            T[p + "dt_bias"] = n(mx.dt_bias)
            T[p + "A_log"] = n(mx.A_log)
            T[p + "D"] = n(mx.D)
            T[p + "gnorm"] = n(mx.norm.weight)
            T[p + "out_proj"] = n(mx.out_proj.weight)
    ids = torch.randint(0, V, (Bsz, L))
    with torch.no_grad():
        logits = m(input_ids=ids, use_cache=False).logits
    blob = ckpt.pack(dims, T)
    return {"blob": np.frombuffer(blob, np.uint8), "ids": n(ids).astype(np.uint32),
            "logits": n(logits)}


def main():
    np.savez(os.path.join(HERE, "hf_kernels.npz"), **kernels())
    for kind, seed in (("mamba1", 1011), ("mamba2", 1012)):
        np.savez(os.path.join(HERE, f"hf_model_{kind}.npz"), **hf_model_fixture(kind, seed))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
