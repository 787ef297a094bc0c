/*
 * ssm_oracle.h -- CPU restatement of the Mamba SSM forward path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker for the HIP path in ssmjs_amd/csrc. Only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load it. The
 * product path never calls it.
 *
 * The reference (SeanHogg/ssmjs) keeps all SSM arithmetic in the un-vendored npm package
 * @seanhogg/mambacode.js@2026.3.21 (package-lock.json:1231-1241), which is absent here.
 * The functions below restate the published algorithms that package names as its
 * "Mamba-1/2 SSM math" (README.md:19, src/index.ts:5):
 *   - Mamba-1 selective scan: Gu & Dao 2023 (arXiv:2312.00752) section 3.2, Algorithm 2;
 *   - Mamba-2 SSD: Dao & Gu 2024 (arXiv:2405.21060) section 6 (chunked SSD);
 *   - causal depthwise conv1d + SiLU, RMSNorm, gated RMSNorm (Mamba-2 block).
 * The reference's call sites: model.forward (src/session/streaming.ts:31-35),
 * model.generate (src/session/session.ts:421-425), new HybridMambaModel (session.ts:359).
 *
 * All arrays are float32, row-major, last index fastest. Accumulation is in double.
 * "ld" arguments are row strides (in elements) between consecutive time steps; the
 * batch stride is L*ld.
 */
#ifndef SSM_ORACLE_H
#define SSM_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads the OpenMP loops use; outputs are independent of it. */
int orc_num_threads(void);

/* y[b,t,c] = act(bias[c] + sum_k w[c,k] * x[b,t-K+1+k,c]); x at t<0 is state_in[b,c,K-1+t]
 * (zero when state_in is NULL). state_out[b,c,:] receives the last K-1 inputs. */
void orc_causal_conv1d(const float* x, long ldx, const float* w, const float* bias,
                       float* y, long ldy, int B, int L, int C, int K, int silu,
                       const float* state_in, float* state_out);

/* Mamba-1 selective scan (Algorithm 2): dt' = softplus(dt + dt_bias) (if softplus);
 * h_t = exp(dt' A) h_{t-1} + dt' B_t u_t; y_t = C_t . h_t + Dsk u_t; y_t *= silu(z_t).
 * u, dt, z: (B,L,D); Bm, Cm: (B,L,N); A: (D,N); h0/hT: (B,D,N) (either may be NULL). */
void orc_selective_scan(const float* u, long ldu, const float* dt, long lddt,
                        const float* dt_bias, int softplus, const float* A,
                        const float* Bm, long ldb, const float* Cm, long ldc,
                        const float* Dsk, const float* z, long ldz, float* y, long ldy,
                        int B, int L, int D, int N, const float* h0, float* hT);

/* Mamba-2 SSD, sequential (recurrent) form with scalar A per head:
 * dt' = clamp(softplus(dt + dt_bias)); h_t[p,n] = exp(dt' A_h) h_{t-1}[p,n] + dt' x_t[p] B_t[g,n];
 * y_t[p] = sum_n C_t[g,n] h_t[p,n] + Dsk_h x_t[p]  (g = h / (H/G)); optional y *= silu(z).
 * x, z: (B,L,H,P); dt: (B,L,H); Bm, Cm: (B,L,G,N); h0/hT: (B,H,P,N). */
void orc_ssd_sequential(const float* x, long ldx, const float* dt, long lddt,
                        const float* dt_bias, int softplus, float dt_min, float dt_max,
                        const float* A, const float* Bm, long ldb, const float* Cm, long ldc,
                        const float* Dsk, const float* z, long ldz, float* y, long ldy,
                        int B, int L, int H, int P, int G, int N,
                        const float* h0, float* hT);

/* The same map computed by the chunked SSD algorithm (Dao & Gu 2024, section 6):
 * intra-chunk (C B^T . decay) X, chunk states, inter-chunk recurrence, state-to-output.
 * Chunk length Q; L need not be a multiple of Q. */
void orc_ssd_chunked(const float* x, long ldx, const float* dt, long lddt,
                     const float* dt_bias, int softplus, float dt_min, float dt_max,
                     const float* A, const float* Bm, long ldb, const float* Cm, long ldc,
                     const float* Dsk, const float* z, long ldz, float* y, long ldy,
                     int B, int L, int H, int P, int G, int N, int Q,
                     const float* h0, float* hT);

/* One-token conv update: window = [state[b,c,0..K-2], x[b,c]]; y = act(bias + w . window);
 * state shifts left by one and takes x. x, y: (B,C); state: (B,C,K-1) in place. */
void orc_conv_update(const float* x, const float* w, const float* bias, float* y,
                     float* state, int B, int C, int K, int silu);

/* One-token Mamba-1 state update: x, dt, z, y: (B,D); Bm, Cm: (B,N); h: (B,D,N) in place. */
void orc_m1_state_update(const float* x, const float* dt, const float* dt_bias, int softplus,
                         const float* A, const float* Bm, const float* Cm, const float* Dsk,
                         const float* z, float* y, float* h, int B, int D, int N);

/* One-token Mamba-2 state update: x, y: (B,H,P); dt: (B,H); Bm, Cm: (B,G,N);
 * h: (B,H,P,N) in place; z may be NULL. */
void orc_m2_state_update(const float* x, const float* dt, const float* dt_bias, int softplus,
                         float dt_min, float dt_max, const float* A, const float* Bm,
                         const float* Cm, const float* Dsk, const float* z, float* y, float* h,
                         int B, int H, int P, int G, int N);

/* y = x W^T (+ bias): x (M,K) ld ldx, W (Nout,K), y (M,Nout) ld ldy; accumulate if acc. */
void orc_linear(const float* x, long ldx, const float* W, const float* bias, float* y, long ldy,
                int M, int K, int Nout, int acc);

/* RMSNorm over rows of length n: y = x / sqrt(mean(x^2)+eps) * w. */
void orc_rmsnorm(const float* x, const float* w, float* y, int M, int n, float eps);

/* Gated RMSNorm (Mamba-2, norm after gate): y = norm_groups(x * silu(z)) * w, groups of
 * size n/G. x, z, y: (M,n) with row strides ldx, ldz, ldy. */
void orc_gated_rmsnorm(const float* x, long ldx, const float* z, long ldz, const float* w,
                       float* y, long ldy, int M, int n, int G, float eps);

/* sampleToken (src/session/streaming.ts:53-97) with Math.random() = u: scaled = float(logit /
 * max(T, 1e-7)); e = float(exp(scaled - max scaled)) (double arithmetic, float stores);
 * sumE = sum of e in index order; the topK largest e in a stable descending order; nucleus =
 * that list up to the first cumulative e/sumE >= topP; returns the first nucleus index whose
 * running e sum reaches u * (nucleus sum), else the nucleus's last index. -1 if topK < 1 or
 * n < 1 (the reference then returns undefined). */
int orc_sample_token(const float* logits, int n, double temperature, int topK, double topP,
                     double u);

/* ---- model level: weights in the ssmjs_amd checkpoint format (magic "SSMW") ---- */
typedef struct orc_model orc_model;

/* Parse a checkpoint image; returns NULL and fills err (if non-NULL) on failure. */
orc_model* orc_model_open(const void* blob, size_t size, char* err, int errlen);
void orc_model_close(orc_model* m);
int orc_model_vocab(const orc_model* m);

/* One mixer (no norm, no residual) of layer `layer` over hidden states x (B,L,d) -> out. */
void orc_mixer_forward(const orc_model* m, int layer, const float* x, int B, int L, float* out);

/* Full prefill forward: ids (B,L) -> logits (B,L,V) (zero initial state). */
void orc_model_forward(const orc_model* m, const uint32_t* ids, int B, int L, float* logits);

/* Recurrent state: allocate for batch B, zero it; run prefill over ids (B,L) updating the state
 * and writing last-position logits (B,V); then decode single tokens. */
typedef struct orc_state orc_state;
orc_state* orc_state_new(const orc_model* m, int B);
void orc_state_free(orc_state* s);
void orc_model_prefill(const orc_model* m, orc_state* s, const uint32_t* ids, int L,
                       float* last_logits);
void orc_model_decode(const orc_model* m, orc_state* s, const uint32_t* ids, float* logits);
/* State image: for each layer, its ssm state then its conv state (float32). */
size_t orc_state_floats(const orc_state* s);
void orc_state_read(const orc_model* m, const orc_state* s, float* out);
void orc_state_write(const orc_model* m, orc_state* s, const float* in);

#ifdef __cplusplus
}
#endif
#endif
