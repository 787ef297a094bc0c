/*
 * ssm_hip.h -- C ABI of libssm_hip.so, the MI355X (gfx950) backend for the Mamba SSM
 * forward path that ssmjs's MambaSession drives.
 *
 * It replaces the module interface of @seanhogg/mambacode.js@2026.3.21 (absent from the
 * reference; pinned at package-lock.json:1231-1241) as the reference's session layer uses it:
 *   initWebGPU / adapter.requestDevice      src/session/session.ts:263,274-277
 *   device.destroy()                        src/session/session.ts:592
 *   new HybridMambaModel(device, config)    src/session/session.ts:359
 *   model.forward(ids, batch, seqLen)       src/session/streaming.ts:31-35
 *   model.generate(ids, n, sampling)        src/session/session.ts:421-425
 *   model.loadWeights(buf)                  src/session/session.ts:394,575
 *   model.exportWeights()                   src/session/session.ts:518
 *   model.config.{vocabSize,eosId}          src/session/streaming.ts:24
 * plus the WGSL compute kernels behind them (README.md:19, src/index.ts:5).
 *
 * Conventions
 *   - Every call returns an ssm_status; 0 is success. ssm_last_error() returns a
 *     thread-local message for the last failure on the calling thread.
 *   - Kernel-level entry points take DEVICE pointers and a HIP stream (hipStream_t passed
 *     as void*, NULL = the null stream). Model-level entry points take HOST buffers unless
 *     the name ends in _device.
 *   - Tensors are row-major, last index fastest. An "ld" argument is the stride, in
 *     elements, between consecutive time steps (rows); the batch stride is L*ld.
 *   - Nothing here allocates device memory except ssm_ctx_create, ssm_malloc,
 *     ssm_model_create, ssm_state_create and the model-level forward calls (which grow a
 *     model-owned workspace).
 */
#ifndef SSM_HIP_H
#define SSM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status codes */
/* Codes map onto SessionErrorCode (src/session/errors.ts:5-13) and SSMErrorCode
 * (src/errors/SSMError.ts:9-15); ssm_status_name gives the reference's string. */
typedef int ssm_status;
#define SSM_OK 0
#define SSM_ERR_INVALID_ARG 1         /* 'UNKNOWN' (bad shape / pointer / option)      */
#define SSM_ERR_GPU_UNAVAILABLE 2     /* 'GPU_UNAVAILABLE' (session.ts:262-270)        */
#define SSM_ERR_CHECKPOINT_INVALID 3  /* 'CHECKPOINT_INVALID' (session.ts:393-401)     */
#define SSM_ERR_DESTROYED 4           /* 'SESSION_DESTROYED' (session.ts:608-615)      */
#define SSM_ERR_HIP 5                 /* 'UNKNOWN' (HIP runtime / launch failure)       */
#define SSM_ERR_OUT_OF_MEMORY 6       /* 'UNKNOWN'                                      */
#define SSM_ERR_UNSUPPORTED 7         /* 'UNKNOWN' (layer type or shape this backend
                                         does not implement, e.g. 'attention')          */

const char* ssm_last_error(void);
const char* ssm_status_name(ssm_status s);
int ssm_abi_version(void);
/* Failure injection for tests of the error contract (no counterpart in the reference; its
 * GPU_UNAVAILABLE / CHECKPOINT_INVALID paths are session.ts:262-270,393-401): kind
 * "nodevice" (ssm_ctx_create finds no device), "alloc" (every device allocation of the
 * library fails with SSM_ERR_OUT_OF_MEMORY), "launch" (every launch check reports
 * SSM_ERR_HIP after the kernel ran normally), "" (none). It holds for the whole process until
 * the next call; NULL hands control back to the environment variable SSM_HIP_FAULT, which
 * each ssm_ctx_create then reads. Unknown kinds: SSM_ERR_INVALID_ARG. */
ssm_status ssm_set_fault_injection(const char* kind);

/* ------------------------------------------------------------------ device context */
typedef struct ssm_ctx ssm_ctx;

/* Open HIP device `device_ordinal` (replaces initWebGPU + requestDevice, session.ts:263,274).
 * Creates a default-priority stream and a BLAS handle bound to it. */
ssm_status ssm_ctx_create(int device_ordinal, ssm_ctx** out);
/* Release the context (replaces device.destroy(), session.ts:592). */
ssm_status ssm_ctx_destroy(ssm_ctx* ctx);
/* Run all context work on `stream` (a hipStream_t) instead of the context's own stream.
 * NULL restores the context's stream. The caller keeps ownership of `stream`. */
ssm_status ssm_ctx_set_stream(ssm_ctx* ctx, void* stream);
void* ssm_ctx_stream(ssm_ctx* ctx);
ssm_status ssm_ctx_synchronize(ssm_ctx* ctx);
/* Opt-in stage profiler (no counterpart in the reference, whose only timing is Date.now()
 * deltas, e.g. src/session/session.ts:486,498): when enabled, model-level calls record HIP
 * events around each stage (projection GEMMs, conv, scan/SSD, norms). The report
 * synchronises, then writes one "stage launches total_ms" line per stage into buf and
 * clears the record. */
ssm_status ssm_ctx_profile(ssm_ctx* ctx, int enable);
ssm_status ssm_ctx_profile_report(ssm_ctx* ctx, char* buf, size_t cap);
/* Device name (e.g. "gfx950") and compute-unit count. */
ssm_status ssm_ctx_info(ssm_ctx* ctx, char* arch, int arch_len, int* compute_units,
                        size_t* total_mem);

/* Device memory helpers for hosts without a GPU runtime of their own (the Node-API addon). */
ssm_status ssm_malloc(ssm_ctx* ctx, size_t bytes, void** dptr);
ssm_status ssm_free(ssm_ctx* ctx, void* dptr);
ssm_status ssm_memcpy_h2d(ssm_ctx* ctx, void* dst, const void* src, size_t bytes);
ssm_status ssm_memcpy_d2h(ssm_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ------------------------------------------------------------------ kernel level */
/* Element types for the SSD inputs x, B, C (y is always float32). */
#define SSM_F32 0
#define SSM_BF16 1

/* K1. Causal depthwise conv1d (+ bias, + SiLU) over (B,L,C):
 *   y[b,t,c] = act(bias[c] + sum_k w[c,k] x[b,t-K+1+k,c]),
 * x at t<0 taken from state_in[b,c,K-1+t] (zero when NULL); state_out[b,c,:] (may be NULL,
 * may alias state_in) receives the last K-1 inputs. w (C,K); bias may be NULL; 1<=K<=8.
 * The WGSL conv kernel of MambaCode.js's Mamba-1/2 layers (prefill path). */
ssm_status ssm_causal_conv1d(const float* x, long ldx, const float* w, const float* bias,
                             float* y, long ldy, int B, int L, int C, int K, int silu,
                             const float* state_in, float* state_out, void* stream);

/* K1 decode: one token. window = [state[b,c,0..K-2], x[b,c]], y = act(bias + w . window),
 * state shifted in place. x (B,ldx), y (B,ldy), state (B,C,K-1). */
ssm_status ssm_conv1d_update(const float* x, long ldx, const float* w, const float* bias,
                             float* y, long ldy, float* state, int B, int C, int K, int silu,
                             void* stream);

/* K2. Mamba-1 selective scan (Gu & Dao 2023, Alg. 2):
 *   dt' = softplus(dt + dt_bias) if softplus else dt + dt_bias
 *   h_t = exp(dt' A) h_{t-1} + dt' B_t u_t;  y_t = C_t . h_t + Dsk u_t;  y_t *= silu(z_t)
 * u, dt, z, y: (B,L,D) with row strides; Bm, Cm: (B,L,N) with row strides; A: (D,N);
 * dt_bias, Dsk, z, h0, hT may be NULL; h0/hT: (B,D,N). N <= 64.
 * `workspace` must hold ssm_selective_scan_workspace(B,L,D,N) bytes (device memory). */
size_t ssm_selective_scan_workspace(int B, int L, int D, int N);
ssm_status ssm_selective_scan(const float* u, long ldu, const float* dt, long lddt,
                              const float* dt_bias, int softplus, const float* A,
                              const float* Bm, long ldb, const float* Cm, long ldc,
                              const float* Dsk, const float* z, long ldz, float* y, long ldy,
                              int B, int L, int D, int N, const float* h0, float* hT,
                              void* workspace, size_t workspace_bytes, void* stream);

/* K2 decode: one-token Mamba-1 state update, h (B,D,N) in place.
 * x, dt, z, y: (B,*) with row strides; Bm, Cm: (B,*) with row strides ldb/ldc. */
ssm_status ssm_m1_state_update(const float* x, long ldx, const float* dt, long lddt,
                               const float* dt_bias, int softplus, const float* A,
                               const float* Bm, long ldb, const float* Cm, long ldc,
                               const float* Dsk, const float* z, long ldz, float* y, long ldy,
                               float* h, int B, int D, int N, void* stream);

/* K3-K6. Mamba-2 SSD (Dao & Gu 2024, section 6), fused chunked form:
 *   dt' = clamp(softplus(dt + dt_bias), dt_min, dt_max);  per head h with scalar A_h:
 *   S_t = exp(dt'_t A_h) S_{t-1} + dt'_t x_t B_t^T  (P x N);  y_t = S_t C_t + Dsk_h x_t.
 * x: (B,L,H,P) elements of `in_dtype` with row stride ldx; dt: (B,L,H) float, row stride
 * lddt; Bm, Cm: (B,L,G,N) of `in_dtype`, row strides ldb/ldc; y: (B,L,H,P) float, ldy;
 * h0/hT: (B,H,P,N) float (may be NULL). P = 64 with N in {64, 128} runs the fused MFMA
 * kernel. Other shapes: with G = 1, N <= 64, float inputs, a dt clamp that cannot bind and
 * the workspace, the Mamba-1 chunked scan over H*P channels; otherwise a sequential kernel
 * (no workspace needed). The chunk length of the reference config (chunkLen) does not change
 * the result; the kernel uses its own internal chunk. `workspace` holds
 * ssm_ssd_workspace(...) bytes: segment states for long sequences and, for float inputs, the
 * C B^T tiles of every chunk (a workspace with room for the segment states only gives the
 * same result more slowly). */
size_t ssm_ssd_workspace(int B, int L, int H, int P, int G, int N);
ssm_status ssm_ssd_chunk_scan(int in_dtype, const void* x, long ldx, const float* dt, long lddt,
                              const float* dt_bias, int softplus, float dt_min, float dt_max,
                              const float* A, const void* Bm, long ldb, const void* Cm,
                              long ldc, const float* Dsk, float* y, long ldy, int B, int L,
                              int H, int P, int G, int N, const float* h0, float* hT,
                              void* workspace, size_t workspace_bytes, void* stream);

/* K7. One-token Mamba-2 state update, h (B,H,P,N) in place:
 *   h = exp(dt' A_h) h + dt' x B^T;  y = h C + Dsk_h x  (optionally y *= silu(z)).
 * x, y, z: (B,H*P) with row strides; dt: (B,H) stride lddt; Bm, Cm: (B,G*N) strides. */
ssm_status ssm_m2_state_update(const float* x, long ldx, const float* dt, long lddt,
                               const float* dt_bias, int softplus, float dt_min, float dt_max,
                               const float* A, const float* Bm, long ldb, const float* Cm,
                               long ldc, const float* Dsk, const float* z, long ldz, float* y,
                               long ldy, float* h, int B, int H, int P, int G, int N,
                               void* stream);

/* RMSNorm rows of length n (eps added to the mean square). */
ssm_status ssm_rmsnorm(const float* x, long ldx, const float* w, float* y, long ldy, int M,
                       int n, float eps, void* stream);
/* Mamba-2 gated RMSNorm, norm after gate: y = norm_groups(x * silu(z)) * w, G groups. */
ssm_status ssm_gated_rmsnorm(const float* x, long ldx, const float* z, long ldz,
                             const float* w, float* y, long ldy, int M, int n, int G, float eps,
                             void* stream);

/* Projection of a few rows (one per decoded sequence, 1 <= M <= 64) with the block's norm
 * fused in front of it (the per-token Linear layers of the MambaCode.js model behind
 * model.forward / model.generate, streaming.ts:31-35, session.ts:421-425):
 *   y[m,n] = beta*y[m,n] + s[m] * sum_k p[m,k] W[n,k],   W (N,K) row-major
 *   mode 0: p = x,                  s = 1
 *   mode 1: p = x*g[k],             s = rsqrt(mean_k x^2 + eps)               (RMSNorm)
 *   mode 2: p = x*silu(z)*g[k],     s = rsqrt(mean_k (x*silu(z))^2 + eps)      (gated RMSNorm)
 * K % 4 == 0; x, z, g, W 16-byte aligned with row strides multiple of 4. fp32 MFMA; W is
 * read once. With `workspace` of ssm_linear_rows_workspace(M, N, K) bytes (0 when the shape
 * never splits) a narrow, long-K product is split over K across workgroups and finished by a
 * second launch that adds the slices in a fixed order; NULL runs it unsplit. Results do not
 * depend on scheduling either way. One workspace serves one stream at a time. */
size_t ssm_linear_rows_workspace(int M, int N, int K);
ssm_status ssm_linear_rows(int mode, const float* x, long ldx, const float* z, long ldz,
                           const float* g, const float* W, float* y, long ldy, int M, int N, int K,
                           float beta, float eps, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Projection of any number of rows (the Linear layers of the MambaCode.js model behind
 * model.forward at prefill, streaming.ts:31-35: the Mamba blocks' in_proj, x_proj, dt_proj
 * and out_proj):
 *   y[m,n] = beta*y[m,n] + sum_k x[m,k] W[n,k] (+ bias[n] when bias is not NULL)
 * W (N,K) row-major with row stride ldw. fp32 arithmetic on the fp32 matrix cores; the sum
 * over k is in a fixed order (results do not depend on scheduling). K % 4 == 0; x and W
 * 16-byte aligned with ldx, ldw multiples of 4; 128 rows of any operand span < 2 GiB. */
ssm_status ssm_linear(const float* x, long ldx, const float* W, long ldw, const float* bias,
                      float* y, long ldy, int M, int N, int K, float beta, void* stream);

/* The Mamba-1 block's x_proj and dt_proj in one pass over x (the conv output), for the
 * Linear layers between the conv and the scan in MambaCode.js's Mamba-1 block behind
 * model.forward (streaming.ts:31-35):
 *   dbl[t, :] = x[t, :] Wx^T            (T, R + 2N): dt_low | B | C, row stride lddbl
 *   dt[t, :]  = dbl[t, 0:R] Wdt^T        (T, D), row stride lddt (before bias and softplus)
 * Wx (R + 2N, D) and Wdt (D, R) row-major. fp32 matrix cores, sums in a fixed order.
 * Needs D % 4 == 0, R % 4 == 0, R <= 64, R + 2N <= 128; x, Wx, Wdt 16-byte aligned with
 * ldx % 4 == 0 (SSM_ERR_INVALID_ARG otherwise). */
ssm_status ssm_m1_xproj_dt(const float* x, long ldx, const float* Wx, const float* Wdt,
                           float* dbl, long lddbl, float* dt, long lddt, int T, int D, int R,
                           int N, void* stream);

/* Greedy pick per row (sampleToken with topK = 1, src/session/streaming.ts:74-75): index
 * of the largest value, lowest index among equal maxima; NaN never wins (0 for an all-NaN
 * row). x (rows, n) with row stride ldx; out (rows) uint32. */
ssm_status ssm_argmax(const float* x, long ldx, int rows, int n, uint32_t* out, void* stream);

/* sampleToken(logits, {temperature, topK, topP}) per row (src/session/streaming.ts:53-97),
 * with the uniform draw Math.random() (streaming.ts:91) passed in: u (rows) doubles in
 * [0, 1), device. logits (rows, n) fp32 with row stride ld; out (rows) uint32, device.
 * Temperature is clamped to >= 1e-7 (streaming.ts:11,61); the division and exp are in
 * double with float stores; the topK largest exps are taken in a stable descending order
 * (equal exps: lower index first); the nucleus ends at the first cumulative exp/sumE >=
 * topP; the pick is the first nucleus entry whose running exp sum reaches u * (nucleus
 * sum). Needs 1 <= n <= 262144 and min(topK, n) <= 1024 (SSM_ERR_UNSUPPORTED otherwise) and
 * topK >= 1. Logits may be -inf (e = 0, as in the reference) but not NaN or +inf, and a
 * row needs one finite logit. workspace: device memory of ssm_sample_workspace(rows,
 * n) bytes (scaled values, keys, slice maxima and sums), one stream at a time. */
size_t ssm_sample_workspace(int rows, int n);
ssm_status ssm_sample(const float* logits, long ld, int rows, int n, double temperature,
                      int top_k, double top_p, const double* u, uint32_t* out, void* workspace,
                      size_t workspace_bytes, void* stream);
/* ssm_sample without a workspace argument and without any device allocation. No counterpart
 * in the reference: it is for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The workspace is a static 32 MiB
 * device array per GPU (the library holds it until the process ends), so rows and n must
 * satisfy ssm_sample_workspace(rows, n) <= 32 MiB (e.g. 64 rows of 128000 logits);
 * larger calls return SSM_ERR_UNSUPPORTED. Its device address is resolved by ssm_ctx_create
 * (else on the first call on a device, for the device current on the calling thread). Calls
 * that overlap on one GPU share the array and race: serialise them. Results are identical to
 * ssm_sample's. */
ssm_status ssm_sample_noalloc(const float* logits, long ld, int rows, int n, double temperature,
                              int top_k, double top_p, const double* u, uint32_t* out,
                              void* stream);

/* ------------------------------------------------------------------ model level */
#define SSM_LAYER_MAMBA1 1
#define SSM_LAYER_MAMBA2 2
#define SSM_LAYER_MAMBA3 3     /* accepted by the schema, rejected with SSM_ERR_UNSUPPORTED */
#define SSM_LAYER_ATTENTION 4  /* accepted by the schema, rejected with SSM_ERR_UNSUPPORTED */

/* HybridMambaModelConfig (src/session/presets.ts:107-120). dt_rank 0 = ceil(d_model/16);
 * norm_eps 0 = 1e-5. layer_types has n_layers entries (SSM_LAYER_*). */
typedef struct ssm_config {
    int vocab_size, d_model, n_layers, d_state, d_conv, expand, n_heads, n_groups;
    int chunk_len, mimo_group, eos_id, dt_rank;
    float norm_eps;
    const int* layer_types;
} ssm_config;

typedef struct ssm_model ssm_model;
typedef struct ssm_state ssm_state;

/* new HybridMambaModel(device, config) (session.ts:359): allocate the weights on the device
 * and fill them with the documented random init from `seed`. */
ssm_status ssm_model_create(ssm_ctx* ctx, const ssm_config* cfg, uint64_t seed,
                            ssm_model** out);
ssm_status ssm_model_destroy(ssm_model* m);
/* Read back the resolved config (dt_rank, eps filled in); layer_types is not written. */
ssm_status ssm_model_config(ssm_model* m, ssm_config* out);
/* model.loadWeights(buf) (session.ts:394,575): validates magic, version, dims and size
 * (src/session/errors.ts:9) -> SSM_ERR_CHECKPOINT_INVALID on mismatch. */
ssm_status ssm_model_load_weights(ssm_model* m, const void* buf, size_t bytes);
/* model.exportWeights() (session.ts:518). buf NULL: only *bytes is written. dtype SSM_F32
 * or 2 (= float16 payload). */
ssm_status ssm_model_export_weights(ssm_model* m, int f16, void* buf, size_t cap,
                                    size_t* bytes);

/* model.forward(ids, batch, seqLen) (streaming.ts:31-35): host ids (B,L) -> host logits
 * (B,L,V), zero initial state. */
ssm_status ssm_forward(ssm_model* m, const uint32_t* ids, int B, int L, float* logits);
/* Same with device buffers, enqueued on the context stream (no host synchronisation). */
ssm_status ssm_forward_device(ssm_model* m, const uint32_t* d_ids, int B, int L,
                              float* d_logits);
/* One mixer (layer `layer`, no norm / residual) over device hidden states (B,L,d_model). */
ssm_status ssm_mixer_forward_device(ssm_model* m, int layer, const float* d_x, float* d_y,
                                    int B, int L);
/* The same Mamba-2 mixer with bf16 operands and fp32 accumulation: x, in_proj and out_proj
 * weights, the SSD's x / B / C and out_proj's input rounded to bf16 (round to nearest even);
 * dt, the conv, the state pass and every sum stay fp32. No counterpart in the reference: the
 * bf16-input variant of the layer prefill that the benchmark configuration asks for, for
 * tests and benches. */
ssm_status ssm_mixer_forward_device_bf16(ssm_model* m, int layer, const float* d_x, float* d_y,
                                         int B, int L);

/* Recurrent decode state (ssm + conv state of every layer) for B sequences. */
ssm_status ssm_state_create(ssm_model* m, int B, ssm_state** out);
ssm_status ssm_state_destroy(ssm_state* s);
ssm_status ssm_state_reset(ssm_state* s);
/* Host image: for each layer, its ssm state then its conv state, float32. */
size_t ssm_state_floats(ssm_state* s);
ssm_status ssm_state_read(ssm_state* s, float* out);
ssm_status ssm_state_write(ssm_state* s, const float* in);
/* Device pointers of layer `layer`'s ssm and conv state (for tests and benches). */
ssm_status ssm_state_layer(ssm_state* s, int layer, float** ssm, float** conv);

/* Prefill ids (B,L) (host) continuing from the state; writes the last position's logits
 * (B,V) and/or greedy ids (B) to host buffers (either may be NULL). */
ssm_status ssm_prefill(ssm_model* m, ssm_state* s, const uint32_t* ids, int L,
                       float* last_logits, uint32_t* argmax);
/* One recurrent token step for all B sequences (host ids (B)). */
ssm_status ssm_decode_step(ssm_model* m, ssm_state* s, const uint32_t* ids, float* logits,
                           uint32_t* argmax);
/* Device variant: ids and outputs are device pointers; no host synchronisation. */
ssm_status ssm_decode_step_device(ssm_model* m, ssm_state* s, const uint32_t* d_ids,
                                  float* d_logits, uint32_t* d_argmax);
/* Greedy generation (topK = 1 in sampleToken, streaming.ts:74-75: argmax, lowest index on
 * ties): prefill prompt (B,Lp), then n_new recurrent steps with on-device argmax. out_ids
 * (B,n_new) host. All n_new steps run; the caller cuts each row after its eos id
 * (streaming.ts:47). */
ssm_status ssm_generate_greedy(ssm_model* m, ssm_state* s, const uint32_t* prompt, int Lp,
                               int n_new, uint32_t* out_ids);
/* Sampled generation (the generate loop of streaming.ts:17-49 with sampleToken on the
 * device, as ssm_sample): prefill prompt (B,Lp) (host), then n_new - 1 recurrent steps;
 * token k of row b is drawn with u_host[k*B + b] (host, n_new*B doubles in [0, 1), the
 * Math.random() values of streaming.ts:91 in the order the reference draws them). out_ids
 * (B,n_new) host. All n_new steps run; the caller cuts each row after its eos id. Same
 * limits as ssm_sample on the vocabulary size and topK. */
ssm_status ssm_generate_sample(ssm_model* m, ssm_state* s, const uint32_t* prompt, int Lp,
                               int n_new, double temperature, int top_k, double top_p,
                               const double* u_host, uint32_t* out_ids);

#ifdef __cplusplus
}
#endif
#endif /* SSM_HIP_H */
