// Launch helpers shared between the glue kernels (glue.hip) and the model code (model.hip).
#pragma once
#include "common.hpp"

enum {
    SSM_INIT_CONST = 0,
    SSM_INIT_UNIFORM = 1,      // U(a0, a1)
    SSM_INIT_NORMAL = 2,       // N(0, a0^2)
    SSM_INIT_ARANGE_LOG = 3,   // log(1 + (i mod row)): S4D-real A_log for Mamba-1
    SSM_INIT_LOG_UNIFORM = 4,  // log U(a0, a1): Mamba-2 A_log
    SSM_INIT_DT_BIAS = 5,      // softplus^-1(dt), dt log-uniform in [a0, a1]
};

namespace ssm {
ssm_status launch_embed(const uint32_t* ids, const float* emb, float* out, long T, int d, int V,
                        int* bad, hipStream_t st);
ssm_status launch_gather_rows(const float* x, long row_stride, long first, float* out, int rows,
                              int d, hipStream_t st);
ssm_status launch_argmax(const float* x, long ldx, int rows, int n, uint32_t* out,
                         hipStream_t st);
// sampleToken on the device (sample.hip): sample_ok says whether (n, topK) is supported.
bool sample_ok(int n, int top_k);
size_t sample_workspace(int rows, int n);
// Device address of ssm_sample_noalloc's static scratch on the current device.
ssm_status sample_scratch(void** out);
ssm_status launch_sample(const float* logits, long ld, int rows, int n, double temperature,
                         int top_k, double top_p, const double* u, uint32_t* out,
                         void* workspace, hipStream_t st);
ssm_status launch_init(float* p, long n, int kind, float a0, float a1, uint64_t seed,
                       uint64_t tensor_id, int row, hipStream_t st);
ssm_status launch_neg_exp(const float* x, float* y, long n, hipStream_t st);
// Few-row projection with fused RMSNorm (mode 1) / gated RMSNorm (mode 2) prologue
// (rowgemm.hip); rowgemm_ok says whether the shape is supported. With rowgemm_workspace
// bytes it may split K over workgroups (plus a finishing launch); with less it runs unsplit.
// With g2 and nout, a split finish also writes nout = RMSNorm(Y) * g2 (row stride ldn) and
// sets *normed; otherwise *normed is false and the caller normalises Y itself.
bool rowgemm_ok(int M, int N, int K);
size_t rowgemm_workspace(int M, int N, int K);
ssm_status launch_rowgemm(int mode, const float* X, long ldx, const float* Z, long ldz,
                          const float* g, const float* W, float* Y, long ldy, int M, int N, int K,
                          float beta, float eps, void* workspace, size_t workspace_bytes,
                          hipStream_t st, const float* g2 = nullptr, float* nout = nullptr,
                          long ldn = 0, bool* normed = nullptr);

// One-token step projections (stepproj.hip): v = s[m] * X W^T on 16 x 16 tiles with an
// epilogue; s[m] = 1 / sqrt(sum_j ssq[m * nssq + j] * inv_div + eps) when ssq is given.
// X (M rows, padded to whole 16-row tiles) and W (N rows, likewise) are in fragment order.
constexpr int kStepProjMaxRows = 64;
constexpr int kStepProjMaxSsq = 256;

// Fragment order of a (rows, K) matrix, K % 16 == 0, KB = K / 16: the 16-row tile t and
// k-block kb form 256 contiguous floats at (t * KB + kb) * 256, lane-major: lane 16 q + i
// holds row 16 t + i, k = 16 kb + 4 q .. 4 q + 3 (one MFMA operand fragment per b128 load).
__host__ __device__ inline long frag_off(int m, int k, int KB) {
    return ((long)(m >> 4) * KB + (k >> 4)) * 256 + (((k >> 2) & 3) * 16 + (m & 15)) * 4 + (k & 3);
}
size_t frag_floats(int rows, int K);

enum { EPI_STORE = 0, EPI_CONV = 1, EPI_RESID = 2 };
struct StepProj {
    const float* X = nullptr;              // (M, K) fragment order
    const float* W = nullptr;              // (N, K) fragment order (launch_pack_frag)
    int M = 0, N = 0, K = 0;
    const float* ssq = nullptr; int nssq = 0; float inv_div = 0.f, eps = 0.f;
    float* Y = nullptr; long ldy = 0; float beta = 0.f;
    // EPI_CONV: columns [c0, c0 + C) -> conv update (weights (C, Kc), bias, state (M, C, Kc-1))
    int c0 = 0, C = 0, Kc = 0;
    const float* cw = nullptr; const float* cb = nullptr; float* cst = nullptr;
    float* Yc = nullptr; long ldyc = 0;
    // EPI_RESID with g2: xg = Y * g2 in fragment order (K = N), ssq_out (M, N / 16)
    const float* g2 = nullptr; float* xg = nullptr; float* ssq_out = nullptr;
    // EPI_CONV: the conv outputs also in fragment order (K = C, C % 16 == 0; rows M .. 16 mt - 1
    // written as zeros), the operand of the step's next projection
    float* Yf = nullptr;
    // EPI_CONV with xpart: the next projection (the Mamba-1 step's x_proj, RN outputs) summed
    // over each conv tile's 16 channels, xpart[(ct, m, j)] = sum_{c in tile ct} u[m, c]
    // wxt[c, j] with wxt (C, RN) row-major (RN <= kXpartMaxRN, c0 and C multiples of 16); the
    // partials, (C / 16, 16 mt, RN), are added by the step's state update
    const float* wxt = nullptr; int RN = 0; float* xpart = nullptr;
    int mt = 0, nt = 0, rotate = 0;        // tiles and k-start rotation (set by the launcher)
};
constexpr int kXpartMaxRN = 128;
bool stepproj_ok(int M, int N, int K);
ssm_status launch_stepproj(int epi, StepProj a, hipStream_t st);
// W (N, K) row stride ldw -> fragment order in out (frag_floats(N, K) floats).
ssm_status launch_pack_frag(const float* W, long ldw, int N, int K, float* out, hipStream_t st);
// Mamba-1 one-token state update (scan_m1.hip): ykb = 0 writes y (B, D) with row stride ldy,
// ykb > 0 in fragment order with K = 16 ykb. dtr given: the raw dt (before bias and softplus)
// is formed in the kernel as dtr (B, R) [ld lddtr] times Wdt^T (Wdt (D, R) row-major, 16-byte
// aligned, R % 4 == 0; D % 64 == 0) instead of read from dt.
ssm_status launch_m1_update(const float* x, long ldx, const float* dt, long lddt,
                            const float* dt_bias, int softplus, const float* A, const float* Bm,
                            long ldb, const float* Cm, long ldc, const float* Dsk, const float* z,
                            long ldz, float* y, long ldy, int ykb, float* h, int B, int D, int N,
                            hipStream_t st, const float* dtr, long lddtr, const float* Wdt,
                            int R);
// The fused step's update: dt_proj formed in the kernel, softplus on, y in fragment order
// (K = D, D % 64 == 0), the input of the step's out_proj.
ssm_status launch_m1_update_frag(const float* x, long ldx, const float* dtr, long lddtr,
                                 const float* Wdt, int R, const float* dt_bias, const float* A,
                                 const float* Bm, long ldb, const float* Cm, long ldc,
                                 const float* Dsk, const float* z, long ldz, float* yf, float* h,
                                 int B, int D, int N, hipStream_t st);
// The fused Mamba-1 step's x_proj reduction, dt_proj and state update in one launch: x_proj
// arrives as the conv epilogue's per-tile partials xpart (D / 16, M16, RN) (M16 = B rounded up
// to 16; RN = R + 2N = (dt_r, B, C)), added per sequence in a fixed order; dt = softplus(dt_r
// Wdt^T + dt_bias) with Wdt (D, R) in quads (launch_pack_q4); y = (C.h + D x) silu(z) in
// fragment order (K = D, rows B .. M16-1 zero), the out_proj's operand.
bool m1_step_update_ok(int D, int N, int R);
ssm_status launch_m1_step_update(const float* x, long ldx, const float* xpart, int RN, int M16,
                                 const float* Wdt, int R, const float* dt_bias, const float* A,
                                 const float* Dsk, const float* z, long ldz, float* yf, float* h,
                                 int B, int D, int N, hipStream_t st);
// W (N, K) row stride ldw -> its transpose (K, N) row-major in out.
ssm_status launch_pack_t(const float* W, long ldw, int N, int K, float* out, hipStream_t st);
// W (N, K) row-major (K % 4 == 0) -> quads: out[((k / 4) N + n) 4 + k % 4] = W[n, k].
ssm_status launch_pack_q4(const float* W, int N, int K, float* out, hipStream_t st);
// The one-token LM head (head.hip): y (M, V) [ldy] = s[m] xg E^T with xg (M, K) in fragment
// order, s[m] = 1 / sqrt(inv_div sum_j ssq[m, j] + eps), Ef the fragment-order copy of E
// (V, K); with argmax, also the greedy pick per row (largest logit, lowest index among equal
// maxima). part: head_parts(V) pairs per row of workspace.
bool head_ok(int M, int V, int K);
int head_parts(int V);
ssm_status launch_head(const float* xg, const float* ssq, int nssq, float inv_div, float eps,
                       const float* Ef, float* y, long ldy, int M, int V, int K, float* part,
                       uint32_t* argmax, hipStream_t st);
// xg = x * g in fragment order (K = d) and ssq (M, d / 16) partial sums of x^2: the first
// RMSNorm of a step.
ssm_status launch_xg_ssq(const float* x, long ldx, const float* g, float* xg, float* ssq, int M,
                         int d, hipStream_t st);
// The one-token step's embedding gather with the first norm's operand in the same pass:
// hid = E[ids] (M, d), then as launch_xg_ssq on hid with g; ids >= V flag *bad.
ssm_status launch_embed_xg(const uint32_t* ids, const float* emb, float* hid, const float* g,
                           float* xg, float* ssq, int M, int d, int V, int* bad, hipStream_t st);
// Prefill projection (gemm.hip): Y = beta * Y + s[m] X W^T (+ bias) on the fp32 matrix
// cores; with ssq, s[m] = 1 / sqrt(inv_div * sum_j ssq[m nssq + j] + eps) (a row RMSNorm of
// X applied after the product), else 1.
bool gemm_ok(int M, int N, int K, long ldx, long ldw, long ldy);
// gate_c0 (a multiple of 16): columns n >= gate_c0 are stored as silu(value) (the Mamba-1
// block's z half of in_proj, the scan's gate).
// part (part_floats floats, 16-byte aligned): workspace of the split-K mode, used when the
// tiles alone leave most CUs idle and part holds gemm_split_floats(M, N, K) floats; null
// runs unsplit.
ssm_status launch_gemm(const float* X, long ldx, const float* W, long ldw, const float* bias,
                       float* Y, long ldy, int M, int N, int K, float beta, hipStream_t st,
                       const float* ssq = nullptr, int nssq = 0, float inv_div = 0.f,
                       float eps = 0.f, int gate_c0 = 0x7fffffff, float* part = nullptr,
                       size_t part_floats = 0);
size_t gemm_split_floats(int M, int N, int K);
// The Mamba-1 block's x_proj and dt_proj in one pass (gemm.hip): dbl = x Wx^T (T, R + 2N),
// dt = dbl[:, :R] Wdt^T (T, D); given dt_bias, dt = softplus(dbl[:, :R] Wdt^T + dt_bias) (the
// scan's dt').
bool xproj_dt_ok(int T, int D, int R, int N, long ldx, long lddbl, long lddt);
ssm_status launch_xproj_dt(const float* x, long ldx, const float* Wx, const float* Wdt,
                           float* dbl, long lddbl, float* dt, long lddt, int T, int D, int R,
                           int N, hipStream_t st, const float* dt_bias = nullptr);
// The bf16-input layer's element-wise stages: fp32 -> bf16 (round to nearest even) row
// copies (glue.hip), the forward conv with bf16 outputs and a zero initial state
// (conv1d.hip), the gated RMSNorm with bf16 outputs (glue.hip).
ssm_status launch_cast_bf16(const float* x, long ldx, __bf16* y, long ldy, long rows, int cols,
                            hipStream_t st);
ssm_status launch_conv1d_bf16(const float* x, long ldx, const float* w, const float* bias,
                              __bf16* y, long ldy, int B, int L, int C, int K, int silu,
                              hipStream_t st);
ssm_status launch_gated_rmsnorm_bf16(const float* x, long ldx, const float* z, long ldz,
                                     const float* w, __bf16* y, long ldy, int M, int n, int G,
                                     float eps, hipStream_t st);
// ssm_selective_scan (scan_m1.hip); zgated = 1: z already holds silu(z).
ssm_status selective_scan(const float* u, long ldu, const float* dt, long lddt,
                          const float* dt_bias, int softplus, const float* A, const float* Bm,
                          long ldb, const float* Cm, long ldc, const float* Dsk, const float* z,
                          long ldz, int zgated, float* y, long ldy, int B, int L, int D, int N,
                          const float* h0, float* hT, void* workspace, size_t workspace_bytes,
                          void* stream);
// The Mamba-2 one-token state update with the gated RMSNorm's element-wise part:
// y = (C.h + D x) * silu(z) * gn in fragment order (K = H P), and per workgroup the partial sum
// of ((C.h + D x) silu(z))^2 into ssq (B, m2_gated_nssq(H, P, N)). ssd.hip.
int m2_gated_nssq(int H, int P, int N);
ssm_status launch_m2_update_gated(const float* x, long ldx, const float* dt, long lddt,
                                  const float* dt_bias, const float* A, const float* Bm, long ldb,
                                  const float* Cm, long ldc, const float* Dsk, const float* z,
                                  long ldz, const float* gn, float* y, float* ssq, float* h, int B,
                                  int H, int Pd, int G, int N, hipStream_t st);
}  // namespace ssm
