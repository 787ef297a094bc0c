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
}  // namespace ssm
