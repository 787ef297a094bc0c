// Internal interface between the SSD entry point (ssd.hip) and the fp32 matrix-core kernel
// (ssd_f32.hip).
#pragma once

#include "common.hpp"

namespace ssm {

// Head dim 64 with d_state 64 or 128: the shapes the fp32 kernel takes.
bool ssd_f32_shape(int Pd, int N);
// Workspace bytes of ssd_f32 (segment states when long sequences are cut into segments).
size_t ssd_f32_workspace(int B, int L, int H, int Pd, int N);
// The SSD of ssm_ssd_chunk_scan for float32 inputs (arguments as there; shapes checked by the
// caller). With ssq, the output carries the gated RMSNorm's element-wise part instead of y:
// y <- u * gn with u = y * silu(z) (z (B*L, H*P), row stride ldz; gn (H*P)), and
// ssq[(b L + t) H + h] = sum over head h's P channels of u^2.
ssm_status ssd_f32(const float* x, long ldx, const float* dt, long lddt, const float* dt_bias,
                   int softplus, float dt_min, float dt_max, const float* A, const float* Bm,
                   long ldb, const float* Cm, long ldc, const float* Dsk, float* y, long ldy,
                   int B, int L, int H, int G, int N, const float* h0, float* hT,
                   void* workspace, size_t workspace_bytes, hipStream_t st,
                   const float* z = nullptr, long ldz = 0, const float* gn = nullptr,
                   float* ssq = nullptr);

// Whether ssd_f32 with the gated output applies (one norm group; offsets and alignments).
bool ssd_gated_ok(int Pd, int G, int N, long ldx, long lddt, long ldb, long ldc, long ldy,
                  long ldz, const void* x, const void* Bm, const void* Cm, const float* y,
                  const float* z, const float* gn);

}  // namespace ssm
