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
// caller).
ssm_status ssd_f32(const float* x, long ldx, const float* dt, long lddt, const float* dt_bias,
                   int softplus, float dt_min, float dt_max, const float* A, const float* Bm,
                   long ldb, const float* Cm, long ldc, const float* Dsk, float* y, long ldy,
                   int B, int L, int H, int G, int N, const float* h0, float* hT,
                   void* workspace, size_t workspace_bytes, hipStream_t st);

}  // namespace ssm
