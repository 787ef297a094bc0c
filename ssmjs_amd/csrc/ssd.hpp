// Internal interface between the SSD entry point (ssd.hip) and the fp32 matrix-core kernel
// (ssd_f32.hip).
#pragma once

#include "common.hpp"

namespace ssm {

// Head dim 64 with d_state 64 or 128: the shapes the fp32 kernel takes.
bool ssd_f32_shape(int Pd, int N);
// Workspace bytes of ssd_f32 (segment states when long sequences are cut into segments).
size_t ssd_f32_workspace(int B, int L, int H, int G, int Pd, int N);
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

// Segment entering states of the segmented SSD, one thread per element e of a (b, h) state of
// PN elements: slot[s] <- carry, carry = 2^(decay2[s]) carry + local[s], carry starting at h0
// (or 0). decay2[s] is the segment's sum of dt' A in log2 units (the caller passes its own
// decays times dscale to get there). The last slot's local state is never read by the result:
// the state-only pass does not produce it. The slots' loads are issued in groups of 16 before
// their stores, so that each group waits for memory once (a loop that stored slot s before
// loading slot s + 1 waited for every load in turn).
__device__ __forceinline__ void seg_prefix_elem(float* seg_state, const float* seg_decay,
                                                const float* h0, int nseg, int PN, long bh,
                                                int e, float dscale) {
    constexpr int GS = 16;
    float carry = h0 ? h0[bh * PN + e] : 0.f;
    float* st = seg_state + bh * nseg * (long)PN + e;
    const float* dc = seg_decay + bh * nseg;
    for (int s0 = 0; s0 < nseg; s0 += GS) {
        float loc[GS], dec[GS];
#pragma unroll
        for (int j = 0; j < GS; ++j) {
            const int s = min(s0 + j, nseg - 1);   // past nseg: an in-range slot, not used
            loc[j] = st[(long)s * PN];
            dec[j] = dc[s];
        }
#pragma unroll
        for (int j = 0; j < GS; ++j) {
            if (s0 + j >= nseg) break;
            st[(long)(s0 + j) * PN] = carry;
            carry = fmaf(ex2(dec[j] * dscale), carry, loc[j]);
        }
    }
}

}  // namespace ssm
