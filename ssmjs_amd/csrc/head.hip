// The one-token LM head (decode, M <= 64 rows) on the gfx950 fp32 matrix cores, with the final
// RMSNorm's scale and the greedy pick folded in:
//
//   logits[m, n] = s[m] * sum_k xg[m, k] E[n, k]      E (V, K): the tied embedding
//   s[m]         = 1 / sqrt(sum_j ssq[m, j] * inv_div + eps)
//
// xg = x * g_final (the final RMSNorm's operand, fragment order) and the partial sums ssq come
// from the last layer's out_proj epilogue (stepproj.hip), so the normalised row never goes
// through memory, as with every other norm of the step. E is read from its fragment-order copy
// (pack_frag): one b128 load per lane brings a whole 16 x 16 fragment as 8 full lines.
//
// Decomposition. A workgroup owns 128 columns (8 column tiles; 250 workgroups for a 32000-word
// vocabulary, one round on 256 CUs) and all rows and all of K. Its 4 waves take 2 column tiles
// each against all row tiles: per 16-wide k-block a wave loads MT + 2 fragments (MT = row
// tiles) and issues 4 (MT x 2) MFMAs on independent accumulators, with kPD k-blocks of loads in
// flight (one wave per SIMD, so the ring can be deep). The X fragments are the same for the
// four waves (L1 hits after the first); E streams from HBM once.
//
// Greedy pick. Each workgroup also writes, per row, the largest logit among its columns with
// the lowest index among equal maxima (NaN never wins), as (value, index) pairs; the finishing
// kernel merges a row's pairs. The merge takes the larger value, or the lower index of equal
// values: a maximum under a total order, so any merge order gives the same pick, which is the
// full-row argmax of the stored logits (glue.hip's argmax_kernel).
#include "common.hpp"
#include "glue.hpp"

namespace ssm {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kHW = 4;                  // waves per workgroup
constexpr int kHT = 2;                  // column tiles per wave
constexpr int kHBN = 16 * kHT * kHW;    // columns per workgroup
constexpr int kPD = 8;                  // k-blocks of loads in flight per wave
constexpr unsigned kOOR = 0x80000000u;  // a buffer offset past every descriptor's range

struct HeadArgs {
    const float* xg; const float* ssq; int nssq; float inv_div, eps;
    const float* Ef;                    // fragment order, nt 16-row tiles
    float* y; long ldy;
    int M, V, K, nt;
    float* part; int nparts;            // (M, nparts) pairs: value, index (as float bits)
};

// greedy order: v wins over (best, bi) when larger, or equal with a lower index
__device__ __forceinline__ void pick(float v, int i, float& best, int& bi) {
    if (v > best || (v == best && i < bi)) { best = v; bi = i; }
}

// KBT: K / 16 when it is a compile-time constant (the loop is then unrolled, so that each
// k-block waits for its own loads only; rolled, the compiler waits for every load in flight at
// the top of each group of kPD blocks), 0 for any K.
template <int MT, int KBT>
__global__ __launch_bounds__(64 * kHW, 1) void head_kernel(HeadArgs a) {
    __shared__ float sm[64];
    __shared__ float pv[kHW][64];
    __shared__ int pi[kHW][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int cb = blockIdx.x;
    const int KB = KBT ? KBT : a.K >> 4;

    // Row scales: thread t takes row t / 4 and the quarter t % 4 of its partial sums (in order),
    // then the quarters are added pairwise (the same sums in every lane of the row). The first
    // 16 of the quarter are loaded here, ahead of the operands (clamped indices, masked when
    // added), and added after the main loop.
    const int srow = tid >> 2, sqp = tid & 3;
    const int per = (a.nssq + 3) >> 2;
    const int j0 = sqp * per, j1 = min(a.nssq, j0 + per);
    const float* sq = a.ssq + (long)min(srow, a.M - 1) * a.nssq;
    float sp[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) sp[u] = sq[min(j0 + u, a.nssq - 1)];

    // fragment loads of k-block kb: X row tiles 0 .. MT-1, E column tiles of this wave
    const auto rx = rsrc(a.xg, (unsigned)(MT * KB) * 1024u);
    const auto re = rsrc(a.Ef, (unsigned)((long)a.nt * KB * 1024));
    const int tn0 = cb * (kHBN / 16) + kHT * w;
    float4 xa[kPD][MT], eb[kPD][kHT];
    auto load = [&](int s, int kb) {
        const unsigned ko = kb < KB ? (unsigned)kb * 1024u + (unsigned)lane * 16u : kOOR;
#pragma unroll
        for (int i = 0; i < MT; ++i)
            xa[s][i] = bload16<float4>(rx, ko == kOOR ? kOOR : ko + (unsigned)(i * KB) * 1024u);
#pragma unroll
        for (int j = 0; j < kHT; ++j) {
            const int tn = tn0 + j;
            eb[s][j] = bload16<float4>(
                re, ko == kOOR || tn >= a.nt ? kOOR : ko + (unsigned)(tn * KB) * 1024u);
        }
    };
#pragma unroll
    for (int s = 0; s < kPD; ++s) load(s, s);
    __builtin_amdgcn_sched_barrier(0);   // the whole ring in flight before the first MFMA

    floatx4 acc[MT][kHT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < kHT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int ng = (KB + kPD - 1) / kPD;
#pragma unroll KBT ? KBT / kPD + 1 : 1
    for (int g = 0; g < ng; ++g) {
#pragma unroll
        for (int s = 0; s < kPD; ++s) {
            // MFMA t of a block takes component t of both fragments (k = 4q + t for lane group q)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < kHT; ++j) {
                    acc[i][j] = mfma4(xa[s][i].x, eb[s][j].x, acc[i][j]);
                    acc[i][j] = mfma4(xa[s][i].y, eb[s][j].y, acc[i][j]);
                    acc[i][j] = mfma4(xa[s][i].z, eb[s][j].z, acc[i][j]);
                    acc[i][j] = mfma4(xa[s][i].w, eb[s][j].w, acc[i][j]);
                }
            load(s, (g + 1) * kPD + s);
            // keep each refill right behind the MFMAs that free its registers
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    {
        float t = 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u) t += j0 + u < j1 ? sp[u] : 0.f;
        for (int j = j0 + 16; j < j1; ++j) t += sq[j];
        t += __shfl_xor(t, 1, 64);
        t += __shfl_xor(t, 2, 64);
        if (sqp == 0 && srow < 64)
            sm[srow] = srow < a.M ? 1.f / sqrtf(t * a.inv_div + a.eps) : 0.f;
    }
    __syncthreads();   // sm

    // epilogue: lane (l16, q) of tile (i, j) holds rows 16 i + 4 q + r of column 16 tn + l16
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * i + 4 * q + r;
            const float sc = sm[row];
            float best = -INFINITY;
            int bi = a.V;   // none yet
#pragma unroll
            for (int j = 0; j < kHT; ++j) {
                const int n = 16 * (tn0 + j) + l16;
                const float v = sc * acc[i][j][r];
                if (n < a.V) {
                    if (row < a.M) a.y[(long)row * a.ldy + n] = v;
                    // ascending n within the lane: the first of equal maxima stays
                    if (v > best || (bi == a.V && v == best)) { best = v; bi = n; }
                }
            }
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) {
                const float ov = __shfl_xor(best, o, 16);
                const int oi = __shfl_xor(bi, o, 16);
                pick(ov, oi, best, bi);
            }
            if (l16 == 0) { pv[w][row] = best; pi[w][row] = bi; }
        }
    __syncthreads();
    if (tid < 16 * MT && tid < a.M) {
        float best = pv[0][tid];
        int bi = pi[0][tid];
#pragma unroll
        for (int k = 1; k < kHW; ++k) pick(pv[k][tid], pi[k][tid], best, bi);
        float* dst = a.part + ((long)tid * a.nparts + cb) * 2;
        dst[0] = best;
        dst[1] = __int_as_float(bi);
    }
}

// One workgroup per row: the row's pairs merged by a wave-shuffle and LDS tree.
constexpr int kFin = 256;
__global__ __launch_bounds__(kFin) void head_argmax_kernel(const float* __restrict__ part,
                                                           int nparts, int V,
                                                           uint32_t* __restrict__ out) {
    __shared__ float sv[kFin / 64];
    __shared__ int si[kFin / 64];
    const int row = blockIdx.x;
    const float* p = part + (long)row * nparts * 2;
    float best = -INFINITY;
    int bi = V;
    for (int c = threadIdx.x; c < nparts; c += kFin)
        pick(p[2 * c], __float_as_int(p[2 * c + 1]), best, bi);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        pick(ov, oi, best, bi);
    }
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) { sv[w] = best; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kFin / 64; ++k) pick(sv[k], si[k], best, bi);
        out[row] = bi < V ? (uint32_t)bi : 0u;
    }
}

}  // namespace

bool head_ok(int M, int V, int K) {
    const long nt = (V + 15) / 16;
    return M >= 1 && M <= kStepProjMaxRows && V >= 1 && K >= 16 && K % 16 == 0 &&
           K / 16 <= kStepProjMaxSsq && nt * (K / 16) * 1024 < (1L << 31);
}

int head_parts(int V) { return (int)cdiv(V, kHBN); }

ssm_status launch_head(const float* xg, const float* ssq, int nssq, float inv_div, float eps,
                       const float* Ef, float* y, long ldy, int M, int V, int K, float* part,
                       uint32_t* argmax, hipStream_t st) {
    SSM_REQUIRE(head_ok(M, V, K) && xg && ssq && Ef && y && part && ldy >= V && nssq >= 1 &&
                    ((uintptr_t)xg & 15) == 0 && ((uintptr_t)Ef & 15) == 0,
                "head: unsupported arguments (%d x %d x %d)", M, V, K);
    HeadArgs a;
    a.xg = xg; a.ssq = ssq; a.nssq = nssq; a.inv_div = inv_div; a.eps = eps; a.Ef = Ef;
    a.y = y; a.ldy = ldy; a.M = M; a.V = V; a.K = K; a.nt = (V + 15) / 16;
    a.part = part; a.nparts = head_parts(V);
    const unsigned grid = (unsigned)a.nparts;
    const int mt = (M + 15) / 16, kb = K / 16;
#define HEAD_MT(KBV)                                                                 \
    switch (mt) {                                                                    \
        case 1: head_kernel<1, KBV><<<grid, 64 * kHW, 0, st>>>(a); break;            \
        case 2: head_kernel<2, KBV><<<grid, 64 * kHW, 0, st>>>(a); break;            \
        case 3: head_kernel<3, KBV><<<grid, 64 * kHW, 0, st>>>(a); break;            \
        default: head_kernel<4, KBV><<<grid, 64 * kHW, 0, st>>>(a); break;           \
    }
    // unrolled for d_model 768 and 1024 (the bench's decode models), rolled otherwise
    if (kb == 64) HEAD_MT(64)
    else if (kb == 48) HEAD_MT(48)
    else HEAD_MT(0)
#undef HEAD_MT
    const ssm_status e = check_launch("head");
    if (e != SSM_OK || !argmax) return e;
    head_argmax_kernel<<<(unsigned)M, kFin, 0, st>>>(part, a.nparts, V, argmax);
    return check_launch("head_argmax");
}

}  // namespace ssm
