// Projections of the one-token step (decode: one row per sequence, M <= 64) on the gfx950
// fp32 matrix cores, with the step's neighbouring element-wise work in the epilogue:
//
//   v[m, n] = s[m] * sum_k X[m, k] W[n, k]          W (N, K)
//   s[m]    = 1 / sqrt(sum_j ssq[m, j] * inv_div + eps)    (ssq given; else s = 1)
//
//   EPI_STORE  Y[m, n] = v + beta * Y[m, n]
//   EPI_CONV   columns c0 .. c0+C-1 go through the depthwise causal-conv update + SiLU (the
//              Mamba conv1d on one new token, state (M, C, Kc-1) shifted in place) into Yc;
//              the other columns are stored to Y
//   EPI_RESID  Y[m, n] += v (the residual add); then, when g2 is given, the next RMSNorm's
//              operand xg[m, n] = Y[m, n] * g2[n] (in fragment order, below) and the row's
//              partial sum of squares over the tile's 16 columns, ssq_out[m, n / 16]
//   Yf         EPI_CONV: the conv outputs also written in fragment order, the operand of the
//              step's next projection (the Mamba-1 step's x_proj as its own launch)
//   xpart      EPI_CONV: that next projection summed over each conv tile's 16 channels (one
//              partial row per tile and row), so that no launch of its own is needed: the
//              Mamba-1 step's state update adds the partials
//
// The RMSNorms of the step are carried this way: the producer of a row writes x * g and
// partial sums of x^2 per 16 columns, and the consumer's epilogue applies 1 / rms(x) as the
// row scale s[m]; the gated norm's y * silu(z) * g and its partial sums come from the state
// update (ssd.hip). The partial sums are added in a fixed order, identical in every
// workgroup, so s[m] is the same wherever it is formed and every result is deterministic.
//
// Operand order. An MFMA operand puts 16 different rows in every 16 lanes (lane (i, q) =
// (lane % 16, lane / 16) holds row i, k = 4q .. 4q+3 of a 16-wide k-block), so loading it
// from a row-major matrix touches 16 cache lines per 16 lanes for 16 bytes each; measured,
// that runs at a fraction of the L1's line rate (22 us for the 64 x 4384 x 1024 in_proj).
// Both operands are therefore stored in fragment order (frag_off in glue.hpp): the 1 KB of
// a (16-row tile, k-block) is contiguous, lane-major, and one b128 load per lane brings a
// whole fragment as 8 full lines. W is packed once from the checkpoint layout (pack_frag
// below, redone when the weights change); X is written in that order by its producer.
//
// Decomposition. A workgroup owns one 16 x 16 output tile and all of K, which its 4 waves
// split into contiguous quarters; the quarters are added in LDS in wave order. At the decode
// shapes (64 rows) that is 4 * N / 16 workgroups: 256 for an out_proj into d_model 1024,
// 1096 for a 4384-column in_proj. Larger tiles reuse operands more, but 64 x 16 tiles give
// 274 workgroups for 256 CUs, and the 18 CUs that run two set the time (twice the mean); at
// 16 x 16 the most loaded CU runs 5 tiles against a mean of 4.3. Each wave streams its
// fragments PD k-blocks ahead; MFMA t of a block takes component t of both fragments
// (k = 4q + t for lane group q), so its four MFMAs cover the block's 16 k exactly once.
//
// Tile order: workgroups are dispatched to the 8 XCDs round-robin by linear id, so the row
// tiles of one column tile get ids 8 apart (same XCD): W, the only operand that comes from
// HBM, is fetched once into that XCD's L2 and read from there by the other row tiles. W goes
// through streaming (non-temporal) loads: its lines are wanted only while the row tiles of
// their column tile run, and X, read by every column tile, keeps the rest of the cache
// (measured: out_proj 8.00 -> 7.72 us at cfg4, 7.28 -> 6.88 us in the Mamba-1 step).
#include "common.hpp"
#include "glue.hpp"

namespace ssm {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kNW = 4;                  // waves per workgroup
constexpr unsigned kOOR = 0x80000000u;  // a buffer offset past every descriptor's range
constexpr int kSsqPer = kStepProjMaxSsq / 16;   // partial sums per epilogue thread
// EPI_CONV with xpart as a kernel of its own (its B fragments need registers that the plain
// conv epilogue's occupancy target does not leave)
constexpr int EPI_CONVX = 3;

__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 16);
    return v;
}

template <int PD, int EPI>
__global__ __launch_bounds__(64 * kNW, EPI == EPI_CONVX ? 4 : PD > 4 ? (EPI == EPI_CONV ? 4 : 5) : EPI == EPI_CONV ? 6 : 8) void stepproj_kernel(
    StepProj a) {
    constexpr bool CONV = EPI == EPI_CONV || EPI == EPI_CONVX;
    __shared__ float red[kNW][16][17];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int b = blockIdx.x, r8 = b >> 3;
    const int tm = r8 % a.mt, tn = (r8 / a.mt) * 8 + (b & 7);
    if (tn >= a.nt) return;   // the id space is padded to whole groups of 8 column tiles
    const int m0 = tm * 16, n0 = tn * 16;

    // The epilogue's element (thread t: row t / 16, column t % 16 of the tile), and the
    // partial sums of its row's scale, loaded ahead of the operands so that waiting for them
    // overlaps the operands' latency (rows past M and sums past nssq read 0).
    const int ei = tid >> 4, ej = tid & 15;
    const int em = m0 + ei, en = n0 + ej;
    float sp[kSsqPer];
    if (a.ssq) {
        const auto rs = rsrc(a.ssq, (unsigned)(a.M * a.nssq) * 4u);
#pragma unroll
        for (int u = 0; u < kSsqPer; ++u) {
            const int j = u * 16 + ej;
            sp[u] = bload4(rs, j < a.nssq ? (unsigned)(em * a.nssq + j) * 4u : kOOR);
        }
    }

    // The conv epilogue's inputs (the cached inputs, the taps and the bias of this thread's
    // channel), loaded here with the operands: they do not depend on the product, and loaded
    // in the epilogue each would be a memory latency after the last MFMA (the state loads and
    // the shift stores of one channel alias, so they were also serial there). Widths up to
    // kConvPre; wider kernels keep the epilogue's own loads.
    constexpr int kConvPre = 4;
    const int ec = en - a.c0;
    const bool conv_pre = CONV && em < a.M && en < a.N && ec >= 0 && ec < a.C && a.Kc <= kConvPre;
    float csv[kConvPre - 1] = {}, cwv[kConvPre] = {}, cbv = 0.f;
    if constexpr (CONV) {
        if (conv_pre) {
            const float* st = a.cst + ((long)em * a.C + ec) * (a.Kc - 1);
#pragma unroll
            for (int k = 0; k < kConvPre - 1; ++k)
                if (k < a.Kc - 1) csv[k] = st[k];
#pragma unroll
            for (int k = 0; k < kConvPre; ++k)
                if (k < a.Kc) cwv[k] = a.cw[(long)ec * a.Kc + k];
            if (a.cb) cbv = a.cb[ec];
        }
    }

    // The residual epilogue's inputs (this thread's element of Y and the next norm's weight),
    // loaded here for the same reason; only this thread reads and writes that element.
    float rsv = 0.f, g2v = 0.f;
    if constexpr (EPI == EPI_RESID) {
        if (em < a.M && en < a.N) rsv = a.Y[(long)em * a.ldy + en];
        if (a.g2 && en < a.N) g2v = a.g2[en];
    }

    // EPI_CONV with xpart: a tile of conv columns (16 channels; c0 and C are multiples of 16)
    // also projects its 16 x 16 conv outputs onto the next projection's RN columns on the
    // matrix cores (the tile's outputs as the A operand, its 16 rows of wxt as B). Wave w takes
    // the 16-column blocks w, w + 4, ...; its B fragments are loaded here (lane (j, k) of
    // k-step s: wxt[channel 4s + k][16 block + j]) so that they arrive with the operands.
    constexpr int kXpBlk = kXpartMaxRN / 16 / kNW;   // column blocks per wave
    const bool xp_tile = EPI == EPI_CONVX && n0 >= a.c0 && n0 < a.c0 + a.C;
    float wxb[kXpBlk][4];
    if constexpr (EPI == EPI_CONVX) {
        if (xp_tile) {
#pragma unroll
            for (int t = 0; t < kXpBlk; ++t) {
                const int col = 16 * (w + kNW * t) + l16;
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4)
                    wxb[t][s4] = col < a.RN ? a.wxt[(long)(n0 - a.c0 + 4 * s4 + q) * a.RN + col]
                                            : 0.f;
            }
        }
    }

    // this wave's k-blocks [kb0, kb0 + nb); fragment kb of a tile is 1 KB at kb * 1024
    const int KB = a.K / 16;
    const int bpw = (KB + kNW - 1) / kNW;
    const int kb0 = w * bpw;
    const int nb = min(bpw, KB - kb0);
    const int ng = nb > 0 ? (nb + PD - 1) / PD : 0;
    const auto ra = rsrc(a.X + (long)tm * KB * 256, (unsigned)KB * 1024u);
    const auto rw = rsrc(a.W + (long)tn * KB * 256, (unsigned)KB * 1024u);
    const unsigned o0 = (unsigned)kb0 * 1024u + (unsigned)lane * 16u;
    // The column tiles that share an XCD read the same X fragments; each starts its k-blocks
    // at its own rotation so that they do not all ask one L2 channel for one line at once.
    // The row tiles of a column tile keep one rotation: they share W's lines in that L2.
    const int rot = a.rotate && nb > 0 ? (r8 / a.mt) % nb : 0;
    auto off = [&](int j) -> unsigned {   // j-th k-block of this wave, rotated
        if (j >= nb) return kOOR;
        const int jr = j + rot < nb ? j + rot : j + rot - nb;
        return o0 + (unsigned)jr * 1024u;
    };

    float4 pa[PD], pb[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) {
        pa[j] = bload16<float4>(ra, off(j));
        pb[j] = ssm::bload16_nt<float4>(rw, off(j));   // W: streaming (see below)
    }
    float scale = 1.f;
    if (a.ssq) {
        float t = sp[0];
#pragma unroll
        for (int u = 1; u < kSsqPer; ++u) t += sp[u];
        t = sum16(t);
        scale = 1.f / sqrtf(t * a.inv_div + a.eps);
    }
    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    for (int g = 0; g < ng; ++g) {
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            acc0 = mfma4(pa[j].x, pb[j].x, acc0);
            acc1 = mfma4(pa[j].y, pb[j].y, acc1);
            acc0 = mfma4(pa[j].z, pb[j].z, acc0);
            acc1 = mfma4(pa[j].w, pb[j].w, acc1);
            const int nj = (g + 1) * PD + j;
            pa[j] = bload16<float4>(ra, off(nj));
            pb[j] = ssm::bload16_nt<float4>(rw, off(nj));
            // keep each refill right behind the MFMAs that free its registers, so that PD
            // blocks stay in flight (left alone, the scheduler sinks all refills to the end
            // of the group and the next group waits a full memory latency)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // lane (l16, q) holds D[4q + r][l16]
#pragma unroll
    for (int r = 0; r < 4; ++r) red[w][4 * q + r][l16] = acc0[r] + acc1[r];
    __syncthreads();
    float v = red[0][ei][ej];
#pragma unroll
    for (int k = 1; k < kNW; ++k) v += red[k][ei][ej];
    v *= scale;
    const bool ok = em < a.M && en < a.N;
    if constexpr (EPI == EPI_STORE) {
        if (ok) {
            float* y = a.Y + (long)em * a.ldy + en;
            *y = a.beta != 0.f ? v + a.beta * *y : v;
        }
    } else if constexpr (CONV) {
        const int c = en - a.c0;
        const bool in_conv = c >= 0 && c < a.C;
        float u = 0.f;   // the conv output; 0 on padding rows
        if (ok && !in_conv) a.Y[(long)em * a.ldy + en] = v;
        if (conv_pre) {
            // same arithmetic order as the conv update kernel (conv1d.hip), on the prefetched
            // inputs
            const int Kc = a.Kc;
            float* st = a.cst + ((long)em * a.C + c) * (Kc - 1);
            float acc = cbv;
#pragma unroll
            for (int k = 0; k < kConvPre - 1; ++k)
                if (k < Kc - 1) acc = fmaf(cwv[k], csv[k], acc);
            float wl = cwv[0];
#pragma unroll
            for (int k = 1; k < kConvPre; ++k)
                if (k == Kc - 1) wl = cwv[k];
            acc = fmaf(wl, v, acc);
#pragma unroll
            for (int k = 1; k < kConvPre - 1; ++k)   // shift the cached inputs down
                if (k < Kc - 1) st[k - 1] = csv[k];
            if (Kc > 1) st[Kc - 2] = v;
            u = silu_fast(acc);
            a.Yc[(long)em * a.ldyc + c] = u;
        } else if (ok && in_conv) {
            // same arithmetic order as the conv update kernel (conv1d.hip)
            const int Kc = a.Kc;
            const float* wc = a.cw + (long)c * Kc;
            float* s = a.cst + ((long)em * a.C + c) * (Kc - 1);
            float acc = a.cb ? a.cb[c] : 0.f;
            for (int k = 0; k < Kc - 1; ++k) {   // taps on the cached inputs, shifting them down
                const float sv = s[k];
                acc = fmaf(wc[k], sv, acc);
                if (k > 0) s[k - 1] = sv;
            }
            acc = fmaf(wc[Kc - 1], v, acc);
            if (Kc > 1) s[Kc - 2] = v;
            u = silu_fast(acc);
            a.Yc[(long)em * a.ldyc + c] = u;
        }
        // padding rows of the fragment-order copy get zeros for the next projection
        if (a.Yf && in_conv && en < a.N) a.Yf[frag_off(em, c, a.C >> 4)] = u;
        if constexpr (EPI == EPI_CONVX) {
            if (xp_tile) {   // uniform over the workgroup
                __shared__ float us[16][17];
                us[ei][ej] = u;
                __syncthreads();
                // D[i][j] = sum_s sum_k u[i][4s + k] wxt[4s + k][j]; lane (j, q) holds
                // rows 4q .. 4q + 3
                const int ct = (n0 - a.c0) >> 4;
#pragma unroll
                for (int t = 0; t < kXpBlk; ++t) {
                    const int blk = w + kNW * t;
                    if (16 * blk >= a.RN) break;   // wave-uniform
                    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4)
                        acc = mfma4(us[l16][4 * s4 + q], wxb[t][s4], acc);
                    const int col = 16 * blk + l16;
                    if (col < a.RN) {
                        float* dst = a.xpart + ((long)ct * 16 * a.mt + m0 + 4 * q) * a.RN + col;
#pragma unroll
                        for (int r = 0; r < 4; ++r) dst[(long)r * a.RN] = acc[r];
                    }
                }
            }
        }
    } else {   // EPI_RESID
        float o = 0.f;
        if (ok) {
            o = rsv + v;
            a.Y[(long)em * a.ldy + en] = o;
        }
        if (a.g2) {
            // rows past M (up to the tile's 16) get zeros: the next projection reads whole tiles
            if (en < a.N) a.xg[frag_off(em, en, a.nt)] = ok ? o * g2v : 0.f;
            const float t = sum16(o * o);
            if (ej == 0 && em < a.M) a.ssq_out[(long)em * a.nt + tn] = t;
        }
    }
}

// x * g in fragment order and the partial sums of x^2 per 16 columns, for the first RMSNorm
// of the step (d % 16 == 0: every 16-lane group is one row's 16 columns). Rows M .. M16-1
// (the last row tile's padding) are written as zeros.
__global__ __launch_bounds__(256) void xg_ssq_kernel(const float* __restrict__ x, long ldx,
                                                     const float* __restrict__ g,
                                                     float* __restrict__ xg,
                                                     float* __restrict__ ssq, int M, int d) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int m = (int)(i / d), n = (int)(i % d);
    const bool ok = m < M;
    const float v = ok ? x[(long)m * ldx + n] : 0.f;
    xg[frag_off(m, n, d / 16)] = v * g[n];
    const float t = sum16(v * v);
    if (ok && (n & 15) == 0) ssq[(long)m * (d / 16) + n / 16] = t;
}

// The embedding gather of a one-token step fused with the first RMSNorm's operand: hid (M, d)
// = E[ids], xg = hid * g in fragment order and the partial sums of hid^2 per 16 columns, as
// embed_kernel and xg_ssq_kernel would write them one after the other (ids past V flag *bad
// and read row 0). M16 * d threads, d % 16 == 0, so the grid is whole blocks of 256.
__global__ __launch_bounds__(256) void embed_xg_kernel(const uint32_t* __restrict__ ids,
                                                       const float* __restrict__ emb,
                                                       float* __restrict__ hid,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ xg,
                                                       float* __restrict__ ssq, int M, int d,
                                                       int V, int* bad) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int m = (int)(i / d), n = (int)(i % d);
    const bool ok = m < M;
    float v = 0.f;
    if (ok) {
        uint32_t id = ids[m];
        if (id >= (uint32_t)V) {
            if (n == 0) atomicOr(bad, 1);
            id = 0;
        }
        v = emb[(long)id * d + n];
        hid[(long)m * d + n] = v;
    }
    xg[frag_off(m, n, d / 16)] = v * g[n];
    const float t = sum16(v * v);
    if (ok && (n & 15) == 0) ssq[(long)m * (d / 16) + n / 16] = t;
}

// W (N, K) row stride ldw -> fragment order, N padded with zero rows to whole 16-row tiles.
// One thread per 16 bytes of the output; W is read as scalars (a layer's weights start at any
// float offset of the checkpoint buffer, and this runs once per weight change).
__global__ __launch_bounds__(256) void pack_frag_kernel(const float* __restrict__ W, long ldw,
                                                        int N, int K, float* __restrict__ out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;   // float4 index
    const int KB = K / 16;
    const long total = (long)((N + 15) / 16) * KB * 64;
    if (i >= total) return;
    const int lane = (int)(i & 63);
    const long blk = i >> 6;
    const int kb = (int)(blk % KB), tn = (int)(blk / KB);
    const int n = tn * 16 + (lane & 15), k = kb * 16 + 4 * (lane >> 4);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n < N) {
        const float* r = W + (long)n * ldw + k;
        v = make_float4(r[0], r[1], r[2], r[3]);
    }
    reinterpret_cast<float4*>(out)[i] = v;
}

// W (N, K) row stride ldw -> W^T (K, N) row-major, out[k N + n] = W[n ldw + k]: the conv
// epilogue's x_proj slice of a tile is then 16 contiguous rows. One thread per element (runs
// once per weight change).
__global__ __launch_bounds__(256) void pack_t_kernel(const float* __restrict__ W, long ldw,
                                                     int N, int K, float* __restrict__ out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)N * K) return;
    const int k = (int)(i / N), n = (int)(i % N);
    out[i] = W[(long)n * ldw + k];
}

// W (N, K) row-major -> quads, out[((k / 4) N + n) 4 + k % 4] = W[n K + k]: a thread that owns
// row n reads its quads as float4s that are contiguous across a wave (the Mamba-1 step's
// dt_proj rows). One thread per quad (runs once per weight change).
__global__ __launch_bounds__(256) void pack_q4_kernel(const float* __restrict__ W, int N, int K,
                                                      float4* __restrict__ out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;   // quad index (k / 4) N + n
    if (i >= (long)N * (K / 4)) return;
    const int n = (int)(i % N), k4 = (int)(i / N);
    const float* r = W + (long)n * K + 4 * k4;
    out[i] = make_float4(r[0], r[1], r[2], r[3]);
}

template <int PD>
ssm_status launch_pd(int epi, const StepProj& a, unsigned grid, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: stepproj_kernel<PD, EPI_STORE><<<grid, 64 * kNW, 0, st>>>(a); break;
        case EPI_CONV:
            if (a.xpart) stepproj_kernel<PD, EPI_CONVX><<<grid, 64 * kNW, 0, st>>>(a);
            else stepproj_kernel<PD, EPI_CONV><<<grid, 64 * kNW, 0, st>>>(a);
            break;
        default: stepproj_kernel<PD, EPI_RESID><<<grid, 64 * kNW, 0, st>>>(a); break;
    }
    return check_launch("stepproj");
}

}  // namespace

bool stepproj_ok(int M, int N, int K) {
    return M >= 1 && M <= kStepProjMaxRows && N >= 1 && K >= 16 && K % 16 == 0 &&
           (long)K * 64 < (1L << 31);
}

size_t frag_floats(int rows, int K) { return (size_t)((rows + 15) / 16) * 16 * K; }

ssm_status launch_pack_frag(const float* W, long ldw, int N, int K, float* out, hipStream_t st) {
    SSM_REQUIRE(K % 16 == 0 && ldw >= K && ((uintptr_t)out & 15) == 0,
                "pack_frag: K %d / ldw %ld / alignment", K, ldw);
    const long n4 = (long)frag_floats(N, K) / 4;
    if (n4 == 0) return SSM_OK;
    pack_frag_kernel<<<(unsigned)cdiv(n4, 256), 256, 0, st>>>(W, ldw, N, K, out);
    return check_launch("pack_frag");
}

ssm_status launch_pack_t(const float* W, long ldw, int N, int K, float* out, hipStream_t st) {
    SSM_REQUIRE(W && out && N >= 1 && K >= 1 && ldw >= K, "pack_t: arguments");
    const long n = (long)N * K;
    pack_t_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(W, ldw, N, K, out);
    return check_launch("pack_t");
}

ssm_status launch_pack_q4(const float* W, int N, int K, float* out, hipStream_t st) {
    SSM_REQUIRE(W && out && N >= 1 && K >= 4 && K % 4 == 0 && ((uintptr_t)out & 15) == 0,
                "pack_q4: arguments");
    const long n = (long)N * (K / 4);
    pack_q4_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(W, N, K, (float4*)out);
    return check_launch("pack_q4");
}

ssm_status launch_stepproj(int epi, StepProj a, hipStream_t st) {
    SSM_REQUIRE(stepproj_ok(a.M, a.N, a.K) && ((uintptr_t)a.X & 15) == 0 &&
                    ((uintptr_t)a.W & 15) == 0,
                "stepproj: unsupported shape %d x %d x %d", a.M, a.N, a.K);
    SSM_REQUIRE(!a.ssq || (a.nssq >= 1 && a.nssq <= kStepProjMaxSsq), "stepproj: nssq");
    SSM_REQUIRE(epi != EPI_CONV || (a.Kc >= 1 && a.Kc <= 8 && a.cw && a.cst && a.Yc),
                "stepproj: conv epilogue arguments");
    SSM_REQUIRE(epi != EPI_RESID || !a.g2 || (a.xg && a.ssq_out && a.N % 16 == 0),
                "stepproj: residual epilogue arguments");
    SSM_REQUIRE(!a.Yf || (epi == EPI_CONV && a.C % 16 == 0),
                "stepproj: fragment-order copy arguments");
    SSM_REQUIRE(!a.xpart || (epi == EPI_CONV && a.wxt && a.RN >= 1 && a.RN <= kXpartMaxRN &&
                             a.c0 % 16 == 0 && a.C % 16 == 0),
                "stepproj: x_proj partial arguments");
    a.mt = (a.M + 15) / 16;
    a.nt = (a.N + 15) / 16;
    const unsigned grid = (unsigned)(8L * a.mt * ((a.nt + 7) / 8));
    // Measured at 64 rows (K 1024 .. 2048): with about one tile per CU, 8 k-blocks in flight
    // per wave and no rotation (5.5 us for 1024 x 2048, against 6.3 rotated and 6.4 with 16
    // blocks); with several tiles per CU, 4 blocks and rotated starts (12.8 us for 4384 x 1024,
    // against 13.5 with 8 blocks and 14.3 unrotated).
    if ((long)a.mt * a.nt <= 512) {
        a.rotate = 0;
        return launch_pd<8>(epi, a, grid, st);
    }
    a.rotate = 1;
    return launch_pd<4>(epi, a, grid, st);
}

ssm_status launch_embed_xg(const uint32_t* ids, const float* emb, float* hid, const float* g,
                           float* xg, float* ssq, int M, int d, int V, int* bad, hipStream_t st) {
    SSM_REQUIRE(d % 16 == 0 && d / 16 <= kStepProjMaxSsq && M >= 0 && M <= kStepProjMaxRows,
                "embed_xg: d_model %d, rows %d", d, M);
    const long n = (long)((M + 15) / 16) * 16 * d;
    if (n == 0) return SSM_OK;
    embed_xg_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(ids, emb, hid, g, xg, ssq, M, d, V,
                                                             bad);
    return check_launch("embed_xg");
}

ssm_status launch_xg_ssq(const float* x, long ldx, const float* g, float* xg, float* ssq, int M,
                         int d, hipStream_t st) {
    SSM_REQUIRE(d % 16 == 0 && d / 16 <= kStepProjMaxSsq, "xg_ssq: d_model %d", d);
    const long n = (long)((M + 15) / 16) * 16 * d;
    if (n == 0) return SSM_OK;
    xg_ssq_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(x, ldx, g, xg, ssq, M, d);
    return check_launch("xg_ssq");
}

}  // namespace ssm
