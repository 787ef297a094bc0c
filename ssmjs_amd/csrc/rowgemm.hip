// Projection GEMM for few rows (decode: one row per sequence, M <= 64) on gfx950, with the
// Mamba block's normalisations fused into its operand prologue:
//
//   Y[m, n] = beta * Y[m, n] + s[m] * sum_k P[m, k] W[n, k]        W (N, K) row-major
//   mode PLAIN  P = X                 s = 1
//   mode RMS    P = X * g[k]          s = rsqrt(mean_k X^2 + eps)             (RMSNorm -> proj)
//   mode GATED  P = X * silu(Z) * g   s = rsqrt(mean_k (X silu(Z))^2 + eps)   (gated norm -> proj)
//
// The row scale s[m] is independent of n, so it is applied once per output; the normalised
// activations never go to memory. fp32 MFMA (v_mfma_f32_16x16x4_f32) throughout: MFMA t of a
// 16-wide k step uses k = 4q + t for lane group q (lanes 16q .. 16q+15) on both operands.
//
// With M <= 64 the product streams W (N x K) once while the small X (L2-resident) is read
// again by every column tile, so a workgroup owns ALL rows and 64 output columns: W is read
// exactly once. K runs in blocks of 32 whose X (with the prologue applied) and W go through a
// double-buffered LDS tile with whole-line loads issued three blocks ahead of their use (HBM
// latency is several blocks of MFMA work); the 4 waves (2 x 2) each own a 32 x 32 quarter of
// the tile as 2 x 2 accumulators.
//
// When the column tiles alone cannot fill the chip (narrow N, long K: the gated out_proj),
// K is split into S slices over S workgroups per tile, which write their partial tiles (and
// their slice's row sums of squares) to a workspace; a second kernel adds the slices in
// slice order (deterministic), applies s[m] and beta, and stores Y. The kernel boundary
// orders the two: a device-scope release/acquire per workgroup, which would let the last
// workgroup finish the tile instead, costs far more on this chip (each XCD's L2 is written
// back and invalidated).
#include <algorithm>

#include "common.hpp"
#include "glue.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 64;        // most rows per launch
constexpr int kTileN = 64;       // output columns per workgroup
constexpr int kKB = 32;          // K per block
constexpr int kPitch = kKB + 4;  // LDS row pitch (floats)
constexpr int kMaxSplit = 16;
// The finishing kernels read all kMaxSplit slots from clamped (in-bounds) slice indices and
// mask the unused ones afterwards: with `s < S ? load : 0` the compiler put each load behind
// its own branch and waited for it before issuing the next.
constexpr int kTargetWG = 256;   // (tile, slice) workgroups worth splitting K for

enum { MODE_PLAIN = 0, MODE_RMS = 1, MODE_GATED = 2 };

struct RgArgs {
    const float* X; long ldx;
    const float* Z; long ldz;
    const float* g;
    const float* W;
    float* Y; long ldy;
    int M, N, K;
    float beta, eps;
    int S, kslice, ntiles;     // splits of K, K per split (multiple of 4 blocks), column tiles
    float* part;               // (S, M, N) partial products (S > 1)
    float* ssqp;               // (S, M) partial row sums of squares (S > 1, norm modes)
};

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// P = X (* silu(Z)); the caller multiplies by g after taking the sum of squares
template <int MODE>
__device__ __forceinline__ float4 prologue(float4 x, float4 z) {
    if (MODE == MODE_GATED) {
        x.x *= ssm::silu_fast(z.x);
        x.y *= ssm::silu_fast(z.y);
        x.z *= ssm::silu_fast(z.z);
        x.w *= ssm::silu_fast(z.w);
    }
    return x;
}

__device__ __forceinline__ float sumsq(float4 p, float s) {
    s = fmaf(p.x, p.x, s);
    s = fmaf(p.y, p.y, s);
    s = fmaf(p.z, p.z, s);
    return fmaf(p.w, p.w, s);
}

__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void rowgemm_kernel(RgArgs a) {
    __shared__ __attribute__((aligned(16))) float xs[2][kRows][kPitch];
    __shared__ __attribute__((aligned(16))) float wsm[2][kTileN][kPitch];
    __shared__ float ssq[kRows];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q = lane >> 4;
    const int wm = w >> 1, wn = w & 1;            // this wave's 32 x 32 quarter
    // split-major order, remapped so that consecutive workgroups (one slice's column tiles,
    // which read the same slice of X) share an XCD and its L2
    const int per = gridDim.x / 8;
    const int wg = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (wg >= a.ntiles * a.S) return;
    const int s = wg / a.ntiles, tile = wg % a.ntiles;
    const int n0 = tile * kTileN;
    const int k0 = s * a.kslice;
    const int M = a.M, K = a.K;
    const int klen = min(a.kslice, K - k0);
    // blocks in groups of four (the tail of the last group reads zeros)
    const int nblk = (klen + 4 * kKB - 1) / (4 * kKB) * 4;

    // Global -> register staging: thread t covers rows (t / 8) + 32 h, k = 4 (t % 8) + 0..3 of a
    // block (8 threads read one row's 128 bytes). Rows past M / N and k past the slice read
    // zeros through the descriptors' ranges, so every block issues the same loads.
    const int sr = tid >> 3, sk = 4 * (tid & 7);
    const auto rx = ssm::rsrc(a.X + k0, (unsigned)(((long)(M - 1) * a.ldx + klen) * 4));
    const auto rz = ssm::rsrc(MODE == MODE_GATED ? a.Z + k0 : a.X,
                              MODE == MODE_GATED ? (unsigned)(((long)(M - 1) * a.ldz + klen) * 4) : 0u);
    const auto rw = ssm::rsrc(a.W + (long)n0 * K + k0,
                              (unsigned)(((long)(min(a.N - n0, kTileN) - 1) * K + klen) * 4));
    const auto rg = ssm::rsrc(a.g ? a.g + k0 : a.X, a.g ? (unsigned)klen * 4u : 0u);
    struct Regs { float4 x[2], z[2], w[2], g; };
    auto gload = [&](Regs& r, int b) {
        // k past the slice reads zeros: the offset lies beyond every range (the slice length
        // is a multiple of 4, so a float4 is all in or out)
        const int k = kKB * b + sk;
        const unsigned kb = k < klen ? (unsigned)k * 4u : 0x80000000u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = sr + 32 * h;
            r.x[h] = ssm::bload16<float4>(rx, (unsigned)(row * a.ldx) * 4u + kb);
            if (MODE == MODE_GATED) r.z[h] = ssm::bload16<float4>(rz, (unsigned)(row * a.ldz) * 4u + kb);
            r.w[h] = ssm::bload16<float4>(rw, (unsigned)(row * K) * 4u + kb);
        }
        if (MODE != MODE_PLAIN) r.g = ssm::bload16<float4>(rg, kb);
    };
    float ss[2] = {0.f, 0.f};
    auto lstore = [&](const Regs& r, int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float4 p = prologue<MODE>(r.x[h], r.z[h]);
            if (MODE != MODE_PLAIN) {
                ss[h] = sumsq(p, ss[h]);
                p = mul4(p, r.g);
            }
            *reinterpret_cast<float4*>(&xs[buf][sr + 32 * h][sk]) = p;
            *reinterpret_cast<float4*>(&wsm[buf][sr + 32 * h][sk]) = r.w[h];
        }
    };

    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            float4 av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                av[i] = *reinterpret_cast<const float4*>(&xs[buf][32 * wm + 16 * i + l16][16 * hh + 4 * q]);
                bv[i] = *reinterpret_cast<const float4*>(&wsm[buf][32 * wn + 16 * i + l16][16 * hh + 4 * q]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = mfma4(av[i].x, bv[j].x, acc[i][j]);
                    acc[i][j] = mfma4(av[i].y, bv[j].y, acc[i][j]);
                    acc[i][j] = mfma4(av[i].z, bv[j].z, acc[i][j]);
                    acc[i][j] = mfma4(av[i].w, bv[j].w, acc[i][j]);
                }
        }
    };

    // pipeline: block j computes from LDS buffer j % 2 while block j + 1 is stored into the
    // other buffer from register set (j + 1) % 4, which then takes the loads of block j + 5:
    // every block's loads are issued three blocks before they are needed. The loop body is one
    // group of four blocks with no exit inside, so the register sets stay distinct;
    // sched_barrier keeps the next block's prologue arithmetic from being hoisted above the
    // LDS barrier (which would make the wave wait for newer loads).
    Regs r0, r1, r2, r3;
    gload(r0, 0);
    gload(r1, 1);
    gload(r2, 2);
    gload(r3, 3);
    lstore(r0, 0);
    gload(r0, 4);
    __syncthreads();
    auto phase = [&](int buf, Regs& nxt, int nb) {
        compute(buf);
        lstore(nxt, buf ^ 1);
        gload(nxt, nb);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int b = 0; b < nblk; b += 4) {
        phase(0, r1, b + 5);   // computes block b, stores b + 1
        phase(1, r2, b + 6);
        phase(0, r3, b + 7);
        phase(1, r0, b + 8);
    }

    // row sums of squares: the 8 threads of a row hold its k-slices
    if (MODE != MODE_PLAIN) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float v = ss[h];
            v += __shfl_xor(v, 1, 64);
            v += __shfl_xor(v, 2, 64);
            v += __shfl_xor(v, 4, 64);
            if ((tid & 7) == 0) ssq[sr + 32 * h] = v;
        }
    }
    __syncthreads();

    // lane holds rows 32wm + 16i + 4q + r, column 32wn + 16j + l16 of acc[i][j]
    if (a.S == 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 32 * wm + 16 * i + 4 * q + r;
                if (m >= M) continue;
                const float sc = MODE != MODE_PLAIN ? rsqrtf(ssq[m] / (float)K + a.eps) : 1.f;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int n = n0 + 32 * wn + 16 * j + l16;
                    if (n >= a.N) continue;
                    float* yp = a.Y + (long)m * a.ldy + n;
                    float o = acc[i][j][r] * sc;
                    if (a.beta != 0.f) o = fmaf(a.beta, *yp, o);
                    *yp = o;
                }
            }
        return;
    }
    // split K: this slice's partial tile, and (from the first column tile) its row sums of
    // squares, for the finishing kernel
    float* pp = a.part + (long)s * M * a.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 32 * wm + 16 * i + 4 * q + r;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + 32 * wn + 16 * j + l16;
                if (n < a.N) pp[(long)m * a.N + n] = acc[i][j][r];
            }
        }
    if (MODE != MODE_PLAIN && tile == 0 && tid < M) a.ssqp[(long)s * M + tid] = ssq[tid];
}

// Direct-W variant for slices of at most 256 (most decode projections): a workgroup owns all
// rows, 64 output columns (16 per wave) and one K slice of KS = 16 NU. Each wave loads its 16
// W rows of the slice straight into registers in MFMA operand order, all at once (lane
// (l16, q) of k group kg holds W[n0 + 16w + l16][16 kg + 4q .. +3]: one 16-byte load per
// lane and group), while the workgroup stages the slice's operand P (X, or X silu(Z), times g)
// in LDS; each k group is then 4 b128 LDS reads (the A fragments of the 4 row tiles) and 16
// MFMAs against the W registers. The whole slice's HBM traffic is in flight together and the
// MFMAs of a k group start as soon as its W arrives, with no barrier between the first and the
// last MFMA. The row scale s[m] of the norm modes is left
// to the finishing kernel, which computes it from X (and Z) itself, so this kernel always
// writes partial tiles (S >= 2).
template <int MODE, int NU>
__global__ __launch_bounds__(256, NU > 16 ? 1 : 2) void rowgemm_direct_kernel(RgArgs a) {
    constexpr int KS = 16 * NU;          // slice length
    constexpr int XP = KS + 4;           // LDS row pitch (floats)
    constexpr int FPR = KS / 4;          // float4 per staged row (64 FPR = 256 NU in all)
    __shared__ __attribute__((aligned(16))) float xs[kRows][XP];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q = lane >> 4;
    const int per = gridDim.x / 8;
    const int wg = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (wg >= a.ntiles * a.S) return;
    const int s = wg / a.ntiles, tile = wg % a.ntiles;
    const int n0 = tile * kTileN;
    const int k0 = s * KS;
    const int M = a.M, K = a.K;
    const int klen = min(KS, K - k0);   // a multiple of 4

    // P staging: float4 j of thread t is element e = t + 256 j of the slice in row-major
    // order (row e / FPR, float4 column e % FPR), so a row's loads are consecutive lanes; rows
    // past M and k past the slice read zeros
    const auto rx = ssm::rsrc(a.X + k0, (unsigned)(((long)(M - 1) * a.ldx + klen) * 4));
    const auto rz = ssm::rsrc(MODE == MODE_GATED ? a.Z + k0 : a.X,
                              MODE == MODE_GATED ? (unsigned)(((long)(M - 1) * a.ldz + klen) * 4) : 0u);
    const auto rg = ssm::rsrc(a.g ? a.g + k0 : a.X, a.g ? (unsigned)klen * 4u : 0u);
    auto col_of = [&](int j) { return (tid + 256 * j) % FPR; };
    auto row_of = [&](int j) { return (tid + 256 * j) / FPR; };
    auto kb_of = [&](int j) { return 4 * col_of(j) < klen ? (unsigned)col_of(j) * 16u : 0x80000000u; };
    float4 xv[NU], zv[NU], gv[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int row = row_of(j);
        xv[j] = ssm::bload16<float4>(rx, (unsigned)(row * a.ldx) * 4u + kb_of(j));
        if (MODE == MODE_GATED) zv[j] = ssm::bload16<float4>(rz, (unsigned)(row * a.ldz) * 4u + kb_of(j));
        // the g float4 of the column: one load when every j has the same column
        if (MODE != MODE_PLAIN)
            gv[j] = (j == 0 || 256 % FPR != 0) ? ssm::bload16<float4>(rg, kb_of(j)) : gv[0];
    }

    // W rows n0 + 16w + l16 of the slice, issued after the (L2-resident) P operands so that the
    // staging below waits for those only; the k groups' MFMAs then consume W as it arrives.
    // Rows past N and k past the slice read zeros.
    const int nrw = min(a.N - n0 - 16 * w, 16);
    const auto rw = ssm::rsrc(a.W + (long)(n0 + 16 * w) * K + k0,
                              nrw > 0 ? (unsigned)(((long)(nrw - 1) * K + klen) * 4) : 0u);
    float4 wr[NU];
#pragma unroll
    for (int kg = 0; kg < NU; ++kg) {
        const int k = 16 * kg + 4 * q;
        wr[kg] = ssm::bload16<float4>(rw, k < klen ? (unsigned)(l16 * K + k) * 4u : 0x80000000u);
    }
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        float4 v = prologue<MODE>(xv[j], zv[j]);
        if (MODE != MODE_PLAIN) v = mul4(v, gv[j]);
        *reinterpret_cast<float4*>(&xs[row_of(j)][4 * col_of(j)]) = v;
    }
    __syncthreads();

    // k group kg: MFMA t uses k = 16 kg + 4q + t for lane group q on both operands. The A
    // fragments of group kg + 1 are read while group kg computes, and consecutive MFMAs go
    // to the four independent row-tile accumulators.
    floatx4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float4 av[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) av[0][i] = *reinterpret_cast<const float4*>(&xs[16 * i + l16][4 * q]);
#pragma unroll
    for (int kg = 0; kg < NU; ++kg) {
        const int cb = kg & 1;
        if (kg + 1 < NU) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                av[cb ^ 1][i] = *reinterpret_cast<const float4*>(&xs[16 * i + l16][16 * (kg + 1) + 4 * q]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma4(av[cb][i].x, wr[kg].x, acc[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma4(av[cb][i].y, wr[kg].y, acc[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma4(av[cb][i].z, wr[kg].z, acc[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma4(av[cb][i].w, wr[kg].w, acc[i]);
    }

    // lane holds rows 16i + 4q + r, column n0 + 16w + l16 of this slice's partial tile
    const int n = n0 + 16 * w + l16;
    if (n < a.N) {
        float* pp = a.part + (long)s * M * a.N + n;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * i + 4 * q + r;
                if (m < M) pp[(long)m * a.N] = acc[i][r];
            }
    }
}

// Row scale of the norm modes from the operands themselves: s[m] = rsqrt(mean_k P[m, k]^2 +
// eps) with P = X or X silu(Z), summed by the threads of a workgroup in thread order and then
// over the waves (deterministic). Every thread of the workgroup returns the same value.
template <int MODE, int NT>
__device__ __forceinline__ float row_scale(const RgArgs& a, int m, float* red) {
    const int tid = threadIdx.x;
    float ss = 0.f;
    for (int k = 4 * tid; k < a.K; k += 4 * NT) {
        float4 p = *reinterpret_cast<const float4*>(a.X + (long)m * a.ldx + k);
        if (MODE == MODE_GATED) p = prologue<MODE>(p, *reinterpret_cast<const float4*>(a.Z + (long)m * a.ldz + k));
        ss = sumsq(p, ss);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int v = 0; v < NT / 64; ++v) t += red[v];
    return rsqrtf(t / (float)a.K + a.eps);
}

// Finish of the direct kernel's slices: a workgroup per (row m, 256 x CPT columns); the norm
// modes' row scale is computed here from X / Z.
template <int MODE>
__global__ __launch_bounds__(256) void rowgemm_direct_reduce(RgArgs a) {
    __shared__ float red[4];
    const int m = blockIdx.y;
    const float rs = MODE != MODE_PLAIN ? row_scale<MODE, 256>(a, m, red) : 1.f;
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= a.N) return;
    const long MN = (long)a.M * a.N;
    const float* pm = a.part + (long)m * a.N + n;
    float pv[kMaxSplit];
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s) pv[s] = pm[(s < a.S ? s : 0) * MN];   // clamped
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s) v += s < a.S ? pv[s] : 0.f;
    v *= rs;
    float* yp = a.Y + (long)m * a.ldy + n;
    if (a.beta != 0.f) v = fmaf(a.beta, *yp, v);
    *yp = v;
}

// Split-K finish: Y = beta * Y + s[m] * (sum of the slices in slice order), one thread per
// output; every slice's load is issued before the sum consumes them.
template <int MODE>
__global__ __launch_bounds__(256) void rowgemm_reduce(RgArgs a) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long MN = (long)a.M * a.N;
    if (i >= MN) return;
    const int m = (int)(i / a.N), n = (int)(i % a.N);
    float pv[kMaxSplit], tv[kMaxSplit];
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s) {
        const int sc = s < a.S ? s : 0;   // clamped, not branched
        pv[s] = a.part[sc * MN + i];
        tv[s] = MODE != MODE_PLAIN ? a.ssqp[(long)sc * a.M + m] : 0.f;
    }
    float v = 0.f, t = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s) {
        v += s < a.S ? pv[s] : 0.f;
        t += s < a.S ? tv[s] : 0.f;
    }
    if (MODE != MODE_PLAIN) v *= rsqrtf(t / (float)a.K + a.eps);
    float* yp = a.Y + (long)m * a.ldy + n;
    if (a.beta != 0.f) v = fmaf(a.beta, *yp, v);
    *yp = v;
}

// Split-K finish fused with the next layer's RMSNorm (decode: the out_proj's result is the
// residual stream that the next in_proj normalises): one 1024-thread workgroup per row m
// finishes the row as rowgemm_reduce does (a thread per column, its slice loads issued
// together), keeps it in LDS, and writes nout[m, :] = Y[m, :] * g2 *
// rsqrt(mean(Y[m, :]^2) + eps). FROMX: the row scale of the norm modes comes from X / Z (the
// direct kernel) instead of the slices' sums of squares.
constexpr int kNormCols = 8192;   // widest row the fused finish keeps in LDS
template <int MODE, bool FROMX>
__global__ __launch_bounds__(1024) void rowgemm_reduce_norm(RgArgs a, const float* __restrict__ g2,
                                                           float* __restrict__ nout, long ldn) {
    __shared__ float row[kNormCols];
    __shared__ float part_ss[16];
    const int m = blockIdx.x, tid = threadIdx.x;
    const long MN = (long)a.M * a.N;
    float rs = 1.f;
    if (MODE != MODE_PLAIN && FROMX) {
        rs = row_scale<MODE, 1024>(a, m, part_ss);
        __syncthreads();   // part_ss is reused below
    } else if (MODE != MODE_PLAIN) {
        float tv[kMaxSplit];
#pragma unroll
        for (int s = 0; s < kMaxSplit; ++s) tv[s] = a.ssqp[(long)(s < a.S ? s : 0) * a.M + m];
        float t = 0.f;
#pragma unroll
        for (int s = 0; s < kMaxSplit; ++s) t += s < a.S ? tv[s] : 0.f;
        rs = rsqrtf(t / (float)a.K + a.eps);
    }
    const float* pm = a.part + (long)m * a.N;
    float* ym = a.Y + (long)m * a.ldy;
    float ss = 0.f;
    for (int n = tid; n < a.N; n += 1024) {
        float pv[kMaxSplit];
#pragma unroll
        for (int s = 0; s < kMaxSplit; ++s) pv[s] = pm[(s < a.S ? s : 0) * MN + n];   // clamped
        float v = 0.f;
#pragma unroll
        for (int s = 0; s < kMaxSplit; ++s) v += s < a.S ? pv[s] : 0.f;
        v *= rs;
        if (a.beta != 0.f) v = fmaf(a.beta, ym[n], v);
        ym[n] = v;
        row[n] = v;
        ss = fmaf(v, v, ss);
    }
    // block sum of squares (16 waves)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) part_ss[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) tot += part_ss[v];
    const float r2 = rsqrtf(tot / (float)a.N + a.eps);
    float* om = nout + (long)m * ldn;
    for (int n = tid; n < a.N; n += 1024) om[n] = row[n] * r2 * g2[n];
}

// Splits of K for a shape: enough (column tile, slice) workgroups to fill the chip. The
// direct-W kernel takes slices of 16 NU (NU in kDirectNU) with at most one workgroup per CU
// (ntiles S <= kTargetWG, so no CU gets two while others idle); otherwise the LDS-staged kernel
// splits into slices of whole groups of four K blocks.
struct Split {
    int S, kslice, ntiles;
    int NU;   // > 0: direct-W kernel with slices of 16 NU
};

constexpr int kDirectNU[] = {8, 16, 24};

Split choose(int N, int K, bool can_split) {
    Split p{};
    p.ntiles = (int)ssm::cdiv(N, kTileN);
    if (can_split && p.ntiles < kTargetWG) {
        const int S = std::min(kMaxSplit, kTargetWG / p.ntiles);
        const int need = (int)ssm::cdiv(K, 16 * S);
        for (int nu : kDirectNU)
            if (nu >= need) {
                const int Sd = (int)ssm::cdiv(K, 16 * nu);
                if (Sd >= 2) {
                    p.S = Sd;
                    p.NU = nu;
                    p.kslice = 16 * nu;
                    return p;
                }
                break;
            }
    }
    const int blocks = (int)ssm::cdiv(K, kKB);
    int S = 1;
    if (can_split && p.ntiles < kTargetWG) {
        S = (int)ssm::cdiv(kTargetWG, p.ntiles);
        S = std::min(S, kMaxSplit);
        S = std::min(S, std::max(1, blocks / 4));
    }
    p.kslice = 4 * kKB * (int)ssm::cdiv(blocks, 4 * S);
    p.S = (int)ssm::cdiv(K, p.kslice);
    return p;
}

size_t split_bytes(const Split& p, int M, int N) {
    if (p.S <= 1) return 0;
    return sizeof(float) * (size_t)p.S * M * ((size_t)N + 1);
}

}  // namespace

namespace ssm {

bool rowgemm_ok(int M, int N, int K) { return M >= 1 && M <= kRows && N >= 1 && K >= 4 && K % 4 == 0; }

size_t rowgemm_workspace(int M, int N, int K) {
    if (!rowgemm_ok(M, N, K)) return 0;
    return split_bytes(choose(N, K, true), M, N);
}

ssm_status launch_rowgemm(int mode, const float* X, long ldx, const float* Z, long ldz,
                          const float* g, const float* W, float* Y, long ldy, int M, int N, int K,
                          float beta, float eps, void* workspace, size_t workspace_bytes,
                          hipStream_t st, const float* g2, float* nout, long ldn, bool* normed) {
    if (normed) *normed = false;
    if (!rowgemm_ok(M, N, K))
        return fail(SSM_ERR_UNSUPPORTED, "row GEMM: need 1 <= M <= %d and K %% 4 == 0 (M=%d K=%d)",
                    kRows, M, K);
    // the kernel addresses X, Z and one tile's W rows with 32-bit byte offsets
    if ((long)kRows * ldx * 4 >= (1L << 31) || (long)kRows * ldz * 4 >= (1L << 31) ||
        (long)kTileN * K * 4 >= (1L << 31))
        return fail(SSM_ERR_UNSUPPORTED, "row GEMM: operands too large for 32-bit offsets");
    Split p = choose(N, K, true);
    if (p.S > 1 && (!workspace || workspace_bytes < split_bytes(p, M, N))) p = choose(N, K, false);
    RgArgs a{};
    a.X = X; a.ldx = ldx; a.Z = Z; a.ldz = ldz; a.g = g; a.W = W; a.Y = Y; a.ldy = ldy;
    a.M = M; a.N = N; a.K = K; a.beta = beta; a.eps = eps;
    a.S = p.S; a.kslice = p.kslice; a.ntiles = p.ntiles;
    if (p.S > 1) {
        a.part = (float*)workspace;
        a.ssqp = a.part + (size_t)p.S * M * N;
    }
    const unsigned grid = (unsigned)(8 * cdiv((long)p.ntiles * p.S, 8));
    const unsigned rgrid = (unsigned)cdiv((long)M * N, 256);
    // the next RMSNorm rides on the split finish when there is one and the row fits in LDS
    const bool fuse = g2 && nout && p.S > 1 && N <= kNormCols;
    if (fuse && normed) *normed = true;
    // the direct-W kernel's finish computes the norm modes' row scale itself
    const bool direct = p.S > 1 && p.NU > 0;
    const dim3 dgrid((unsigned)cdiv(N, 256), (unsigned)M);
#define RG_LAUNCH(MD)                                                                         \
    if (direct) {                                                                             \
        if (p.NU == 8) rowgemm_direct_kernel<MD, 8><<<grid, 256, 0, st>>>(a);                 \
        else if (p.NU == 16) rowgemm_direct_kernel<MD, 16><<<grid, 256, 0, st>>>(a);          \
        else rowgemm_direct_kernel<MD, 24><<<grid, 256, 0, st>>>(a);                          \
        if (fuse) rowgemm_reduce_norm<MD, true><<<(unsigned)M, 1024, 0, st>>>(a, g2, nout, ldn); \
        else rowgemm_direct_reduce<MD><<<dgrid, 256, 0, st>>>(a);                             \
    } else {                                                                                  \
        rowgemm_kernel<MD><<<grid, 256, 0, st>>>(a);                                          \
        if (fuse) rowgemm_reduce_norm<MD, false><<<(unsigned)M, 1024, 0, st>>>(a, g2, nout, ldn); \
        else if (p.S > 1) rowgemm_reduce<MD><<<rgrid, 256, 0, st>>>(a);                       \
    }
    switch (mode) {
        case 0: RG_LAUNCH(MODE_PLAIN); break;
        case 1: RG_LAUNCH(MODE_RMS); break;
        default: RG_LAUNCH(MODE_GATED); break;
    }
#undef RG_LAUNCH
    return check_launch("rowgemm");
}

}  // namespace ssm

extern "C" size_t ssm_linear_rows_workspace(int M, int N, int K) {
    return ssm::rowgemm_workspace(M, N, K);
}

extern "C" ssm_status ssm_linear_rows(int mode, const float* x, long ldx, const float* z, long ldz,
                                      const float* g, const float* W, float* y, long ldy, int M,
                                      int N, int K, float beta, float eps, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    SSM_REQUIRE(x && W && y, "ssm_linear_rows: null x/W/y");
    SSM_REQUIRE(mode >= 0 && mode <= 2, "ssm_linear_rows: mode must be 0, 1 or 2");
    SSM_REQUIRE(mode == 0 || g, "ssm_linear_rows: norm modes need the weight g");
    SSM_REQUIRE(mode != 2 || z, "ssm_linear_rows: gated mode needs z");
    SSM_REQUIRE(ldx >= K && ldy >= N && (mode != 2 || ldz >= K), "ssm_linear_rows: bad strides");
    SSM_REQUIRE(ldx % 4 == 0 && (mode != 2 || ldz % 4 == 0) && (uintptr_t)x % 16 == 0 &&
                    (uintptr_t)W % 16 == 0 && (!z || (uintptr_t)z % 16 == 0) &&
                    (!g || (uintptr_t)g % 16 == 0),
                "ssm_linear_rows: x, z, g, W must be 16-byte aligned with ld % 4 == 0");
    if (M == 0 || N == 0) return SSM_OK;
    return ssm::launch_rowgemm(mode, x, ldx, z, ldz, g, W, y, ldy, M, N, K, beta, eps, workspace,
                               workspace_bytes, (hipStream_t)stream, nullptr, nullptr, 0, nullptr);
}
