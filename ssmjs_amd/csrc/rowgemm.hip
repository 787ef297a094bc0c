// Projection GEMM for few rows (decode: one row per sequence, M <= 64) on gfx950, with the
// Mamba block's normalisations fused into its operand prologue:
//
//   Y[m, n] = beta * Y[m, n] + s[m] * sum_k P[m, k] W[n, k]        W (N, K) row-major
//   mode PLAIN  P = X                 s = 1
//   mode RMS    P = X * g[k]          s = rsqrt(mean_k X^2 + eps)             (RMSNorm -> proj)
//   mode GATED  P = X * silu(Z) * g   s = rsqrt(mean_k (X silu(Z))^2 + eps)   (gated norm -> proj)
//
// The row scale s[m] is independent of n, so it is applied once per output; the normalised
// activations never go to memory. Work split: a workgroup owns 16 rows and 16*NB output
// columns (grid = column tiles x row blocks, padded to a multiple of 8 and remapped so one
// tile's row blocks share an XCD and its L2); its 4 waves take interleaved 16-wide chunks of K, issue 8 chunks' loads at a
// time, and meet in LDS at the end.
// Per chunk a lane loads one float4 of each operand row it covers (row l%16, k = k0 + 4(l/16)
// + 0..3) and issues 4 v_mfma_f32_16x16x4_f32 per (row block, column block): MFMA j uses
// k-slots {k0 + 4q + j}, the same permutation on both operands. fp32 MFMA throughout.
#include "common.hpp"
#include "glue.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 64;   // most rows per launch (row blocks of 16)

enum { MODE_PLAIN = 0, MODE_RMS = 1, MODE_GATED = 2 };

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int MODE, int NB>
__global__ __launch_bounds__(256) void rowgemm_kernel(
    const float* __restrict__ X, long ldx, const float* __restrict__ Z, long ldz,
    const float* __restrict__ g, const float* __restrict__ W, float* __restrict__ Y, long ldy,
    int M, int N, int K, float beta, float eps, int rbs, int ntiles_rbs) {
    constexpr int WAVES = 4, U = 4, NT = 16 * NB;
    __shared__ floatx4 part[WAVES][NB][64];
    __shared__ float ssq[WAVES][16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q = lane >> 4;
    // the grid is padded to a multiple of 8 so that consecutive logical workgroups (a column
    // tile's row blocks) land on one XCD and read the tile's W rows through one L2
    const int wg = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
    if (wg >= ntiles_rbs) return;
    const int rb = wg % rbs, n0 = (wg / rbs) * NT, m0 = 16 * rb;

    // rows past M and columns past N read zeros through the descriptors' ranges
    const auto rx = ssm::rsrc(X + (long)m0 * ldx, (unsigned)(((long)(min(M - m0, 16) - 1) * ldx + K) * 4));
    const auto rz = ssm::rsrc(MODE == MODE_GATED ? Z + (long)m0 * ldz : X,
                              MODE == MODE_GATED ? (unsigned)(((long)(min(M - m0, 16) - 1) * ldz + K) * 4) : 0u);
    const auto rw = ssm::rsrc(W + (long)n0 * K, (unsigned)(((long)(min(N - n0, NT) - 1) * K + K) * 4));
    const auto rg = ssm::rsrc(g ? g : X, g ? (unsigned)K * 4u : 0u);
    const unsigned ox = (unsigned)(l16 * ldx) * 4u, oz = (unsigned)(l16 * ldz) * 4u;

    floatx4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;

    // wave w takes the 16-wide k chunks w, w + 4, ...; rounds of U chunks are double-buffered
    // (round r + 1's loads are in flight while round r computes). Every load is issued: a
    // chunk past K gets an out-of-range offset and reads zeros, so the compiler's vmcnt waits
    // count exactly.
    const int nchunks = K / 16;
    const int rounds = ((nchunks + WAVES - 1) / WAVES + U - 1) / U;
    struct Buf { float4 w[U][NB], x[U], z[U], g[U]; };
    auto load = [&](Buf& bf, int r) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = w + WAVES * (U * r + u);
            const unsigned kb = c < nchunks ? (unsigned)(16 * c + 4 * q) * 4u : 0x80000000u;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                bf.w[u][nb] = ssm::bload16<float4>(rw, (unsigned)((16 * nb + l16) * K) * 4u + kb);
            bf.x[u] = ssm::bload16<float4>(rx, ox + kb);
            if (MODE == MODE_GATED) bf.z[u] = ssm::bload16<float4>(rz, oz + kb);
            if (MODE != MODE_PLAIN) bf.g[u] = ssm::bload16<float4>(rg, kb);
        }
    };
    auto compute = [&](const Buf& bf) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float4 p = bf.x[u];
            if (MODE == MODE_GATED) {
                p.x *= ssm::silu_fast(bf.z[u].x);
                p.y *= ssm::silu_fast(bf.z[u].y);
                p.z *= ssm::silu_fast(bf.z[u].z);
                p.w *= ssm::silu_fast(bf.z[u].w);
            }
            if (MODE != MODE_PLAIN) {
                ss = fmaf(p.x, p.x, ss);
                ss = fmaf(p.y, p.y, ss);
                ss = fmaf(p.z, p.z, ss);
                ss = fmaf(p.w, p.w, ss);
                p.x *= bf.g[u].x;
                p.y *= bf.g[u].y;
                p.z *= bf.g[u].z;
                p.w *= bf.g[u].w;
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc[nb] = mfma4(p.x, bf.w[u][nb].x, acc[nb]);
                acc[nb] = mfma4(p.y, bf.w[u][nb].y, acc[nb]);
                acc[nb] = mfma4(p.z, bf.w[u][nb].z, acc[nb]);
                acc[nb] = mfma4(p.w, bf.w[u][nb].w, acc[nb]);
            }
        }
    };
    // (a round past the last one loads and multiplies zeros: no branch breaks the counting)
    Buf ba, bb;
    load(ba, 0);
    for (int r = 0; r < rounds; r += 2) {
        load(bb, r + 1);
        compute(ba);
        load(ba, r + 2);
        compute(bb);
    }

    // ---- cross-wave reduction: partial tiles and row sums of squares through LDS
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) part[w][nb][lane] = acc[nb];
    if (MODE != MODE_PLAIN) {
        // lanes l, l^16, l^32, l^48 hold the same row's four k-slots
        float v = ss;
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        if (q == 0) ssq[w][l16] = v;
    }
    __syncthreads();
    // epilogue: wave nb finishes column block nb; lane holds rows m0 + 4q + r, column l16
    for (int nb = w; nb < NB; nb += WAVES) {
        floatx4 s = part[0][nb][lane];
#pragma unroll
        for (int v = 1; v < WAVES; ++v) s += part[v][nb][lane];
        const int n = n0 + 16 * nb + l16;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float scale = 1.f;
            if (MODE != MODE_PLAIN) {
                const float tot = ssq[0][4 * q + r] + ssq[1][4 * q + r] + ssq[2][4 * q + r] +
                                  ssq[3][4 * q + r];
                scale = rsqrtf(tot / (float)K + eps);
            }
            o[r] = s[r] * scale;
        }
        const bool col_ok = n < N;
        if (beta != 0.f) {
            float old[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 4 * q + r;
                old[r] = (m < M && col_ok) ? Y[(long)m * ldy + n] : 0.f;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = fmaf(beta, old[r], o[r]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 4 * q + r;
            if (m < M && col_ok) Y[(long)m * ldy + n] = o[r];
        }
    }
}

template <int MODE, int NB>
void launch(const float* X, long ldx, const float* Z, long ldz, const float* g, const float* W,
            float* Y, long ldy, int M, int N, int K, float beta, float eps, hipStream_t st) {
    const int rbs = (int)ssm::cdiv(M, 16);
    const int work = (int)(ssm::cdiv(N, 16 * NB) * rbs);
    const unsigned grid = (unsigned)(8 * ssm::cdiv(work, 8));
    rowgemm_kernel<MODE, NB><<<grid, 256, 0, st>>>(X, ldx, Z, ldz, g, W, Y, ldy, M, N, K, beta,
                                                    eps, rbs, work);
}

template <int MODE>
void pick(const float* X, long ldx, const float* Z, long ldz, const float* g, const float* W,
          float* Y, long ldy, int M, int N, int K, float beta, float eps, hipStream_t st) {
    // 32 columns per workgroup when that still gives about 512+ workgroups
    if ((long)ssm::cdiv(N, 32) * ssm::cdiv(M, 16) >= 512)
        launch<MODE, 2>(X, ldx, Z, ldz, g, W, Y, ldy, M, N, K, beta, eps, st);
    else
        launch<MODE, 1>(X, ldx, Z, ldz, g, W, Y, ldy, M, N, K, beta, eps, st);
}

}  // namespace

namespace ssm {

bool rowgemm_ok(int M, int N, int K) { return M >= 1 && M <= kRows && N >= 1 && K >= 16 && K % 16 == 0; }

ssm_status launch_rowgemm(int mode, const float* X, long ldx, const float* Z, long ldz,
                          const float* g, const float* W, float* Y, long ldy, int M, int N, int K,
                          float beta, float eps, hipStream_t st) {
    if (!rowgemm_ok(M, N, K))
        return fail(SSM_ERR_UNSUPPORTED, "row GEMM: need 1 <= M <= %d and K %% 16 == 0 (M=%d K=%d)",
                    kRows, M, K);
    // the kernel addresses X, Z and one workgroup's W rows with 32-bit byte offsets
    if ((long)M * ldx * 4 >= (1L << 31) || (long)M * ldz * 4 >= (1L << 31) ||
        (long)32 * K * 4 >= (1L << 31))
        return fail(SSM_ERR_UNSUPPORTED, "row GEMM: operands too large for 32-bit offsets");
    switch (mode) {
        case 0: pick<MODE_PLAIN>(X, ldx, Z, ldz, g, W, Y, ldy, M, N, K, beta, eps, st); break;
        case 1: pick<MODE_RMS>(X, ldx, Z, ldz, g, W, Y, ldy, M, N, K, beta, eps, st); break;
        default: pick<MODE_GATED>(X, ldx, Z, ldz, g, W, Y, ldy, M, N, K, beta, eps, st); break;
    }
    return check_launch("rowgemm");
}

}  // namespace ssm

extern "C" ssm_status ssm_linear_rows(int mode, const float* x, long ldx, const float* z, long ldz,
                                      const float* g, const float* W, float* y, long ldy, int M,
                                      int N, int K, float beta, float eps, void* stream) {
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
    return ssm::launch_rowgemm(mode, x, ldx, z, ldz, g, W, y, ldy, M, N, K, beta, eps,
                               (hipStream_t)stream);
}
