// K2: Mamba-1 selective scan (Gu & Dao 2023, Algorithm 2) for gfx950, and its one-token
// decode update.
//
// Work split: one lane per channel d (64 adjacent channels per wave, so u/dt/z/y rows are
// read and written as 256-byte runs) holding all N state entries in registers. B_t and C_t
// are the same for every channel, so their loads are wave-uniform and the compiler issues
// them as scalar loads. Time is cut into NC chunks so that B*D/64*NC waves fill the chip:
//   pass A  scan_chunk_state : each chunk from a zero state -> chunk-end state + sum(dt')
//   pass B  scan_chunk_prefix: per (b,n,d) sequential combine over chunks -> state entering
//                               each chunk (h_in[c] = exp(A*sum_dt[c-1]) h_in[c-1] + hend[c-1]),
//                               final state
//   pass C  scan_chunk_output: re-run each chunk from its entering state, emit y with the D
//                               skip and SiLU(z) gate.
// exp(dt A) is computed as exp2(dt * (A log2 e)) with A pre-scaled once per lane.
#include "common.hpp"

namespace {

constexpr int kWave = 64;
constexpr int kMinChunk = 16;
constexpr int kTargetWaves = 4096;

struct ScanArgs {
    const float* u; long ldu;
    const float* dt; long lddt;
    const float* dt_bias; int softplus;
    const float* A;
    const float* Bm; long ldb;
    const float* Cm; long ldc;
    const float* Dsk;
    const float* z; long ldz;
    float* y; long ldy;
    int B, L, D, N;
    int T;        // chunk length
    int NC;       // number of chunks
    float* hc;    // (B, NC, N, D): chunk-end state (pass A), then state entering chunk (pass B)
    float* sdt;   // (B, NC, D): sum of dt' over the chunk
    const float* h0;
    float* hT;
};

__device__ __forceinline__ float delta_at(const ScanArgs& a, long r, int d, float bias) {
    float v = a.dt[r * a.lddt + d] + bias;
    return a.softplus ? ssm::softplus(v) : v;
}

template <int NS>
__global__ __launch_bounds__(kWave) void scan_chunk_state(ScanArgs a) {
    const int d = blockIdx.x * kWave + threadIdx.x;
    const int c = blockIdx.y, b = blockIdx.z;
    if (d >= a.D) return;
    float A2[NS], h[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        A2[n] = n < a.N ? a.A[(long)d * a.N + n] * ssm::kLog2e : 0.f;
        h[n] = 0.f;
    }
    const float bias = a.dt_bias ? a.dt_bias[d] : 0.f;
    const int t0 = c * a.T, t1 = min(t0 + a.T, a.L);
    float sdt = 0.f;
    for (int t = t0; t < t1; ++t) {
        const long r = (long)b * a.L + t;
        const float dl = delta_at(a, r, d, bias);
        const float du = dl * a.u[r * a.ldu + d];
        sdt += dl;
        const float* Br = a.Bm + r * a.ldb;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < a.N) h[n] = fmaf(ssm::ex2(dl * A2[n]), h[n], du * Br[n]);
    }
    float* hc = a.hc + (((long)b * a.NC + c) * a.N) * a.D + d;
#pragma unroll
    for (int n = 0; n < NS; ++n)
        if (n < a.N) hc[(long)n * a.D] = h[n];
    a.sdt[((long)b * a.NC + c) * a.D + d] = sdt;
}

// One thread per (b, n, d); d fastest so the chunk-state rows are read coalesced.
__global__ void scan_chunk_prefix(ScanArgs a) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)a.B * a.N * a.D) return;
    const int d = (int)(i % a.D);
    const int n = (int)((i / a.D) % a.N);
    const int b = (int)(i / ((long)a.D * a.N));
    const float A2 = a.A[(long)d * a.N + n] * ssm::kLog2e;
    float carry = a.h0 ? a.h0[((long)b * a.D + d) * a.N + n] : 0.f;
    for (int c = 0; c < a.NC; ++c) {
        float* p = a.hc + (((long)b * a.NC + c) * a.N + n) * a.D + d;
        const float hend = *p;
        *p = carry;
        carry = fmaf(ssm::ex2(A2 * a.sdt[((long)b * a.NC + c) * a.D + d]), carry, hend);
    }
    if (a.hT) a.hT[((long)b * a.D + d) * a.N + n] = carry;
}

template <int NS>
__global__ __launch_bounds__(kWave) void scan_chunk_output(ScanArgs a) {
    const int d = blockIdx.x * kWave + threadIdx.x;
    const int c = blockIdx.y, b = blockIdx.z;
    if (d >= a.D) return;
    float A2[NS], h[NS];
    const float* hc = a.hc + (((long)b * a.NC + c) * a.N) * a.D + d;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        A2[n] = n < a.N ? a.A[(long)d * a.N + n] * ssm::kLog2e : 0.f;
        h[n] = n < a.N ? hc[(long)n * a.D] : 0.f;
    }
    const float bias = a.dt_bias ? a.dt_bias[d] : 0.f;
    const float Dd = a.Dsk ? a.Dsk[d] : 0.f;
    const int t0 = c * a.T, t1 = min(t0 + a.T, a.L);
    for (int t = t0; t < t1; ++t) {
        const long r = (long)b * a.L + t;
        const float dl = delta_at(a, r, d, bias);
        const float uu = a.u[r * a.ldu + d];
        const float du = dl * uu;
        const float* Br = a.Bm + r * a.ldb;
        const float* Cr = a.Cm + r * a.ldc;
        float acc = 0.f;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < a.N) {
                h[n] = fmaf(ssm::ex2(dl * A2[n]), h[n], du * Br[n]);
                acc = fmaf(h[n], Cr[n], acc);
            }
        acc = fmaf(Dd, uu, acc);
        if (a.z) acc *= ssm::silu(a.z[r * a.ldz + d]);
        a.y[r * a.ldy + d] = acc;
    }
}

int pick_chunk(int B, int L, int D) {
    const long waves_per_chunk = (long)B * ssm::cdiv(D, kWave);
    long nc = ssm::cdiv(kTargetWaves, waves_per_chunk > 0 ? waves_per_chunk : 1);
    long T = ssm::cdiv(L, nc > 0 ? nc : 1);
    if (T < kMinChunk) T = kMinChunk;
    return (int)T;
}

template <int NS>
void launch_all(ScanArgs& a, hipStream_t st) {
    dim3 grid((unsigned)ssm::cdiv(a.D, kWave), (unsigned)a.NC, (unsigned)a.B);
    scan_chunk_state<NS><<<grid, kWave, 0, st>>>(a);
    const long nthr = (long)a.B * a.N * a.D;
    scan_chunk_prefix<<<(unsigned)ssm::cdiv(nthr, 256), 256, 0, st>>>(a);
    scan_chunk_output<NS><<<grid, kWave, 0, st>>>(a);
}

// One-token update: one thread per (b, d) with the N state entries in registers.
template <int NS>
__global__ void m1_update_kernel(const float* __restrict__ x, long ldx,
                                 const float* __restrict__ dt, long lddt,
                                 const float* __restrict__ dt_bias, int softplus,
                                 const float* __restrict__ A, const float* __restrict__ Bm,
                                 long ldb, const float* __restrict__ Cm, long ldc,
                                 const float* __restrict__ Dsk, const float* __restrict__ z,
                                 long ldz, float* __restrict__ y, long ldy,
                                 float* __restrict__ h, int B, int D, int N) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * D) return;
    const int b = (int)(i / D), d = (int)(i % D);
    float dl = dt[(long)b * lddt + d] + (dt_bias ? dt_bias[d] : 0.f);
    if (softplus) dl = ssm::softplus(dl);
    const float xx = x[(long)b * ldx + d];
    const float du = dl * xx;
    float* hp = h + i * N;
    float acc = 0.f;
#pragma unroll
    for (int n = 0; n < NS; ++n)
        if (n < N) {
            const float v = fmaf(ssm::ex2(dl * A[(long)d * N + n] * ssm::kLog2e), hp[n],
                                 du * Bm[(long)b * ldb + n]);
            hp[n] = v;
            acc = fmaf(v, Cm[(long)b * ldc + n], acc);
        }
    if (Dsk) acc = fmaf(Dsk[d], xx, acc);
    if (z) acc *= ssm::silu(z[(long)b * ldz + d]);
    y[(long)b * ldy + d] = acc;
}

}  // namespace

extern "C" size_t ssm_selective_scan_workspace(int B, int L, int D, int N) {
    if (B <= 0 || L <= 0 || D <= 0 || N <= 0) return 0;
    const int T = pick_chunk(B, L, D);
    const long NC = ssm::cdiv(L, T);
    return sizeof(float) * (size_t)B * NC * D * ((size_t)N + 1);
}

extern "C" ssm_status ssm_selective_scan(const float* u, long ldu, const float* dt, long lddt,
                                         const float* dt_bias, int softplus, const float* A,
                                         const float* Bm, long ldb, const float* Cm, long ldc,
                                         const float* Dsk, const float* z, long ldz, float* y,
                                         long ldy, int B, int L, int D, int N, const float* h0,
                                         float* hT, void* workspace, size_t workspace_bytes,
                                         void* stream) {
    SSM_REQUIRE(u && dt && A && Bm && Cm && y, "ssm_selective_scan: null input");
    SSM_REQUIRE(B >= 0 && L >= 0 && D >= 0 && N >= 1 && N <= 64,
                "ssm_selective_scan: need 1 <= N <= 64 (got %d)", N);
    SSM_REQUIRE(ldu >= D && lddt >= D && ldy >= D && ldb >= N && ldc >= N &&
                    (!z || ldz >= D),
                "ssm_selective_scan: row stride below row width");
    if (B == 0 || D == 0) return SSM_OK;
    if (L == 0) {
        if (hT) {
            if (h0) SSM_HIP_TRY(hipMemcpyAsync(hT, h0, sizeof(float) * (size_t)B * D * N,
                                                hipMemcpyDeviceToDevice, (hipStream_t)stream));
            else SSM_HIP_TRY(hipMemsetAsync(hT, 0, sizeof(float) * (size_t)B * D * N,
                                            (hipStream_t)stream));
        }
        return SSM_OK;
    }
    const size_t need = ssm_selective_scan_workspace(B, L, D, N);
    SSM_REQUIRE(workspace && workspace_bytes >= need,
                "ssm_selective_scan: workspace of %zu bytes needed", need);
    ScanArgs a;
    a.u = u; a.ldu = ldu; a.dt = dt; a.lddt = lddt; a.dt_bias = dt_bias; a.softplus = softplus;
    a.A = A; a.Bm = Bm; a.ldb = ldb; a.Cm = Cm; a.ldc = ldc; a.Dsk = Dsk; a.z = z; a.ldz = ldz;
    a.y = y; a.ldy = ldy; a.B = B; a.L = L; a.D = D; a.N = N;
    a.T = pick_chunk(B, L, D);
    a.NC = (int)ssm::cdiv(L, a.T);
    a.hc = (float*)workspace;
    a.sdt = a.hc + (size_t)B * a.NC * N * D;
    a.h0 = h0; a.hT = hT;
    hipStream_t st = (hipStream_t)stream;
    if (N <= 8) launch_all<8>(a, st);
    else if (N <= 16) launch_all<16>(a, st);
    else if (N <= 32) launch_all<32>(a, st);
    else launch_all<64>(a, st);
    return ssm::check_launch("selective_scan");
}

extern "C" ssm_status ssm_m1_state_update(const float* x, long ldx, const float* dt, long lddt,
                                          const float* dt_bias, int softplus, const float* A,
                                          const float* Bm, long ldb, const float* Cm, long ldc,
                                          const float* Dsk, const float* z, long ldz, float* y,
                                          long ldy, float* h, int B, int D, int N,
                                          void* stream) {
    SSM_REQUIRE(x && dt && A && Bm && Cm && y && h, "ssm_m1_state_update: null input");
    SSM_REQUIRE(B >= 0 && D >= 0 && N >= 1 && N <= 64, "ssm_m1_state_update: need N <= 64");
    if (B == 0 || D == 0) return SSM_OK;
    const long n = (long)B * D;
    const unsigned g = (unsigned)ssm::cdiv(n, 256);
    hipStream_t st = (hipStream_t)stream;
#define M1U(NS)                                                                              \
    m1_update_kernel<NS><<<g, 256, 0, st>>>(x, ldx, dt, lddt, dt_bias, softplus, A, Bm, ldb, \
                                            Cm, ldc, Dsk, z, ldz, y, ldy, h, B, D, N)
    if (N <= 8) M1U(8);
    else if (N <= 16) M1U(16);
    else if (N <= 32) M1U(32);
    else M1U(64);
#undef M1U
    return ssm::check_launch("m1_state_update");
}
