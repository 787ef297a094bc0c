// K2: Mamba-1 selective scan (Gu & Dao 2023, Algorithm 2) for gfx950, and its one-token
// decode update.
//
// Work split: one lane per channel d (64 adjacent channels per wave, so u/dt/z/y rows are
// read and written as 256-byte runs) holding all N state entries in registers (N is a
// template constant, so the state loop is straight-line code). B_t and C_t are the same for
// every channel: their addresses are wave-uniform and the pointers are read-only restrict
// parameters, so they are fetched with scalar loads into SGPRs. Time is cut into NC chunks
// so that B*D/64*NC waves fill the chip:
//   pass A  scan_chunk_state : each chunk from a zero state -> chunk-end state + sum(dt')
//   pass B  scan_chunk_prefix: per (b,n,d) sequential combine over chunks -> state entering
//                               each chunk (h_in[c] = exp(A*sum_dt[c-1]) h_in[c-1] + hend[c-1]),
//                               final state
//   pass C  scan_chunk_output: re-run each chunk from its entering state, emit y with the D
//                               skip and SiLU(z) gate.
// exp(dt A) is exp2(dt * (A log2 e)) with A pre-scaled once per lane (one v_exp_f32 each).
#include "common.hpp"

namespace {

constexpr int kWave = 64;
constexpr int kMinChunk = 16;
constexpr int kTargetWaves = 4096;

__device__ __forceinline__ float delta_of(float raw, float bias, int softplus) {
    const float v = raw + bias;
    return softplus ? ssm::softplus_sel(v) : v;
}

// Inner loops of both passes. Per step every lane loads its u / dt (/ z) element through a
// chunk-wide buffer descriptor (32-bit offsets; the prefetch one row past the chunk reads
// zeros instead of faulting) and the wave-uniform B_t row through scalar loads one step
// ahead (C_t's scalar load is issued at the top of its own step). `#pragma unroll 2` lets the compiler rename the carried registers instead of
// copying them back every step.
template <int N, bool EXACT>
struct Rows {
    const float* base;   // row 0 of the chunk
    long ld;
    int last;            // index of the chunk's last row
    int Nr;
    __device__ __forceinline__ void load(int k, float (&v)[N], const float (&msk)[N]) const {
        const float* r = base + (long)min(k, last) * ld;
#pragma unroll
        for (int n = 0; n < N; ++n) v[n] = EXACT ? r[n] : r[n < Nr ? n : Nr - 1] * msk[n];
    }
};

// N: state size the kernel is compiled for; Nr: runtime size (<= N). Entries n >= Nr get
// A = 0 and B = C = 0 (clamped loads times a zero mask), so they stay exactly zero and add
// nothing to y.
template <int N, bool EXACT>
__global__ __launch_bounds__(kWave) void scan_chunk_state(
    const float* __restrict__ u, long ldu, const float* __restrict__ dt, long lddt,
    const float* __restrict__ dt_bias, int softplus, const float* __restrict__ A,
    const float* __restrict__ Bm, long ldb, int L, int D, int Nr, int T, int NC,
    float* __restrict__ hc, float* __restrict__ sdt_out) {
    const int d = blockIdx.x * kWave + threadIdx.x;
    const int c = blockIdx.y, b = blockIdx.z;
    if (d >= D) return;
    if (EXACT) Nr = N;
    float A2[N], h[N], msk[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const int nn = EXACT ? n : (n < Nr ? n : Nr - 1);
        msk[n] = (EXACT || n < Nr) ? 1.f : 0.f;
        A2[n] = A[(long)d * Nr + nn] * ssm::kLog2e * msk[n];
        h[n] = 0.f;
    }
    const float bias = dt_bias ? dt_bias[d] : 0.f;
    const int t0 = c * T, steps = min(T, L - t0);
    const long r0 = (long)b * L + t0;
    const auto ru = ssm::rsrc(u + r0 * ldu, (unsigned)(((long)(steps - 1) * ldu + D) * 4));
    const auto rd = ssm::rsrc(dt + r0 * lddt, (unsigned)(((long)(steps - 1) * lddt + D) * 4));
    const unsigned su = (unsigned)ldu * 4u, sd = (unsigned)lddt * 4u;
    unsigned ou = (unsigned)d * 4u, od = (unsigned)d * 4u;
    const Rows<N, EXACT> Br{Bm + r0 * ldb, ldb, steps - 1, Nr};
    float sdt = 0.f;
    float dtv = ssm::bload4(rd, od), uv = ssm::bload4(ru, ou);
    float bc[N];
    Br.load(0, bc, msk);
#pragma unroll 2
    for (int k = 0; k < steps; ++k) {
        ou += su;
        od += sd;
        const float dtn = ssm::bload4(rd, od), un = ssm::bload4(ru, ou);
        float bn[N];
        Br.load(k + 1, bn, msk);
        const float dl = delta_of(dtv, bias, softplus);
        const float du = dl * uv;
        sdt += dl;
#pragma unroll
        for (int n = 0; n < N; ++n) h[n] = fmaf(ssm::ex2(dl * A2[n]), h[n], du * bc[n]);
        dtv = dtn;
        uv = un;
#pragma unroll
        for (int n = 0; n < N; ++n) bc[n] = bn[n];
    }
    float* hp = hc + (((long)b * NC + c) * Nr) * D + d;
#pragma unroll
    for (int n = 0; n < N; ++n)
        if (n < Nr) hp[(long)n * D] = h[n];
    sdt_out[((long)b * NC + c) * D + d] = sdt;
}

// One thread per (b, n, d); d fastest so the chunk-state rows are read coalesced.
__global__ void scan_chunk_prefix(const float* __restrict__ A, int L, int D, int N, int NC,
                                  long total, float* __restrict__ hc,
                                  const float* __restrict__ sdt, const float* __restrict__ h0,
                                  float* __restrict__ hT) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int d = (int)(i % D);
    const int n = (int)((i / D) % N);
    const int b = (int)(i / ((long)D * N));
    const float A2 = A[(long)d * N + n] * ssm::kLog2e;
    float carry = h0 ? h0[((long)b * D + d) * N + n] : 0.f;
    // the chunk-end states and dt sums of kPre chunks are loaded before the carry chain
    // consumes them (the chain itself has no memory latency in it)
    constexpr int kPre = 8;
    const long cstride = (long)N * D;
    float* p0 = hc + ((long)b * NC * N + n) * D + d;
    const float* s0 = sdt + (long)b * NC * D + d;
    for (int c0 = 0; c0 < NC; c0 += kPre) {
        float he[kPre], sd[kPre];
#pragma unroll
        for (int u = 0; u < kPre; ++u) {
            const bool live = c0 + u < NC;
            he[u] = live ? p0[(long)(c0 + u) * cstride] : 0.f;
            sd[u] = live ? s0[(long)(c0 + u) * D] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kPre; ++u) {
            if (c0 + u >= NC) break;
            p0[(long)(c0 + u) * cstride] = carry;
            carry = fmaf(ssm::ex2(A2 * sd[u]), carry, he[u]);
        }
    }
    if (hT) hT[((long)b * D + d) * N + n] = carry;
}

template <int N, bool EXACT>
__global__ __launch_bounds__(kWave) void scan_chunk_output(
    const float* __restrict__ u, long ldu, const float* __restrict__ dt, long lddt,
    const float* __restrict__ dt_bias, int softplus, const float* __restrict__ A,
    const float* __restrict__ Bm, long ldb, const float* __restrict__ Cm, long ldc,
    const float* __restrict__ Dsk, const float* __restrict__ z, long ldz, float* __restrict__ y,
    long ldy, int L, int D, int Nr, int T, int NC, const float* __restrict__ hc) {
    const int d = blockIdx.x * kWave + threadIdx.x;
    const int c = blockIdx.y, b = blockIdx.z;
    if (d >= D) return;
    if (EXACT) Nr = N;
    float A2[N], h[N], msk[N];
    const float* hp = hc + (((long)b * NC + c) * Nr) * D + d;
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const int nn = EXACT ? n : (n < Nr ? n : Nr - 1);
        msk[n] = (EXACT || n < Nr) ? 1.f : 0.f;
        A2[n] = A[(long)d * Nr + nn] * ssm::kLog2e * msk[n];
        h[n] = hp[(long)nn * D] * msk[n];
    }
    const float bias = dt_bias ? dt_bias[d] : 0.f;
    const float Dd = Dsk ? Dsk[d] : 0.f;
    const int t0 = c * T, steps = min(T, L - t0);
    const long r0 = (long)b * L + t0;
    const auto ru = ssm::rsrc(u + r0 * ldu, (unsigned)(((long)(steps - 1) * ldu + D) * 4));
    const auto rd = ssm::rsrc(dt + r0 * lddt, (unsigned)(((long)(steps - 1) * lddt + D) * 4));
    // without z the descriptor is empty: its loads read zeros and the gate is skipped
    const auto rz = ssm::rsrc(z ? z + r0 * ldz : u, z ? (unsigned)(((long)(steps - 1) * ldz + D) * 4) : 0u);
    const auto ry = ssm::rsrc(y + r0 * ldy, (unsigned)(((long)(steps - 1) * ldy + D) * 4));
    const unsigned su = (unsigned)ldu * 4u, sd = (unsigned)lddt * 4u,
                   sz = z ? (unsigned)ldz * 4u : 0u, sy = (unsigned)ldy * 4u;
    unsigned ou = (unsigned)d * 4u, od = ou, oz = ou, oy = ou;
    const Rows<N, EXACT> Br{Bm + r0 * ldb, ldb, steps - 1, Nr};
    const Rows<N, EXACT> Cr{Cm + r0 * ldc, ldc, steps - 1, Nr};
    float dtv = ssm::bload4(rd, od), uv = ssm::bload4(ru, ou), zv = ssm::bload4(rz, oz);
    float bc[N], cc[N];
    Br.load(0, bc, msk);
#pragma unroll 2
    for (int k = 0; k < steps; ++k) {
        ou += su;
        od += sd;
        oz += sz;
        const float dtn = ssm::bload4(rd, od), un = ssm::bload4(ru, ou), zn = ssm::bload4(rz, oz);
        float bn[N];
        Br.load(k + 1, bn, msk);   // B one step ahead; C (used after the state update) in-step
        Cr.load(k, cc, msk);
        const float dl = delta_of(dtv, bias, softplus);
        const float du = dl * uv;
        float acc = Dd * uv;
#pragma unroll
        for (int n = 0; n < N; ++n) {
            h[n] = fmaf(ssm::ex2(dl * A2[n]), h[n], du * bc[n]);
            acc = fmaf(h[n], cc[n], acc);
        }
        if (z) acc *= ssm::silu_fast(zv);
        ssm::bstore4(acc, ry, oy);
        oy += sy;
        dtv = dtn;
        uv = un;
        zv = zn;
#pragma unroll
        for (int n = 0; n < N; ++n) bc[n] = bn[n];
    }
}

int pick_chunk(int B, int L, int D) {
    const long waves_per_chunk = (long)B * ssm::cdiv(D, kWave);
    long nc = ssm::cdiv(kTargetWaves, waves_per_chunk > 0 ? waves_per_chunk : 1);
    long T = ssm::cdiv(L, nc > 0 ? nc : 1);
    if (T < kMinChunk) T = kMinChunk;
    return (int)T;
}

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
    int B, L, D, N, T, NC;
    float* hc;
    float* sdt;
    const float* h0;
    float* hT;
};

template <int N, bool EXACT>
void launch_all(const ScanArgs& a, hipStream_t st) {
    dim3 grid((unsigned)ssm::cdiv(a.D, kWave), (unsigned)a.NC, (unsigned)a.B);
    scan_chunk_state<N, EXACT><<<grid, kWave, 0, st>>>(a.u, a.ldu, a.dt, a.lddt, a.dt_bias, a.softplus,
                                                a.A, a.Bm, a.ldb, a.L, a.D, a.N, a.T, a.NC, a.hc,
                                                a.sdt);
    const long nthr = (long)a.B * a.N * a.D;
    scan_chunk_prefix<<<(unsigned)ssm::cdiv(nthr, 256), 256, 0, st>>>(
        a.A, a.L, a.D, a.N, a.NC, nthr, a.hc, a.sdt, a.h0, a.hT);
    scan_chunk_output<N, EXACT><<<grid, kWave, 0, st>>>(a.u, a.ldu, a.dt, a.lddt, a.dt_bias,
                                                 a.softplus, a.A, a.Bm, a.ldb, a.Cm, a.ldc,
                                                 a.Dsk, a.z, a.ldz, a.y, a.ldy, a.L, a.D, a.N,
                                                 a.T, a.NC, a.hc);
}

// One-token update: one thread per (b, d) with the N state entries in registers.
template <int N>
__global__ void m1_update_kernel(const float* __restrict__ x, long ldx,
                                 const float* __restrict__ dt, long lddt,
                                 const float* __restrict__ dt_bias, int softplus,
                                 const float* __restrict__ A, const float* __restrict__ Bm,
                                 long ldb, const float* __restrict__ Cm, long ldc,
                                 const float* __restrict__ Dsk, const float* __restrict__ z,
                                 long ldz, float* __restrict__ y, long ldy,
                                 float* __restrict__ h, int B, int D, int Nr, int vec) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * D) return;
    const int b = (int)(i / D), d = (int)(i % D);
    const float dl = delta_of(dt[(long)b * lddt + d], dt_bias ? dt_bias[d] : 0.f, softplus);
    const float xx = x[(long)b * ldx + d];
    const float du = dl * xx;
    float* hp = h + i * Nr;
    // per group of up to 16 states: all loads first, then the arithmetic. When the state
    // count is the template's and the rows are 16-byte aligned (vec), h and A come in float4
    // loads; otherwise from clamped (in-bounds) scalar indices. (Loads behind a per-n branch
    // were each waited for before the next.)
    constexpr int G = N < 16 ? N : 16;
    float acc = 0.f;
    if (Nr == N && vec) {
#pragma unroll
        for (int n0 = 0; n0 < N; n0 += G) {
            float hv[G], av[G], bv[G], cv[G];
#pragma unroll
            for (int q = 0; q < G; q += 4) {
                const float4 h4 = *reinterpret_cast<const float4*>(hp + n0 + q);
                const float4 a4 = *reinterpret_cast<const float4*>(A + (long)d * N + n0 + q);
                hv[q] = h4.x; hv[q + 1] = h4.y; hv[q + 2] = h4.z; hv[q + 3] = h4.w;
                av[q] = a4.x; av[q + 1] = a4.y; av[q + 2] = a4.z; av[q + 3] = a4.w;
            }
#pragma unroll
            for (int q = 0; q < G; ++q) {
                bv[q] = Bm[(long)b * ldb + n0 + q];
                cv[q] = Cm[(long)b * ldc + n0 + q];
            }
#pragma unroll
            for (int q = 0; q < G; q += 4) {
                float4 v;
                v.x = fmaf(ssm::ex2(dl * av[q] * ssm::kLog2e), hv[q], du * bv[q]);
                v.y = fmaf(ssm::ex2(dl * av[q + 1] * ssm::kLog2e), hv[q + 1], du * bv[q + 1]);
                v.z = fmaf(ssm::ex2(dl * av[q + 2] * ssm::kLog2e), hv[q + 2], du * bv[q + 2]);
                v.w = fmaf(ssm::ex2(dl * av[q + 3] * ssm::kLog2e), hv[q + 3], du * bv[q + 3]);
                *reinterpret_cast<float4*>(hp + n0 + q) = v;
                acc = fmaf(v.x, cv[q], acc);
                acc = fmaf(v.y, cv[q + 1], acc);
                acc = fmaf(v.z, cv[q + 2], acc);
                acc = fmaf(v.w, cv[q + 3], acc);
            }
        }
    } else
#pragma unroll
    for (int n0 = 0; n0 < N; n0 += G) {
        if (n0 >= Nr) break;
        float hv[G], av[G], bv[G], cv[G];
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int nn = n0 + q < Nr ? n0 + q : Nr - 1;
            hv[q] = hp[nn];
            av[q] = A[(long)d * Nr + nn];
            bv[q] = Bm[(long)b * ldb + nn];
            cv[q] = Cm[(long)b * ldc + nn];
        }
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const float v = fmaf(ssm::ex2(dl * av[q] * ssm::kLog2e), hv[q], du * bv[q]);
            if (n0 + q < Nr) {
                hp[n0 + q] = v;
                acc = fmaf(v, cv[q], acc);
            }
        }
    }
    if (Dsk) acc = fmaf(Dsk[d], xx, acc);
    if (z) acc *= ssm::silu_fast(z[(long)b * ldz + d]);
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
    switch (N) {
        case 4: launch_all<4, true>(a, st); break;
        case 8: launch_all<8, true>(a, st); break;
        case 16: launch_all<16, true>(a, st); break;
        case 32: launch_all<32, true>(a, st); break;
        case 64: launch_all<64, true>(a, st); break;
        default:
            if (N < 8) launch_all<8, false>(a, st);
            else if (N < 16) launch_all<16, false>(a, st);
            else if (N < 32) launch_all<32, false>(a, st);
            else launch_all<64, false>(a, st);
    }
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
    // float4 access to h and A rows when N is a template size and the rows are aligned
    const int vec = (N == 8 || N == 16 || N == 32 || N == 64) && (uintptr_t)h % 16 == 0 &&
                    (uintptr_t)A % 16 == 0;
#define M1U(NS)                                                                              \
    m1_update_kernel<NS><<<g, 256, 0, st>>>(x, ldx, dt, lddt, dt_bias, softplus, A, Bm, ldb, \
                                            Cm, ldc, Dsk, z, ldz, y, ldy, h, B, D, N, vec)
    if (N <= 8) M1U(8);
    else if (N <= 16) M1U(16);
    else if (N <= 32) M1U(32);
    else M1U(64);
#undef M1U
    return ssm::check_launch("m1_state_update");
}
