// K2: Mamba-1 selective scan (Gu & Dao 2023, Algorithm 2) for gfx950, and its one-token
// decode update. Two designs, chosen by how many waves the channels alone give:
//
// Single pass (scan_single_kernel, when B * D * N / 64 waves give every SIMD one): lane
// (c, n) holds state h[d, n] in a register and walks the whole sequence once; the inputs of
// a 64- or 128-step block are staged in LDS by the workgroup, and the per-step outputs
// y = C_t . h_t are reduced over the N lanes of a channel through LDS. One v_exp_f32 per
// (t, d, n); no intermediate state leaves the CU. Its own description is below.
//
// Chunked (when the channels are too few, e.g. one sequence of 512 channels): one lane per
// channel d (64 adjacent channels per wave, so u/dt/z/y rows are read and written as 256-byte
// runs) holding all N state entries in registers (N is a template constant, so the state loop
// is straight-line code). B_t and C_t are the same for every channel: their addresses are
// wave-uniform and the pointers are read-only restrict parameters, so they are fetched with
// scalar loads into SGPRs. Time is cut into NC chunks so that B*D/64*NC waves fill the chip:
//   pass A  scan_chunk_state : each chunk from a zero state -> chunk-end state + sum(dt')
//   pass B  scan_chunk_prefix: per (b,n,d) sequential combine over chunks -> state entering
//                               each chunk (h_in[c] = exp(A*sum_dt[c-1]) h_in[c-1] + hend[c-1]),
//                               final state
//   pass C  scan_chunk_output: re-run each chunk from its entering state, emit y with the D
//                               skip and SiLU(z) gate.
// exp(dt A) is exp2(dt * (A log2 e)) with A pre-scaled once per lane (one v_exp_f32 each).
#include <algorithm>

#include "common.hpp"
#include "glue.hpp"

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
    long ldy, int L, int D, int Nr, int T, int NC, const float* __restrict__ hc, int zgated) {
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
        if (z) acc *= zgated ? zv : ssm::silu_fast(zv);
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
    int zgated;          // z already holds silu(z) (written so by its producer)
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
                                                 a.T, a.NC, a.hc, a.zgated);
}

// ---------------------------------------------------------------- single-pass scan
// When the channels alone give every SIMD a wave, the whole sequence is walked once and each
// exp(dt A) is evaluated once (the chunked passes above evaluate it twice: a v_exp_f32 costs
// about three FMAs on this chip and does not overlap them, so that second evaluation is the
// larger part of their cost).
//
// Lane (c, n) of a wave holds the state h[d, n] of channel d = c0 + c in a register, with
// 64 / N channels per wave and N lanes per channel; a workgroup of W waves covers CW adjacent
// channels of one sequence b. The sequence goes by in blocks of TK = 64 or 128 steps:
//   staging  the block's u, dt, z (TK x CW) and B_t, C_t rows (TK x N), loaded one block
//            ahead into registers, go to LDS as dt' = softplus(dt + bias), dt' u, silu(z),
//            D u, B and C;
//   then, per sub-block of SB = N steps:
//   scan     lane (c, n), each step: h = exp2(dt' A log2 e) h + dt' u B_t[n]; h goes to LDS;
//   output   lane (c, t) of the same wave: y = (sum_n h_t[c, n] C_t[n] + D u) silu(z);
//   and the block's outputs are stored by the workgroup as whole rows of CW channels.
// The scan's inner step is one multiply, one v_exp_f32, one multiply and one FMA per (t, d, n)
// and the output's one FMA; only the final state goes to memory. State entries n >= Nr have
// A = 0 and B = C = 0 and stay exactly zero.
template <int N>
struct Scan1 {
    static constexpr int W = (N == 4 || N == 64) ? 4 : 8;   // waves (LDS <= 110 KB)
    static constexpr int CPW = 64 / N;     // channels per wave
    static constexpr int CW = W * CPW;     // channels per workgroup
    // steps per block: the block's loads are issued one block ahead, so a block's work must
    // outlast a memory latency under load (a 64-step block at N = 16, about 1.2 us of
    // arithmetic, measured latency-bound); 128 where the LDS (160 KB) holds it
    static constexpr int TK = N >= 16 ? 128 : 64;
    static constexpr int SB = N;           // steps per output sub-block (64 lanes = CPW x SB)
    static constexpr int NT = 64 * W;      // threads
    static constexpr int UE = TK * CW / NT;        // u/dt/z values per thread and block
    static constexpr int BE = (TK * N + NT - 1) / NT;   // B (and C) values per thread and block
    // Row paddings keep the LDS accesses free of bank conflicts (32 banks): [channel][step]
    // rows are read as one float per lane for N = 16 (odd pitch) and as float4 otherwise.
    static constexpr int PD = N == 16 ? TK + 1 : TK + 4;
    static constexpr int PT = TK + 4;      // [n][step] rows (float4 reads)
    static constexpr int PC = CW + 1;      // [step][channel] rows
    static constexpr int RR = CW * N + 4;  // padded row of one step's states
    struct Smem {
        float dl[CW][PD], du[CW][PD];      // dt', dt' u
        float bt[N][PT];                   // B_t[n]
        float ct[TK][N + 4];               // C_t[n]
        float gz[TK][PC], dx[TK][PC];      // silu(z), D u
        float red[SB][RR];                 // h_t[c, n] of one sub-block
        float ys[TK][PC];                  // outputs
    };
};

// Value of lane j of this lane's 16-lane row (DPP row_newbcast); as an operand of a VALU
// instruction the compiler folds it into that instruction.
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + J, 0xF, 0xF, true));
}

// Value of lane q ^ X of this lane's quad (DPP quad_perm), folded into its user.
template <int X>
__device__ __forceinline__ float quad_xor(float v) {
    constexpr int ctrl = X == 1 ? 0xB1 : 0x4E;   // quad_perm [1,0,3,2] / [2,3,0,1]
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, true));
}

template <int N, bool EXACT>
__global__ __launch_bounds__(64 * Scan1<N>::W) void scan_single_kernel(ScanArgs a) {
    using S = Scan1<N>;
    constexpr int CPW = S::CPW, CW = S::CW, TK = S::TK, SB = S::SB, NT = S::NT, UE = S::UE,
                  BE = S::BE;
    __shared__ __attribute__((aligned(16))) typename S::Smem sm;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b = blockIdx.y, c0 = blockIdx.x * CW;
    const int D = a.D, L = a.L, Nr = EXACT ? N : a.N;

    // scan lane: channel cl of the workgroup, state n
    const int cl = w * CPW + lane / N, n = lane % N;
    const int d = c0 + cl;
    const bool live = d < D && n < Nr;
    const float A2 = live ? a.A[(long)d * Nr + n] * ssm::kLog2e : 0.f;
    float h = (live && a.h0) ? a.h0[((long)b * D + d) * Nr + n] : 0.f;
    // output lane: channel cl2 of the workgroup (of this wave), step ot of the sub-block
    const int cl2 = w * CPW + lane / SB, ot = lane % SB;
    // staging elements: channel sc (fixed per thread: NT is a multiple of CW), steps
    // st0 + e * (NT / CW)
    constexpr int SR = NT / CW;            // steps covered by one pass of the threads
    const int sc = tid % CW, st0 = tid / CW, sd = c0 + sc;
    const bool sdok = sd < D;
    const float bias = (sdok && a.dt_bias) ? a.dt_bias[sd] : 0.f;
    const float Dd = (sdok && a.Dsk) ? a.Dsk[sd] : 0.f;
    const float spf = a.softplus ? 1.f : 0.f, gzf = a.z ? 1.f : 0.f;

    // Descriptors of block k (rows k TK .. k TK + TK - 1 of sequence b), rebuilt per block
    // from wave-uniform values so that every offset stays within 32 bits however long the
    // sequence is (the host checks TK rows of the widest stride fit): rows past L, and every
    // row of the block past the last, read zeros and take no stores.
    const long r0 = (long)b * L;
    auto blk = [&](const float* p, long ld, int width, int k) {
        const int rows = min(TK, L - k * TK);
        return rows > 0 ? ssm::rsrc(p + (r0 + (long)k * TK) * ld,
                                    (unsigned)(((long)(rows - 1) * ld + width) * 4))
                        : ssm::rsrc(p, 0u);
    };
    const float* zp = a.z ? a.z : a.u;
    const long ldz = a.z ? a.ldz : 0;

    // Block k's values of this thread, loaded one block ahead. The offsets carry no select
    // (a lane-dependent `cond ? offset : out-of-range` was split by the compiler into two
    // branches, each with its own load, whose join waited for every load in flight): rows
    // past the block's last read zeros through the descriptor's range, and a channel past D
    // or a state past Nr reads some in-range value that the staging never uses.
    float uv[UE], dv[UE], zv[UE], bv[BE], cv[BE];
    auto load = [&](int k) {
        const auto ru = blk(a.u, a.ldu, D, k), rd = blk(a.dt, a.lddt, D, k);
        const auto rz = a.z ? blk(zp, ldz, D, k) : ssm::rsrc(zp, 0u);
        const auto rb = blk(a.Bm, a.ldb, Nr, k), rc = blk(a.Cm, a.ldc, Nr, k);
#pragma unroll
        for (int e = 0; e < UE; ++e) {
            const unsigned t = (unsigned)(st0 + e * SR);
            uv[e] = ssm::bload4(ru, (t * (unsigned)a.ldu + (unsigned)sd) * 4u);
            dv[e] = ssm::bload4(rd, (t * (unsigned)a.lddt + (unsigned)sd) * 4u);
            zv[e] = ssm::bload4(rz, (t * (unsigned)ldz + (unsigned)sd) * 4u);
        }
#pragma unroll
        for (int j = 0; j < BE; ++j) {
            const int i = (tid + NT * j) % (TK * N), nn = i % N;
            const unsigned t = (unsigned)(i / N);
            bv[j] = ssm::bload4(rb, (t * (unsigned)a.ldb + (unsigned)nn) * 4u);
            cv[j] = ssm::bload4(rc, (t * (unsigned)a.ldc + (unsigned)nn) * 4u);
        }
    };

    const int nblk = (L + TK - 1) / TK;
    load(0);
    for (int k = 0; k < nblk; ++k) {
        // staging (no data-dependent branch: the flags blend arithmetically)
#pragma unroll
        for (int e = 0; e < UE; ++e) {
            const int st = st0 + e * SR;
            const float ok = (sdok && k * TK + st < L) ? 1.f : 0.f;   // past L: dt' = 0
            const float raw = dv[e] + bias;
            const float dl = ok * (spf * ssm::softplus_sel(raw) + (1.f - spf) * raw);
            sm.dl[sc][st] = dl;
            sm.du[sc][st] = dl * uv[e];
            sm.gz[st][sc] = a.zgated ? (a.z ? zv[e] : 1.f) : fmaf(gzf, ssm::silu_fast(zv[e]) - 1.f, 1.f);
            sm.dx[st][sc] = Dd * uv[e];
        }
#pragma unroll
        for (int j = 0; j < BE; ++j) {
            // threads past the block's TK x N values repeat the first ones (the same value to
            // the same place), so no thread branches around its write
            const int i = (tid + NT * j) % (TK * N);
            const float nm = (EXACT || i % N < Nr) ? 1.f : 0.f;
            sm.bt[i % N][i / N] = nm * bv[j];
            sm.ct[i / N][i % N] = nm * cv[j];
        }
        load(k + 1);   // the next block's loads have this whole block to arrive
        __syncthreads();
#pragma unroll 1
        for (int s0 = 0; s0 < TK; s0 += SB) {
            if constexpr (N == 16) {
                // A channel's 16 lanes are one DPP row: lane (c, j) fetches dt' and dt' u of
                // step s0 + j and step j broadcasts them across the row, inside the multiplies;
                // B_t[n] of the 16 steps comes in four float4 reads.
                const float dlr = sm.dl[cl][s0 + n], dur = sm.du[cl][s0 + n];
                float bq[16];
#pragma unroll
                for (int q = 0; q < 16; q += 4) {
                    const float4 b4 = *reinterpret_cast<const float4*>(&sm.bt[n][s0 + q]);
                    bq[q] = b4.x; bq[q + 1] = b4.y; bq[q + 2] = b4.z; bq[q + 3] = b4.w;
                }
#define SCAN_STEP(J)                                                                         \
                h = fmaf(ssm::ex2(row_bcast<J>(dlr) * A2), h, row_bcast<J>(dur) * bq[J]);   \
                sm.red[J][cl * N + n] = h;
                SCAN_STEP(0) SCAN_STEP(1) SCAN_STEP(2) SCAN_STEP(3)
                SCAN_STEP(4) SCAN_STEP(5) SCAN_STEP(6) SCAN_STEP(7)
                SCAN_STEP(8) SCAN_STEP(9) SCAN_STEP(10) SCAN_STEP(11)
                SCAN_STEP(12) SCAN_STEP(13) SCAN_STEP(14) SCAN_STEP(15)
#undef SCAN_STEP
            } else {
                // four steps per LDS read
#pragma unroll
                for (int t4 = 0; t4 < SB; t4 += 4) {
                    const float4 dl4 = *reinterpret_cast<const float4*>(&sm.dl[cl][s0 + t4]);
                    const float4 du4 = *reinterpret_cast<const float4*>(&sm.du[cl][s0 + t4]);
                    const float4 b4 = *reinterpret_cast<const float4*>(&sm.bt[n][s0 + t4]);
                    h = fmaf(ssm::ex2(dl4.x * A2), h, du4.x * b4.x);
                    sm.red[t4][cl * N + n] = h;
                    h = fmaf(ssm::ex2(dl4.y * A2), h, du4.y * b4.y);
                    sm.red[t4 + 1][cl * N + n] = h;
                    h = fmaf(ssm::ex2(dl4.z * A2), h, du4.z * b4.z);
                    sm.red[t4 + 2][cl * N + n] = h;
                    h = fmaf(ssm::ex2(dl4.w * A2), h, du4.w * b4.w);
                    sm.red[t4 + 3][cl * N + n] = h;
                }
            }
            // output: the same wave's states, one (channel, step) per lane
            float acc = sm.dx[s0 + ot][cl2];
#pragma unroll
            for (int q = 0; q < N; q += 4) {
                const float4 r4 = *reinterpret_cast<const float4*>(&sm.red[ot][cl2 * N + q]);
                const float4 c4 = *reinterpret_cast<const float4*>(&sm.ct[s0 + ot][q]);
                acc = fmaf(r4.x, c4.x, acc);
                acc = fmaf(r4.y, c4.y, acc);
                acc = fmaf(r4.z, c4.z, acc);
                acc = fmaf(r4.w, c4.w, acc);
            }
            sm.ys[s0 + ot][cl2] = acc * sm.gz[s0 + ot][cl2];
        }
        __syncthreads();
        const auto ry = blk(a.y, a.ldy, D, k);
#pragma unroll
        for (int e = 0; e < UE; ++e) {
            // rows past L fall outside the descriptor (dropped); so does a channel past D
            const int st = st0 + e * SR;
            const unsigned off = ((unsigned)st * (unsigned)a.ldy + (unsigned)sd) * 4u;
            ssm::bstore4(sm.ys[st][sc], ry, off | (sdok ? 0u : 0x80000000u));
        }
    }
    if (live && a.hT) a.hT[((long)b * D + d) * Nr + n] = h;
}

// ---------------------------------------------------------------- single pass, N = 16
// The same walk for N = 16, laid out for the LDS of gfx950, which serves a ds_read_b128 16
// lanes (256 bytes, all 64 banks) at a time at about 1 KB per 1.8 ns per CU while writes
// cost three to four times as much per byte; the design keeps LDS writes to one per staged
// value and one per state, with every access touching distinct banks:
//   staging  per block of TK steps the workgroup loads u, dt, z as whole rows of its CW
//            channels (and B_t, C_t), one block ahead, and writes one float4 {dt', dt' u,
//            silu(z), D u} per (step, channel), dt' = softplus(dt + bias) (slots XOR-swizzled
//            by the step so that 16 steps of one channel fall in 16 bank groups). The Mamba-1
//            block hands over dt' and silu(z) already formed by their producers (zgated, no
//            bias, no softplus), which takes the transcendentals out of this kernel;
//   scan     lane (c, j) reads the float4 of step s0 + j of its channel; lane (c, n) then
//            takes dt' and dt' u of step J from lane J of the channel's row (row_newbcast
//            inside the multiplies): h = exp2(dt' A log2 e) h + dt' u B_t[n] for 16 steps,
//            B_t[n] of the 16 steps in four ds_read_b128;
//   output   the 16 states per lane go to the wave's own LDS region in four ds_write_b128
//            (4 steps each, slots XOR-swizzled by the step quad so that both the writes and
//            the reads below touch 64 different banks per 16 lanes); lane (c, tq, nq) reads
//            the 4 x 4 (step, state) block t = 4 tq .. 4 tq + 3, n = 4 nq .. 4 nq + 3 and the
//            matching C, forms 4 partial sums (independent FMA chains) and reduces them over
//            the 4 lanes of its quad (two DPP exchange levels). Lane (c, tq, nq) ends with the
//            sum of step 4 tq + nq = j: the lane that read that step's gate and skip term,
//            so y = (sum + D u) silu(z) is formed and stored there.
// Staging buffers are double-buffered, so a block needs one barrier; within a block each
// sub-block's output reduction is issued next to the following sub-block's scan. The sum over
// n runs as four sums of 4 states added pairwise across the quad (the oracle adds the 16 in
// order; the fp32 rounding differs only).
template <int W>
struct ScanW16 {
    static constexpr int CW = 4 * W;     // channels per workgroup (4 per wave)
    static constexpr int TK = 64;        // steps per block
    static constexpr int NSB = TK / 16;  // sub-blocks of 16 steps per block
    // Every wave stages a share of each block. (Staging on only the two waves that are alone
    // on a SIMD, waves 2 and 3 of a six-wave group, measured slower: their share became the
    // block's critical path.)
    static constexpr int NST = 64 * W;                   // staging threads
    static constexpr int UE = TK * CW / NST;             // staged (step, channel) per thread
    static constexpr int BE = (TK * 16 + NST - 1) / NST; // B (and C) values per thread
    static constexpr int SW = (CW + 15) / 16 * 16;       // slots per staged row
    static constexpr int PB = TK + 4;    // [n][t] rows: n rows 4 banks apart
    static constexpr int PC = 20;        // [t][n] rows: t rows 20 banks apart
    struct Smem {
        float4 sx[2][TK][SW];            // {dt', dt' u, silu(z), D u}, slot c ^ (t % 16)
        float bt[2][16][PB];             // B_t[n]
        float ct[2][TK][PC];             // C_t[n]
        float hx[W][1024];               // each wave's states of one sub-block
        float2 par[CW];                  // dt bias, D of the workgroup's channels
    };
};

template <int W>
__global__ __launch_bounds__(64 * W) void scan_w16_kernel(ScanArgs a) {
    using S = ScanW16<W>;
    constexpr int TK = S::TK, NSB = S::NSB, NST = S::NST, BE = S::BE, UE = S::UE, CW = S::CW;
    static_assert((TK * CW) % NST == 0, "staging layout");
    __shared__ __attribute__((aligned(16))) typename S::Smem sm;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = lane >> 4, j = lane & 15;
    // Workgroups go to the 8 XCDs round-robin by id; XCD x takes the x-th contiguous run of
    // (sequence, channel block) tiles, so that the channel blocks sharing a row's 128-byte
    // lines (CW * 4 bytes need not be a whole line) mostly share one L2.
    const int nwg = (int)gridDim.x, nb = (a.D + CW - 1) / CW;
    const int xcd = blockIdx.x % 8, q = nwg / 8, rem = nwg % 8;
    const int tile = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + blockIdx.x / 8;
    const int b = tile / nb, c0 = (tile % nb) * CW;
    const int D = a.D, L = a.L;
    const int cw = 4 * w + c;            // this lane's channel within the workgroup
    const int d = c0 + cw;
    const bool dok = d < D;
    const unsigned dmask = dok ? 0u : 0x80000000u;   // a channel past D stores nothing
    const float A2 = a.A[(long)(dok ? d : D - 1) * 16 + j] * ssm::kLog2e;
    float h = (dok && a.h0) ? a.h0[((long)b * D + d) * 16 + j] : 0.f;
    if (tid < CW) {
        const int pd = min(c0 + tid, D - 1);
        sm.par[tid] = make_float2(a.dt_bias ? a.dt_bias[pd] : 0.f, a.Dsk ? a.Dsk[pd] : 0.f);
    }
    // staging thread st: elements i = st + NST e, step i / CW, channel i % CW
    const int st = tid;

    // rows k TK .. k TK + TK - 1 of sequence b through a descriptor rebuilt per block
    // (32-bit offsets however long the sequence); rows past L read zeros, take no stores
    const long r0 = (long)b * L;
    auto blk = [&](const float* p, long ld, int width, int k) {
        const int rows = min(TK, L - k * TK);
        return rows > 0 ? ssm::rsrc(p + (r0 + (long)k * TK) * ld,
                                    (unsigned)(((long)(rows - 1) * ld + width) * 4))
                        : ssm::rsrc(p, 0u);
    };
    // block k's values of this staging thread, loaded one block ahead (a channel past D reads
    // the last channel's value, never used; rows past the last read zeros)
    float uv[UE], dv[UE], zv[UE], bv[BE], cv[BE];
    auto load = [&](int k) {
        const auto ru = blk(a.u, a.ldu, D, k), rd = blk(a.dt, a.lddt, D, k);
        const auto rz = a.z ? blk(a.z, a.ldz, D, k) : ssm::rsrc(a.u, 0u);
        const auto rb = blk(a.Bm, a.ldb, 16, k), rc = blk(a.Cm, a.ldc, 16, k);
#pragma unroll
        for (int e = 0; e < UE; ++e) {
            const int i = st + NST * e;
            const unsigned t = (unsigned)(i / CW), sd = (unsigned)min(c0 + i % CW, D - 1);
            uv[e] = ssm::bload4(ru, (t * (unsigned)a.ldu + sd) * 4u);
            dv[e] = ssm::bload4(rd, (t * (unsigned)a.lddt + sd) * 4u);
            zv[e] = ssm::bload4(rz, (t * (unsigned)a.ldz + sd) * 4u);
        }
#pragma unroll
        for (int e = 0; e < BE; ++e) {
            // value i = step i / 16, state i % 16; threads past the block's values repeat the
            // first ones (the same value to the same place)
            const int i = (st + NST * e) % (TK * 16);
            const unsigned t = (unsigned)(i >> 4), nn = (unsigned)(i & 15);
            bv[e] = ssm::bload4(rb, (t * (unsigned)a.ldb + nn) * 4u);
            cv[e] = ssm::bload4(rc, (t * (unsigned)a.ldc + nn) * 4u);
        }
    };
    auto stage = [&](int k, int buf) {
#pragma unroll
        for (int e = 0; e < UE; ++e) {
            const int i = st + NST * e, t = i / CW, sc = i % CW;
            const float2 pr = sm.par[sc];
            float dl = dv[e] + pr.x;
            if (a.softplus) dl = ssm::softplus_sel(dl);
            dl = (k * TK + t < L) ? dl : 0.f;            // past L: dt' = 0, the state is kept
            const float gz = a.z ? (a.zgated ? zv[e] : ssm::silu_fast(zv[e])) : 1.f;
            sm.sx[buf][t][sc ^ (t & 15)] = make_float4(dl, dl * uv[e], gz, pr.y * uv[e]);
        }
#pragma unroll
        for (int e = 0; e < BE; ++e) {
            const int i = (st + NST * e) % (TK * 16);
            sm.bt[buf][i & 15][i >> 4] = bv[e];
            sm.ct[buf][i >> 4][i & 15] = cv[e];
        }
    };

    float* hw = sm.hx[w];
    const int tq = j >> 2, nq = j & 3;
    const bool x2 = (nq & 2) != 0, x1 = (nq & 1) != 0;
    const int nblk = (L + TK - 1) / TK;
    __syncthreads();                     // par
    load(0);
    stage(0, 0);
    load(1);
    __syncthreads();
    for (int k = 0; k < nblk; ++k) {
        const int buf = k & 1;
        // fill the other buffer (last read in block k - 1, which every wave finished before
        // the previous barrier) and issue the loads of the block after it
        stage(k + 1, buf ^ 1);           // past the last block: zeros, never read
        load(k + 2);
        const auto ry = blk(a.y, a.ldy, D, k);
        // Sub-block s: its inputs (the staged float4 of step 16 s + j, B of its 16 steps) are
        // read one sub-block ahead; its output reduction runs in the next sub-block, next to
        // that sub-block's scan, so the scan's exp -> FMA chain and the LDS round trips fill
        // each other's stalls. One wave-scope fence per sub-block orders the transposition's
        // writes before its reads (other lanes of the same wave read them).
        float4 in, hv[4], cq[4];
        float bq[16];
        auto read_in = [&](int s, float4& iv, float (&bb)[16]) {
            iv = sm.sx[buf][16 * s + j][cw ^ j];   // (16 s + j) % 16 == j
#pragma unroll
            for (int q = 0; q < 16; q += 4) {
                const float4 b4 = *reinterpret_cast<const float4*>(&sm.bt[buf][j][16 * s + q]);
                bb[q] = b4.x; bb[q + 1] = b4.y; bb[q + 2] = b4.z; bb[q + 3] = b4.w;
            }
        };
        // reduce sub-block s's products (hv, cq read earlier) and store its outputs
        auto output = [&](int s, float gz, float dx) {
            float p[4];
            p[0] = fmaf(hv[3].x, cq[0].w, fmaf(hv[2].x, cq[0].z, fmaf(hv[1].x, cq[0].y, hv[0].x * cq[0].x)));
            p[1] = fmaf(hv[3].y, cq[1].w, fmaf(hv[2].y, cq[1].z, fmaf(hv[1].y, cq[1].y, hv[0].y * cq[1].x)));
            p[2] = fmaf(hv[3].z, cq[2].w, fmaf(hv[2].z, cq[2].z, fmaf(hv[1].z, cq[2].y, hv[0].z * cq[2].x)));
            p[3] = fmaf(hv[3].w, cq[3].w, fmaf(hv[2].w, cq[3].z, fmaf(hv[1].w, cq[3].y, hv[0].w * cq[3].x)));
            // sum over the quad: lanes nq and nq ^ 2 exchange halves, then nq and nq ^ 1
            const float k0 = x2 ? p[2] : p[0], s0 = x2 ? p[0] : p[2];
            const float k1 = x2 ? p[3] : p[1], s1 = x2 ? p[1] : p[3];
            const float r0s = k0 + quad_xor<2>(s0), r1s = k1 + quad_xor<2>(s1);
            const float kk = x1 ? r1s : r0s, ss = x1 ? r0s : r1s;
            const float ysum = kk + quad_xor<1>(ss);
            ssm::bstore4((ysum + dx) * gz, ry,
                         (((unsigned)(16 * s + j) * (unsigned)a.ldy + (unsigned)d) * 4u) | dmask);
        };
        read_in(0, in, bq);
        float gzp = 0.f, dxp = 0.f;
#pragma unroll
        for (int s = 0; s < NSB; ++s) {
            float4 inn;
            float bqn[16];
            if (s + 1 < NSB) read_in(s + 1, inn, bqn);
            const float dl = in.x, du = in.y;
            float hs[16];
#define SCANW_STEP(J)                                                                        \
            h = fmaf(ssm::ex2(row_bcast<J>(dl) * A2), h, row_bcast<J>(du) * bq[J]);          \
            hs[J] = h;
            SCANW_STEP(0) SCANW_STEP(1) SCANW_STEP(2) SCANW_STEP(3)
            SCANW_STEP(4) SCANW_STEP(5) SCANW_STEP(6) SCANW_STEP(7)
            SCANW_STEP(8) SCANW_STEP(9) SCANW_STEP(10) SCANW_STEP(11)
            SCANW_STEP(12) SCANW_STEP(13) SCANW_STEP(14) SCANW_STEP(15)
#undef SCANW_STEP
            if (s > 0) output(s - 1, gzp, dxp);
            // states of steps 4 q .. 4 q + 3 to slot (c, n ^ q) of quad q
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4*>(&hw[q * 256 + c * 64 + 4 * (j ^ q)]) =
                    make_float4(hs[4 * q], hs[4 * q + 1], hs[4 * q + 2], hs[4 * q + 3]);
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            // hv[i]: steps 4 tq .. 4 tq + 3 of state 4 nq + i; cq[u]: C of step 4 tq + u,
            // states 4 nq .. 4 nq + 3
#pragma unroll
            for (int i = 0; i < 4; ++i)
                hv[i] = *reinterpret_cast<const float4*>(
                    &hw[tq * 256 + c * 64 + 4 * (4 * nq + (i ^ tq))]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                cq[u] = *reinterpret_cast<const float4*>(&sm.ct[buf][16 * s + 4 * tq + u][4 * nq]);
            gzp = in.z;
            dxp = in.w;
            if (s + 1 < NSB) {
                in = inn;
#pragma unroll
                for (int q = 0; q < 16; ++q) bq[q] = bqn[q];
            }
        }
        output(NSB - 1, gzp, dxp);
        __syncthreads();
    }
    if (dok && a.hT) a.hT[((long)b * D + d) * 16 + j] = h;
}

// Six waves (24 channels) per workgroup: cfg2's 1536 channels x 4 sequences give one
// workgroup per CU on all 256 (eight-wave groups leave 64 CUs idle: 108 against 104 us).
void launch_w16(const ScanArgs& a, hipStream_t st) {
    constexpr int W = 6;
    const long nwg = ssm::cdiv(a.D, ScanW16<W>::CW) * a.B;
    scan_w16_kernel<W><<<(unsigned)nwg, 64 * W, 0, st>>>(a);
}

template <int N, bool EXACT>
void launch_single(const ScanArgs& a, hipStream_t st) {
    using S = Scan1<N>;
    dim3 grid((unsigned)ssm::cdiv(a.D, S::CW), (unsigned)a.B);
    scan_single_kernel<N, EXACT><<<grid, S::NT, 0, st>>>(a);
}

// Whether the single pass has at least one wave per SIMD (256 CUs x 4).
template <int N>
bool single_ok_n(int B, int D) {
    using S = Scan1<N>;
    return (long)B * ssm::cdiv(D, S::CW) * S::W >= 1024;
}
bool single_ok(int B, int D, int Np) {
    switch (Np) {
        case 4: return single_ok_n<4>(B, D);
        case 8: return single_ok_n<8>(B, D);
        case 16: return single_ok_n<16>(B, D);
        case 32: return single_ok_n<32>(B, D);
        default: return single_ok_n<64>(B, D);
    }
}
// The single pass also for sequences of up to kShortL steps, however few the channels: its
// walk costs about 50 ns a step, less than the chunked passes' three launches (about 20 us
// for one sequence of 1536 channels at 16 to 200 steps, measured).
constexpr int kShortL = 256;
bool use_single(int B, int L, int D, int Np) { return L <= kShortL || single_ok(B, D, Np); }

// One-token update: one thread per (b, d) with the N state entries in registers. ykb > 0:
// y goes to fragment order with K = D = 16 ykb (the input of the fused step's out_proj).
// dtr given: the raw dt is dt_proj formed here, sum over r < R of dtr[b, r] Wdt[d, r] (Wdt
// (D, R) rows 16-byte aligned, R % 4 == 0), and the grid is (D / 64) x ceil(B / 4) workgroups:
// wave w of workgroup (g, j) takes d = 64 g + lane of sequence b = 4 j + w, so the four waves
// read the same 64 rows of Wdt (from L2 once, then L1) and each wave's row of dtr is uniform
// (scalar loads). Otherwise one thread per i = b D + d.
template <int N>
__global__ void m1_update_kernel(const float* __restrict__ x, long ldx,
                                 const float* __restrict__ dt, long lddt,
                                 const float* __restrict__ dt_bias, int softplus,
                                 const float* __restrict__ A, const float* __restrict__ Bm,
                                 long ldb, const float* __restrict__ Cm, long ldc,
                                 const float* __restrict__ Dsk, const float* __restrict__ z,
                                 long ldz, float* __restrict__ y, long ldy,
                                 float* __restrict__ h, int B, int D, int Nr, int vec, int ykb,
                                 const float* __restrict__ dtr, long lddtr,
                                 const float* __restrict__ Wdt, int R) {
    int b, d;
    long i;
    if (dtr) {
        const int nd = D >> 6;
        b = 4 * (int)(blockIdx.x / nd) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        d = 64 * (int)(blockIdx.x % nd) + (threadIdx.x & 63);
        if (b >= B) return;
        i = (long)b * D + d;
    } else {
        i = (long)blockIdx.x * blockDim.x + threadIdx.x;
        if (i >= (long)B * D) return;
        b = (int)(i / D);
        d = (int)(i % D);
    }
    float* hp = h + i * Nr;
    // per group of up to 16 states: all loads first, then the arithmetic. When the state
    // count is the template's and the rows are 16-byte aligned (vec), h and A come in float4
    // loads; otherwise from clamped (in-bounds) scalar indices. (Loads behind a per-n branch
    // were each waited for before the next.) The first group's loads, x and z are issued
    // before dt is formed, so that their latency overlaps dt_proj's.
    constexpr int G = N < 16 ? N : 16;
    struct Grp {
        float h[G], a[G], b[G], c[G];
    };
    auto load_grp = [&](int n0) {
        Grp g;
#pragma unroll
        for (int q = 0; q < G; q += 4) {
            const float4 h4 = *reinterpret_cast<const float4*>(hp + n0 + q);
            const float4 a4 = *reinterpret_cast<const float4*>(A + (long)d * N + n0 + q);
            g.h[q] = h4.x; g.h[q + 1] = h4.y; g.h[q + 2] = h4.z; g.h[q + 3] = h4.w;
            g.a[q] = a4.x; g.a[q + 1] = a4.y; g.a[q + 2] = a4.z; g.a[q + 3] = a4.w;
        }
#pragma unroll
        for (int q = 0; q < G; ++q) {
            g.b[q] = Bm[(long)b * ldb + n0 + q];
            g.c[q] = Cm[(long)b * ldc + n0 + q];
        }
        return g;
    };
    const bool vpath = Nr == N && vec;
    Grp g0;
    if (vpath) g0 = load_grp(0);
    const float xx = x[(long)b * ldx + d];
    const float zz = z ? z[(long)b * ldz + d] : 0.f;
    float raw;
    if (dtr) {
        const float* dr = dtr + (long)b * lddtr;
        const float* wr = Wdt + (long)d * R;
        float s = 0.f;
        for (int r = 0; r < R; r += 4) {
            const float4 w4 = *reinterpret_cast<const float4*>(wr + r);
            s = fmaf(dr[r], w4.x, s);
            s = fmaf(dr[r + 1], w4.y, s);
            s = fmaf(dr[r + 2], w4.z, s);
            s = fmaf(dr[r + 3], w4.w, s);
        }
        raw = s;
    } else {
        raw = dt[(long)b * lddt + d];
    }
    const float dl = delta_of(raw, dt_bias ? dt_bias[d] : 0.f, softplus);
    const float du = dl * xx;
    float acc = 0.f;
    if (vpath) {
#pragma unroll
        for (int n0 = 0; n0 < N; n0 += G) {
            const Grp gg = n0 == 0 ? g0 : load_grp(n0);
#pragma unroll
            for (int q = 0; q < G; q += 4) {
                float4 v;
                v.x = fmaf(ssm::ex2(dl * gg.a[q] * ssm::kLog2e), gg.h[q], du * gg.b[q]);
                v.y = fmaf(ssm::ex2(dl * gg.a[q + 1] * ssm::kLog2e), gg.h[q + 1], du * gg.b[q + 1]);
                v.z = fmaf(ssm::ex2(dl * gg.a[q + 2] * ssm::kLog2e), gg.h[q + 2], du * gg.b[q + 2]);
                v.w = fmaf(ssm::ex2(dl * gg.a[q + 3] * ssm::kLog2e), gg.h[q + 3], du * gg.b[q + 3]);
                *reinterpret_cast<float4*>(hp + n0 + q) = v;
                acc = fmaf(v.x, gg.c[q], acc);
                acc = fmaf(v.y, gg.c[q + 1], acc);
                acc = fmaf(v.z, gg.c[q + 2], acc);
                acc = fmaf(v.w, gg.c[q + 3], acc);
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
    if (z) acc *= ssm::silu_fast(zz);
    if (ykb) y[ssm::frag_off(b, d, ykb)] = acc;
    else y[(long)b * ldy + d] = acc;
}

// The fused Mamba-1 step's x_proj reduction, dt_proj and state update (launch_m1_step_update).
// Workgroup (g, b): sequence b, channels [CPW g, CPW g + CPW), one thread per channel.
// - x_proj of sequence b: dbl[j] = sum over the NP = D / 16 conv tiles of xpart[t, b, j], in a
//   fixed order that every workgroup of b repeats (Q contiguous runs of tiles, one thread per
//   (run, j), then the runs in order), into LDS. These loads are issued first (they come from
//   L2), then the thread's own: its N states and A row (float4), x, z, D, dt_bias, and its W_dt
//   row, stored in quads (W_dt[c, 4i .. 4i+3] at (i D + c) 4, so that a wave's float4 loads are
//   contiguous); all are in flight before the first wait.
// - dt = softplus(dt_r . W_dt[c] + dt_bias[c]) with dt_r = dbl[0, R) (r in order), then
//   h = exp(dt A) h + dt x B, y = (C . h + D x) silu(z), with B = dbl[R, R + N) and
//   C = dbl[R + N, R + 2N) read from LDS.
// Workgroups of the padding rows (b in [B, M16)) write zeros to their rows of y's fragment
// order (the out_proj reads whole 16-row tiles) and do nothing else. Workgroups go to the 8
// XCDs round-robin by id; the ids are mapped so that the D / CPW workgroups of a sequence share
// one XCD, whose L2 then serves its x_proj partials to all of them after the first read.
struct M1StepArgs {
    const float* x; long ldx;
    const float* xpart; int RN, NP, M16;
    const float* Wdt; int R;
    const float* dt_bias; const float* A; const float* Dsk;
    const float* z; long ldz;
    float* yf; float* h;
    int B, D;
};
constexpr int kM1StepMaxQ = 8;
constexpr int kM1StepMaxRQ = 16;   // W_dt quads per thread (R <= 64)

template <int N>
__global__ __launch_bounds__(384) void m1_step_update_kernel(M1StepArgs a) {
    __shared__ float red[kM1StepMaxQ][ssm::kXpartMaxRN];
    __shared__ __attribute__((aligned(16))) float dbl[ssm::kXpartMaxRN];
    const int CPW = blockDim.x;
    const int tid = threadIdx.x;
    const int nq = a.D / CPW;
    const int id = blockIdx.x, k = id >> 3;
    const int b = (id & 7) + 8 * (k / nq);
    const int d = (k % nq) * CPW + tid;
    const int kb = a.D >> 4;
    if (b >= a.B) {
        a.yf[ssm::frag_off(b, d, kb)] = 0.f;
        return;
    }
    // x_proj of sequence b from the partials. Thread (q, j) adds the tiles of run q in order;
    // its loads are issued before the thread's own (HBM) loads below, in groups of kPer with
    // clamped indices (a term past the run adds +0), so that one L2 latency covers a group.
    const int RN = a.RN;
    // Q runs of at least one tile each (NP = D / 16 >= 4)
    const int Q = max(1, min(min(kM1StepMaxQ, CPW / RN), a.NP));
    constexpr int kPer = 32;
    const long step = (long)a.M16 * RN;
    const bool red_thread = tid < RN * Q;   // one (q, j) per thread (RN Q <= CPW, else loop)
    float part = 0.f;
    int pq = 0, pj = 0, t0 = 0, t1 = 0;
    if (red_thread) {
        pj = tid % RN; pq = tid / RN;
        t0 = pq * a.NP / Q; t1 = (pq + 1) * a.NP / Q;
    }
    const float* pbase = a.xpart + (long)b * RN + pj;
    float pv[kPer];
    if (red_thread) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) pv[u] = pbase[(long)min(t0 + u, t1 - 1) * step];
    }

    float* hp = a.h + ((long)b * a.D + d) * N;
    float4 hv[N / 4], av[N / 4];
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
        hv[q] = *reinterpret_cast<const float4*>(hp + 4 * q);
        av[q] = *reinterpret_cast<const float4*>(a.A + (long)d * N + 4 * q);
    }
    const float xx = a.x[(long)b * a.ldx + d];
    const float zz = a.z[(long)b * a.ldz + d];
    const float dsk = a.Dsk ? a.Dsk[d] : 0.f;
    const float bias = a.dt_bias ? a.dt_bias[d] : 0.f;
    const int rq = a.R >> 2;
    float4 wq[kM1StepMaxRQ];   // quads past rq repeat the last one (in bounds, unused)
#pragma unroll
    for (int i = 0; i < kM1StepMaxRQ; ++i)
        wq[i] = *reinterpret_cast<const float4*>(a.Wdt + ((long)min(i, rq - 1) * a.D + d) * 4);

    if (red_thread) {
        for (int g = t0;;) {
#pragma unroll
            for (int u = 0; u < kPer; ++u) part += g + u < t1 ? pv[u] : 0.f;
            g += kPer;
            if (g >= t1) break;
#pragma unroll
            for (int u = 0; u < kPer; ++u) pv[u] = pbase[(long)min(g + u, t1 - 1) * step];
        }
        red[pq][pj] = part;
    }
    // (RN Q > CPW: the remaining (q, j) pairs, with the same order of terms)
    for (int i = tid + CPW; i < RN * Q; i += CPW) {
        const int j = i % RN, q = i / RN;
        const int u0 = q * a.NP / Q, u1 = (q + 1) * a.NP / Q;
        const float* p = a.xpart + ((long)u0 * a.M16 + b) * RN + j;
        float sum = 0.f;
        for (int t = u0; t < u1; ++t, p += step) sum += *p;
        red[q][j] = sum;
    }
    __syncthreads();
    for (int j = tid; j < RN; j += CPW) {
        float sum = red[0][j];
        for (int q = 1; q < Q; ++q) sum += red[q][j];
        dbl[j] = sum;
    }
    __syncthreads();

    // dt_proj, r in order
    float raw = 0.f;
#pragma unroll
    for (int i = 0; i < kM1StepMaxRQ; ++i) {
        if (i < rq) {   // (uniform; a break here would send wq to scratch memory)
            const float4 d4 = *reinterpret_cast<const float4*>(dbl + 4 * i);
            raw = fmaf(d4.x, wq[i].x, raw);
            raw = fmaf(d4.y, wq[i].y, raw);
            raw = fmaf(d4.z, wq[i].z, raw);
            raw = fmaf(d4.w, wq[i].w, raw);
        }
    }
    const float dl = delta_of(raw, bias, 1);
    const float du = dl * xx;
    const float* Bv = dbl + a.R;
    const float* Cv = Bv + N;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
        float4 v;
        v.x = fmaf(ssm::ex2(dl * av[q].x * ssm::kLog2e), hv[q].x, du * Bv[4 * q]);
        v.y = fmaf(ssm::ex2(dl * av[q].y * ssm::kLog2e), hv[q].y, du * Bv[4 * q + 1]);
        v.z = fmaf(ssm::ex2(dl * av[q].z * ssm::kLog2e), hv[q].z, du * Bv[4 * q + 2]);
        v.w = fmaf(ssm::ex2(dl * av[q].w * ssm::kLog2e), hv[q].w, du * Bv[4 * q + 3]);
        *reinterpret_cast<float4*>(hp + 4 * q) = v;
        acc = fmaf(v.x, Cv[4 * q], acc);
        acc = fmaf(v.y, Cv[4 * q + 1], acc);
        acc = fmaf(v.z, Cv[4 * q + 2], acc);
        acc = fmaf(v.w, Cv[4 * q + 3], acc);
    }
    if (a.Dsk) acc = fmaf(dsk, xx, acc);
    acc *= ssm::silu_fast(zz);
    a.yf[ssm::frag_off(b, d, kb)] = acc;
}

}  // namespace

namespace {
int pad_n(int N) { return N <= 4 ? 4 : N <= 8 ? 8 : N <= 16 ? 16 : N <= 32 ? 32 : 64; }
// Both designs address rows through 32-bit offsets from a base they rebuild per block (single
// pass: 128 rows) or per chunk (chunked passes: T rows), so a stride only has to fit that
// many rows; the plan itself depends on (B, D, N) alone, and so does the workspace query.
constexpr long kOffMax = 1L << 31;
bool rows_fit(long rows, long ld, int D) { return ((rows - 1) * ld + D) * 4 < kOffMax; }
size_t chunked_workspace(int B, int L, int D, int N) {
    const int T = pick_chunk(B, L, D);
    const long NC = ssm::cdiv(L, T);
    return sizeof(float) * (size_t)B * NC * D * ((size_t)N + 1);
}
}  // namespace

extern "C" size_t ssm_selective_scan_workspace(int B, int L, int D, int N) {
    if (B <= 0 || L <= 0 || D <= 0 || N <= 0 || N > 64) return 0;
    if (use_single(B, L, D, pad_n(N))) return 0;   // the single pass needs none
    return chunked_workspace(B, L, D, N);
}

namespace ssm {

// ssm_selective_scan with one more input form: zgated = 1 when z already holds silu(z) (the
// Mamba-1 block writes it so from in_proj's epilogue).
ssm_status selective_scan(const float* u, long ldu, const float* dt, long lddt,
                          const float* dt_bias, int softplus, const float* A, const float* Bm,
                          long ldb, const float* Cm, long ldc, const float* Dsk, const float* z,
                          long ldz, int zgated, float* y, long ldy, int B, int L, int D, int N,
                          const float* h0, float* hT, void* workspace, size_t workspace_bytes,
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
    const int Np = pad_n(N);
    const long ldmax = std::max({ldu, lddt, ldy, z ? ldz : 0L, ldb, ldc});
    const bool single = use_single(B, L, D, Np);
    const long rows = single ? std::min<long>(L, 128) : pick_chunk(B, L, D);
    SSM_REQUIRE(rows_fit(rows, ldmax, D),
                "ssm_selective_scan: row stride %ld too large for 32-bit block offsets", ldmax);
    const size_t need = single ? 0 : chunked_workspace(B, L, D, N);
    SSM_REQUIRE(need == 0 || (workspace && workspace_bytes >= need),
                "ssm_selective_scan: workspace of %zu bytes needed", need);
    ScanArgs a;
    a.u = u; a.ldu = ldu; a.dt = dt; a.lddt = lddt; a.dt_bias = dt_bias; a.softplus = softplus;
    a.A = A; a.Bm = Bm; a.ldb = ldb; a.Cm = Cm; a.ldc = ldc; a.Dsk = Dsk; a.z = z; a.ldz = ldz;
    a.y = y; a.ldy = ldy; a.B = B; a.L = L; a.D = D; a.N = N;
    a.zgated = z ? zgated : 0;
    a.T = pick_chunk(B, L, D);
    a.NC = (int)ssm::cdiv(L, a.T);
    a.hc = (float*)workspace;
    a.sdt = a.hc + (size_t)B * a.NC * N * D;
    a.h0 = h0; a.hT = hT;
    hipStream_t st = (hipStream_t)stream;
    if (single) {
        const bool exact = N == Np;
        switch (Np) {
            case 4: exact ? launch_single<4, true>(a, st) : launch_single<4, false>(a, st); break;
            case 8: exact ? launch_single<8, true>(a, st) : launch_single<8, false>(a, st); break;
            case 16: exact ? launch_w16(a, st) : launch_single<16, false>(a, st); break;
            case 32: exact ? launch_single<32, true>(a, st) : launch_single<32, false>(a, st); break;
            default: exact ? launch_single<64, true>(a, st) : launch_single<64, false>(a, st); break;
        }
        return ssm::check_launch("selective_scan");
    }
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

}  // namespace ssm

extern "C" ssm_status ssm_selective_scan(const float* u, long ldu, const float* dt, long lddt,
                                         const float* dt_bias, int softplus, const float* A,
                                         const float* Bm, long ldb, const float* Cm, long ldc,
                                         const float* Dsk, const float* z, long ldz, float* y,
                                         long ldy, int B, int L, int D, int N, const float* h0,
                                         float* hT, void* workspace, size_t workspace_bytes,
                                         void* stream) {
    return ssm::selective_scan(u, ldu, dt, lddt, dt_bias, softplus, A, Bm, ldb, Cm, ldc, Dsk, z,
                               ldz, 0, y, ldy, B, L, D, N, h0, hT, workspace, workspace_bytes,
                               stream);
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
    hipStream_t st = (hipStream_t)stream;
    return ssm::launch_m1_update(x, ldx, dt, lddt, dt_bias, softplus, A, Bm, ldb, Cm, ldc, Dsk,
                                 z, ldz, y, ldy, 0, h, B, D, N, st, nullptr, 0, nullptr, 0);
}

namespace ssm {

ssm_status launch_m1_update(const float* x, long ldx, const float* dt, long lddt,
                            const float* dt_bias, int softplus, const float* A, const float* Bm,
                            long ldb, const float* Cm, long ldc, const float* Dsk, const float* z,
                            long ldz, float* y, long ldy, int ykb, float* h, int B, int D, int N,
                            hipStream_t st, const float* dtr, long lddtr, const float* Wdt,
                            int R) {
    const long n = (long)B * D;
    const unsigned g = dtr ? (unsigned)((D / 64) * ssm::cdiv(B, 4)) : (unsigned)ssm::cdiv(n, 256);
    // float4 access to h and A rows when N is a template size and the rows are aligned
    const int vec = (N == 8 || N == 16 || N == 32 || N == 64) && (uintptr_t)h % 16 == 0 &&
                    (uintptr_t)A % 16 == 0;
#define M1U(NS)                                                                              \
    m1_update_kernel<NS><<<g, 256, 0, st>>>(x, ldx, dt, lddt, dt_bias, softplus, A, Bm, ldb, \
                                            Cm, ldc, Dsk, z, ldz, y, ldy, h, B, D, N, vec, ykb, \
                                            dtr, lddtr, Wdt, R)
    if (N <= 8) M1U(8);
    else if (N <= 16) M1U(16);
    else if (N <= 32) M1U(32);
    else M1U(64);
#undef M1U
    return ssm::check_launch("m1_state_update");
}

ssm_status launch_m1_update_frag(const float* x, long ldx, const float* dtr, long lddtr,
                                 const float* Wdt, int R, const float* dt_bias, const float* A,
                                 const float* Bm, long ldb, const float* Cm, long ldc,
                                 const float* Dsk, const float* z, long ldz, float* yf, float* h,
                                 int B, int D, int N, hipStream_t st) {
    SSM_REQUIRE(x && dtr && Wdt && A && Bm && Cm && yf && h && B >= 1 && D % 64 == 0 &&
                    N >= 1 && N <= 64 && R >= 4 && R % 4 == 0 && ((uintptr_t)Wdt & 15) == 0,
                "m1_update_frag: arguments");
    return launch_m1_update(x, ldx, nullptr, 0, dt_bias, 1, A, Bm, ldb, Cm, ldc, Dsk, z, ldz, yf,
                            0, D / 16, h, B, D, N, st, dtr, lddtr, Wdt, R);
}

}  // namespace ssm

namespace ssm {

bool m1_step_update_ok(int D, int N, int R) {
    // (N = 64 would hold 128 state and A registers per thread next to the prefetched rows)
    return D % 64 == 0 && (N == 4 || N == 8 || N == 16 || N == 32) && R >= 4 &&
           R % 4 == 0 && R <= 4 * kM1StepMaxRQ && R + 2 * N <= kXpartMaxRN;
}

ssm_status launch_m1_step_update(const float* x, long ldx, const float* xpart, int RN, int M16,
                                 const float* Wdt, int R, const float* dt_bias, const float* A,
                                 const float* Dsk, const float* z, long ldz, float* yf, float* h,
                                 int B, int D, int N, hipStream_t st) {
    SSM_REQUIRE(x && xpart && Wdt && A && z && yf && h && B >= 1 && M16 >= B && M16 % 16 == 0 &&
                    RN == R + 2 * N && m1_step_update_ok(D, N, R) &&
                    ((uintptr_t)Wdt & 15) == 0 && ((uintptr_t)h & 15) == 0 &&
                    ((uintptr_t)A & 15) == 0,
                "m1_step_update: arguments");
    // channels per workgroup: the largest of 384, 256, 192, 128, 64 that divides D
    int cpw = 64;
    for (int c : {384, 256, 192, 128})
        if (D % c == 0) { cpw = c; break; }
    M1StepArgs a;
    a.x = x; a.ldx = ldx; a.xpart = xpart; a.RN = RN; a.NP = D / 16; a.M16 = M16;
    a.Wdt = Wdt; a.R = R; a.dt_bias = dt_bias; a.A = A; a.Dsk = Dsk; a.z = z; a.ldz = ldz;
    a.yf = yf; a.h = h; a.B = B; a.D = D;
    const unsigned grid = (unsigned)(D / cpw) * (unsigned)M16;   // M16 % 8 == 0
    switch (N) {
        case 4: m1_step_update_kernel<4><<<grid, cpw, 0, st>>>(a); break;
        case 8: m1_step_update_kernel<8><<<grid, cpw, 0, st>>>(a); break;
        case 16: m1_step_update_kernel<16><<<grid, cpw, 0, st>>>(a); break;
        default: m1_step_update_kernel<32><<<grid, cpw, 0, st>>>(a); break;
    }
    return check_launch("m1_step_update");
}

}  // namespace ssm
