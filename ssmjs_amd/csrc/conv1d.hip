// K1: causal depthwise conv1d (+bias, +SiLU) for gfx950.
//
// Replaces the conv stage of MambaCode.js's Mamba-1/2 layers (called through model.forward,
// src/session/streaming.ts:31-35). HBM-bound: every input element is read once (plus a K-1
// row halo per time run, served from L2) and every output written once.
//
// Layout: x, y (B, L, C) row-major with row strides ldx/ldy (x is usually a column slice of
// the in_proj output). A thread owns VEC adjacent channels and a run of TT time steps and
// slides a K-deep register window down the run; threadIdx.x walks channels so a wave reads
// 64*VEC*4 contiguous bytes per time step.
#include "common.hpp"

namespace {

constexpr int kTT = 16;      // time steps per thread
constexpr int kRuns = 4;     // threadIdx.y extent (time runs per block)
constexpr int kChan = 64;    // threadIdx.x extent (channel groups per block)

template <int VEC>
struct vec_t;
template <>
struct vec_t<1> { using type = float; };
template <>
struct vec_t<4> { using type = float4; };

// a run's own rows, read by no other thread: streaming loads (ssm::load_nt4)
template <int VEC>
__device__ __forceinline__ void load_nt(const float* p, float (&v)[VEC]) {
    if constexpr (VEC == 4) {
        const float4 q = ssm::load_nt4(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
        v[0] = __builtin_nontemporal_load(p);
    }
}

template <int VEC>
__device__ __forceinline__ void load_v(const float* p, float (&v)[VEC]) {
    if constexpr (VEC == 4) {
        float4 q = *reinterpret_cast<const float4*>(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
        v[0] = *p;
    }
}

// outputs are read by the next launch only: streaming stores
template <int VEC>
__device__ __forceinline__ void store_v(float* p, const float (&v)[VEC]) {
    if constexpr (VEC == 4) {
        ssm::store_nt4(make_float4(v[0], v[1], v[2], v[3]), p);
    } else {
        __builtin_nontemporal_store(v[0], p);
    }
}

// bf16 outputs (round to nearest even), for the bf16-input layer's SSD operands
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
template <int VEC>
__device__ __forceinline__ void store_v(__bf16* p, const float (&v)[VEC]) {
    if constexpr (VEC == 4) {
        __builtin_nontemporal_store(bf16x4_t{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]},
                                    reinterpret_cast<bf16x4_t*>(p));
    } else {
        __builtin_nontemporal_store((__bf16)v[0], p);
    }
}

template <int K, int VEC, typename OT>
__global__ __launch_bounds__(256) void conv1d_fwd(const float* __restrict__ x, long ldx,
                                                  const float* __restrict__ w,
                                                  const float* __restrict__ bias,
                                                  OT* __restrict__ y, long ldy, int L, int C,
                                                  int silu, const float* __restrict__ state_in) {
    const int c0 = (blockIdx.x * kChan + threadIdx.x) * VEC;
    const int t0 = (blockIdx.y * kRuns + threadIdx.y) * kTT;
    const int b = blockIdx.z;
    if (c0 >= C || t0 >= L) return;
    const float* xb = x + (long)b * L * ldx + c0;
    OT* yb = y + (long)b * L * ldy + c0;

    float wk[K][VEC], bv[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
#pragma unroll
        for (int k = 0; k < K; ++k) wk[k][v] = w[(long)(c0 + v) * K + k];
        bv[v] = bias ? bias[c0 + v] : 0.f;
    }
    // window[k] holds x[t - (K-1) + k] for the next output t
    float win[K][VEC];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
        const int ts = t0 - (K - 1) + k;
        if (ts >= 0) {
            load_v<VEC>(xb + (long)ts * ldx, win[k]);
        } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                win[k][v] = state_in
                                ? state_in[((long)b * C + c0 + v) * (K - 1) + (K - 1) + ts]
                                : 0.f;
        }
    }
    if (t0 + kTT <= L) {
        // full run: all kTT input rows are issued before the first use (kTT + K - 1 loads in
        // flight per thread), then the window slides over registers. The last K - 1 rows are
        // also the next run's window (ordinary loads: that thread finds them in L2); the
        // others stream.
        float xs[kTT][VEC];
#pragma unroll
        for (int i = 0; i < kTT; ++i) {
            if (i < kTT - (K - 1)) load_nt<VEC>(xb + (long)(t0 + i) * ldx, xs[i]);
            else load_v<VEC>(xb + (long)(t0 + i) * ldx, xs[i]);
        }
#pragma unroll
        for (int i = 0; i < kTT; ++i) {
            float out[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                float acc = bv[v];
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const int src = i - (K - 1) + k;   // < 0: from the carried window
                    acc = fmaf(wk[k][v], src < 0 ? win[K - 1 + src][v] : xs[src][v], acc);
                }
                out[v] = silu ? ssm::silu_fast(acc) : acc;
            }
            store_v<VEC>(yb + (long)(t0 + i) * ldy, out);
        }
        return;
    }
    const int tend = min(t0 + kTT, L);
    for (int t = t0; t < tend; ++t) {
        load_v<VEC>(xb + (long)t * ldx, win[K - 1]);
        float out[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            float acc = bv[v];
#pragma unroll
            for (int k = 0; k < K; ++k) acc = fmaf(wk[k][v], win[k][v], acc);
            out[v] = silu ? ssm::silu_fast(acc) : acc;
        }
        store_v<VEC>(yb + (long)t * ldy, out);
#pragma unroll
        for (int k = 0; k < K - 1; ++k)
#pragma unroll
            for (int v = 0; v < VEC; ++v) win[k][v] = win[k + 1][v];
    }
}

// state_out[b,c,j] = x[b, L-(K-1)+j, c] (or the carried state when L < K-1). One thread per
// (b,c); j ascends, and the source index of an in-place shift is always ahead of j.
__global__ void conv1d_state_out(const float* __restrict__ x, long ldx, int B, int L, int C,
                                 int K, const float* state_in, float* state_out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * C) return;
    const int b = (int)(i / C), c = (int)(i % C);
    for (int j = 0; j < K - 1; ++j) {
        const int ts = L - (K - 1) + j;
        float v;
        if (ts >= 0) v = x[((long)b * L + ts) * ldx + c];
        else if (state_in) v = state_in[i * (K - 1) + (K - 1) + ts];
        else v = 0.f;
        state_out[i * (K - 1) + j] = v;
    }
}

// One decode token: thread per (b, c).
// One-token update, a thread per (b, c): the window is the (K-1)-deep state plus x. KC is
// the width when known at compile time (every load is then issued before the first use);
// KC = 0 takes it from K at run time.
template <int KC>
__global__ void conv1d_update_kernel(const float* __restrict__ x, long ldx,
                                     const float* __restrict__ w, const float* __restrict__ bias,
                                     float* __restrict__ y, long ldy, float* __restrict__ state,
                                     int B, int C, int Kr, int silu) {
    const int K = KC > 0 ? KC : Kr;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * C) return;
    const int b = (int)(i / C), c = (int)(i % C);
    float* st = state + i * (K - 1);
    const float xn = x[(long)b * ldx + c];
    float acc = bias ? bias[c] : 0.f;
    if (KC > 0) {
        float wv[KC > 0 ? KC : 1], sv[KC > 1 ? KC - 1 : 1];
#pragma unroll
        for (int k = 0; k < KC; ++k) wv[k] = w[(long)c * KC + k];
#pragma unroll
        for (int k = 0; k < KC - 1; ++k) sv[k] = st[k];
#pragma unroll
        for (int k = 0; k < KC - 1; ++k) acc = fmaf(wv[k], sv[k], acc);
        acc = fmaf(wv[KC - 1], xn, acc);
#pragma unroll
        for (int k = 0; k + 1 < KC - 1; ++k) st[k] = sv[k + 1];
        if (KC > 1) st[KC - 2] = xn;
    } else {
        for (int k = 0; k < K - 1; ++k) acc = fmaf(w[(long)c * K + k], st[k], acc);
        acc = fmaf(w[(long)c * K + K - 1], xn, acc);
        for (int k = 0; k + 1 < K - 1; ++k) st[k] = st[k + 1];
        if (K > 1) st[K - 2] = xn;
    }
    y[(long)b * ldy + c] = silu ? ssm::silu_fast(acc) : acc;
}

template <int K, typename OT>
ssm_status launch_fwd(const float* x, long ldx, const float* w, const float* bias, OT* y,
                      long ldy, int B, int L, int C, int silu, const float* state_in,
                      hipStream_t st) {
    const bool v4 = (C % 4 == 0) && (ldx % 4 == 0) && (ldy % 4 == 0) &&
                    ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % (4 * sizeof(OT)) == 0);
    const dim3 block(kChan, kRuns);
    if (v4) {
        dim3 grid((unsigned)ssm::cdiv(C / 4, kChan), (unsigned)ssm::cdiv(L, kRuns * kTT), B);
        conv1d_fwd<K, 4, OT><<<grid, block, 0, st>>>(x, ldx, w, bias, y, ldy, L, C, silu, state_in);
    } else {
        dim3 grid((unsigned)ssm::cdiv(C, kChan), (unsigned)ssm::cdiv(L, kRuns * kTT), B);
        conv1d_fwd<K, 1, OT><<<grid, block, 0, st>>>(x, ldx, w, bias, y, ldy, L, C, silu, state_in);
    }
    return ssm::check_launch("conv1d_fwd");
}

}  // namespace

namespace ssm {

// The forward conv with bf16 outputs and a zero initial state (the bf16-input layer).
ssm_status launch_conv1d_bf16(const float* x, long ldx, const float* w, const float* bias,
                              __bf16* y, long ldy, int B, int L, int C, int K, int silu,
                              hipStream_t st) {
    SSM_REQUIRE(x && w && y && B >= 0 && L >= 0 && C >= 0 && ldx >= C && ldy >= C,
                "conv1d_bf16: bad args");
    if (B == 0 || L == 0 || C == 0) return SSM_OK;
    switch (K) {
        case 2: return launch_fwd<2>(x, ldx, w, bias, y, ldy, B, L, C, silu, nullptr, st);
        case 3: return launch_fwd<3>(x, ldx, w, bias, y, ldy, B, L, C, silu, nullptr, st);
        case 4: return launch_fwd<4>(x, ldx, w, bias, y, ldy, B, L, C, silu, nullptr, st);
        default: return fail(SSM_ERR_INVALID_ARG, "conv1d_bf16: kernel width %d", K);
    }
}

}  // namespace ssm

extern "C" ssm_status ssm_causal_conv1d(const float* x, long ldx, const float* w,
                                        const float* bias, float* y, long ldy, int B, int L,
                                        int C, int K, int silu, const float* state_in,
                                        float* state_out, void* stream) {
    SSM_REQUIRE(x && w && y, "ssm_causal_conv1d: null x/w/y");
    SSM_REQUIRE(B >= 0 && L >= 0 && C >= 0 && K >= 1 && K <= 8, "ssm_causal_conv1d: bad shape");
    SSM_REQUIRE(ldx >= C && ldy >= C, "ssm_causal_conv1d: row stride below C");
    SSM_REQUIRE(!state_out || state_out != (float*)x, "ssm_causal_conv1d: state_out aliases x");
    hipStream_t st = (hipStream_t)stream;
    if (B == 0 || C == 0) return SSM_OK;
    if (L > 0) {
        ssm_status s;
        switch (K) {
            case 1: s = launch_fwd<1>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            case 2: s = launch_fwd<2>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            case 3: s = launch_fwd<3>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            case 4: s = launch_fwd<4>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            case 5: s = launch_fwd<5>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            case 6: s = launch_fwd<6>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            case 7: s = launch_fwd<7>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
            default: s = launch_fwd<8>(x, ldx, w, bias, y, ldy, B, L, C, silu, state_in, st); break;
        }
        if (s != SSM_OK) return s;
    }
    if (state_out && K > 1) {
        const long n = (long)B * C;
        conv1d_state_out<<<(unsigned)ssm::cdiv(n, 256), 256, 0, st>>>(x, ldx, B, L, C, K,
                                                                       state_in, state_out);
        return ssm::check_launch("conv1d_state_out");
    }
    return SSM_OK;
}

extern "C" ssm_status ssm_conv1d_update(const float* x, long ldx, const float* w,
                                        const float* bias, float* y, long ldy, float* state,
                                        int B, int C, int K, int silu, void* stream) {
    SSM_REQUIRE(x && w && y && (state || K == 1), "ssm_conv1d_update: null pointer");
    SSM_REQUIRE(B >= 0 && C >= 0 && K >= 1 && K <= 8 && ldx >= C && ldy >= C,
                "ssm_conv1d_update: bad shape");
    if (B == 0 || C == 0) return SSM_OK;
    const long n = (long)B * C;
    const unsigned grid = (unsigned)ssm::cdiv(n, 256);
    hipStream_t st = (hipStream_t)stream;
    switch (K) {
        case 2: conv1d_update_kernel<2><<<grid, 256, 0, st>>>(x, ldx, w, bias, y, ldy, state, B, C, K, silu); break;
        case 3: conv1d_update_kernel<3><<<grid, 256, 0, st>>>(x, ldx, w, bias, y, ldy, state, B, C, K, silu); break;
        case 4: conv1d_update_kernel<4><<<grid, 256, 0, st>>>(x, ldx, w, bias, y, ldy, state, B, C, K, silu); break;
        default: conv1d_update_kernel<0><<<grid, 256, 0, st>>>(x, ldx, w, bias, y, ldy, state, B, C, K, silu); break;
    }
    return ssm::check_launch("conv1d_update");
}
