// sampleToken (src/session/streaming.ts:53-97) on the device, one 1024-thread workgroup per
// row of logits, so that sampled generation needs no logits readback:
//   scaled_i = float(logit_i / max(T, 1e-7))          (double division, float store)
//   e_i      = float(exp(double(scaled_i) - maxL))     (double exp, float store)
//   sumE     = sum_i double(e_i)
//   the topK largest e in a stable descending order (ties: lower index first), the nucleus
//   cut at the first cumulative e / sumE >= topP, and the draw: the first nucleus entry whose
//   running sum of e reaches u * (sum of the nucleus's e), u in [0, 1) given per row.
// Order of work inside the row:
//   1. every thread holds up to kEPT elements (index tid + 1024 j) in registers;
//   2. the K-th largest e is found exactly by a 4-pass radix select over the 32-bit keys
//      (bits of e + 1, monotonic for e >= 0; 0 marks padding), with per-wave histograms;
//   3. the elements above it, then the lowest-index ones equal to it, go to LDS;
//   4. a bitonic sort orders the K candidates (key descending, index ascending);
//   5. one thread walks the nucleus and the draw in double, in that order.
// sumE is summed per thread in index order and then over threads and waves in a fixed
// order: the reference adds in plain index order, so sumE can differ in its last bits, which
// moves the nucleus cut only if a cumulative probability lies within ~1e-15 of topP.
#include <cstdint>

#include "common.hpp"
#include "glue.hpp"

namespace {

constexpr int kThreads = 1024;
constexpr int kEPT = 32;                        // elements per thread: rows up to 32768
constexpr int kMaxN = kThreads * kEPT;
constexpr int kMaxK = 1024;                     // topK handled on the device
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__global__ __launch_bounds__(kThreads) void sample_kernel(const float* __restrict__ logits,
                                                          long ld, int n, double temp, int K,
                                                          double top_p,
                                                          const double* __restrict__ u,
                                                          uint32_t* __restrict__ out) {
    __shared__ float redf[kWaves];
    __shared__ double redd[kWaves];
    __shared__ unsigned hist[kWaves][256];
    __shared__ unsigned ckey[kMaxK];
    __shared__ unsigned cidx[kMaxK];
    __shared__ unsigned sel_digit, sel_left;
    __shared__ unsigned gcount;
    __shared__ unsigned wcount[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* row = logits + (long)blockIdx.x * ld;

    // 1. scaled values and their maximum (NaN never becomes the maximum, as in the reference)
    float e[kEPT];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kEPT; ++j) {
        const int i = tid + kThreads * j;
        e[j] = i < n ? (float)((double)row[i] / temp) : -INFINITY;
        mx = fmaxf(mx, e[j]);
    }
    mx = wave_max(mx);
    if (lane == 0) redf[w] = mx;
    __syncthreads();
    mx = redf[0];
    for (int v = 1; v < kWaves; ++v) mx = fmaxf(mx, redf[v]);

    // exponentials, their sum, and the keys (e >= 0: float bits are monotonic; + 1 so that
    // padding, key 0, sorts below every real element)
    double part = 0.0;
    unsigned key[kEPT];
#pragma unroll
    for (int j = 0; j < kEPT; ++j) {
        const int i = tid + kThreads * j;
        if (i < n) {
            e[j] = (float)exp((double)e[j] - (double)mx);
            part += (double)e[j];
            key[j] = __float_as_uint(e[j]) + 1u;
        } else {
            key[j] = 0u;
        }
    }
    part = wave_sum(part);
    if (lane == 0) redd[w] = part;
    __syncthreads();
    double sumE = 0.0;
    for (int v = 0; v < kWaves; ++v) sumE += redd[v];

    // 2. radix select: the K-th largest key, and how many of the elements equal to it belong
    // to the top K (left)
    unsigned prefix = 0u, pmask = 0u, left = (unsigned)K;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int b = lane; b < 256; b += 64) hist[w][b] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kEPT; ++j)
            if ((key[j] & pmask) == prefix) atomicAdd(&hist[w][(key[j] >> shift) & 255u], 1u);
        __syncthreads();
        // bin totals over the waves: thread b < 256 owns bin b
        unsigned tot = 0u;
        if (tid < 256)
            for (int v = 0; v < kWaves; ++v) tot += hist[v][tid];
        __syncthreads();
        if (tid < 256) hist[0][tid] = tot;
        __syncthreads();
        if (tid == 0) {
            unsigned cum = 0u, d = 0u;
            for (int b = 255; b >= 0; --b) {
                if (cum + hist[0][b] >= left) {
                    d = (unsigned)b;
                    break;
                }
                cum += hist[0][b];
            }
            sel_digit = d;
            sel_left = left - cum;
        }
        __syncthreads();
        prefix |= sel_digit << shift;
        pmask |= 255u << shift;
        left = sel_left;
        __syncthreads();
    }
    const unsigned kth = prefix;
    const unsigned above = (unsigned)K - left;   // elements with a key above kth

    // 3. candidates: every key above kth (in any order; the sort below orders them), then the
    // `left` lowest-index elements equal to kth (index order = slice j, then thread)
    if (tid == 0) gcount = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kEPT; ++j)
        if (key[j] > kth) {
            const unsigned pos = atomicAdd(&gcount, 1u);
            ckey[pos] = key[j];
            cidx[pos] = (unsigned)(tid + kThreads * j);
        }
    unsigned taken = 0u;   // equal elements placed so far (the same in every thread)
#pragma unroll
    for (int j = 0; j < kEPT; ++j) {
        if (taken < left) {   // uniform over the workgroup
            const bool eq = key[j] == kth;
            const unsigned long long bal = __ballot(eq);
            const unsigned below_in_wave = __popcll(bal & ((1ull << lane) - 1ull));
            if (lane == 0) wcount[w] = (unsigned)__popcll(bal);
            __syncthreads();
            unsigned before = 0u, total = 0u;
            for (int v = 0; v < kWaves; ++v) {
                if (v < w) before += wcount[v];
                total += wcount[v];
            }
            const unsigned rank = taken + before + below_in_wave;
            if (eq && rank < left) {
                ckey[above + rank] = key[j];
                cidx[above + rank] = (unsigned)(tid + kThreads * j);
            }
            taken += total;
            __syncthreads();
        }
    }
    // padding up to the sort size
    for (int t = K + tid; t < kMaxK; t += kThreads) {
        ckey[t] = 0u;
        cidx[t] = 0xffffffffu;
    }
    __syncthreads();

    // 4. bitonic sort of kMaxK entries: key descending, then index ascending
    for (int size = 2; size <= kMaxK; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int t = tid;
            const int p = t ^ stride;
            if (p > t) {
                const bool desc_block = (t & size) == 0;
                const unsigned ka = ckey[t], kb = ckey[p];
                const unsigned ia = cidx[t], ib = cidx[p];
                // "a before b" in the final order
                const bool a_first = ka > kb || (ka == kb && ia < ib);
                if (a_first != desc_block) {
                    ckey[t] = kb; ckey[p] = ka;
                    cidx[t] = ib; cidx[p] = ia;
                }
            }
            __syncthreads();
        }
    }

    // 5. nucleus and draw, in the reference's order, in double
    if (tid == 0) {
        double cum = 0.0;
        int m = 0;
        for (int t = 0; t < K; ++t) {
            cum += (double)__uint_as_float(ckey[t] - 1u) / sumE;
            m = t + 1;
            if (cum >= top_p) break;
        }
        double nsum = 0.0;
        for (int t = 0; t < m; ++t) nsum += (double)__uint_as_float(ckey[t] - 1u);
        const double thr = u[blockIdx.x] * nsum;
        double acc = 0.0;
        unsigned pick = cidx[m - 1];
        for (int t = 0; t < m; ++t) {
            acc += (double)__uint_as_float(ckey[t] - 1u);
            if (acc >= thr) {
                pick = cidx[t];
                break;
            }
        }
        out[blockIdx.x] = pick;
    }
}

}  // namespace

namespace ssm {

bool sample_ok(int n, int top_k) {
    return n >= 1 && n <= kMaxN && top_k >= 1 && (top_k < n ? top_k : n) <= kMaxK;
}

ssm_status launch_sample(const float* logits, long ld, int rows, int n, double temperature,
                         int top_k, double top_p, const double* u, uint32_t* out,
                         hipStream_t st) {
    if (rows == 0) return SSM_OK;
    const double t = temperature > 1e-7 ? temperature : 1e-7;   // streaming.ts:11,61
    const int K = top_k < n ? top_k : n;                         // slice(0, topK)
    sample_kernel<<<rows, kThreads, 0, st>>>(logits, ld, n, t, K, top_p, u, out);
    return check_launch("sample");
}

}  // namespace ssm

extern "C" ssm_status ssm_sample(const float* logits, long ld, int rows, int n,
                                 double temperature, int top_k, double top_p, const double* u,
                                 uint32_t* out, void* stream) {
    SSM_REQUIRE(logits && u && out, "ssm_sample: null logits/u/out");
    SSM_REQUIRE(rows >= 0 && n >= 1 && ld >= n, "ssm_sample: bad shape");
    SSM_REQUIRE(top_k >= 1, "ssm_sample: topK must be at least 1");
    if (!ssm::sample_ok(n, top_k))
        return ssm::fail(SSM_ERR_UNSUPPORTED,
                         "ssm_sample: needs n <= %d and topK <= %d (n=%d topK=%d)", kMaxN, kMaxK,
                         n, top_k);
    return ssm::launch_sample(logits, ld, rows, n, temperature, top_k, top_p, u, out,
                              (hipStream_t)stream);
}
