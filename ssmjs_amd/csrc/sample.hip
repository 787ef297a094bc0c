// sampleToken (src/session/streaming.ts:53-97) on the device, so that sampled generation
// needs no logits readback:
//   scaled_i = float(logit_i / max(T, 1e-7))          (double division, float store)
//   e_i      = float(exp(double(scaled_i) - maxL))     (double exp, float store)
//   sumE     = sum_i double(e_i)
//   the topK largest e in a stable descending order (ties: lower index first), the nucleus
//   cut at the first cumulative e / sumE >= topP, and the draw: the first nucleus entry whose
//   running sum of e reaches u * (sum of the nucleus's e), u in [0, 1) given per row.
// Three launches per batch of rows:
//   scale  (slices of 2048 logits per workgroup): scaled values to the workspace, slice maxima;
//   exp    (same slices): e as a sortable key (bits of e + 1: monotonic for e >= 0, and 0
//          marks padding) over the scaled values, and each slice's sum of e;
//   pick   (one 1024-thread workgroup per row; keys in registers up to 32768 per row, read
//          again from the workspace for longer rows): a bound on the K-th largest key, the
//          candidates above it gathered to LDS (an exact radix select when too many tie),
//          sorted (key descending, index ascending), then the nucleus and the draw.
// The double division and exp are the costly part (about 35 double operations per logit),
// which is why they are spread over many workgroups instead of the one that owns the row.
// sumE adds per thread in index order, then over threads, waves and slices in a fixed order:
// the reference adds in plain index order, so sumE can differ in its last bits, which moves
// the nucleus cut only if a cumulative probability lies within ~1e-15 of topP.
#include <cstdint>

#include <mutex>

#include "common.hpp"
#include "glue.hpp"

// The slice loops are unrolled fully for register-held keys (a constant 32 slices) and stay
// loops for keys read from the workspace; clang warns about the latter.
#pragma clang diagnostic ignored "-Wpass-failed"

namespace {

constexpr int kSlice = 2048;                    // logits per scale / exp workgroup
constexpr int kSliceThreads = 256;
constexpr int kPer = kSlice / kSliceThreads;    // 8 per thread
constexpr int kThreads = 1024;                  // pick workgroup
constexpr int kEPT = 32;                        // keys per pick thread held in registers
constexpr int kRegN = kThreads * kEPT;          // rows up to 32768 keep their keys in registers
constexpr int kMaxN = 262144;                   // longer rows re-read them from the workspace
constexpr int kMaxK = 1024;                     // topK handled on the device; sort capacity
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSlices = (kMaxN + kSlice - 1) / kSlice;   // 128

struct Ws {
    uint32_t* keys;   // (rows, n): scaled floats, then keys
    float* smax;      // (rows, S)
    double* ssum;     // (rows, S)
};

size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t ws_bytes(int rows, int n, int S) {
    return up256((size_t)rows * n * 4) + up256((size_t)rows * S * 4) + up256((size_t)rows * S * 8);
}

Ws ws_split(void* base, int rows, int n, int S) {
    char* p = (char*)base;
    Ws w;
    w.keys = (uint32_t*)p;
    p += up256((size_t)rows * n * 4);
    w.smax = (float*)p;
    p += up256((size_t)rows * S * 4);
    w.ssum = (double*)p;
    return w;
}

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

__device__ __forceinline__ double readlane_d(double v, int l) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), l);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// scaled = float(logit / t) (streaming.ts:60-61) and the slice maximum (:64-65; NaN never
// becomes the maximum, fmaxf skips it as the reference's `>` does)
__global__ __launch_bounds__(kSliceThreads) void sample_scale_kernel(
    const float* __restrict__ logits, long ld, int n, double t, Ws ws) {
    __shared__ float red[kSliceThreads / 64];
    const int row = blockIdx.y, S = gridDim.x;
    const float* x = logits + (long)row * ld;
    float* out = (float*)ws.keys + (long)row * n;
    const int base = blockIdx.x * kSlice + threadIdx.x;
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + kSliceThreads * j;
        v[j] = x[i < n ? i : n - 1];   // clamped, not branched: all loads in flight at once
    }
    // every element is computed (past the row's end on a clamped copy) so that the eight
    // divisions overlap; only the stores and the maximum are masked
    float sc[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) sc[j] = (float)((double)v[j] / t);
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + kSliceThreads * j;
        if (i < n) out[i] = sc[j];
        mx = fmaxf(mx, i < n ? sc[j] : -INFINITY);
    }
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0];
        for (int v2 = 1; v2 < kSliceThreads / 64; ++v2) m = fmaxf(m, red[v2]);
        ws.smax[(long)row * S + blockIdx.x] = m;
    }
}

// e = float(exp(scaled - maxL)) (:66-71) stored as key bits(e) + 1, and the slice's sum of e
__global__ __launch_bounds__(kSliceThreads) void sample_exp_kernel(int n, Ws ws) {
    __shared__ double red[kSliceThreads / 64];
    __shared__ float redm[kSliceThreads / 64];
    const int row = blockIdx.y, S = gridDim.x;
    float mx = (int)threadIdx.x < S ? ws.smax[(long)row * S + threadIdx.x] : -INFINITY;
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) redm[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    uint32_t* keys = ws.keys + (long)row * n;
    const int base = blockIdx.x * kSlice + threadIdx.x;
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + kSliceThreads * j;
        v[j] = __uint_as_float(keys[i < n ? i : n - 1]);   // clamped: loads in flight at once
    }
    float e[kPer];   // all eight exps overlap, as in the scale kernel
#pragma unroll
    for (int j = 0; j < kPer; ++j) e[j] = (float)exp((double)v[j] - (double)mx);
    double part = 0.0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + kSliceThreads * j;
        if (i < n) keys[i] = __float_as_uint(e[j]) + 1u;
        part += i < n ? (double)e[j] : 0.0;
    }
    part = wave_sum(part);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0.0;
        for (int v2 = 0; v2 < kSliceThreads / 64; ++v2) s += red[v2];
        ws.ssum[(long)row * S + blockIdx.x] = s;
    }
}

// "a comes before b" in the final order: key descending, then index ascending
__device__ __forceinline__ bool before(unsigned ka, unsigned ia, unsigned kb, unsigned ib) {
    return ka > kb || (ka == kb && ia < ib);
}

// A row's keys as thread tid sees them: slice j holds index tid + 1024 j. Rows up to 32768
// keep them in registers; longer rows read them from the workspace at every use (the row
// stays in L2 / the MALL between the passes).
template <bool REG>
struct RowKeys;

template <>
struct RowKeys<true> {
    unsigned k[kEPT];
    __device__ void init(const uint32_t* src, int n) {
#pragma unroll
        for (int j = 0; j < kEPT; ++j) {
            const int i = threadIdx.x + kThreads * j;
            const unsigned v = src[i < n ? i : n - 1];   // clamped, not branched
            k[j] = i < n ? v : 0u;
        }
    }
    __device__ constexpr int slices() const { return kEPT; }
    __device__ unsigned get(int j) const { return k[j]; }
};

template <>
struct RowKeys<false> {
    const uint32_t* src;
    int n;
    __device__ void init(const uint32_t* s, int nn) {
        src = s;
        n = nn;
    }
    __device__ int slices() const { return (n + kThreads - 1) / kThreads; }
    // any j >= 0: past the row's end it reads the last key (in bounds) and returns 0; a
    // branch around the load instead would wait for each load before issuing the next
    __device__ unsigned get(int j) const {
        const int i = threadIdx.x + kThreads * j;
        const unsigned v = src[i < n ? i : n - 1];
        return i < n ? v : 0u;
    }
};

// The K-th largest key by a 4-pass radix select: kth, how many elements equal to it belong
// to the top K (left), and how many equal it in all (eq_total). Padding (key 0) is left out
// of the counts; there are always at least K real elements.
template <bool REG>
__device__ void radix_select(const RowKeys<REG>& ks, unsigned K, unsigned (*hist)[256],
                             unsigned* wtot, unsigned* sel, unsigned& kth, unsigned& left,
                             unsigned& eq_total) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    unsigned prefix = 0u, pmask = 0u;
    left = K;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int b = lane; b < 256; b += 64) hist[w][b] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ks.slices(); ++j) {
            const unsigned key = ks.get(j);
            if (key != 0u && (key & pmask) == prefix)
                atomicAdd(&hist[w][(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        // thread t < 256 owns bin 255 - t: an inclusive scan over t counts the elements in
        // this bin and every higher one
        unsigned tot = 0u, inc = 0u;
        if (tid < 256) {
            const int b = 255 - tid;
            for (int v = 0; v < kWaves; ++v) tot += hist[v][b];
            inc = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned y = __shfl_up(inc, off, 64);
                if (lane >= off) inc += y;
            }
            if (lane == 63) wtot[w] = inc;
        }
        __syncthreads();
        if (tid < 256) {
            unsigned pre = 0u;
            for (int v = 0; v < w; ++v) pre += wtot[v];
            const unsigned incl = pre + inc, excl = incl - tot;
            if (excl < left && incl >= left) {   // exactly one bin
                sel[0] = 255u - (unsigned)tid;
                sel[1] = left - excl;
                sel[2] = tot;
            }
        }
        __syncthreads();
        prefix |= sel[0] << shift;
        pmask |= 255u << shift;
        left = sel[1];
        eq_total = sel[2];
    }
    kth = prefix;
}

// Appends the lanes' flagged entries of G slices (starting at slice j0) to the LDS list, with
// one LDS atomic per wave on the list's count (which keeps counting past the capacity).
template <int G>
__device__ __forceinline__ void append(const bool (&flag)[G], const unsigned (&key)[G], int j0,
                                       unsigned* count, unsigned* ckey, unsigned* cidx,
                                       unsigned cap) {
    const int tid = threadIdx.x, lane = tid & 63;
    const unsigned long long below = (1ull << lane) - 1ull;
    unsigned long long bal[G];
    unsigned total = 0u;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        bal[j] = __ballot(flag[j]);
        total += (unsigned)__popcll(bal[j]);
    }
    if (total == 0u) return;
    unsigned base = 0u;
    if (lane == 0) base = atomicAdd(count, total);
    base = (unsigned)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const unsigned pos = base + (unsigned)__popcll(bal[j] & below);
        if (flag[j] && pos < cap) {
            ckey[pos] = key[j];
            cidx[pos] = (unsigned)(tid + kThreads * (j0 + j));
        }
        base += (unsigned)__popcll(bal[j]);
    }
}

// Every key in [lo, hi) (lo <= key < hi, key != 0) to the list, in groups of 16 slices.
template <bool REG>
__device__ __forceinline__ void append_range(const RowKeys<REG>& ks, unsigned lo, unsigned hi,
                                             unsigned* count, unsigned* ckey, unsigned* cidx) {
#pragma unroll
    for (int j0 = 0; j0 < ks.slices(); j0 += 16) {
        bool f[16];
        unsigned k[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) k[q] = ks.get(REG ? (j0 + q) % kEPT : j0 + q);
#pragma unroll
        for (int q = 0; q < 16; ++q) f[q] = k[q] != 0u && k[q] >= lo && k[q] < hi;
        append<16>(f, k, j0, count, ckey, cidx, (unsigned)kMaxK);
    }
}

template <bool REG>
__global__ __launch_bounds__(kThreads) void sample_pick_kernel(int n, int S, int K, double top_p,
                                                               const double* __restrict__ u,
                                                               Ws ws,
                                                               uint32_t* __restrict__ out) {
    __shared__ unsigned hist[kWaves][256];   // radix histograms; thread maxima before that
    __shared__ unsigned ckey[kMaxK];
    __shared__ unsigned cidx[kMaxK];
    __shared__ double acc[kMaxK];   // running sums of e along the sorted candidates
    __shared__ double pd[kMaxK];    // e / sumE of the sorted candidates
    __shared__ double sum_s;
    __shared__ unsigned wtot[4];
    __shared__ unsigned sel[3];
    __shared__ unsigned gcount;
    __shared__ unsigned wcount[kWaves];
    __shared__ unsigned flags[2][kWaves];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int row = blockIdx.x;

    RowKeys<REG> ks;
    ks.init(ws.keys + (long)row * n, n);
    unsigned tmax = 0u;
#pragma unroll
    for (int j0 = 0; j0 < ks.slices(); j0 += 16) {   // 16 loads in flight per group
        unsigned k[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) k[q] = ks.get(REG ? (j0 + q) % kEPT : j0 + q);
#pragma unroll
        for (int q = 0; q < 16; ++q) tmax = k[q] > tmax ? k[q] : tmax;
    }
    // sumE from the slice sums: lane l of wave 0 adds slices l, l + 64 (S <= 128), then a
    // fixed butterfly over the lanes
    if (w == 0) {
        const long b = (long)row * S;
        double part = lane < S ? ws.ssum[b + lane] : 0.0;
        if (lane + 64 < S) part += ws.ssum[b + lane + 64];
        part = wave_sum(part);
        if (lane == 0) sum_s = part;
    }
    const double ur = u[row];

    // 1. a lower bound tau for the K-th largest key: the K-th largest of the 1024 thread
    // maxima (K threads hold a key >= tau, so at least K keys are >= tau), to 16 bits (keys
    // are below 2^30 as e <= 1; bits 13..0 of tau stay 0, which only lowers it). Four rounds
    // of 4 bits: wave v counts the maxima >= tau | v << shift, and tau takes the largest v
    // whose count reaches K.
    unsigned* tm = &hist[0][0];
    tm[tid] = tmax;
    if (tid == 0) gcount = 0u;
    __syncthreads();
    unsigned v[kWaves];
#pragma unroll
    for (int q = 0; q < kWaves; ++q) v[q] = tm[q * 64 + lane];
    unsigned tau = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int shift = 26 - 4 * r;
        const unsigned cand = tau | ((unsigned)w << shift);
        unsigned c = 0u;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) c += v[q] >= cand ? 1u : 0u;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
        if (lane == 0) flags[r & 1][w] = c >= (unsigned)K ? 1u : 0u;
        __syncthreads();
        unsigned nv = 0u;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) nv += flags[r & 1][q];
        tau |= (nv - 1u) << shift;   // wave 0's count always reaches K
    }

    // 2. candidates: every key >= tau (they include the top K, ties and all), when they fit
    append_range(ks, tau, 0xffffffffu, &gcount, ckey, cidx);
    __syncthreads();
    unsigned C = gcount;
    if (C > (unsigned)kMaxK) {
        // too many (ties at the bound, or K near the list's capacity): select the K-th key
        // exactly, then take every key above it and the lowest-index ones equal to it
        unsigned kth, left, eq_total;
        radix_select(ks, (unsigned)K, hist, wtot, sel, kth, left, eq_total);
        const unsigned above = (unsigned)K - left;
        if (tid == 0) gcount = 0u;
        __syncthreads();
        const bool all_eq = above + eq_total <= (unsigned)kMaxK;
        append_range(ks, all_eq ? kth : kth + 1u, 0xffffffffu, &gcount, ckey, cidx);
        C = all_eq ? above + eq_total : (unsigned)K;
        if (!all_eq) {
            // index order is slice j, then thread
            unsigned taken = 0u;   // equal elements placed so far (the same in every thread)
#pragma unroll
            for (int j = 0; j < ks.slices(); ++j) {
                if (taken < left) {   // uniform over the workgroup
                    const bool eq = ks.get(j) == kth;
                    const unsigned long long bal = __ballot(eq);
                    const unsigned below_in_wave = __popcll(bal & ((1ull << lane) - 1ull));
                    if (lane == 0) wcount[w] = (unsigned)__popcll(bal);
                    __syncthreads();
                    unsigned pre = 0u, total = 0u;
                    for (int v2 = 0; v2 < kWaves; ++v2) {
                        if (v2 < w) pre += wcount[v2];
                        total += wcount[v2];
                    }
                    const unsigned rank = taken + pre + below_in_wave;
                    if (eq && rank < left) {
                        ckey[above + rank] = kth;
                        cidx[above + rank] = (unsigned)(tid + kThreads * j);
                    }
                    taken += total;
                    __syncthreads();
                }
            }
        }
        __syncthreads();
    }
    const double sum_e = sum_s;

    // 3. sort the C candidates (padded to a power of two with key 0, which sorts last)
    unsigned S2 = 64u;
    while (S2 < C) S2 <<= 1;
    if (S2 == 64u) {
        if (w == 0) {   // one wave, in registers
            unsigned k = lane < (int)C ? ckey[lane] : 0u;
            unsigned ix = lane < (int)C ? cidx[lane] : 0xffffffffu;
#pragma unroll
            for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    const unsigned ok = __shfl_xor(k, stride, 64);
                    const unsigned oi = __shfl_xor(ix, stride, 64);
                    const bool lower = (lane & stride) == 0;
                    const bool desc = (lane & size) == 0;
                    if (before(k, ix, ok, oi) != (lower == desc)) {
                        k = ok;
                        ix = oi;
                    }
                }
            }
            ckey[lane] = k;
            cidx[lane] = ix;
        }
    } else {
        for (unsigned t = C + tid; t < S2; t += kThreads) {
            ckey[t] = 0u;
            cidx[t] = 0xffffffffu;
        }
        __syncthreads();
        for (unsigned size = 2; size <= S2; size <<= 1) {
            for (unsigned stride = size >> 1; stride > 0; stride >>= 1) {
                if ((unsigned)tid < S2 / 2) {
                    const unsigned lo = ((unsigned)tid / stride) * 2u * stride + (unsigned)tid % stride;
                    const unsigned hi = lo + stride;
                    const bool desc = (lo & size) == 0;
                    const unsigned ka = ckey[lo], kb = ckey[hi];
                    const unsigned ia = cidx[lo], ib = cidx[hi];
                    if (before(ka, ia, kb, ib) != desc) {
                        ckey[lo] = kb; ckey[hi] = ka;
                        cidx[lo] = ib; cidx[hi] = ia;
                    }
                }
                __syncthreads();
            }
        }
    }
    __syncthreads();

    // 4. nucleus and draw (:79-96) in the reference's order and in double: e / sumE for the
    // first K entries in parallel, then one running sum of them for the cut and one of e,
    // whose value after entry t is also the draw's `acc` after entry t. Lane 0 of wave 0
    // adds them eight entries at a time (adding 0.0 past the end changes neither sum) before
    // looking for the cut among the eight; the draw is then a parallel search.
    {
        const double sumE = sum_e;
        const int Kp = (K + 7) & ~7;
        for (int t = tid; t < Kp; t += kThreads) {
            const double ev = t < K ? (double)__uint_as_float(ckey[t] - 1u) : 0.0;
            pd[t] = ev / sumE;
            acc[t] = ev;
        }
    }
    __syncthreads();
    if (w == 0) {
        int m = K;
        double nsum = 0.0;
        if (lane == 0) {
            double cum = 0.0, es = 0.0;
            for (int t0 = 0; t0 < K; t0 += 8) {
                double cs[8], ss[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    cum += pd[t0 + q];
                    es += acc[t0 + q];
                    cs[q] = cum;
                    ss[q] = es;
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) acc[t0 + q] = ss[q];
                int hit = 8;
#pragma unroll
                for (int q = 7; q >= 0; --q)
                    if (t0 + q < K && cs[q] >= top_p) hit = q;
                if (hit < 8) {
                    m = t0 + hit + 1;
                    es = ss[hit];
                    break;
                }
            }
            nsum = es;
        }
        m = __builtin_amdgcn_readfirstlane(m);
        nsum = readlane_d(nsum, 0);
        const double thr = ur * nsum;
        unsigned pick = cidx[m - 1];
        for (int base = 0; base < m; base += 64) {
            const int t = base + lane;
            const unsigned long long bal = __ballot(t < m && acc[t] >= thr);
            if (bal) {
                pick = cidx[base + __builtin_ctzll(bal)];
                break;
            }
        }
        if (lane == 0) out[row] = pick;
    }
}

}  // namespace

namespace ssm {

bool sample_ok(int n, int top_k) {
    return n >= 1 && n <= kMaxN && top_k >= 1 && (top_k < n ? top_k : n) <= kMaxK;
}

size_t sample_workspace(int rows, int n) {
    if (rows <= 0 || n <= 0) return 0;
    return ws_bytes(rows, n, (n + kSlice - 1) / kSlice);
}

ssm_status launch_sample(const float* logits, long ld, int rows, int n, double temperature,
                         int top_k, double top_p, const double* u, uint32_t* out,
                         void* workspace, hipStream_t st) {
    if (rows == 0) return SSM_OK;
    const double t = temperature > 1e-7 ? temperature : 1e-7;   // streaming.ts:11,61
    const int K = top_k < n ? top_k : n;                         // slice(0, topK)
    const int S = (n + kSlice - 1) / kSlice;
    const Ws w = ws_split(workspace, rows, n, S);
    sample_scale_kernel<<<dim3(S, rows), kSliceThreads, 0, st>>>(logits, ld, n, t, w);
    ssm_status r = check_launch("sample scale");
    if (r != SSM_OK) return r;
    sample_exp_kernel<<<dim3(S, rows), kSliceThreads, 0, st>>>(n, w);
    r = check_launch("sample exp");
    if (r != SSM_OK) return r;
    if (n <= kRegN)
        sample_pick_kernel<true><<<rows, kThreads, 0, st>>>(n, S, K, top_p, u, w, out);
    else
        sample_pick_kernel<false><<<rows, kThreads, 0, st>>>(n, S, K, top_p, u, w, out);
    return check_launch("sample pick");
}

}  // namespace ssm

static_assert(kMaxSlices <= 128, "the pick kernel adds at most two slice sums per lane");
static_assert(kEPT % 16 == 0, "register keys are visited in groups of 16 slices");
static_assert(kMaxSlices <= kSliceThreads, "one slice maximum per exp-kernel thread");

extern "C" size_t ssm_sample_workspace(int rows, int n) { return ssm::sample_workspace(rows, n); }

// ---------------------------------------------------------------- allocation-free variant
// ssm_sample_noalloc runs the kernels of ssm_sample with their workspace in `scratch`, a
// file-scope device array of kScratchBytes that each GPU holds from the library's load until
// the process ends. Host code never passes the array's name to a kernel (on the host it is
// only a stand-in symbol): its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and kept in g_scratch. Every call on a GPU
// shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race on it.
// The kernels write every workspace slot before they read it, so nothing is cleared.
namespace {

constexpr size_t kScratchBytes = (size_t)32 << 20;   // 32 MiB per GPU
constexpr int kMaxDevices = 64;

__device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

}  // namespace

namespace ssm {

// Device address of `scratch` on the current device (looked up on the first call per device).
ssm_status sample_scratch(void** out) {
    int dev = 0;
    SSM_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(SSM_ERR_INVALID_ARG, "sample scratch: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return from_hip(e, "hipGetSymbolAddress(sample scratch)");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return SSM_OK;
}

}  // namespace ssm

extern "C" ssm_status ssm_sample_noalloc(const float* logits, long ld, int rows, int n,
                                         double temperature, int top_k, double top_p,
                                         const double* u, uint32_t* out, void* stream) {
    SSM_REQUIRE(logits && u && out, "ssm_sample_noalloc: null logits/u/out");
    SSM_REQUIRE(rows >= 0 && n >= 1 && ld >= n, "ssm_sample_noalloc: bad shape");
    SSM_REQUIRE(top_k >= 1, "ssm_sample_noalloc: topK must be at least 1");
    if (!ssm::sample_ok(n, top_k))
        return ssm::fail(SSM_ERR_UNSUPPORTED,
                         "ssm_sample_noalloc: needs n <= %d and topK <= %d (n=%d topK=%d)", kMaxN,
                         kMaxK, n, top_k);
    const size_t need = ssm::sample_workspace(rows, n);
    if (need > kScratchBytes)
        return ssm::fail(SSM_ERR_UNSUPPORTED,
                         "ssm_sample_noalloc: %d rows of %d logits need %zu bytes of scratch; the "
                         "static scratch holds %zu (use ssm_sample with a workspace)",
                         rows, n, need, kScratchBytes);
    if (rows == 0) return SSM_OK;
    void* ws = nullptr;
    ssm_status r = ssm::sample_scratch(&ws);
    if (r != SSM_OK) return r;
    return ssm::launch_sample(logits, ld, rows, n, temperature, top_k, top_p, u, out, ws,
                              (hipStream_t)stream);
}

extern "C" ssm_status ssm_sample(const float* logits, long ld, int rows, int n,
                                 double temperature, int top_k, double top_p, const double* u,
                                 uint32_t* out, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    SSM_REQUIRE(logits && u && out, "ssm_sample: null logits/u/out");
    SSM_REQUIRE(rows >= 0 && n >= 1 && ld >= n, "ssm_sample: bad shape");
    SSM_REQUIRE(top_k >= 1, "ssm_sample: topK must be at least 1");
    if (!ssm::sample_ok(n, top_k))
        return ssm::fail(SSM_ERR_UNSUPPORTED,
                         "ssm_sample: needs n <= %d and topK <= %d (n=%d topK=%d)", kMaxN, kMaxK,
                         n, top_k);
    SSM_REQUIRE(rows == 0 || (workspace && workspace_bytes >= ssm::sample_workspace(rows, n)),
                "ssm_sample: workspace smaller than ssm_sample_workspace(rows, n)");
    return ssm::launch_sample(logits, ld, rows, n, temperature, top_k, top_p, u, out, workspace,
                              (hipStream_t)stream);
}
