// Model glue for gfx950: RMSNorm, gated RMSNorm (Mamba-2), embedding gather, last-row
// gather, greedy argmax and the counter-based weight initialiser. All row kernels use one
// workgroup per row with a block reduction; they are HBM-bound.
#include "common.hpp"
#include "glue.hpp"

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
    return t;
}

__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const float* __restrict__ x, long ldx,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ y, long ldy, int n,
                                                         float eps) {
    __shared__ float red[kBlock / 64];
    const float* xr = x + (long)blockIdx.x * ldx;
    float* yr = y + (long)blockIdx.x * ldy;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) ss = fmaf(xr[i], xr[i], ss);
    const float r = rsqrtf(block_sum(ss, red) / n + eps);
    for (int i = threadIdx.x; i < n; i += kBlock) yr[i] = xr[i] * r * w[i];
}

// y = norm_g(x * silu(z)) * w over G groups of n/G. Row values are staged in LDS-free
// registers by re-reading x and z (rows are short and L2 resident).
template <typename OT>
__global__ __launch_bounds__(kBlock) void gated_rmsnorm_kernel(
    const float* __restrict__ x, long ldx, const float* __restrict__ z, long ldz,
    const float* __restrict__ w, OT* __restrict__ y, long ldy, int n, int G, float eps) {
    __shared__ float red[kBlock / 64];
    const int gs = n / G;
    const float* xr = x + (long)blockIdx.x * ldx;
    const float* zr = z + (long)blockIdx.x * ldz;
    OT* yr = y + (long)blockIdx.x * ldy;
    for (int g = 0; g < G; ++g) {
        float ss = 0.f;
        for (int i = g * gs + threadIdx.x; i < (g + 1) * gs; i += kBlock) {
            const float v = xr[i] * ssm::silu(zr[i]);
            ss = fmaf(v, v, ss);
        }
        const float r = rsqrtf(block_sum(ss, red) / gs + eps);
        for (int i = g * gs + threadIdx.x; i < (g + 1) * gs; i += kBlock)
            yr[i] = (OT)(xr[i] * ssm::silu(zr[i]) * r * w[i]);
    }
}

// x (rows, cols) fp32, row stride ldx -> y bf16 (round to nearest even), row stride ldy.
// V4: cols, ldx, ldy multiples of 4 and 16/8-byte aligned rows, four values per thread.
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
template <bool V4>
__global__ __launch_bounds__(256) void cast_bf16_kernel(const float* __restrict__ x, long ldx,
                                                        __bf16* __restrict__ y, long ldy,
                                                        long rows, int cols) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int cw = V4 ? cols / 4 : cols;
    if (i >= rows * cw) return;
    const long r = i / cw;
    const int c = (int)(i % cw);
    if constexpr (V4) {
        // streaming: each value is read and written once
        const float4 v = ssm::load_nt4(x + r * ldx + 4 * c);
        __builtin_nontemporal_store(bf16x4_t{(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w},
                                    reinterpret_cast<bf16x4_t*>(y + r * ldy + 4 * c));
    } else {
        y[r * ldy + c] = (__bf16)x[r * ldx + c];
    }
}

// One group, rows of n <= 4 * 256 * R floats held in registers: x and z are read once, as
// float4 (n, ldx, ldz multiples of 4, rows 16-byte aligned); same arithmetic per element as
// gated_rmsnorm_kernel, the sum of squares added per thread and then across the block.
template <typename OT, int R>
__global__ __launch_bounds__(kBlock) void gated_rmsnorm_row_kernel(
    const float* __restrict__ x, long ldx, const float* __restrict__ z, long ldz,
    const float* __restrict__ w, OT* __restrict__ y, long ldy, int n, float eps) {
    __shared__ float red[kBlock / 64];
    const float* xr = x + (long)blockIdx.x * ldx;
    const float* zr = z + (long)blockIdx.x * ldz;
    OT* yr = y + (long)blockIdx.x * ldy;
    float4 u[R];
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int e = 4 * (threadIdx.x + kBlock * r);
        u[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e < n) {
            const float4 xv = ssm::load_nt4(xr + e);   // x, z and y stream (used once)
            const float4 zv = ssm::load_nt4(zr + e);
            u[r] = make_float4(xv.x * ssm::silu(zv.x), xv.y * ssm::silu(zv.y),
                               xv.z * ssm::silu(zv.z), xv.w * ssm::silu(zv.w));
        }
        ss = fmaf(u[r].x, u[r].x, ss);
        ss = fmaf(u[r].y, u[r].y, ss);
        ss = fmaf(u[r].z, u[r].z, ss);
        ss = fmaf(u[r].w, u[r].w, ss);
    }
    const float rs = rsqrtf(block_sum(ss, red) / n + eps);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int e = 4 * (threadIdx.x + kBlock * r);
        if (e >= n) continue;
        const float4 wv = *reinterpret_cast<const float4*>(w + e);
        const float o0 = u[r].x * rs * wv.x, o1 = u[r].y * rs * wv.y, o2 = u[r].z * rs * wv.z,
                    o3 = u[r].w * rs * wv.w;
        if constexpr (sizeof(OT) == 2) {
            __builtin_nontemporal_store(bf16x4_t{(__bf16)o0, (__bf16)o1, (__bf16)o2, (__bf16)o3},
                                        reinterpret_cast<bf16x4_t*>(yr + e));
        } else {
            ssm::store_nt4(make_float4(o0, o1, o2, o3), yr + e);
        }
    }
}

__global__ void embed_kernel(const uint32_t* __restrict__ ids, const float* __restrict__ emb,
                             float* __restrict__ out, long T, int d, int V, int* bad) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * d) return;
    const long t = i / d;
    const int c = (int)(i % d);
    uint32_t id = ids[t];
    if (id >= (uint32_t)V) {
        if (c == 0) atomicOr(bad, 1);
        id = 0;
    }
    out[i] = emb[(long)id * d + c];
}

__global__ void gather_rows_kernel(const float* __restrict__ x, long row_stride, long first,
                                   float* __restrict__ out, int rows, int d) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)rows * d) return;
    const int r = (int)(i / d), c = (int)(i % d);
    out[i] = x[(first + (long)r * row_stride) * d + c];
}

// Greedy pick: largest logit, lowest index among equal maxima (the order a stable
// descending sort gives, src/session/streaming.ts:74-75). NaN never wins. One 1024-thread
// workgroup per row: groups of eight float4 loads keep a whole vocabulary row (32000 logits
// = 128 KB) in flight at once; each thread scans ascending indices, then wave shuffles and
// LDS combine (value, index) pairs.
constexpr int kArgBlock = 1024;

__device__ __forceinline__ void arg_take(float v, int i, float& best, int& bi, int n) {
    if (v > best || (bi == n && v == best)) { best = v; bi = i; }
}

__device__ __forceinline__ void arg_merge(float ov, int oi, float& best, int& bi) {
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
}

__global__ __launch_bounds__(kArgBlock) void argmax_kernel(const float* __restrict__ x, long ldx,
                                                           int n, int vec, uint32_t* __restrict__ out) {
    __shared__ float sv[kArgBlock / 64];
    __shared__ int si[kArgBlock / 64];
    const float* xr = x + (long)blockIdx.x * ldx;
    float best = -INFINITY;
    int bi = n;
    int tail = 0;
    if (vec && n >= 4) {
        const int n4 = n / 4;
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        // eight loads per group from clamped (in-bounds) addresses, all in flight before the
        // first is used; a branch around each load would wait for it before the next
        for (int g = threadIdx.x; g < n4; g += 8 * kArgBlock) {
            float4 v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int i = g + q * kArgBlock;
                v[q] = x4[i < n4 ? i : n4 - 1];
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int i = g + q * kArgBlock;
                if (i < n4) {
                    arg_take(v[q].x, 4 * i, best, bi, n);
                    arg_take(v[q].y, 4 * i + 1, best, bi, n);
                    arg_take(v[q].z, 4 * i + 2, best, bi, n);
                    arg_take(v[q].w, 4 * i + 3, best, bi, n);
                }
            }
        }
        tail = 4 * n4;
    }
    for (int i = tail + threadIdx.x; i < n; i += kArgBlock) arg_take(xr[i], i, best, bi, n);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        arg_merge(ov, oi, best, bi);
    }
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) { sv[w] = best; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kArgBlock / 64; ++k) arg_merge(sv[k], si[k], best, bi);
        out[blockIdx.x] = bi < n ? (uint32_t)bi : 0u;
    }
}

// ---- counter-based random init: value i of tensor `tid` depends only on (seed, tid, i)
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float unif01(uint64_t key, uint64_t i) {
    // (0, 1): 24 random bits, offset by half an ulp so 0 never appears
    return ((float)(mix64(key ^ mix64(i)) >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

__global__ void init_kernel(float* __restrict__ p, long n, int kind, float a0, float a1,
                            uint64_t key, int row) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v;
    switch (kind) {
        case SSM_INIT_CONST: v = a0; break;
        case SSM_INIT_UNIFORM: v = a0 + (a1 - a0) * unif01(key, (uint64_t)i); break;
        case SSM_INIT_NORMAL: {
            const float u1 = unif01(key, 2 * (uint64_t)i), u2 = unif01(key, 2 * (uint64_t)i + 1);
            v = a0 * sqrtf(-2.f * logf(u1)) * cospif(2.f * u2);
            break;
        }
        case SSM_INIT_ARANGE_LOG: v = logf((float)(i % row) + 1.f); break;
        case SSM_INIT_LOG_UNIFORM: v = logf(a0 + (a1 - a0) * unif01(key, (uint64_t)i)); break;
        default: {  // SSM_INIT_DT_BIAS: softplus^-1 of dt ~ log-uniform[a0, a1], dt >= 1e-4
            const float la = logf(a0), lb = logf(a1);
            float dt = expf(la + (lb - la) * unif01(key, (uint64_t)i));
            dt = fmaxf(dt, 1e-4f);
            v = dt + logf(-expm1f(-dt));
            break;
        }
    }
    p[i] = v;
}

__global__ void neg_exp_kernel(const float* __restrict__ x, float* __restrict__ y, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = -expf(x[i]);
}

}  // namespace

namespace ssm {

ssm_status launch_embed(const uint32_t* ids, const float* emb, float* out, long T, int d, int V,
                        int* bad, hipStream_t st) {
    const long n = T * d;
    if (n == 0) return SSM_OK;
    embed_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(ids, emb, out, T, d, V, bad);
    return check_launch("embed");
}

ssm_status launch_gather_rows(const float* x, long row_stride, long first, float* out, int rows,
                              int d, hipStream_t st) {
    const long n = (long)rows * d;
    if (n == 0) return SSM_OK;
    gather_rows_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(x, row_stride, first, out, rows, d);
    return check_launch("gather_rows");
}

ssm_status launch_argmax(const float* x, long ldx, int rows, int n, uint32_t* out,
                         hipStream_t st) {
    if (rows == 0) return SSM_OK;
    const int vec = ((uintptr_t)x % 16 == 0 && ldx % 4 == 0) ? 1 : 0;
    argmax_kernel<<<rows, kArgBlock, 0, st>>>(x, ldx, n, vec, out);
    return check_launch("argmax");
}

ssm_status launch_init(float* p, long n, int kind, float a0, float a1, uint64_t seed,
                       uint64_t tensor_id, int row, hipStream_t st) {
    if (n == 0) return SSM_OK;
    const uint64_t key = seed * 0x2545F4914F6CDD1Dull ^ (tensor_id * 0x9E3779B97F4A7C15ull + 1);
    init_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(p, n, kind, a0, a1, key, row > 0 ? row : 1);
    return check_launch("init");
}

ssm_status launch_neg_exp(const float* x, float* y, long n, hipStream_t st) {
    if (n == 0) return SSM_OK;
    neg_exp_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(x, y, n);
    return check_launch("neg_exp");
}

ssm_status launch_cast_bf16(const float* x, long ldx, __bf16* y, long ldy, long rows, int cols,
                            hipStream_t st) {
    const long n = rows * cols;
    if (n == 0) return SSM_OK;
    const bool v4 = cols % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
                    ((uintptr_t)y & 7) == 0;
    if (v4) cast_bf16_kernel<true><<<(unsigned)cdiv(n / 4, 256), 256, 0, st>>>(x, ldx, y, ldy, rows, cols);
    else cast_bf16_kernel<false><<<(unsigned)cdiv(n, 256), 256, 0, st>>>(x, ldx, y, ldy, rows, cols);
    return check_launch("cast_bf16");
}

ssm_status launch_gated_rmsnorm_bf16(const float* x, long ldx, const float* z, long ldz,
                                     const float* w, __bf16* y, long ldy, int M, int n, int G,
                                     float eps, hipStream_t st) {
    if (M == 0) return SSM_OK;
    const bool rowreg = G == 1 && n % 4 == 0 && n <= 4 * kBlock * 4 && ldx % 4 == 0 &&
                        ldz % 4 == 0 && ldy % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
                        ((uintptr_t)z & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
                        ((uintptr_t)y & 7) == 0;
    if (rowreg) gated_rmsnorm_row_kernel<__bf16, 4><<<M, kBlock, 0, st>>>(x, ldx, z, ldz, w, y, ldy, n, eps);
    else gated_rmsnorm_kernel<<<M, kBlock, 0, st>>>(x, ldx, z, ldz, w, y, ldy, n, G, eps);
    return check_launch("gated_rmsnorm_bf16");
}

}  // namespace ssm

extern "C" ssm_status ssm_rmsnorm(const float* x, long ldx, const float* w, float* y, long ldy,
                                  int M, int n, float eps, void* stream) {
    SSM_REQUIRE(x && w && y && M >= 0 && n > 0 && ldx >= n && ldy >= n, "ssm_rmsnorm: bad args");
    if (M == 0) return SSM_OK;
    rmsnorm_kernel<<<M, kBlock, 0, (hipStream_t)stream>>>(x, ldx, w, y, ldy, n, eps);
    return ssm::check_launch("rmsnorm");
}

extern "C" ssm_status ssm_gated_rmsnorm(const float* x, long ldx, const float* z, long ldz,
                                        const float* w, float* y, long ldy, int M, int n, int G,
                                        float eps, void* stream) {
    SSM_REQUIRE(x && z && w && y && M >= 0 && n > 0 && G > 0 && n % G == 0 && ldx >= n &&
                    ldz >= n && ldy >= n,
                "ssm_gated_rmsnorm: bad args");
    if (M == 0) return SSM_OK;
    const bool rowreg = G == 1 && n % 4 == 0 && n <= 4 * kBlock * 4 && ldx % 4 == 0 &&
                        ldz % 4 == 0 && ldy % 4 == 0 && (((uintptr_t)x | (uintptr_t)z |
                                                          (uintptr_t)w | (uintptr_t)y) & 15) == 0;
    if (rowreg)
        gated_rmsnorm_row_kernel<float, 4><<<M, kBlock, 0, (hipStream_t)stream>>>(
            x, ldx, z, ldz, w, y, ldy, n, eps);
    else
        gated_rmsnorm_kernel<<<M, kBlock, 0, (hipStream_t)stream>>>(x, ldx, z, ldz, w, y, ldy, n,
                                                                    G, eps);
    return ssm::check_launch("gated_rmsnorm");
}

extern "C" ssm_status ssm_argmax(const float* x, long ldx, int rows, int n, uint32_t* out,
                                 void* stream) {
    SSM_REQUIRE(x && out, "ssm_argmax: null x/out");
    SSM_REQUIRE(rows >= 0 && n >= 1 && ldx >= n, "ssm_argmax: bad shape");
    return ssm::launch_argmax(x, ldx, rows, n, out, (hipStream_t)stream);
}
