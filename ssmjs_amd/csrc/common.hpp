// Shared helpers for the gfx950 SSM kernels and the C ABI (include/ssm_hip.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/ssm_hip.h"

namespace ssm {

// Thread-local message behind ssm_last_error().
void set_error(const char* fmt, ...);
ssm_status fail(ssm_status code, const char* fmt, ...);
// Map a HIP error from a launch or runtime call to SSM_ERR_HIP (or GPU_UNAVAILABLE / OOM).
ssm_status from_hip(hipError_t e, const char* what);
// hipGetLastError after a launch (an injected "launch" fault makes it report a failure).
ssm_status check_launch(const char* what);
// hipMalloc, failing with hipErrorOutOfMemory under an injected "alloc" fault.
hipError_t dev_malloc(void** p, size_t bytes);

inline long cdiv(long a, long b) { return (a + b - 1) / b; }

}  // namespace ssm

#define SSM_HIP_TRY(expr)                                                   \
    do {                                                                    \
        hipError_t _e = (expr);                                             \
        if (_e != hipSuccess) return ::ssm::from_hip(_e, #expr);            \
    } while (0)

#define SSM_REQUIRE(cond, ...)                                              \
    do {                                                                    \
        if (!(cond)) return ::ssm::fail(SSM_ERR_INVALID_ARG, __VA_ARGS__);  \
    } while (0)

// ---------------------------------------------------------------- device math
namespace ssm {

constexpr float kLog2e = 1.4426950408889634f;

// v_exp_f32: 2^x.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// softplus(x) = log(1 + e^x), written as max(x,0) + log1p(e^-|x|) so it neither overflows
// nor loses the small tail; x > 20 returns x (the float32 value of log1p(e^-20) is below
// half an ulp of 20).
__device__ __forceinline__ float softplus(float x) {
    if (x > 20.f) return x;
    return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
}

__device__ __forceinline__ float silu(float z) { return z / (1.f + expf(-z)); }

// softplus on the hardware exp/log (v_exp_f32 / v_log_f32). Below -8 it returns e^x, whose
// relative distance from log1p(e^x) is under e^x / 2 < 1.7e-4 of a value < 3.4e-4, i.e. an
// absolute error below 6e-8; above 20 it returns x. In between log(1 + e^x) has
// 1 + e^x >= 1.0003, so no cancellation.
__device__ __forceinline__ float softplus_fast(float x) {
    if (x > 20.f) return x;
    const float e = __expf(x);
    return x < -8.f ? e : __logf(1.f + e);
}

// z * sigmoid(z) with v_exp_f32 and v_rcp_f32 (about 1 ulp each).
__device__ __forceinline__ float silu_fast(float z) {
    return z * __builtin_amdgcn_rcpf(1.f + __expf(-z));
}

// softplus_fast without branches (every lane evaluates both transcendentals): v_exp_f32 and
// v_log_f32 (log2) times ln 2; same three regions and bounds as softplus_fast.
__device__ __forceinline__ float softplus_sel(float x) {
    const float e = ex2(fminf(x, 20.f) * kLog2e);
    const float l = __builtin_amdgcn_logf(1.f + e) * 0.6931471805599453f;
    return x > 20.f ? x : (x < -8.f ? e : l);
}

// ---------------------------------------------------------------- buffer access
// Raw buffer resources (stride 0; dword 3 = 0x00020000 on gfx9): a lane whose byte offset
// lies at or past num_records reads zeros and its stores are dropped, so a descriptor that
// ends with a tensor's last valid row makes tail rows branch-free. Offsets are 32-bit.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

template <typename V>
__device__ __forceinline__ V bload16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ float bload4(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ void bstore4(float v, __amdgpu_buffer_rsrc_t r, unsigned off) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, 0);
}

__device__ __forceinline__ void bstore16(float4 v, __amdgpu_buffer_rsrc_t r, unsigned off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
}

// ---------------------------------------------------------------- streaming access
// Non-temporal loads and stores for data a launch touches once (its inputs read once, its
// outputs read only by a later launch): the caches keep their lines for the data that is
// reused. On MI355X a 137 MB read + write stream runs at 6.3 TB/s this way and at 4.8 TB/s
// with ordinary accesses.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 load_nt4(const float* p) {
    const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void store_nt4(float4 v, float* p) {
    __builtin_nontemporal_store(f32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4_t*>(p));
}

// the buffer forms: cache-policy bit nt (bit 1 of the instruction's cache-policy field)
constexpr int kPolicyNT = 2;

template <typename V>
__device__ __forceinline__ V bload16_nt(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kPolicyNT));
}

__device__ __forceinline__ float bload4_nt(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kPolicyNT));
}

__device__ __forceinline__ void bstore4_nt(float v, __amdgpu_buffer_rsrc_t r, unsigned off) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, kPolicyNT);
}

__device__ __forceinline__ void bstore16_nt(float4 v, __amdgpu_buffer_rsrc_t r, unsigned off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kPolicyNT);
}

}  // namespace ssm
