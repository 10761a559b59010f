// Shared helpers for the HXQ HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "hxq.h"

namespace hxq {

// ---------------------------------------------------------------------------
// Error reporting: every entry point returns an hxq_status and leaves a
// human-readable message in a thread-local slot read by hxq_last_error().
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
void clear_error();

#define HXQ_REQUIRE(cond, msg)                                                 \
    do {                                                                       \
        if (!(cond)) {                                                         \
            ::hxq::set_error(std::string(__func__) + ": " + (msg));            \
            return HXQ_ERR_INVALID_ARG;                                        \
        }                                                                      \
    } while (0)

#define HXQ_HIP_TRY(expr)                                                      \
    do {                                                                       \
        hipError_t e_ = (expr);                                                \
        if (e_ != hipSuccess) {                                                \
            ::hxq::set_error(std::string(__func__) + ": " #expr " -> " +      \
                             hipGetErrorString(e_));                           \
            return HXQ_ERR_HIP;                                                \
        }                                                                      \
    } while (0)

// Launch check: catches invalid launch configurations immediately.
#define HXQ_LAUNCH_CHECK() HXQ_HIP_TRY(hipGetLastError())

// Number of compute units of the current device (cached per device).
int device_cu_count();

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Numeric conversions (device)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// fp32 -> fp16, round to nearest even (the conversion the ISA performs).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Native 4 x u32 vector (usable with the nontemporal load builtin).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ float load_act(const void *p, int64_t i) {
    if constexpr (DT == HXQ_F32) return static_cast<const float *>(p)[i];
    else if constexpr (DT == HXQ_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_act(void *p, int64_t i, float v) {
    if constexpr (DT == HXQ_F32) static_cast<float *>(p)[i] = v;
    else if constexpr (DT == HXQ_BF16) static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
    else static_cast<uint16_t *>(p)[i] = f32_to_f16(v);
}

// The affine dequant step with its two roundings kept apart:
// fl(fl(c * s) + o).  Contraction into an FMA would change the bits.
__device__ __forceinline__ float affine_exact(float c, float s, float o) {
#pragma clang fp contract(off)
    float t = c * s;
    return t + o;
}

// Workgroup barrier that orders LDS only: it waits for this wave's LDS
// traffic (lgkmcnt) but leaves global loads in flight, so prefetched data
// can stream in across the barrier.  Use it where no global stores need to
// become visible to other waves.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Raw buffer resource over [base, base + bytes): loads at or past `bytes`
// return zero (hardware range check).  bytes must fit in 32 bits.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                             static_cast<int>(static_cast<uint32_t>(bytes)),
                                             0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

__device__ __forceinline__ float buf_loadf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ int32_t buf_loadi(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Full wave64 sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

}  // namespace hxq
