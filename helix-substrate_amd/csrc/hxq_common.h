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
constexpr int kPairCodes = 4096;  // largest pair (2-D) codebook

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

// The affine as one rounding, fl(c * s + o): the form of the reference's GPU
// kernel (a contracted multiply-add) and what the GEMMs take for 16-bit
// operands, which round it to bf16/fp16 right after (2^-9 relative against
// an fp32 difference of at most one ulp).
__device__ __forceinline__ float affine_fma(float c, float s, float o) { return fmaf(c, s, o); }

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

typedef __attribute__((address_space(3))) const float lds_cfloat;

// LDS byte address of a pointer into LDS.
__device__ __forceinline__ uint32_t lds_offset_of(const float *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cfloat *)p));
}

// Codebook lookup of byte B (0..3) of the packed index word w in a table
// that starts at LDS address 0 (the caller checks lds_offset_of(table) == 0).
//   NREP == 64: entry stride is 256 bytes and the lane's replica offset
//   (lane*4 < 256) fits in the low byte, so the LDS byte address is
//   {0, 0, w.byte[B], lane_off} -- one v_perm_b32 builds it, and the load
//   goes straight to that address (no base add).
//   NREP == 32: shift/mask arithmetic.
template <int NREP, int B>
__device__ __forceinline__ float tbl_lookup0(uint32_t lane_off, uint32_t w) {
    uint32_t addr;
    if constexpr (NREP == 64) {
        constexpr uint32_t sel = (12u << 24) | (12u << 16) | (static_cast<uint32_t>(B) << 8) | 4u;
        addr = __builtin_amdgcn_perm(lane_off, w, sel);
    } else {
        addr = ((w >> (8 * B)) & 0xffu) * (NREP * 4) + lane_off;
    }
    return *reinterpret_cast<lds_cfloat *>(static_cast<uintptr_t>(addr));
}

// Wave64 sum via DPP; the total lands in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
    return v + __int_as_float(s);
}

__device__ __forceinline__ float wave_sum_lane63(float v) {
    v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);  // row_mirror: every lane holds its row's sum
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;                    // lane 63 holds the wave total
}

// Sum over each aligned group of L lanes (L a power of two <= 64); every lane
// of a group ends with the group's total.  Lane distance 1 and 2 (quad
// permutes), 4 (row_half_mirror: the quads hold equal sums by then, so the
// mirrored lane of the other quad stands for lane ^ 4), 8 (row_ror:8), 16 and
// 32 (v_permlane16_swap / v_permlane32_swap of the value with itself: the two
// results are the lane's value and that of lane ^ 16 / ^ 32).  Fixed order,
// deterministic, and no LDS round trip (an xor shuffle is an LDS permute).
// Every lane of the wave must be active.
__device__ __forceinline__ float lane_group_sum(float v, int L) {
    if (L > 1) v = dpp_add<0xb1, 0xf>(v);
    if (L > 2) v = dpp_add<0x4e, 0xf>(v);
    if (L > 4) v = dpp_add<0x141, 0xf>(v);
    if (L > 8) v = dpp_add<0x128, 0xf>(v);
    if (L > 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if (L > 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return v;
}

// Full wave64 sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) { return lane_group_sum(v, kWave); }

// A value the kernel only reads and that nothing writes during the launch,
// loaded with a scalar load through the constant address space (the value
// lands in scalar registers; the load counts in lgkmcnt only, so using it
// waits for no vector-memory load).  The address must be wave-uniform.
template <typename T>
__device__ __forceinline__ T kload(const T &ref) {
#if __HIP_DEVICE_COMPILE__
    typedef __attribute__((address_space(4))) const T cT;
    return *__builtin_bit_cast(const cT *, &ref);
#else
    return ref;  // the host pass only parses device functions
#endif
}

}  // namespace hxq
