// Bit-exact reconstruction of HXQ weights (fp32).
//
// Replaces CDNAv3Reader.reconstruct / reconstruct_block
// (helix_substrate/hxq_reader_v3.py:102-187): W = codebook[idx], then the
// per-group affine extension fl(fl(c*s)+o), then sidecar values REPLACE the
// entries at their positions (reader semantics, hxq_reader_v3.py:128-133).
//
// Kernel 1 streams 16 index bytes per lane (one dwordx4 load) and writes 16
// fp32 weights (four dwordx4 stores).  The 1 KiB codebook sits in LDS.
// Kernel 2 walks the CSR sidecar, one thread per output row, in stored order,
// so a duplicated position resolves like numpy's fancy assignment (last wins).
#include "hxq_common.h"

namespace hxq {

template <bool AFFINE>
__global__ __launch_bounds__(256) void dequant_dense_kernel(
    const uint8_t *__restrict__ idx, const float *__restrict__ cb,
    const float *__restrict__ gs, const float *__restrict__ go, int32_t group,
    int64_t K, int64_t row_begin, int64_t n_vec16, float *__restrict__ w) {
    __shared__ float tbl[256];
    tbl[threadIdx.x] = cb[threadIdx.x];
    __syncthreads();

    const int64_t vec_per_row = K / 16;
    const int64_t ngroups = AFFINE ? K / group : 0;
    for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < n_vec16;
         v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = v / vec_per_row;             // row within the block
        const int64_t k0 = (v - r * vec_per_row) * 16; // first column
        const int64_t row = row_begin + r;
        const uint4 q = *reinterpret_cast<const uint4 *>(idx + row * K + k0);
        float s = 1.f, o = 0.f;
        if constexpr (AFFINE) {
            const int64_t g = row * ngroups + k0 / group;
            s = gs[g];
            o = go[g];
        }
        const uint32_t words[4] = {q.x, q.y, q.z, q.w};
        float out[16];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float c = tbl[(words[d] >> (8 * b)) & 0xffu];
                out[d * 4 + b] = AFFINE ? affine_exact(c, s, o) : c;
            }
        }
        float4 *dst = reinterpret_cast<float4 *>(w + r * K + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dst[j] = make_float4(out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]);
    }
}

__global__ __launch_bounds__(256) void dequant_sidecar_kernel(
    const int32_t *__restrict__ row_ptr, const int32_t *__restrict__ col,
    const float *__restrict__ val, int64_t K, int64_t row_begin, int64_t rows,
    float *__restrict__ w) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const int64_t row = row_begin + r;
    for (int32_t j = row_ptr[row]; j < row_ptr[row + 1]; ++j)
        w[r * K + col[j]] = val[j];
}

// Reconstruction for the packed / pair / uint16-index formats: one thread per
// 16 weights.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_fmt_kernel(
    const uint8_t *__restrict__ idx, const float *__restrict__ cb, int32_t n_codes,
    const float *__restrict__ gs, const float *__restrict__ go, int32_t group, int64_t K,
    int64_t row_begin, int64_t n_vec16, float *__restrict__ w) {
    constexpr bool PAIR = FMT == HXQ_FMT_VQ2_U16 || FMT == HXQ_FMT_VQ2_P12;
    constexpr bool U16 = FMT == HXQ_FMT_SCALAR_U16;
    constexpr int QB = U16 ? 32 : FMT == HXQ_FMT_VQ2_U16 ? 16 : 12;
    __shared__ float2 tbl[PAIR ? kPairCodes : 1];
    __shared__ float tbl1[U16 ? kPairCodes : 1];
    if constexpr (PAIR) {
        for (int j = threadIdx.x; j < kPairCodes; j += blockDim.x)
            tbl[j] = j < n_codes ? make_float2(cb[2 * j], cb[2 * j + 1]) : make_float2(0.f, 0.f);
        __syncthreads();
    }
    if constexpr (U16) {
        for (int j = threadIdx.x; j < kPairCodes; j += blockDim.x) tbl1[j] = j < n_codes ? cb[j] : 0.f;
        __syncthreads();
    }
    const int64_t vec_per_row = K / 16;
    const int64_t row_bytes = vec_per_row * QB;
    for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < n_vec16;
         v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = v / vec_per_row;
        const int64_t c16 = v - r * vec_per_row;
        const int64_t row = row_begin + r;
        const uint32_t *src = reinterpret_cast<const uint32_t *>(idx + row * row_bytes + c16 * QB);
        const uint32_t q[4] = {src[0], src[1], src[2], QB >= 16 ? src[3] : 0u};
        auto field = [&](int bit, int width) -> uint32_t {
            const int d = bit >> 5, sh = bit & 31;
            const uint32_t x = sh + width <= 32 ? q[d] >> sh : __builtin_amdgcn_alignbit(q[d + 1], q[d], sh);
            return x & ((1u << width) - 1u);
        };
        float out[16];
        if constexpr (U16) {
            const uint4 hi = *reinterpret_cast<const uint4 *>(src + 4);
            const uint32_t q2[8] = {q[0], q[1], q[2], q[3], hi.x, hi.y, hi.z, hi.w};
            float s = 1.f, o = 0.f;
            if (gs != nullptr) {
                const int64_t g = row * (K / group) + c16 * 16 / group;
                s = gs[g];
                o = go[g];
            }
#pragma unroll
            for (int f = 0; f < 16; ++f) {
                const float c = tbl1[(q2[f >> 1] >> (16 * (f & 1))) & (kPairCodes - 1u)];
                out[f] = gs != nullptr ? affine_exact(c, s, o) : c;
            }
        } else if constexpr (FMT == HXQ_FMT_AF6) {
            const int64_t g = row * (K / group) + c16 * 16 / group;
            const float s = gs[g], o = go[g];
#pragma unroll
            for (int f = 0; f < 16; ++f) out[f] = affine_exact(static_cast<float>(field(6 * f, 6)), s, o);
        } else {
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const uint32_t id = FMT == HXQ_FMT_VQ2_U16 ? (q[p >> 1] >> (16 * (p & 1))) & (kPairCodes - 1u)
                                                           : field(12 * p, 12);
                const float2 c = tbl[id];
                out[2 * p] = c.x;
                out[2 * p + 1] = c.y;
            }
        }
        float4 *dst = reinterpret_cast<float4 *>(w + r * K + c16 * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dst[j] = make_float4(out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]);
    }
}

}  // namespace hxq

using namespace hxq;

extern "C" int hxq_dequant_fmt(int32_t format, const uint8_t *indices, const float *codebook,
                               int32_t n_codes, const float *group_scale,
                               const float *group_offset, int32_t group_size,
                               const int32_t *sc_row_ptr, const int32_t *sc_col,
                               const float *sc_val, int64_t out_features, int64_t in_features,
                               int64_t row_begin, int64_t row_end, float *w_out,
                               hipStream_t stream) {
    clear_error();
    if (format == HXQ_FMT_SCALAR)
        return hxq_dequant_f32(indices, codebook, group_scale, group_offset, group_size,
                               sc_row_ptr, sc_col, sc_val, out_features, in_features, row_begin,
                               row_end, w_out, stream);
    HXQ_REQUIRE(format == HXQ_FMT_VQ2_U16 || format == HXQ_FMT_VQ2_P12 ||
                    format == HXQ_FMT_AF6 || format == HXQ_FMT_SCALAR_U16,
                "unknown index format");
    HXQ_REQUIRE(indices && w_out, "indices and w_out are required");
    HXQ_REQUIRE((reinterpret_cast<uintptr_t>(indices) & 3u) == 0, "indices must be 4-byte aligned");
    HXQ_REQUIRE(format != HXQ_FMT_SCALAR_U16 || (reinterpret_cast<uintptr_t>(indices) & 15u) == 0,
                "uint16 indices must be 16-byte aligned");
    HXQ_REQUIRE((reinterpret_cast<uintptr_t>(w_out) & 15u) == 0, "w_out must be 16-byte aligned");
    HXQ_REQUIRE(out_features > 0 && in_features > 0 && in_features % 16 == 0,
                "in_features must be a positive multiple of 16");
    HXQ_REQUIRE(0 <= row_begin && row_begin <= row_end && row_end <= out_features,
                "row range out of bounds");
    if (format == HXQ_FMT_AF6)
        HXQ_REQUIRE(group_scale && group_offset && group_size > 0 && group_size % 16 == 0 &&
                        in_features % group_size == 0,
                    "6-bit levels need the group affine (group_size a multiple of 16)");
    else if (format == HXQ_FMT_SCALAR_U16)
        HXQ_REQUIRE(codebook && n_codes >= 1 && n_codes <= kPairCodes &&
                        (group_scale != nullptr) == (group_offset != nullptr) &&
                        (!group_scale || (group_size > 0 && group_size % 16 == 0 &&
                                          in_features % group_size == 0)),
                    "uint16 indices need a 1..4096-entry codebook (affine: both factors, "
                    "group_size a multiple of 16 dividing in_features)");
    else
        HXQ_REQUIRE(codebook && n_codes >= 1 && n_codes <= kPairCodes,
                    "pair codebooks need 1..4096 entries");
    HXQ_REQUIRE(!sc_row_ptr || (sc_col && sc_val), "sidecar CSR needs row_ptr, col and val");
    const int64_t rows = row_end - row_begin;
    if (rows == 0) return HXQ_OK;
    const int64_t n_vec16 = rows * (in_features / 16);
    const int grid = static_cast<int>(
        std::min<int64_t>((n_vec16 + 255) / 256, (int64_t)device_cu_count() * 16));
#define HXQ_DQ(F)                                                                                \
    hipLaunchKernelGGL(dequant_fmt_kernel<F>, dim3(grid), dim3(256), 0, stream, indices, codebook, \
                       n_codes, group_scale, group_offset, group_size, in_features, row_begin,   \
                       n_vec16, w_out)
    switch (format) {
        case HXQ_FMT_VQ2_U16: HXQ_DQ(HXQ_FMT_VQ2_U16); break;
        case HXQ_FMT_VQ2_P12: HXQ_DQ(HXQ_FMT_VQ2_P12); break;
        case HXQ_FMT_SCALAR_U16: HXQ_DQ(HXQ_FMT_SCALAR_U16); break;
        default: HXQ_DQ(HXQ_FMT_AF6); break;
    }
#undef HXQ_DQ
    HXQ_LAUNCH_CHECK();
    if (sc_row_ptr) {
        hipLaunchKernelGGL(dequant_sidecar_kernel, dim3(static_cast<int>((rows + 255) / 256)),
                           dim3(256), 0, stream, sc_row_ptr, sc_col, sc_val, in_features,
                           row_begin, rows, w_out);
        HXQ_LAUNCH_CHECK();
    }
    return HXQ_OK;
}

extern "C" int hxq_dequant_f32(const uint8_t *indices, const float *codebook,
                               const float *group_scale, const float *group_offset,
                               int32_t group_size, const int32_t *sc_row_ptr,
                               const int32_t *sc_col, const float *sc_val,
                               int64_t out_features, int64_t in_features,
                               int64_t row_begin, int64_t row_end, float *w_out,
                               hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(indices && codebook && w_out, "indices, codebook and w_out are required");
    HXQ_REQUIRE(out_features > 0 && in_features > 0, "empty matrix");
    HXQ_REQUIRE(in_features % 16 == 0, "in_features must be a multiple of 16");
    HXQ_REQUIRE(0 <= row_begin && row_begin <= row_end && row_end <= out_features,
                "row range out of bounds");
    const bool affine = group_scale != nullptr || group_offset != nullptr;
    HXQ_REQUIRE(!affine || (group_scale && group_offset),
                "group_scale and group_offset must be given together");
    HXQ_REQUIRE(!affine || (group_size > 0 && group_size % 16 == 0 &&
                            in_features % group_size == 0),
                "group_size must be a positive multiple of 16 dividing in_features");
    const bool sidecar = sc_row_ptr != nullptr;
    HXQ_REQUIRE(!sidecar || (sc_col && sc_val), "sidecar CSR needs row_ptr, col and val");
    const int64_t rows = row_end - row_begin;
    if (rows == 0) return HXQ_OK;

    const int64_t n_vec16 = rows * (in_features / 16);
    const int64_t want = (n_vec16 + 255) / 256;
    const int grid = static_cast<int>(std::min<int64_t>(want, (int64_t)device_cu_count() * 16));
    if (affine)
        hipLaunchKernelGGL(dequant_dense_kernel<true>, dim3(grid), dim3(256), 0, stream, indices,
                           codebook, group_scale, group_offset, group_size, in_features,
                           row_begin, n_vec16, w_out);
    else
        hipLaunchKernelGGL(dequant_dense_kernel<false>, dim3(grid), dim3(256), 0, stream,
                           indices, codebook, nullptr, nullptr, 0, in_features, row_begin,
                           n_vec16, w_out);
    HXQ_LAUNCH_CHECK();
    if (sidecar) {
        const int g2 = static_cast<int>((rows + 255) / 256);
        hipLaunchKernelGGL(dequant_sidecar_kernel, dim3(g2), dim3(256), 0, stream, sc_row_ptr,
                           sc_col, sc_val, in_features, row_begin, rows, w_out);
        HXQ_LAUNCH_CHECK();
    }
    return HXQ_OK;
}
