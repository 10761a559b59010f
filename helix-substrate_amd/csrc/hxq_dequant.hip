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

}  // namespace hxq

using namespace hxq;

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
