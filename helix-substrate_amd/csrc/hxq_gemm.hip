// HXQ prefill GEMM: Y[M, OUT] = X[M, K] @ W^T, W dequantised into LDS and fed
// to bf16/fp16 MFMA (v_mfma_f32_32x32x16_{bf16,f16}) with fp32 accumulation.
//
// Replaces fused_vq_matmul's N > 1 path (helix_substrate/triton_vq_matmul.py:
// 634-661 _vq_gather_matmul_tiled_kernel, 693-698 scatter_add sidecar, 724-725
// bias) and the default _forward_buffered materialise-then-BLAS path
// (helix_linear.py:556-634).
//
// Block tile BM x BN (M x OUT) with BK = 64 per K-step, 256 threads (4 waves in
// a 2 x 2 layout, each wave BM/2 x BN/2 = (BM/64) x (BN/64) MFMA 32x32 tiles).
// Per K-step:
//   * X tile [BM, 64] (16-bit) -> LDS;
//   * index tile [BN, 64] (u8) -> codebook lookup (LDS, 16 replicas) ->
//     fma(cb, scale, offset) -> 16-bit -> LDS; sidecar entries of the tile
//     then REPLACE their element (each of the 2 threads of a row keeps a
//     prefetched cursor into its row's CSR entries);
//   * the next K-step's global loads are issued before this step's MFMAs.
// LDS rows are padded by 16 bytes so the MFMA operand reads (16 bytes per
// lane, 32 rows per half-wave) spread over the banks.
// Results are written once per output element: deterministic.
#include <algorithm>

#include "hxq_common.h"

namespace hxq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmThreads = 256;
constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8;   // 16-bit elements per padded LDS row
constexpr int kCbRep = 16;         // codebook replicas (lane % 16)

struct GemmArgs {
    const uint16_t *x;    // [M, K] bf16/fp16
    const uint8_t *idx;   // [OUT, K]
    const float *cb;      // [256]
    const float *gs;      // [OUT, K/G] or null
    const float *go;
    const int32_t *rp;    // CSR [OUT+1] or null
    const int32_t *col;
    const float *val;     // replacement values
    const float *bias;    // [OUT] or null
    void *y;              // [M, OUT]
    int32_t M, OUT, K, group, y_dtype, pad_;
};

template <bool BF16>
__device__ __forceinline__ uint16_t to16(float v) {
    if constexpr (BF16) return f32_to_bf16(v);
    else return f32_to_f16(v);
}

// One K-step worth of global data held in registers between steps.
template <int BM>
struct GemmStage {
    u32x4 a[BM / 32];   // X: BM rows x 128 B; a pass of 256 threads x 16 B covers 32 rows
    u32x4 q[2];         // indices: 32 bytes of one row
    float s, o;         // affine factors of that row's group
};

template <int BM, int BN, bool BF16, bool AFFINE>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_kernel(const GemmArgs g) {
    static_assert(BN == 128, "one index row per thread pair");
    constexpr int WM = BM / 2, WN = BN / 2;          // wave tile
    constexpr int TM = WM / 32, TN = WN / 32;        // MFMA tiles per wave
    __shared__ __attribute__((aligned(16))) uint16_t sA[BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t sB[BN * kLdsRow];
    __shared__ float tbl[256 * kCbRep];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int wm = wave / 2, wn = wave % 2;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = g.K;
    const int nk = K / kBK;

    // codebook replicas: entry j at [j*16 + r]
    for (int e = tid; e < 256 * kCbRep; e += kGemmThreads) tbl[e] = g.cb[e / kCbRep];

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, (int64_t)g.M * K * 2);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(g.idx, (int64_t)g.OUT * K);
    const int ngroups = AFFINE ? K / g.group : 0;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(g.gs, AFFINE ? (int64_t)g.OUT * ngroups * 4 : 0);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(g.go, AFFINE ? (int64_t)g.OUT * ngroups * 4 : 0);

    // X loads: thread t covers row (t / 8) + 32*p, 16-byte column chunk t % 8
    const int a_row = tid / 8, a_cc = tid % 8;
    // index loads: thread t covers row t / 2, half t % 2 (32 bytes)
    const int b_row = tid / 2, b_half = tid % 2;
    const int grow = n0 + b_row;  // global output row of this thread's index slice
    const uint32_t kOob = 0x80000000u;

    auto load_stage = [&](int ks, GemmStage<BM> &st) {
        const int k0 = ks * kBK;
#pragma unroll
        for (int p = 0; p < BM / 32; ++p) {
            const int r = m0 + a_row + 32 * p;
            const uint32_t off = r < g.M ? (uint32_t)((r * K + k0 + a_cc * 8) * 2) : kOob;
            st.a[p] = buf_load16(xr, off);
        }
        const uint32_t qoff = grow < g.OUT ? (uint32_t)(grow * K + k0 + b_half * 32) : kOob;
        st.q[0] = buf_load16(qr, qoff);
        st.q[1] = buf_load16(qr, qoff + 16);
        if constexpr (AFFINE) {
            const uint32_t so = grow < g.OUT ? (uint32_t)((grow * ngroups + k0 / g.group) * 4) : kOob;
            st.s = buf_loadf(sr, so);
            st.o = buf_loadf(orr, so);
        } else {
            st.s = 1.f;
            st.o = 0.f;
        }
    };

    // sidecar cursor of this thread's row: next entry (col, val) prefetched
    const bool has_sc = g.rp != nullptr && grow < g.OUT;
    int32_t sc_j = 0, sc_end = 0;
    int32_t sc_col = 0x7fffffff;
    float sc_val = 0.f;
    if (has_sc) {
        sc_j = g.rp[grow];
        sc_end = g.rp[grow + 1];
        if (sc_j < sc_end) {
            sc_col = g.col[sc_j];
            sc_val = g.val[sc_j];
        }
    }

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    GemmStage<BM> cur;
    load_stage(0, cur);
    const uint32_t rep = (lane % kCbRep) * 4u;

    for (int ks = 0; ks < nk; ++ks) {
        __syncthreads();  // previous MFMAs are done with sA / sB
        // X -> LDS
#pragma unroll
        for (int p = 0; p < BM / 32; ++p)
            *reinterpret_cast<u32x4 *>(&sA[(a_row + 32 * p) * kLdsRow + a_cc * 8]) = cur.a[p];
        // indices -> dequantised 16-bit weights -> LDS
        {
            uint32_t packed[16];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t w = cur.q[h][d];
                    float v[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float c = *reinterpret_cast<const float *>(
                            reinterpret_cast<const char *>(tbl) + ((w >> (8 * b)) & 0xffu) * (kCbRep * 4) + rep);
                        v[b] = AFFINE ? fmaf(c, cur.s, cur.o) : c;
                    }
                    packed[h * 8 + d * 2] = to16<BF16>(v[0]) | (uint32_t(to16<BF16>(v[1])) << 16);
                    packed[h * 8 + d * 2 + 1] = to16<BF16>(v[2]) | (uint32_t(to16<BF16>(v[3])) << 16);
                }
            uint16_t *dst = &sB[b_row * kLdsRow + b_half * 32];
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4)
                *reinterpret_cast<u32x4 *>(dst + c4 * 8) =
                    u32x4{packed[4 * c4], packed[4 * c4 + 1], packed[4 * c4 + 2], packed[4 * c4 + 3]};
            // sidecar: replace entries in [lo, hi) of this row
            const int lo = ks * kBK + b_half * 32, hi = lo + 32;
            while (sc_col < hi) {
                if (sc_col >= lo) sB[b_row * kLdsRow + (sc_col - ks * kBK)] = to16<BF16>(sc_val);
                ++sc_j;
                if (sc_j < sc_end) {
                    sc_col = g.col[sc_j];
                    sc_val = g.val[sc_j];
                } else {
                    sc_col = 0x7fffffff;
                }
            }
        }
        __syncthreads();
        if (ks + 1 < nk) load_stage(ks + 1, cur);
        // MFMAs: 4 k-substeps of 16
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            u32x4 av[TM], bv[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                av[i] = *reinterpret_cast<const u32x4 *>(
                    &sA[(wm * WM + i * 32 + lane % 32) * kLdsRow + kk * 16 + (lane / 32) * 8]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bv[j] = *reinterpret_cast<const u32x4 *>(
                    &sB[(wn * WN + j * 32 + lane % 32) * kLdsRow + kk * 16 + (lane / 32) * 8]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (BF16)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, av[i]), __builtin_bit_cast(bf16x8, bv[j]),
                            acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, av[i]), __builtin_bit_cast(f16x8, bv[j]),
                            acc[i][j], 0, 0, 0);
                }
        }
    }

    // epilogue: acc[i][j][r] = C[row = 8*(r/4) + 4*(lane/32) + r%4][col = lane%32]
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * WN + j * 32 + lane % 32;
        if (n >= g.OUT) continue;
        const float bv = g.bias ? g.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
                if (m < g.M) {
                    const float v = acc[i][j][r] + bv;
                    const int64_t o = (int64_t)m * g.OUT + n;
                    if (g.y_dtype == HXQ_F32) static_cast<float *>(g.y)[o] = v;
                    else if (g.y_dtype == HXQ_BF16) static_cast<uint16_t *>(g.y)[o] = f32_to_bf16(v);
                    else static_cast<uint16_t *>(g.y)[o] = f32_to_f16(v);
                }
            }
    }
}

template <int BM, bool BF16>
static int gemm_launch(const GemmArgs &a, hipStream_t stream) {
    const dim3 grid((a.OUT + 127) / 128, (a.M + BM - 1) / BM);
    if (a.gs)
        hipLaunchKernelGGL((gemm_kernel<BM, 128, BF16, true>), grid, dim3(kGemmThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, 128, BF16, false>), grid, dim3(kGemmThreads), 0, stream, a);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

}  // namespace hxq

using namespace hxq;

extern "C" int hxq_gemm(const void *x, int32_t x_dtype, const uint8_t *indices,
                        const float *codebook, const float *group_scale,
                        const float *group_offset, int32_t group_size,
                        const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                        const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                        int64_t out_features, int64_t in_features, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && indices && codebook && y, "x, indices, codebook and y are required");
    HXQ_REQUIRE(x_dtype == HXQ_BF16 || x_dtype == HXQ_F16,
                "the MFMA GEMM takes bf16 or fp16 activations (fp32 goes through hxq_gemv)");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(m_rows > 0 && out_features > 0 && in_features > 0, "empty problem");
    HXQ_REQUIRE(in_features % kBK == 0, "in_features must be a multiple of 64");
    HXQ_REQUIRE(m_rows * in_features * 2 < (int64_t{1} << 31) &&
                    out_features * in_features < (int64_t{1} << 31) &&
                    m_rows * out_features < (int64_t{1} << 31),
                "problem too large for 32-bit offsets");
    const bool affine = group_scale || group_offset;
    HXQ_REQUIRE(!affine || (group_scale && group_offset),
                "group_scale and group_offset must be given together");
    HXQ_REQUIRE(!affine || (group_size >= kBK && group_size % kBK == 0 &&
                            in_features % group_size == 0),
                "the GEMM needs group_size to be a multiple of 64 dividing in_features");
    HXQ_REQUIRE(!sc_row_ptr || (sc_col && sc_val), "sidecar CSR needs row_ptr, col and val");
    GemmArgs a{static_cast<const uint16_t *>(x), indices, codebook, group_scale, group_offset,
               sc_row_ptr, sc_col, sc_val, bias, y,
               static_cast<int32_t>(m_rows), static_cast<int32_t>(out_features),
               static_cast<int32_t>(in_features), group_size, y_dtype, 0};
    const int64_t tiles256 = ((m_rows + 255) / 256) * ((out_features + 127) / 128);
    const bool big = tiles256 >= device_cu_count();
    if (x_dtype == HXQ_BF16)
        return big ? gemm_launch<256, true>(a, stream) : gemm_launch<128, true>(a, stream);
    return big ? gemm_launch<256, false>(a, stream) : gemm_launch<128, false>(a, stream);
}
