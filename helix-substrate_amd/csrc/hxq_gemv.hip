// HXQ decode GEMV (fp32 accumulation), one or several matrices per launch.
//
// Replaces fused_vq_matmul's N==1 path (helix_substrate/triton_vq_matmul.py:
// 521-633: _vq_decode_dotprod_kernel, _sidecar_fused_kernel, bias).
//
// Math per output row o (G = group_size, g = group of column k):
//   y[o] = sum_g s[o,g] * (sum_{k in g} x[k] * cb[idx[o,k]])
//        + sum_g off[o,g] * (sum_{k in g} x[k])
//        + sum_{sidecar j in row o} x[col_j] * delta_j           + bias[o]
// i.e. the affine step is factored out of the inner loop (one multiply per
// 16 weights instead of one per weight).  This changes rounding relative to
// dequantising first; it stays far inside the 1e-5 relative bound.
//
// Work decomposition (wave64, 512-thread blocks = 8 waves, 1 or 2 blocks per CU):
//   * the index matrix is streamed in "chunks" of 1024 columns: lane l of a
//     wave loads the 16 bytes at columns [16l, 16l+16) with one dwordx4 load,
//     so one wave load covers 1 KiB of one row, fully coalesced;
//   * block b owns the contiguous rows [T*b/G, T*(b+1)/G) of the concatenated
//     row space of all matrices in the launch;
//   * its 8 waves split as S K-slices x (8/S) row lanes; a slice is at most
//     CPS chunks, whose activations stay in registers for the whole kernel;
//   * each wave walks its rows in batches of RB rows, issuing every load of a
//     batch before computing it; two blocks per CU (16 waves) hide the
//     latency of large launches, small ones run one block per CU (fewer
//     codebook tables to build); loads are clamped to valid addresses instead of branched
//     around, and results of out-of-range rows are not stored;
//   * the 256-entry codebook lives in LDS replicated NREP times with entry j
//     of replica r at dword j*NREP + r; lane l reads replica l % NREP, so the
//     random lookups of one wave hit distinct banks (no bank conflicts);
//   * row partials go to LDS; the sidecar products x[col] * delta of the
//     block's entries go to LDS during the stream; a final pass with up to 64
//     lanes per output row adds slices, sidecar entries and bias, the row's
//     lanes reducing in a fixed order by DPP and lane swaps (deterministic,
//     no atomics, no LDS round trips).
#include <algorithm>

#include "hxq_common.h"

namespace hxq {

struct GemvMat {
    const uint8_t *idx;
    const float *cb;
    const float *gs;
    const float *go;
    const int32_t *rp;
    const int32_t *col;
    const float *delta;
    const float *bias;
    void *y;
    int64_t out;
    int64_t ncodes;  // codebook entries (formats with a pair codebook)
    int32_t rpb;     // rows per block (set by the launch plan)
    int32_t pad_;
};

struct GemvMats {
    GemvMat m[HXQ_MAX_MULTI];
};

// Fused activation prologue (one fp32 activation row).
//   XM 1: x_eff = bf16(w * r * rsqrt(mean(r^2) + eps)), r = x + b (b = NULL:
//         r = x); block 0 also stores r to res_out (the updated residual).
//   XM 2: x_eff = bf16(silu(x) * b).
// bf16 rounding matches a separate norm / SiLU kernel writing bf16.
struct GemvPro {
    const float *b;
    const float *w;
    float *res_out;
    float eps;
    int32_t pad_;
};

// Launch header.  It travels as leading scalar kernel arguments so the
// hardware preloads it into SGPRs (no kernarg memory round trip).
struct GemvHeader {
    const void *x;
    int64_t K;
    int32_t group;
    int32_t S;
    int32_t nchunks;
    int32_t x_dtype;
    int32_t y_dtype;
    int32_t n_mats;
    int32_t red_rows;  // LDS reduction slots per block (rows)
    int32_t xlds;      // 1: activations staged in LDS for the sidecar gather
    int32_t fmt;       // HXQ_FMT_*
    int32_t bb[HXQ_MAX_MULTI];  // bb[m]: first block after matrix m (cumulative)
};

constexpr int kChunk = 1024;  // columns per wave load (64 lanes x 16 bytes)

// Load 16 consecutive activations starting at x + base (fp32/bf16/fp16).
__device__ __forceinline__ void load_x16(const void *x, int64_t base, int dt, float (&v)[16]) {
    if (dt == HXQ_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + base);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 f = p[j];
            v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
        }
    } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + base);
        const uint4 a = p[0], b = p[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        if (dt == HXQ_BF16) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[2 * j] = __uint_as_float(w[j] << 16);
                v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[2 * j] = f16_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
                v[2 * j + 1] = f16_to_f32(static_cast<uint16_t>(w[j] >> 16));
            }
        }
    }
}

__device__ __forceinline__ float load_x1(const void *x, int64_t i, int dt) {
    if (dt == HXQ_F32) return static_cast<const float *>(x)[i];
    const uint16_t h = static_cast<const uint16_t *>(x)[i];
    return dt == HXQ_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ void store_y(void *y, int64_t i, int dt, float v) {
    if (dt == HXQ_F32) static_cast<float *>(y)[i] = v;
    else if (dt == HXQ_BF16) static_cast<uint16_t *>(y)[i] = f32_to_bf16(v);
    else static_cast<uint16_t *>(y)[i] = f32_to_f16(v);
}

// One pipeline stage: the index words and affine factors of one row x CPS chunks.
// Index formats (HXQ_FMT_*): bytes of index data per 16 weights, and LDS
// table floats per block.
__host__ __device__ constexpr int fmt_bytes16(int f) {
    return f == HXQ_FMT_SCALAR_U16 ? 32 : (f == HXQ_FMT_VQ2_P12 || f == HXQ_FMT_AF6) ? 12 : 16;
}
__host__ __device__ constexpr int fmt_table_floats(int f, int nrep) {
    return f == HXQ_FMT_SCALAR ? 256 * nrep : f == HXQ_FMT_AF6 ? 0
         : f == HXQ_FMT_SCALAR_U16 ? kPairCodes : 2 * kPairCodes;
}

// Bits [bit, bit + width) of the little-endian 96/128-bit stream q (bit and
// width are constants after unrolling, so this folds to a shift/mask or one
// v_alignbit_b32).
__device__ __forceinline__ uint32_t bitfield(const u32x4 &q, int bit, int width) {
    const int d = bit >> 5, sh = bit & 31;
    const uint32_t v = sh + width <= 32 ? q[d] >> sh : __builtin_amdgcn_alignbit(q[d + 1], q[d], sh);
    return v & ((1u << width) - 1u);
}

__device__ __forceinline__ u32x4 buf_load12(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
    return u32x4{v[0], v[1], v[2], 0u};
}

// QW: 16-byte index words per 16 weights (2 for uint16 scalar indices)
template <int CPS, int QW = 1>
struct GemvItem {
    u32x4 q[CPS * QW];
    float sc[CPS];
    float of[CPS];
};

constexpr int kEntCap = 512;  // sidecar entries per block staged in LDS

// Kernel phases:
//   block -> matrix: the host gives each matrix its own contiguous run of
//             blocks (bb[]); a block owns rows [out*b/nb, out*(b+1)/nb) of it;
//   prologue  every global load the block needs first is issued before the
//             first wait: activations, this thread's codebook slots, row_ptr
//             of the block's rows, and the first batch of index rows;
//   table     codebook -> LDS (NREP replicas, conflict-free float4 writes);
//             activations -> LDS (fp32) when they fit, for the sidecar gather;
//   stream    batches of RB rows per wave, loads of a batch issued together,
//             double-buffered (batch i+1 in flight while batch i computes);
//             rows a wave does not own get an out-of-range buffer offset
//             (no memory traffic) and are not computed; after its first batch
//             (whose wait covers the col/delta loads issued before the loop)
//             each thread writes its sidecar entry's x[col]*delta to LDS;
//   epilogue  LPR lanes per output row (the largest power of two <= 64 that
//             fits the block's rows in one pass): lane q adds slices q, q+LPR,
//             ... and sidecar entries j0+q, j0+q+LPR, ... (CSR order), then
//             the lanes reduce by DPP and lane swaps; bias, store.  Fixed summation
//             order: deterministic.  (One thread per row with a serial loop
//             over the row's entries cost 1.3 us on the config-1 down launch.)
// Barriers order LDS only (lds_barrier), so prefetched loads stay in flight.
// Occupancy target: 4 waves per SIMD (two 8-wave blocks per CU, <= 128 VGPRs);
// the long-row variant (4 chunks per slice) accepts 2.
template <int NREP, int NX, int CPS, int WAVES, bool AFFINE, int RB, int XT, int XM, int FMT>
__global__ __launch_bounds__(WAVES * kWave, CPS == 4 ? 2 : 4) void gemv_kernel(
    const void *__restrict__ x, int32_t K, int32_t group, int32_t S, int32_t nchunks,
    int32_t flags, int32_t red_rows, int32_t bb1, int32_t bb2, int32_t bb3, int32_t bb4,
    int32_t bb5, int32_t bb6, int32_t bb7, const GemvMats mats, const GemvPro pro) {
    constexpr bool XF32 = XT == HXQ_F32;
    static_assert(XM == 0 || (XF32 && NX == 1), "fused prologues take one fp32 row");
    constexpr int NT = WAVES * kWave;
    constexpr int TBLF = fmt_table_floats(FMT, NREP);
    constexpr int TPW = TBLF / (4 * NT);  // table float4 writes per thread
    static_assert(FMT == HXQ_FMT_AF6 || (TPW >= 1 && TBLF % (4 * NT) == 0),
                  "table/thread-count mismatch");
    static_assert(XM == 0 || FMT == HXQ_FMT_SCALAR, "fused prologues take scalar codebooks");
    static_assert((FMT == HXQ_FMT_AF6) == AFFINE || FMT == HXQ_FMT_SCALAR ||
                      FMT == HXQ_FMT_SCALAR_U16,
                  "6-bit levels carry the affine; pair codebooks have none");
    constexpr int QB = fmt_bytes16(FMT);  // index bytes per 16 weights
    constexpr int QW = QB > 16 ? 2 : 1;   // 16-byte words per 16 weights
    constexpr uint32_t kOob = 0x80000000u;      // buffer offset past any range: reads 0
    const int y_dtype = flags & 0xf;
    const bool xlds = (flags >> 4) & 1;

    // ---- block -> matrix (scalar compares on preloaded arguments)
    const int bid = blockIdx.x;
    const int mi = (bid >= bb1) + (bid >= bb2) + (bid >= bb3) + (bid >= bb4) + (bid >= bb5) +
                   (bid >= bb6) + (bid >= bb7);
    const int b_lo = mi == 0 ? 0 : mi == 1 ? bb1 : mi == 2 ? bb2 : mi == 3 ? bb3 : mi == 4 ? bb4
                   : mi == 5 ? bb5 : mi == 6 ? bb6 : bb7;
    const GemvMat &M = mats.m[mi];

    extern __shared__ float smem[];
    float *tbl = smem;                                      // [TBLF]
    float *xl = tbl + TBLF;                                 // [NX * K] when xlds
    float *red = xl + (xlds ? NX * K : 0);                  // [red_rows * NX * S]
    float *ent = red + red_rows * NX * S;                   // [kEntCap * NX]
    float *sumsq = ent + kEntCap * NX;                      // [S] (XM == 1)

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    // S and RG = WAVES / S are powers of two: shifts, not divisions
    const int lg_s = __builtin_ctz(static_cast<uint32_t>(S));
    const int RG = WAVES >> lg_s;
    const int lg_rg = __builtin_ctz(static_cast<uint32_t>(RG));
    const int s_id = wave & (S - 1);
    const int rg = wave >> lg_s;
    const int c_lo = (s_id * nchunks) >> lg_s;
    const int nc = (((s_id + 1) * nchunks) >> lg_s) - c_lo;  // chunks of this slice (<= CPS)
    const uint32_t lane_off = static_cast<uint32_t>(lane % NREP) * 4u;
    uint32_t koff[CPS];
    bool kok[CPS];
#pragma unroll
    for (int ci = 0; ci < CPS; ++ci) {
        const int k0 = (c_lo + ci) * kChunk + lane * 16;
        kok[ci] = ci < nc && k0 < K;
        koff[ci] = static_cast<uint32_t>(k0);
    }

    // rows of this block: [lo, lo + n_rows), rpb rows per block (the last may have fewer)
    const int64_t out = M.out;
    const int32_t rpb = M.rpb;
    const int64_t lo = static_cast<int64_t>(bid - b_lo) * rpb;
    const int32_t n_rows = static_cast<int32_t>(min(static_cast<int64_t>(rpb), out - lo));
    const int64_t ngroups = AFFINE ? K / group : 0;
    const int32_t n_mine = n_rows > rg ? (n_rows - rg + RG - 1) >> lg_rg : 0;
    const bool has_sc = M.rp != nullptr;
    if (lds_offset_of(smem) != 0) {
        // the lookups address the table from LDS 0 (no static LDS in this kernel):
        // never taken, but poison the outputs rather than read a wrong table
        if (threadIdx.x < n_rows * NX)
            store_y(M.y, (threadIdx.x % NX) * out + lo + threadIdx.x / NX, y_dtype, __builtin_nanf(""));
        return;
    }

    // ---- prologue: issue everything, wait later
    constexpr int XV = XF32 ? 4 : 2;  // 16-byte loads per 16 activations
    u32x4 xraw[CPS][NX][XV];
    {
        const int esz = XF32 ? 4 : 2;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (int64_t)NX * K * esz);
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci)
#pragma unroll
            for (int n = 0; n < NX; ++n)
#pragma unroll
                for (int v = 0; v < XV; ++v)
                    xraw[ci][n][v] = buf_load16(xr, (n * K + koff[ci]) * esz + 16u * v);
    }
    // fused prologue operands (b: delta or up; w: norm weight), 16 per chunk
    u32x4 braw[XM != 0 ? CPS : 1][4], wraw[XM == 1 ? CPS : 1][4];
    if constexpr (XM != 0) {
        const __amdgpu_buffer_rsrc_t br = make_rsrc(pro.b, pro.b ? (int64_t)K * 4 : 0);
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(pro.w, XM == 1 ? (int64_t)K * 4 : 0);
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                braw[ci][v] = buf_load16(br, koff[ci] * 4 + 16u * v);
                if constexpr (XM == 1) wraw[ci][v] = buf_load16(wr, koff[ci] * 4 + 16u * v);
            }
    }
    float cbv[FMT == HXQ_FMT_SCALAR ? TPW : 1];
    u32x4 cbq[(FMT == HXQ_FMT_VQ2_U16 || FMT == HXQ_FMT_VQ2_P12 || FMT == HXQ_FMT_SCALAR_U16)
                  ? TPW : 1];
    if constexpr (FMT == HXQ_FMT_SCALAR) {
        const __amdgpu_buffer_rsrc_t cr = make_rsrc(M.cb, 256 * 4);
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const uint32_t e = 4u * (threadIdx.x + k * NT);  // first replica slot
            cbv[k] = buf_loadf(cr, (e / NREP) * 4u);
        }
    } else if constexpr (FMT != HXQ_FMT_AF6) {
        // scalar codebook [ncodes <= 4096] fp32 or pair codebook [ncodes, 2]
        // fp32, one copy.  Four one-dword loads per 16-byte slot: the range
        // check of a single dword is exact, so entries past ncodes read 0
        // whatever ncodes % 4 is (a 16-byte load straddling the end of the
        // table would depend on how the hardware checks a partial range).
        const __amdgpu_buffer_rsrc_t cr =
            make_rsrc(M.cb, M.ncodes * (FMT == HXQ_FMT_SCALAR_U16 ? 4 : 8));
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const uint32_t b = 16u * (threadIdx.x + k * NT);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                cbq[k][j] = static_cast<uint32_t>(buf_loadi(cr, b + 4u * j));
        }
    }
    const __amdgpu_buffer_rsrc_t rp_r = make_rsrc(M.rp, has_sc ? (out + 1) * 4 : 0);
    // final-pass outputs: thread t handles (row lo + t / NX, activation t % NX)
    // final pass: LPR lanes per (row, activation) item, LPR a power of two <= 64
    int lg_lpr = 0;
    while (lg_lpr < 6 && (n_rows * NX) << (lg_lpr + 1) <= NT) ++lg_lpr;
    const int LPR = 1 << lg_lpr;
    const int my_item = static_cast<int>(threadIdx.x) >> lg_lpr, my_q = threadIdx.x & (LPR - 1);
    const int64_t my_rl = my_item / NX;
    const int32_t my_j0 = buf_loadi(rp_r, static_cast<uint32_t>((lo + my_rl) * 4));
    const int32_t my_j1 = buf_loadi(rp_r, static_cast<uint32_t>((lo + my_rl + 1) * 4));
    const int32_t blk_j0 = buf_loadi(rp_r, static_cast<uint32_t>(lo * 4));
    const int32_t blk_j1 = buf_loadi(rp_r, static_cast<uint32_t>((lo + n_rows) * 4));

    const uint32_t row_bytes = static_cast<uint32_t>(K) / 16u * QB;
    const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(M.idx, out * row_bytes);
    const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(M.gs, AFFINE ? out * ngroups * 4 : 0);
    const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(M.go, AFFINE ? out * ngroups * 4 : 0);
    auto load_item = [&](int32_t i, GemvItem<CPS, QW> &it) {
        const bool mine = i < n_mine;
        const uint32_t row = static_cast<uint32_t>(lo + rg + i * RG);
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci) {
            const uint32_t qo = mine ? row * row_bytes + koff[ci] / 16u * QB : kOob;
            if constexpr (QB == 32) {
                it.q[2 * ci] = buf_load16(q_rsrc, qo);
                it.q[2 * ci + 1] = buf_load16(q_rsrc, mine ? qo + 16u : kOob);
            } else if constexpr (QB == 16) {
                it.q[ci] = buf_load16(q_rsrc, qo);
            } else {
                it.q[ci] = buf_load12(q_rsrc, qo);
            }
            if constexpr (AFFINE) {
                const uint32_t g4 =
                    (row * static_cast<uint32_t>(ngroups) + koff[ci] / static_cast<uint32_t>(group)) * 4u;
                it.sc[ci] = buf_loadf(s_rsrc, mine ? g4 : kOob);
                it.of[ci] = buf_loadf(o_rsrc, mine ? g4 : kOob);
            } else {
                it.sc[ci] = 1.f;
                it.of[ci] = 0.f;
            }
        }
    };
    GemvItem<CPS, QW> it[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) load_item(b, it[b]);
    __builtin_amdgcn_sched_barrier(0);  // all prologue loads are issued before any wait

    // ---- table (+ activations to registers / LDS)
    if constexpr (FMT == HXQ_FMT_SCALAR) {
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const int e = 4 * (threadIdx.x + k * NT);
            *reinterpret_cast<float4 *>(tbl + e) = make_float4(cbv[k], cbv[k], cbv[k], cbv[k]);
        }
    } else if constexpr (FMT != HXQ_FMT_AF6) {
        // pair table as float2 entries, or the uint16-index scalar table (one copy)
#pragma unroll
        for (int k = 0; k < TPW; ++k)
            *reinterpret_cast<u32x4 *>(tbl + 4 * (threadIdx.x + k * NT)) = cbq[k];
    }
    float xv[CPS][NX][16];
    float xs[CPS][NX];
#pragma unroll
    for (int ci = 0; ci < CPS; ++ci)
#pragma unroll
        for (int n = 0; n < NX; ++n) {
            if constexpr (XF32) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        xv[ci][n][4 * v + j] = kok[ci] ? __uint_as_float(xraw[ci][n][v][j]) : 0.f;
            } else {
#pragma unroll
                for (int v = 0; v < 2; ++v)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t w = xraw[ci][n][v][j];
                        float a, b;
                        if constexpr (XT == HXQ_BF16) {
                            a = __uint_as_float(w << 16);
                            b = __uint_as_float(w & 0xffff0000u);
                        } else {
                            a = f16_to_f32(static_cast<uint16_t>(w & 0xffffu));
                            b = f16_to_f32(static_cast<uint16_t>(w >> 16));
                        }
                        xv[ci][n][8 * v + 2 * j] = kok[ci] ? a : 0.f;
                        xv[ci][n][8 * v + 2 * j + 1] = kok[ci] ? b : 0.f;
                    }
            }
            if constexpr (XM != 0) {
                // r = x + b (norm) / silu(x) * b (SiLU), kept in xv; norm scaling below
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float bv = __uint_as_float(braw[ci][v][j]);
                        float &e = xv[ci][n][4 * v + j];
                        if constexpr (XM == 1) e = kok[ci] ? e + bv : 0.f;
                        else e = kok[ci] ? bf16_to_f32(f32_to_bf16(e / (1.f + expf(-e)) * bv)) : 0.f;
                    }
            }
            if constexpr (XM == 1) continue;  // sums and LDS copy after the norm
            float t = 0.f;
#pragma unroll
            for (int j = 0; j < 16; ++j) t += xv[ci][n][j];
            xs[ci][n] = t;
            if (xlds && rg == 0 && kok[ci]) {
                float4 *dst = reinterpret_cast<float4 *>(xl + n * K + koff[ci]);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    dst[v] = make_float4(xv[ci][n][4 * v], xv[ci][n][4 * v + 1],
                                         xv[ci][n][4 * v + 2], xv[ci][n][4 * v + 3]);
            }
        }
    float norm_inv = 1.f;
    if constexpr (XM == 1) {
        // block-wide sum of squares: slice partials of row group 0 -> LDS
        float ss = 0.f;
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci)
#pragma unroll
            for (int j = 0; j < 16; ++j) ss = fmaf(xv[ci][0][j], xv[ci][0][j], ss);
        ss = wave_sum(ss);
        if (rg == 0 && lane == 0) sumsq[s_id] = ss;
        // the updated residual, once (block 0, row group 0)
        if (pro.res_out && blockIdx.x == 0 && rg == 0) {
#pragma unroll
            for (int ci = 0; ci < CPS; ++ci)
                if (kok[ci]) {
                    float4 *dst = reinterpret_cast<float4 *>(pro.res_out + koff[ci]);
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        dst[v] = make_float4(xv[ci][0][4 * v], xv[ci][0][4 * v + 1],
                                             xv[ci][0][4 * v + 2], xv[ci][0][4 * v + 3]);
                }
        }
        lds_barrier();
        float tot = 0.f;
        for (int i = 0; i < S; ++i) tot += sumsq[i];
        norm_inv = rsqrtf(tot / K + pro.eps);
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float &e = xv[ci][0][4 * v + j];
                    e = kok[ci] ? bf16_to_f32(f32_to_bf16(__uint_as_float(wraw[ci][v][j]) * (e * norm_inv)))
                                : 0.f;
                }
            float t = 0.f;
#pragma unroll
            for (int j = 0; j < 16; ++j) t += xv[ci][0][j];
            xs[ci][0] = t;
            if (xlds && rg == 0 && kok[ci]) {
                float4 *dst = reinterpret_cast<float4 *>(xl + koff[ci]);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    dst[v] = make_float4(xv[ci][0][4 * v], xv[ci][0][4 * v + 1],
                                         xv[ci][0][4 * v + 2], xv[ci][0][4 * v + 3]);
            }
        }
    }
    lds_barrier();

    // sidecar entries of this block, first round: col/delta loads now
    const int32_t nent = has_sc ? blk_j1 - blk_j0 : 0;
    const __amdgpu_buffer_rsrc_t col_r = make_rsrc(M.col, has_sc ? (int64_t)blk_j1 * 4 : 0);
    const __amdgpu_buffer_rsrc_t dl_r = make_rsrc(M.delta, has_sc ? (int64_t)blk_j1 * 4 : 0);
    const uint32_t e0 = (static_cast<uint32_t>(blk_j0) + threadIdx.x) * 4u;
    const int32_t sc_col0 = buf_loadi(col_r, e0);
    const float sc_dl0 = buf_loadf(dl_r, e0);

    // ---- stream
    auto compute_item = [&](int32_t i, const GemvItem<CPS, QW> &itm) {
        float acc[NX];
#pragma unroll
        for (int n = 0; n < NX; ++n) acc[n] = 0.f;
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci) {
            float part[NX];
#pragma unroll
            for (int n = 0; n < NX; ++n) part[n] = 0.f;
            if constexpr (FMT == HXQ_FMT_SCALAR) {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t w = itm.q[ci][d];
                    const float c0 = tbl_lookup0<NREP, 0>(lane_off, w);
                    const float c1 = tbl_lookup0<NREP, 1>(lane_off, w);
                    const float c2 = tbl_lookup0<NREP, 2>(lane_off, w);
                    const float c3 = tbl_lookup0<NREP, 3>(lane_off, w);
#pragma unroll
                    for (int n = 0; n < NX; ++n) {
                        part[n] = fmaf(xv[ci][n][4 * d + 0], c0, part[n]);
                        part[n] = fmaf(xv[ci][n][4 * d + 1], c1, part[n]);
                        part[n] = fmaf(xv[ci][n][4 * d + 2], c2, part[n]);
                        part[n] = fmaf(xv[ci][n][4 * d + 3], c3, part[n]);
                    }
                }
            } else if constexpr (FMT == HXQ_FMT_SCALAR_U16) {
                // 16 uint16 indices in two words (ids masked to the 4096-entry table)
#pragma unroll
                for (int f = 0; f < 16; ++f) {
                    const uint32_t id =
                        (itm.q[2 * ci + (f >> 3)][(f >> 1) & 3] >> (16 * (f & 1))) & (kPairCodes - 1u);
                    const float c = tbl[id];
#pragma unroll
                    for (int n = 0; n < NX; ++n) part[n] = fmaf(xv[ci][n][f], c, part[n]);
                }
            } else if constexpr (FMT == HXQ_FMT_AF6) {
                // 16 six-bit levels, little-endian bit stream
#pragma unroll
                for (int f = 0; f < 16; ++f) {
                    const float c = static_cast<float>(bitfield(itm.q[ci], 6 * f, 6));
#pragma unroll
                    for (int n = 0; n < NX; ++n) part[n] = fmaf(xv[ci][n][f], c, part[n]);
                }
            } else {
                // 8 pair indices (uint16 in the low 12 bits, or packed 12-bit)
                const float2 *tbl2 = reinterpret_cast<const float2 *>(tbl);
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    const uint32_t id = FMT == HXQ_FMT_VQ2_U16
                                            ? (itm.q[ci][p >> 1] >> (16 * (p & 1))) & (kPairCodes - 1u)
                                            : bitfield(itm.q[ci], 12 * p, 12);
                    const float2 c = tbl2[id];
#pragma unroll
                    for (int n = 0; n < NX; ++n) {
                        part[n] = fmaf(xv[ci][n][2 * p], c.x, part[n]);
                        part[n] = fmaf(xv[ci][n][2 * p + 1], c.y, part[n]);
                    }
                }
            }
#pragma unroll
            for (int n = 0; n < NX; ++n) {
                acc[n] = fmaf(part[n], itm.sc[ci], acc[n]);
                acc[n] = fmaf(itm.of[ci], xs[ci][n], acc[n]);
            }
        }
        const int32_t rl = rg + i * RG;  // row within the block's range
#pragma unroll
        for (int n = 0; n < NX; ++n) {
            const float v = wave_sum_lane63(acc[n]);
            if (lane == kWave - 1) red[(rl * NX + n) * S + s_id] = v;
        }
    };
    auto xval = [&](int n, int32_t c) -> float {
        if (xlds) return xl[n * K + c];
        if constexpr (XM == 1) {
            const float r = static_cast<const float *>(x)[c] + (pro.b ? pro.b[c] : 0.f);
            return bf16_to_f32(f32_to_bf16(pro.w[c] * (r * norm_inv)));
        } else if constexpr (XM == 2) {
            const float g = static_cast<const float *>(x)[c];
            return bf16_to_f32(f32_to_bf16(g / (1.f + expf(-g)) * pro.b[c]));
        }
        return load_x1(x, n * K + c, XT);
    };
    // the sidecar products x[col] * delta of this block's entries, into LDS:
    // after a thread's first batch (its col/delta loads have landed by then)
    bool ent_done = !has_sc;
    auto compute_ent = [&]() {
        const int32_t lim = nent < kEntCap ? nent : kEntCap;
        for (int32_t e = threadIdx.x; e < lim; e += NT) {
            int32_t c;
            float dv;
            if (e == static_cast<int32_t>(threadIdx.x)) {
                c = sc_col0;
                dv = sc_dl0;
            } else {
                c = M.col[blk_j0 + e];
                dv = M.delta[blk_j0 + e];
            }
#pragma unroll
            for (int n = 0; n < NX; ++n) ent[e * NX + n] = xval(n, c) * dv;
        }
        ent_done = true;
    };
    // double-buffered batches: the next batch's loads are issued before the
    // current batch is computed (it2 is the second buffer)
    GemvItem<CPS, QW> it2[RB];
    for (int32_t i0 = 0; i0 < n_mine; i0 += 2 * RB) {
#pragma unroll
        for (int b = 0; b < RB; ++b) load_item(i0 + RB + b, it2[b]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < RB; ++b)
            if (i0 + b < n_mine) compute_item(i0 + b, it[b]);
        if (!ent_done) compute_ent();
        if (i0 + RB >= n_mine) break;
#pragma unroll
        for (int b = 0; b < RB; ++b) load_item(i0 + 2 * RB + b, it[b]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < RB; ++b)
            if (i0 + RB + b < n_mine) compute_item(i0 + RB + b, it2[b]);
    }

    // ---- epilogue
    if (!ent_done) compute_ent();
    lds_barrier();  // red and ent complete
    {
        // lane q of an item adds slices q, q + LPR, ... and sidecar entries
        // j0 + q, j0 + q + LPR, ...; the item's lanes then reduce in a fixed
        // order by DPP and lane swaps (deterministic, no LDS round trips)
        const bool live = my_item < n_rows * NX;
        const int n = my_item % NX;
        float v = 0.f;
        if (live) {
            for (int s2 = my_q; s2 < S; s2 += LPR) v += red[my_item * S + s2];
            if (has_sc) {
                for (int32_t j = my_j0 + my_q; j < my_j1; j += LPR) {
                    const int32_t e = j - blk_j0;
                    v += e < kEntCap ? ent[e * NX + n] : xval(n, M.col[j]) * M.delta[j];
                }
            }
        }
        v = lane_group_sum(v, LPR);
        if (live && my_q == 0) {
            const int64_t row = lo + my_rl;
            store_y(M.y, n * out + row, y_dtype, v + (M.bias ? M.bias[row] : 0.f));
        }
    }
}

// ---------------------------------------------------------------------------
// Host side: validation, launch-shape choice, dispatch.
// ---------------------------------------------------------------------------
constexpr int kWaves = 8;  // waves per block (512 threads; two blocks share a CU)
constexpr int kNrep = 64;  // codebook replicas in LDS (one per lane)

// Launch-shape overrides for tuning sweeps, read once per process:
// HXQ_GEMV_S (K slices), HXQ_GEMV_BPC (blocks per CU).
struct GemvTuning {
    int s, bpc;
};

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v ? atoi(v) : dflt;
}

static const GemvTuning &tuning() {
    static const GemvTuning t{env_int("HXQ_GEMV_S", 0), env_int("HXQ_GEMV_BPC", 0)};
    return t;
}

// Blocks per CU (0 = by size): one-row launches of fewer than 8192 output rows
// run one block per CU -- half the codebook tables to build, and a CU's eight
// waves still keep enough rows in flight (config 1: q+k+v 8.5 -> 6.2 us, o
// 6.4 -> 5.8 us, down 11.4 -> 11.3 us) -- larger ones (gate+up, 22016 rows:
// 13.5 us against 13.9) and multi-row launches two.
static int blocks_per_cu(int64_t total_rows, int n_x) {
    if (tuning().bpc > 0) return tuning().bpc;
    return n_x == 1 && total_rows < 8192 ? 1 : 2;
}

struct GemvPlan {
    int CPS;
    int grid;
};

// Chunks per slice, K slices, and the block partition over matrices.
static int plan_gemv(GemvHeader &h, GemvMats &mats, int n_x, GemvPlan &pl, bool fused_prologue) {
    pl.CPS = 1;
    if (n_x == 1) {
        while (pl.CPS < 4 && pl.CPS * kWaves < h.nchunks) pl.CPS *= 2;
    }
    int64_t total = 0;
    for (int m = 0; m < h.n_mats; ++m) total += mats.m[m].out;
    const int cus = device_cu_count();
    const int64_t target = (int64_t)cus * blocks_per_cu(total, n_x);
    // blocks per matrix proportional to its rows; at most 512/n_x rows a block
    const int64_t max_rows = (kWaves * kWave) / n_x;
    int64_t grid = 0;
    int64_t rows_pb = 1;
    for (int m = 0; m < h.n_mats; ++m) {
        const int64_t out = mats.m[m].out;
        int64_t nb = std::max<int64_t>(1, (target * out + total - 1) / total);
        nb = std::max<int64_t>(nb, (out + max_rows - 1) / max_rows);
        nb = std::min<int64_t>(nb, out);
        // equal runs of rpb rows; the last block of the matrix takes the rest
        const int64_t rpb = (out + nb - 1) / nb;
        nb = (out + rpb - 1) / rpb;
        mats.m[m].rpb = static_cast<int32_t>(rpb);
        grid += nb;
        HXQ_REQUIRE(grid < (int64_t{1} << 30), "too many GEMV blocks");
        h.bb[m] = static_cast<int32_t>(grid);
        rows_pb = std::max<int64_t>(rows_pb, rpb);
    }
    for (int m = h.n_mats; m < HXQ_MAX_MULTI; ++m) h.bb[m] = INT32_MAX;
    pl.grid = static_cast<int>(grid);
    // Enough rows per block for every wave: two chunks per slice, so one
    // cross-lane reduction covers 32 weights per lane instead of 16 (with few
    // rows per block the K split keeps more waves busy instead).
    // (Not with a fused prologue: its extra operand registers would spill.)
    if (n_x == 1 && !fused_prologue && pl.CPS == 1 && h.nchunks >= 2 && rows_pb >= 2 * kWaves)
        pl.CPS = 2;
    int S = 1;
    while (S * pl.CPS < h.nchunks) S *= 2;
    // few rows per block: split K further so more waves have rows
    while (S < kWaves && S < h.nchunks && rows_pb < (int64_t)(kWaves / S)) S *= 2;
    if (tuning().s > 0) S = tuning().s;
    HXQ_REQUIRE(S >= 1 && S <= kWaves && (kWaves % S) == 0,
                "K slices must be a power of two up to the wave count");
    HXQ_REQUIRE((int64_t)S * pl.CPS >= h.nchunks,
                n_x == 1 ? "in_features above 32768 is not supported by the GEMV"
                         : "in_features above 8192 is not supported for 2-4 activation rows");
    h.S = S;
    h.red_rows = static_cast<int32_t>(rows_pb);
    return HXQ_OK;
}

static size_t gemv_lds_bytes(int nrep, int nx, const GemvHeader &h) {
    return ((size_t)fmt_table_floats(h.fmt, nrep) + (h.xlds ? (size_t)nx * h.K : 0) +
            (size_t)h.red_rows * nx * h.S + (size_t)kEntCap * nx + 64) * sizeof(float);
}

template <int NREP, int NX, int CPS, int RB, int XM = 0, int FMT = HXQ_FMT_SCALAR>
static int launch_one(const GemvHeader &h, const GemvMats &mats, int grid, hipStream_t stream,
                      const GemvPro &pro = GemvPro{}) {
    const size_t lds = gemv_lds_bytes(NREP, NX, h);
    const bool aff = mats.m[0].gs != nullptr;
    const dim3 g(grid), b(kWaves * kWave);
    const int32_t flags = h.y_dtype | (h.xlds << 4);
    const int32_t K = static_cast<int32_t>(h.K);
    // all matrices of one launch either carry the affine factors or none do
#define HXQ_GEMV_LAUNCH(AFF, XT)                                                               \
    hipLaunchKernelGGL((gemv_kernel<NREP, NX, CPS, kWaves, AFF, RB, XT, XM, FMT>), g, b, lds, stream, \
                       h.x, K, h.group, h.S, h.nchunks, flags, h.red_rows, h.bb[0], h.bb[1],   \
                       h.bb[2], h.bb[3], h.bb[4], h.bb[5], h.bb[6], mats, pro)
    if constexpr (XM != 0) {
        if (aff) HXQ_GEMV_LAUNCH(true, HXQ_F32); else HXQ_GEMV_LAUNCH(false, HXQ_F32);
    } else if constexpr (FMT != HXQ_FMT_SCALAR && FMT != HXQ_FMT_SCALAR_U16) {
        constexpr bool A = FMT == HXQ_FMT_AF6;
        switch (h.x_dtype) {
            case HXQ_F32: HXQ_GEMV_LAUNCH(A, HXQ_F32); break;
            case HXQ_BF16: HXQ_GEMV_LAUNCH(A, HXQ_BF16); break;
            default: HXQ_GEMV_LAUNCH(A, HXQ_F16); break;
        }
    } else {
        switch (h.x_dtype) {
            case HXQ_F32: if (aff) HXQ_GEMV_LAUNCH(true, HXQ_F32); else HXQ_GEMV_LAUNCH(false, HXQ_F32); break;
            case HXQ_BF16: if (aff) HXQ_GEMV_LAUNCH(true, HXQ_BF16); else HXQ_GEMV_LAUNCH(false, HXQ_BF16); break;
            default: if (aff) HXQ_GEMV_LAUNCH(true, HXQ_F16); else HXQ_GEMV_LAUNCH(false, HXQ_F16); break;
        }
    }
#undef HXQ_GEMV_LAUNCH
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

template <int XM = 0, int FMT = HXQ_FMT_SCALAR>
static int gemv_run(GemvHeader &h, GemvMats &mats, int n_x, hipStream_t stream,
                    const GemvPro &pro = GemvPro{}) {
    h.fmt = FMT;
    GemvPlan pl{};
    const int rc = plan_gemv(h, mats, n_x, pl, XM != 0);
    if (rc != HXQ_OK) return rc;
    // stage activations in LDS (sidecar gather) when two blocks still fit a CU
    constexpr size_t kLdsBudget = 80 * 1024;
    h.xlds = 1;
    if (gemv_lds_bytes(kNrep, n_x, h) > kLdsBudget) h.xlds = 0;
    HXQ_REQUIRE(gemv_lds_bytes(kNrep, n_x, h) <= 160 * 1024, "GEMV LDS budget exceeded");
    // rows per batch (two batches in flight): what fits 128 VGPRs
    if (n_x == 1) {
        switch (pl.CPS) {
            case 1: return launch_one<kNrep, 1, 1, 4, XM, FMT>(h, mats, pl.grid, stream, pro);
            case 2: return launch_one<kNrep, 1, 2, 2, XM, FMT>(h, mats, pl.grid, stream, pro);
            default: return launch_one<kNrep, 1, 4, 1, XM, FMT>(h, mats, pl.grid, stream, pro);
        }
    }
    if constexpr (XM != 0) {
        return HXQ_ERR_INVALID_ARG;
    } else {
        switch (n_x) {
            case 2: return launch_one<kNrep, 2, 1, 2, 0, FMT>(h, mats, pl.grid, stream);
            case 3: return launch_one<kNrep, 3, 1, 1, 0, FMT>(h, mats, pl.grid, stream);
            default: return launch_one<kNrep, 4, 1, 1, 0, FMT>(h, mats, pl.grid, stream);
        }
    }
}

static bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

static int check_mat(const hxq_matrix &m, int64_t K, int32_t group) {
    HXQ_REQUIRE(m.indices && m.codebook && m.y, "indices, codebook and y are required");
    HXQ_REQUIRE(aligned16(m.indices), "indices must be 16-byte aligned");
    HXQ_REQUIRE(m.out_features > 0, "out_features must be positive");
    HXQ_REQUIRE(m.out_features * K + kChunk < (int64_t{1} << 32),
                "index matrix must be smaller than 4 GiB (32-bit buffer offsets)");
    const bool affine = m.group_scale || m.group_offset;
    HXQ_REQUIRE(!affine || (m.group_scale && m.group_offset),
                "group_scale and group_offset must be given together");
    HXQ_REQUIRE(!affine || (group > 0 && group % 16 == 0 && K % group == 0),
                "group_size must be a positive multiple of 16 dividing in_features");
    HXQ_REQUIRE(!m.sc_row_ptr || (m.sc_col && m.sc_delta), "sidecar CSR needs row_ptr, col, delta");
    return HXQ_OK;
}

}  // namespace hxq

using namespace hxq;

extern "C" int hxq_gemv_multi(const void *x, int32_t x_dtype, const hxq_matrix *mats_in,
                              int32_t n_mats, int32_t group_size, int32_t y_dtype,
                              int64_t in_features, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && mats_in, "x and mats are required");
    HXQ_REQUIRE(n_mats >= 1 && n_mats <= HXQ_MAX_MULTI, "n_mats must be in [1, HXQ_MAX_MULTI]");
    HXQ_REQUIRE(x_dtype >= HXQ_F32 && x_dtype <= HXQ_F16, "bad x_dtype");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(in_features > 0 && in_features % 16 == 0, "in_features must be a positive multiple of 16");
    HXQ_REQUIRE(aligned16(x), "x must be 16-byte aligned");
    HXQ_REQUIRE(in_features <= INT32_MAX / 4, "in_features too large");
    GemvHeader h{};
    h.x = x;
    h.K = in_features;
    h.group = group_size;
    h.n_mats = n_mats;
    h.nchunks = static_cast<int32_t>((in_features + kChunk - 1) / kChunk);
    h.x_dtype = x_dtype;
    h.y_dtype = y_dtype;
    GemvMats mats{};
    for (int i = 0; i < n_mats; ++i) {
        const int rc = check_mat(mats_in[i], in_features, group_size);
        if (rc != HXQ_OK) return rc;
        HXQ_REQUIRE((mats_in[i].group_scale != nullptr) == (mats_in[0].group_scale != nullptr),
                    "all matrices of one launch must agree on having the group affine");
        const hxq_matrix &m = mats_in[i];
        mats.m[i] = GemvMat{m.indices, m.codebook, m.group_scale, m.group_offset, m.sc_row_ptr,
                            m.sc_col, m.sc_delta, m.bias, m.y, m.out_features};
    }
    return gemv_run(h, mats, 1, stream);
}

extern "C" int hxq_gemv(const void *x, int32_t x_dtype, const uint8_t *indices,
                        const float *codebook, const float *group_scale,
                        const float *group_offset, int32_t group_size,
                        const int32_t *sc_row_ptr, const int32_t *sc_col,
                        const float *sc_delta, const float *bias, void *y, int32_t y_dtype,
                        int64_t n_rows, int64_t out_features, int64_t in_features,
                        hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(n_rows >= 1 && n_rows <= 4, "n_rows must be in [1, 4]");
    HXQ_REQUIRE(x, "x is required");
    HXQ_REQUIRE(x_dtype >= HXQ_F32 && x_dtype <= HXQ_F16, "bad x_dtype");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(in_features > 0 && in_features % 16 == 0, "in_features must be a positive multiple of 16");
    HXQ_REQUIRE(aligned16(x), "x must be 16-byte aligned");
    hxq_matrix m{indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col, sc_delta,
                 bias, y, out_features};
    const int rc = check_mat(m, in_features, group_size);
    if (rc != HXQ_OK) return rc;
    HXQ_REQUIRE(in_features <= INT32_MAX / 4, "in_features too large");
    GemvHeader h{};
    h.x = x;
    h.K = in_features;
    h.group = group_size;
    h.n_mats = 1;
    h.nchunks = static_cast<int32_t>((in_features + kChunk - 1) / kChunk);
    h.x_dtype = x_dtype;
    h.y_dtype = y_dtype;
    GemvMats mats{};
    mats.m[0] = GemvMat{indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col,
                        sc_delta, bias, y, out_features};
    return gemv_run(h, mats, static_cast<int>(n_rows), stream);
}

// Fused-prologue launches: one fp32 activation row, transformed on load.
static int gemv_fused(int xm, const float *x, const GemvPro &pro, const hxq_matrix *mats_in,
                      int32_t n_mats, int32_t group_size, int32_t y_dtype, int64_t in_features,
                      hipStream_t stream) {
    HXQ_REQUIRE(x && mats_in, "x and mats are required");
    HXQ_REQUIRE(n_mats >= 1 && n_mats <= HXQ_MAX_MULTI, "n_mats must be in [1, HXQ_MAX_MULTI]");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(in_features > 0 && in_features % 16 == 0, "in_features must be a positive multiple of 16");
    HXQ_REQUIRE(aligned16(x) && (!pro.b || aligned16(pro.b)) && (!pro.w || aligned16(pro.w)) &&
                    (!pro.res_out || aligned16(pro.res_out)), "vectors must be 16-byte aligned");
    HXQ_REQUIRE(in_features <= INT32_MAX / 4, "in_features too large");
    GemvHeader h{};
    h.x = x;
    h.K = in_features;
    h.group = group_size;
    h.n_mats = n_mats;
    h.nchunks = static_cast<int32_t>((in_features + kChunk - 1) / kChunk);
    h.x_dtype = HXQ_F32;
    h.y_dtype = y_dtype;
    GemvMats mats{};
    for (int i = 0; i < n_mats; ++i) {
        const int rc = check_mat(mats_in[i], in_features, group_size);
        if (rc != HXQ_OK) return rc;
        HXQ_REQUIRE((mats_in[i].group_scale != nullptr) == (mats_in[0].group_scale != nullptr),
                    "all matrices of one launch must agree on having the group affine");
        const hxq_matrix &m = mats_in[i];
        mats.m[i] = GemvMat{m.indices, m.codebook, m.group_scale, m.group_offset, m.sc_row_ptr,
                            m.sc_col, m.sc_delta, m.bias, m.y, m.out_features};
    }
    return xm == 1 ? gemv_run<1>(h, mats, 1, stream, pro) : gemv_run<2>(h, mats, 1, stream, pro);
}

extern "C" int hxq_gemv_multi_rmsnorm(const float *x, const float *delta, const float *norm_w,
                                      float eps, float *res_out, const hxq_matrix *mats,
                                      int32_t n_mats, int32_t group_size, int32_t y_dtype,
                                      int64_t in_features, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(norm_w, "norm_w is required");
    HXQ_REQUIRE(!res_out || (res_out != x && res_out != delta), "res_out must not alias x or delta");
    const GemvPro pro{delta, norm_w, res_out, eps, 0};
    return gemv_fused(1, x, pro, mats, n_mats, group_size, y_dtype, in_features, stream);
}

extern "C" int hxq_gemv_multi_silu(const float *gate, const float *up, const hxq_matrix *mats,
                                   int32_t n_mats, int32_t group_size, int32_t y_dtype,
                                   int64_t in_features, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(up, "up is required");
    const GemvPro pro{up, nullptr, nullptr, 0.f, 0};
    return gemv_fused(2, gate, pro, mats, n_mats, group_size, y_dtype, in_features, stream);
}

extern "C" int hxq_gemv_fmt(const void *x, int32_t x_dtype, int32_t format, const uint8_t *indices,
                            const float *codebook, int32_t n_codes, const float *group_scale,
                            const float *group_offset, int32_t group_size,
                            const int32_t *sc_row_ptr, const int32_t *sc_col,
                            const float *sc_delta, const float *bias, void *y, int32_t y_dtype,
                            int64_t n_rows, int64_t out_features, int64_t in_features,
                            hipStream_t stream) {
    clear_error();
    if (format == HXQ_FMT_SCALAR)
        return hxq_gemv(x, x_dtype, indices, codebook, group_scale, group_offset, group_size,
                        sc_row_ptr, sc_col, sc_delta, bias, y, y_dtype, n_rows, out_features,
                        in_features, stream);
    HXQ_REQUIRE(format == HXQ_FMT_VQ2_U16 || format == HXQ_FMT_VQ2_P12 ||
                    format == HXQ_FMT_AF6 || format == HXQ_FMT_SCALAR_U16,
                "unknown index format");
    HXQ_REQUIRE(n_rows >= 1 && n_rows <= 4, "n_rows must be in [1, 4]");
    HXQ_REQUIRE(x && indices && y, "x, indices and y are required");
    HXQ_REQUIRE(x_dtype >= HXQ_F32 && x_dtype <= HXQ_F16, "bad x_dtype");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(in_features > 0 && in_features % 16 == 0 && in_features <= INT32_MAX / 4,
                "in_features must be a positive multiple of 16");
    HXQ_REQUIRE(out_features > 0, "out_features must be positive");
    HXQ_REQUIRE(aligned16(x), "x must be 16-byte aligned");
    HXQ_REQUIRE(aligned16(indices) || fmt_bytes16(format) == 12, "indices must be 16-byte aligned");
    HXQ_REQUIRE((reinterpret_cast<uintptr_t>(indices) & 3u) == 0, "indices must be 4-byte aligned");
    HXQ_REQUIRE(out_features * (in_features / 16 * fmt_bytes16(format)) + kChunk <
                    (int64_t{1} << 32), "index data must be smaller than 4 GiB");
    HXQ_REQUIRE(!sc_row_ptr || (sc_col && sc_delta), "sidecar CSR needs row_ptr, col, delta");
    if (format == HXQ_FMT_AF6) {
        HXQ_REQUIRE(group_scale && group_offset, "6-bit levels need group_scale and group_offset");
        HXQ_REQUIRE(group_size > 0 && group_size % 16 == 0 && in_features % group_size == 0,
                    "group_size must be a positive multiple of 16 dividing in_features");
    } else if (format == HXQ_FMT_SCALAR_U16) {
        HXQ_REQUIRE(codebook && n_codes >= 1 && n_codes <= kPairCodes,
                    "uint16-index scalar codebooks need 1..4096 entries");
        HXQ_REQUIRE(aligned16(codebook), "codebook must be 16-byte aligned");
        const bool affine = group_scale || group_offset;
        HXQ_REQUIRE(!affine || (group_scale && group_offset),
                    "group_scale and group_offset must be given together");
        HXQ_REQUIRE(!affine || (group_size > 0 && group_size % 16 == 0 &&
                                in_features % group_size == 0),
                    "group_size must be a positive multiple of 16 dividing in_features");
    } else {
        HXQ_REQUIRE(codebook && n_codes >= 1 && n_codes <= kPairCodes,
                    "pair codebooks need 1..4096 entries");
        HXQ_REQUIRE(!group_scale && !group_offset, "pair codebooks take no group affine");
        HXQ_REQUIRE(aligned16(codebook), "codebook must be 16-byte aligned");
    }
    GemvHeader h{};
    h.x = x;
    h.K = in_features;
    h.group = (format == HXQ_FMT_AF6 || format == HXQ_FMT_SCALAR_U16) ? group_size : 0;
    h.n_mats = 1;
    h.nchunks = static_cast<int32_t>((in_features + kChunk - 1) / kChunk);
    h.x_dtype = x_dtype;
    h.y_dtype = y_dtype;
    GemvMats mats{};
    mats.m[0] = GemvMat{indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col, sc_delta,
                        bias, y, out_features, n_codes};
    const int nx = static_cast<int>(n_rows);
    switch (format) {
        case HXQ_FMT_VQ2_U16: return gemv_run<0, HXQ_FMT_VQ2_U16>(h, mats, nx, stream);
        case HXQ_FMT_VQ2_P12: return gemv_run<0, HXQ_FMT_VQ2_P12>(h, mats, nx, stream);
        case HXQ_FMT_SCALAR_U16: return gemv_run<0, HXQ_FMT_SCALAR_U16>(h, mats, nx, stream);
        default: return gemv_run<0, HXQ_FMT_AF6>(h, mats, nx, stream);
    }
}
