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
// Work decomposition (wave64, 1024-thread blocks = 16 waves):
//   * the index matrix is streamed in "chunks" of 1024 columns: lane l of a
//     wave loads the 16 bytes at columns [16l, 16l+16) with one dwordx4 load,
//     so one wave load covers 1 KiB of one row, fully coalesced;
//   * a block tile is RPB = (16/S)*R rows; the 16 waves split as S K-slices x
//     (16/S) row groups; each wave owns R rows of its K-slice, so every x
//     value it loads is reused R times from registers;
//   * the 256-entry codebook lives in LDS replicated NREP times with entry j
//     of replica r at dword j*NREP + r; lane l reads replica l % NREP, so the
//     random lookups of one wave hit distinct banks (no bank conflicts);
//   * the S partial sums of a row are combined in LDS in a fixed order, so the
//     result is deterministic;
//   * blocks are persistent over tiles; the codebook table is refilled only
//     when a block moves on to the next matrix.
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
    int32_t tile_begin;
    int32_t pad_;
};

struct GemvParams {
    const void *x;
    int64_t K;
    int32_t group;
    int32_t n_mats;
    int32_t n_tiles;
    int32_t S;
    int32_t nchunks;
    int32_t x_dtype;
    int32_t y_dtype;
    int32_t n_x;
    GemvMat m[HXQ_MAX_MULTI];
};

constexpr int kMaxWaves = 16;  // waves per block for n_x == 1 (8 for n_x > 1)
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

// Codebook lookup of byte b (0..3) of the packed index word w.
//   NREP == 64: entry stride is 256 bytes and the lane's replica offset
//   (lane*4 < 256) fits in the low byte, so the LDS byte address is
//   {0, 0, w.byte[b], lane_off} -- one v_perm_b32 builds it.
//   Other NREP: shift/mask arithmetic.
template <int NREP, int B>
__device__ __forceinline__ float tbl_lookup(const float *tbl, uint32_t lane_off, uint32_t w) {
    if constexpr (NREP == 64) {
        constexpr uint32_t sel = (12u << 24) | (12u << 16) | (static_cast<uint32_t>(B) << 8) | 4u;
        const uint32_t addr = __builtin_amdgcn_perm(lane_off, w, sel);
        return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(tbl) + addr);
    } else {
        const uint32_t addr = ((w >> (8 * B)) & 0xffu) * (NREP * 4) + lane_off;
        return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(tbl) + addr);
    }
}

template <int NREP, int R, int NX, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void gemv_kernel(const GemvParams p) {
    constexpr int kGemvThreads = WAVES * kWave;
    constexpr int kGemvWaves = WAVES;
    extern __shared__ float smem[];
    float *tbl = smem;                 // [256 * NREP]
    float *red = smem + 256 * NREP;    // [WAVES * R * NX]

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int S = p.S;
    const int RG = kGemvWaves / S;
    const int s_id = wave % S;
    const int rg = wave / S;
    const int RPB = RG * R;
    const int64_t K = p.K;
    const int c_begin = s_id * p.nchunks / S;
    const int c_end = (s_id + 1) * p.nchunks / S;
    const uint32_t lane_off = static_cast<uint32_t>(lane % NREP) * 4u;
    const int64_t xstride = K;  // activations are [n_x, K]

    int cur = -1;
    for (int tile = blockIdx.x; tile < p.n_tiles; tile += gridDim.x) {
        int mi = 0;
        while (mi + 1 < p.n_mats && tile >= p.m[mi + 1].tile_begin) ++mi;
        const uint8_t *__restrict__ idx = p.m[mi].idx;
        const float *__restrict__ gs = p.m[mi].gs;
        const float *__restrict__ go = p.m[mi].go;
        const int64_t out = p.m[mi].out;
        if (mi != cur) {
            const float *cb = p.m[mi].cb;
            __syncthreads();  // previous matrix's lookups are done
            for (int e = threadIdx.x; e < 256 * NREP; e += kGemvThreads) tbl[e] = cb[e / NREP];
            __syncthreads();
            cur = mi;
        }
        const int64_t row0 = (int64_t)(tile - p.m[mi].tile_begin) * RPB + rg * R;
        const bool affine = gs != nullptr;
        const int64_t ngroups = affine ? K / p.group : 0;

        float acc[R][NX];
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int n = 0; n < NX; ++n) acc[i][n] = 0.f;

        for (int c = c_begin; c < c_end; ++c) {
            const int64_t k0 = (int64_t)c * kChunk + lane * 16;
            if (k0 >= K) continue;
            u32x4 q[R];
            float sc[R], of[R];
            const int64_t g = affine ? k0 / p.group : 0;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int64_t row = row0 + i;
                if (row < out) {
                    q[i] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4 *>(idx + row * K + k0));
                    sc[i] = affine ? gs[row * ngroups + g] : 1.f;
                    of[i] = affine ? go[row * ngroups + g] : 0.f;
                } else {
                    q[i] = u32x4{0u, 0u, 0u, 0u};
                    sc[i] = 0.f;
                    of[i] = 0.f;
                }
            }
            float xv[NX][16];
            float xs[NX];
#pragma unroll
            for (int n = 0; n < NX; ++n) {
                load_x16(p.x, n * xstride + k0, p.x_dtype, xv[n]);
                float t = 0.f;
#pragma unroll
                for (int j = 0; j < 16; ++j) t += xv[n][j];
                xs[n] = t;
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const uint32_t w[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
                float part[NX];
#pragma unroll
                for (int n = 0; n < NX; ++n) part[n] = 0.f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const float c0 = tbl_lookup<NREP, 0>(tbl, lane_off, w[d]);
                    const float c1 = tbl_lookup<NREP, 1>(tbl, lane_off, w[d]);
                    const float c2 = tbl_lookup<NREP, 2>(tbl, lane_off, w[d]);
                    const float c3 = tbl_lookup<NREP, 3>(tbl, lane_off, w[d]);
#pragma unroll
                    for (int n = 0; n < NX; ++n) {
                        part[n] = fmaf(xv[n][4 * d + 0], c0, part[n]);
                        part[n] = fmaf(xv[n][4 * d + 1], c1, part[n]);
                        part[n] = fmaf(xv[n][4 * d + 2], c2, part[n]);
                        part[n] = fmaf(xv[n][4 * d + 3], c3, part[n]);
                    }
                }
#pragma unroll
                for (int n = 0; n < NX; ++n) {
                    acc[i][n] = fmaf(part[n], sc[i], acc[i][n]);
                    acc[i][n] = fmaf(of[i], xs[n], acc[i][n]);
                }
            }
        }

        // Sidecar correction: slice 0 adds x[col] * delta for its rows.
        const int32_t *__restrict__ rp = p.m[mi].rp;
        if (s_id == 0 && rp != nullptr) {
            const int32_t *__restrict__ col = p.m[mi].col;
            const float *__restrict__ delta = p.m[mi].delta;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int64_t row = row0 + i;
                if (row >= out) continue;
                const int32_t jb = rp[row], je = rp[row + 1];
                for (int32_t j = jb + lane; j < je; j += kWave) {
                    const int32_t cc = col[j];
                    const float dv = delta[j];
#pragma unroll
                    for (int n = 0; n < NX; ++n)
                        acc[i][n] = fmaf(load_x1(p.x, n * xstride + cc, p.x_dtype), dv, acc[i][n]);
                }
            }
        }

        const float *__restrict__ bias = p.m[mi].bias;
        void *y = p.m[mi].y;
#pragma unroll
        for (int i = 0; i < R; ++i) {
#pragma unroll
            for (int n = 0; n < NX; ++n) {
                const float v = wave_sum(acc[i][n]);
                const int64_t row = row0 + i;
                if (S == 1) {
                    if (lane == 0 && row < out)
                        store_y(y, n * out + row, p.y_dtype, v + (bias ? bias[row] : 0.f));
                } else if (lane == 0) {
                    red[((rg * R + i) * NX + n) * S + s_id] = v;
                }
            }
        }
        if (S > 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < RPB * NX; t += kGemvThreads) {
                const int rl = t / NX, n = t % NX;
                const int64_t row = (int64_t)(tile - p.m[mi].tile_begin) * RPB + rl;
                if (row < out) {
                    float v = 0.f;
                    for (int s = 0; s < S; ++s) v += red[t * S + s];
                    store_y(y, n * out + row, p.y_dtype, v + (bias ? bias[row] : 0.f));
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// Host side: validation, launch-shape heuristic, dispatch.
// ---------------------------------------------------------------------------
struct GemvShape {
    int R;
    int S;
    int waves;
};

// Launch-shape overrides for tuning sweeps, read once per process:
// HXQ_GEMV_R (rows per wave), HXQ_GEMV_S (K slices), HXQ_GEMV_BPC (blocks
// per CU), HXQ_GEMV_NREP (codebook replicas in LDS: 1, 32 or 64).
struct GemvTuning {
    int r, s, bpc, nrep;
};

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v ? atoi(v) : dflt;
}

static const GemvTuning &tuning() {
    static const GemvTuning t{env_int("HXQ_GEMV_R", 0), env_int("HXQ_GEMV_S", 0),
                              env_int("HXQ_GEMV_BPC", 2), env_int("HXQ_GEMV_NREP", 64)};
    return t;
}

static int64_t count_tiles(const GemvParams &p, int rpb) {
    int64_t tiles = 0;
    for (int m = 0; m < p.n_mats; ++m) tiles += (p.m[m].out + rpb - 1) / rpb;
    return tiles;
}

// Pick rows-per-wave R and K-slices S so that there are at least two tiles
// per CU (persistent blocks stay busy), preferring many rows per wave (more
// loads in flight, x reused from registers) and few slices (less reduction).
static GemvShape pick_shape(const GemvParams &p) {
    const int cus = device_cu_count();
    const int waves = p.n_x == 1 ? kMaxWaves : kMaxWaves / 2;
    if (tuning().r > 0 && tuning().s > 0) return {tuning().r, tuning().s, waves};
    const int max_r = p.n_x == 1 ? 4 : (p.n_x == 2 ? 2 : 1);
    for (int R = max_r; R >= 1; R /= 2) {
        for (int S = 1; S <= waves && S <= p.nchunks; S *= 2) {
            if (count_tiles(p, (waves / S) * R) >= 2 * (int64_t)cus) return {R, S, waves};
        }
    }
    int S = 1;
    while (S * 2 <= waves && S * 2 <= p.nchunks) S *= 2;
    return {1, S, waves};
}

template <int NREP, int R, int NX, int WAVES>
static int launch_one(const GemvParams &p, int grid, hipStream_t stream) {
    const size_t lds = (256 * NREP + WAVES * R * NX) * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<NREP, R, NX, WAVES>), dim3(grid), dim3(WAVES * kWave), lds,
                       stream, p);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

template <int NREP>
static int launch_nx1(const GemvParams &p, int R, int grid, hipStream_t stream) {
    switch (R) {
        case 4: return launch_one<NREP, 4, 1, kMaxWaves>(p, grid, stream);
        case 2: return launch_one<NREP, 2, 1, kMaxWaves>(p, grid, stream);
        default: return launch_one<NREP, 1, 1, kMaxWaves>(p, grid, stream);
    }
}

static int gemv_run(GemvParams &p, hipStream_t stream) {
    const GemvShape sh = pick_shape(p);
    const int max_r = p.n_x == 1 ? 4 : (p.n_x == 2 ? 2 : 1);
    HXQ_REQUIRE(sh.R >= 1 && sh.R <= max_r && (sh.R & (sh.R - 1)) == 0,
                "rows per wave must be 1, 2 or 4 (at most 2 for n_rows 2, 1 above)");
    HXQ_REQUIRE(sh.S >= 1 && sh.S <= sh.waves && (sh.waves % sh.S) == 0,
                "K slices must divide the wave count");
    p.S = sh.S;
    const int rpb = (sh.waves / sh.S) * sh.R;
    int64_t tiles = 0;
    for (int m = 0; m < p.n_mats; ++m) {
        p.m[m].tile_begin = static_cast<int32_t>(tiles);
        tiles += (p.m[m].out + rpb - 1) / rpb;
    }
    HXQ_REQUIRE(tiles < (1LL << 30), "too many rows");
    p.n_tiles = static_cast<int32_t>(tiles);
    const int bpc = std::max(1, tuning().bpc);
    const int grid = static_cast<int>(std::min<int64_t>(tiles, (int64_t)device_cu_count() * bpc));
    if (p.n_x == 1) {
        switch (tuning().nrep) {
            case 1: return launch_nx1<1>(p, sh.R, grid, stream);
            case 32: return launch_nx1<32>(p, sh.R, grid, stream);
            default: return launch_nx1<64>(p, sh.R, grid, stream);
        }
    }
    constexpr int W2 = kMaxWaves / 2;
    switch (p.n_x) {
        case 2:
            return sh.R == 2 ? launch_one<64, 2, 2, W2>(p, grid, stream)
                             : launch_one<64, 1, 2, W2>(p, grid, stream);
        case 3: return launch_one<64, 1, 3, W2>(p, grid, stream);
        default: return launch_one<64, 1, 4, W2>(p, grid, stream);
    }
}

static bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

static int check_mat(const hxq_matrix &m, int64_t K, int32_t group) {
    HXQ_REQUIRE(m.indices && m.codebook && m.y, "indices, codebook and y are required");
    HXQ_REQUIRE(aligned16(m.indices), "indices must be 16-byte aligned");
    HXQ_REQUIRE(m.out_features > 0, "out_features must be positive");
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

extern "C" int hxq_gemv_multi(const void *x, int32_t x_dtype, const hxq_matrix *mats,
                              int32_t n_mats, int32_t group_size, int32_t y_dtype,
                              int64_t in_features, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && mats, "x and mats are required");
    HXQ_REQUIRE(n_mats >= 1 && n_mats <= HXQ_MAX_MULTI, "n_mats must be in [1, HXQ_MAX_MULTI]");
    HXQ_REQUIRE(x_dtype >= HXQ_F32 && x_dtype <= HXQ_F16, "bad x_dtype");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(in_features > 0 && in_features % 16 == 0, "in_features must be a positive multiple of 16");
    HXQ_REQUIRE(aligned16(x), "x must be 16-byte aligned");
    GemvParams p{};
    p.x = x;
    p.K = in_features;
    p.group = group_size;
    p.n_mats = n_mats;
    p.nchunks = static_cast<int32_t>((in_features + kChunk - 1) / kChunk);
    p.x_dtype = x_dtype;
    p.y_dtype = y_dtype;
    p.n_x = 1;
    for (int i = 0; i < n_mats; ++i) {
        const int rc = check_mat(mats[i], in_features, group_size);
        if (rc != HXQ_OK) return rc;
        const hxq_matrix &m = mats[i];
        p.m[i] = GemvMat{m.indices, m.codebook, m.group_scale, m.group_offset, m.sc_row_ptr,
                         m.sc_col, m.sc_delta, m.bias, m.y, m.out_features, 0, 0};
    }
    return gemv_run(p, stream);
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
    GemvParams p{};
    p.x = x;
    p.K = in_features;
    p.group = group_size;
    p.n_mats = 1;
    p.nchunks = static_cast<int32_t>((in_features + kChunk - 1) / kChunk);
    p.x_dtype = x_dtype;
    p.y_dtype = y_dtype;
    p.n_x = static_cast<int32_t>(n_rows);
    p.m[0] = GemvMat{indices, codebook, group_scale, group_offset, sc_row_ptr, sc_col,
                     sc_delta, bias, y, out_features, 0, 0};
    return gemv_run(p, stream);
}
