// Decoder-step kernels around the HXQ GEMVs for batch-1 greedy decoding of a
// Qwen2-shaped model: residual add + RMSNorm, RoPE + KV-cache append, GQA
// decode attention, SiLU(gate) * up, and greedy argmax.  The token position
// is read from device memory, so one captured HIP graph replays every step.
//
// Math follows transformers' Qwen2 (models/qwen2/modeling_qwen2.py):
// Qwen2RMSNorm.forward (:247-253), rotate_half / apply_rotary_pos_emb
// (:105-135) with inv_freq = theta^(-2i/D) (:86), eager attention with
// scaling D^-1/2 and repeat_kv grouping (:138-170), decoder layer residuals
// (:269-300) and Qwen2MLP down(act(gate) * up).  The residual stream is kept
// in fp32; arithmetic is fp32.
#include <algorithm>
#include <cfloat>

#include "hxq_common.h"

namespace hxq {

constexpr int kDecThreads = 256;

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < kDecThreads / kWave; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = -FLT_MAX;
    for (int i = 0; i < kDecThreads / kWave; ++i) t = fmaxf(t, red[i]);
    return t;
}

// x += delta (if any); out = weight * x * rsqrt(mean(x^2) + eps); one block
// per row, each thread keeping its up to kNormPer elements in registers
// (one pass over memory).
constexpr int kNormPer = 16;   // hidden <= 256 * 16

template <int DDT, int ODT>
__global__ __launch_bounds__(kDecThreads) void add_rmsnorm_kernel(float *x, const void *delta,
                                                                  const float *w, float eps,
                                                                  int32_t H, void *out) {
    __shared__ float red[kDecThreads / kWave];
    const int64_t r = blockIdx.x;
    float v[kNormPer];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormPer; ++j) {
        const int i = threadIdx.x + j * kDecThreads;
        v[j] = 0.f;
        if (i < H) {
            v[j] = x[r * H + i];
            if (delta) v[j] += load_act<DDT>(delta, r * H + i);
        }
        ss = fmaf(v[j], v[j], ss);
    }
    const float inv = rsqrtf(block_sum(ss, red) / H + eps);
#pragma unroll
    for (int j = 0; j < kNormPer; ++j) {
        const int i = threadIdx.x + j * kDecThreads;
        if (i < H) {
            if (delta) x[r * H + i] = v[j];
            store_act<ODT>(out, r * H + i, w[i] * (v[j] * inv));
        }
    }
}

// qkv fp32 [n_heads*D | n_kv*D | n_kv*D] of one token at position *pos:
// rotate q and k (rotate_half convention), write q_out fp32 [n_heads*D] and
// k/v into the caches [max_seq, n_kv, D] (cache dtype CDT) at row *pos.
template <int CDT>
__global__ __launch_bounds__(kDecThreads) void rope_append_kernel(
    const float *qkv, const int32_t *pos_p, int32_t n_heads, int32_t n_kv, int32_t D,
    float theta, float *q_out, void *k_cache, void *v_cache, int32_t max_seq) {
    const int pos = *pos_p;
    if (pos < 0 || pos >= max_seq) return;  // the host keeps pos < max_seq
    const int half = D / 2;
    const int total = (n_heads + n_kv) * half;
    for (int e = blockIdx.x * kDecThreads + threadIdx.x; e < total + n_kv * D;
         e += gridDim.x * kDecThreads) {
        if (e < total) {
            const int h = e / half, i = e % half;
            const float inv_freq = powf(theta, -2.f * i / D);
            const float ang = static_cast<float>(pos) * inv_freq;
            float sn, cs;
            sincosf(ang, &sn, &cs);
            const float *src = qkv + (int64_t)h * D;  // q heads then k heads (contiguous)
            const float x1 = src[i], x2 = src[i + half];
            const float o1 = x1 * cs - x2 * sn, o2 = x2 * cs + x1 * sn;
            if (h < n_heads) {
                q_out[(int64_t)h * D + i] = o1;
                q_out[(int64_t)h * D + i + half] = o2;
            } else {
                const int kh = h - n_heads;
                const int64_t base = ((int64_t)pos * n_kv + kh) * D;
                store_act<CDT>(k_cache, base + i, o1);
                store_act<CDT>(k_cache, base + i + half, o2);
            }
        } else {
            const int j = e - total;  // v element
            const int64_t base = (int64_t)pos * n_kv * D;
            store_act<CDT>(v_cache, base + j, qkv[(int64_t)(n_heads + n_kv) * D + j]);
        }
    }
}

// One block per query head: softmax(q . k_t * D^-1/2, t <= pos) . v_t over the
// head's KV group (head h reads kv head h / (n_heads / n_kv)).  D = 128,
// bf16 or fp32 cache.
//   scores: one position per thread; its k row (256 B) arrives as 16
//           independent 16-byte loads, q comes from LDS as broadcasts;
//   output: wave w sums positions w + 4j, eight at a time, lane l owning
//           dims 2l, 2l+1 (a position is one coalesced row); the four wave
//           partials meet in LDS.
constexpr int kAttnD = 128;

// The value a cache of type CDT would return for v.
template <int CDT>
__device__ __forceinline__ float load_back(float v) {
    if constexpr (CDT == HXQ_F32) return v;
    else if constexpr (CDT == HXQ_BF16) return bf16_to_f32(f32_to_bf16(v));
    else return f16_to_f32(f32_to_f16(v));
}

template <int CDT>
__device__ __forceinline__ void load_row8(const void *cache, int64_t elem, float (&v)[8]) {
    if constexpr (CDT == HXQ_F32) {
        const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(cache) + elem);
        const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(cache) + elem + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const u32x4 w = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(cache) + elem);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint16_t lo = static_cast<uint16_t>(w[j] & 0xffffu), hi = static_cast<uint16_t>(w[j] >> 16);
            v[2 * j] = CDT == HXQ_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
            v[2 * j + 1] = CDT == HXQ_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
        }
    }
}

// Rotation of element pair (i, i + D/2) at position pos (rotate_half).
__device__ __forceinline__ void rope_pair(float x1, float x2, int i, int D, int pos, float theta,
                                          float &o1, float &o2) {
    const float inv_freq = powf(theta, -2.f * i / D);
    float sn, cs;
    sincosf(static_cast<float>(pos) * inv_freq, &sn, &cs);
    o1 = x1 * cs - x2 * sn;
    o2 = x2 * cs + x1 * sn;
}

// ROPE = true: q is the fused qkv row of the token; the block rotates its q
// head and its kv head's new key, takes position pos's key and value from
// registers/LDS (rounded to the cache type, as a cache read would give), and
// the first q head of each kv group stores them into the caches (other
// blocks never read row pos of the cache in this launch).
template <int CDT, int ODT, bool ROPE>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(
    const float *q, const void *k_cache, const void *v_cache, const int32_t *pos_p,
    int32_t n_heads, int32_t n_kv, int32_t max_seq, void *out, float theta) {
    extern __shared__ float smem[];
    float *sc = smem;                      // [max_seq]
    __shared__ float qs[kAttnD];
    __shared__ float kn[kAttnD], vn[kAttnD];   // position pos (ROPE)
    __shared__ float part[kDecThreads / kWave][kAttnD];
    __shared__ float red[kDecThreads / kWave];
    constexpr int D = kAttnD;
    const int h = blockIdx.x;
    const int grp = n_heads / n_kv;
    const int kvh = h / grp;
    const int pos = *pos_p;
    if (ROPE && (pos < 0 || pos >= max_seq)) return;  // the host keeps pos < max_seq
    const int n = min(max(pos + 1, 1), max_seq);
    const float scale = rsqrtf(static_cast<float>(D));
    const int lane = threadIdx.x & 63, wave = threadIdx.x / kWave;
    constexpr int NW = kDecThreads / kWave;
    const int64_t row = (int64_t)n_kv * D;  // elements between positions
    if constexpr (ROPE) {
        const float *qh = q + (int64_t)h * D;
        const float *kh = q + (int64_t)(n_heads + kvh) * D;
        const float *vh = q + (int64_t)(n_heads + n_kv + kvh) * D;
        if (threadIdx.x < D / 2) {
            const int i = threadIdx.x;
            float a, b;
            rope_pair(qh[i], qh[i + D / 2], i, D, pos, theta, a, b);
            qs[i] = a * scale;
            qs[i + D / 2] = b * scale;
            rope_pair(kh[i], kh[i + D / 2], i, D, pos, theta, a, b);
            const int64_t base = (int64_t)pos * row + (int64_t)kvh * D;
            if (h % grp == 0) {
                store_act<CDT>(const_cast<void *>(k_cache), base + i, a);
                store_act<CDT>(const_cast<void *>(k_cache), base + i + D / 2, b);
            }
            kn[i] = load_back<CDT>(a);
            kn[i + D / 2] = load_back<CDT>(b);
        } else if (threadIdx.x < D / 2 + D) {
            const int j = threadIdx.x - D / 2;
            if (h % grp == 0)
                store_act<CDT>(const_cast<void *>(v_cache), (int64_t)pos * row + (int64_t)kvh * D + j, vh[j]);
            vn[j] = load_back<CDT>(vh[j]);
        }
    } else {
        if (threadIdx.x < D) qs[threadIdx.x] = q[(int64_t)h * D + threadIdx.x] * scale;
    }
    __syncthreads();
    float mx = -FLT_MAX;
    for (int t = threadIdx.x; t < n; t += kDecThreads) {
        const int64_t base = (int64_t)t * row + (int64_t)kvh * D;
        float s0 = 0.f, s1 = 0.f;
        if (ROPE && t == pos) {
            for (int d = 0; d < D; d += 2) {
                s0 = fmaf(qs[d], kn[d], s0);
                s1 = fmaf(qs[d + 1], kn[d + 1], s1);
            }
        } else {
            float kv[D / 8][8];
#pragma unroll
            for (int c = 0; c < D / 8; ++c) load_row8<CDT>(k_cache, base + 8 * c, kv[c]);
#pragma unroll
            for (int c = 0; c < D / 8; ++c)
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    s0 = fmaf(qs[8 * c + j], kv[c][j], s0);
                    s1 = fmaf(qs[8 * c + j + 1], kv[c][j + 1], s1);
                }
        }
        sc[t] = s0 + s1;
        mx = fmaxf(mx, s0 + s1);
    }
    mx = block_max(mx, red);  // barriers: sc[] complete
    float sum = 0.f;
    for (int t = threadIdx.x; t < n; t += kDecThreads) {
        const float p = expf(sc[t] - mx);
        sc[t] = p;
        sum += p;
    }
    sum = block_sum(sum, red);  // includes a barrier: sc[] complete
    const float inv = 1.f / sum;
    float a0 = 0.f, a1 = 0.f;
    const int64_t voff = (int64_t)kvh * D + 2 * lane;
    for (int t0 = wave; t0 < n; t0 += 8 * NW) {
        float v0[8], v1[8], p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int t = t0 + u * NW;
            const bool ok = t < n && !(ROPE && t == pos);
            const int64_t b = (int64_t)(ok ? t : 0) * row + voff;
            v0[u] = load_act<CDT>(v_cache, b);
            v1[u] = load_act<CDT>(v_cache, b + 1);
            p[u] = ok ? sc[t] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            a0 = fmaf(p[u], v0[u], a0);
            a1 = fmaf(p[u], v1[u], a1);
        }
    }
    if (ROPE && wave == pos % NW) {  // position pos: value from LDS
        a0 = fmaf(sc[pos], vn[2 * lane], a0);
        a1 = fmaf(sc[pos], vn[2 * lane + 1], a1);
    }
    part[wave][2 * lane] = a0;
    part[wave][2 * lane + 1] = a1;
    __syncthreads();
    if (threadIdx.x < D) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += part[w][threadIdx.x];
        store_act<ODT>(out, (int64_t)h * D + threadIdx.x, v * inv);
    }
}

template <int ODT>
__global__ __launch_bounds__(kDecThreads) void silu_mul_kernel(const float *g, const float *u,
                                                               int64_t n, void *out) {
    const int64_t i = blockIdx.x * (int64_t)kDecThreads + threadIdx.x;
    if (i >= n) return;
    const float a = g[i];
    store_act<ODT>(out, i, a / (1.f + expf(-a)) * u[i]);
}

// Greedy argmax over fp32 logits (ties -> lowest index) in two kernels:
// per-block partial maxima, then one block over the partials.
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__device__ __forceinline__ void block_argmax(float &best, int &idx) {
    __shared__ float bv[kDecThreads / kWave];
    __shared__ int bi[kDecThreads / kWave];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(best, m, kWave);
        const int oi = __shfl_xor(idx, m, kWave);
        better(best, idx, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x / 64] = best; bi[threadIdx.x / 64] = idx; }
    __syncthreads();
    for (int w = 0; w < kDecThreads / kWave; ++w) better(best, idx, bv[w], bi[w]);
}

constexpr int kArgBlocks = 256;

__global__ __launch_bounds__(kDecThreads) void argmax_partial_kernel(const float *logits, int32_t n,
                                                                     float *pv, int32_t *pi) {
    float best = -FLT_MAX;
    int idx = n;
    for (int i = blockIdx.x * kDecThreads + threadIdx.x; i < n; i += kArgBlocks * kDecThreads)
        better(best, idx, logits[i], i);
    block_argmax(best, idx);
    if (threadIdx.x == 0) { pv[blockIdx.x] = best; pi[blockIdx.x] = idx; }
}

__global__ __launch_bounds__(kDecThreads) void argmax_final_kernel(const float *pv, const int32_t *pi,
                                                                   int32_t *out_id, int32_t *pos_p) {
    float best = -FLT_MAX;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < kArgBlocks; i += kDecThreads) better(best, idx, pv[i], pi[i]);
    block_argmax(best, idx);
    if (threadIdx.x == 0) {
        *out_id = idx;
        if (pos_p) *pos_p += 1;  // advance the decode position for the next step
    }
}

// Dense bf16 GEMV (the uncompressed LM head): y[r] = sum_k W[r, k] x[k],
// fp32 accumulation and output.  Each wave owns kDenseRowsPerWave rows and
// issues all their 16-byte loads of one 512-column slab before reducing, so
// a wave keeps several KB in flight; x is staged in LDS as fp32.
constexpr int kDenseRowsPerWave = 4;

template <int XDT>
__global__ __launch_bounds__(kDecThreads) void dense_gemv_bf16_kernel(const uint16_t *W,
                                                                      const void *x, int64_t rows,
                                                                      int32_t K, float *y) {
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < K; i += kDecThreads) xs[i] = load_act<XDT>(x, i);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t r0 = ((int64_t)blockIdx.x * (kDecThreads / kWave) + threadIdx.x / kWave) *
                       kDenseRowsPerWave;
    float acc[kDenseRowsPerWave];
#pragma unroll
    for (int j = 0; j < kDenseRowsPerWave; ++j) acc[j] = 0.f;
    for (int c0 = 0; c0 < K / 8; c0 += kWave) {   // 512 columns per pass
        const int c = c0 + lane;
        const bool ok = c < K / 8;
        u32x4 v[kDenseRowsPerWave];
#pragma unroll
        for (int j = 0; j < kDenseRowsPerWave; ++j) {
            const int64_t r = min(r0 + j, rows - 1);  // tail rows re-read the last row
            v[j] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(W + r * K) + c)
                      : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < kDenseRowsPerWave; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[j] = fmaf(bf16_to_f32(static_cast<uint16_t>(v[j][e] & 0xffffu)),
                              ok ? xs[c * 8 + 2 * e] : 0.f, acc[j]);
                acc[j] = fmaf(bf16_to_f32(static_cast<uint16_t>(v[j][e] >> 16)),
                              ok ? xs[c * 8 + 2 * e + 1] : 0.f, acc[j]);
            }
    }
#pragma unroll
    for (int j = 0; j < kDenseRowsPerWave; ++j) {
        const float t = wave_sum(acc[j]);
        if (lane == 0 && r0 + j < rows) y[r0 + j] = t;
    }
}

static bool fdt(int32_t d) { return d == HXQ_F32 || d == HXQ_BF16 || d == HXQ_F16; }

}  // namespace hxq

using namespace hxq;

#define HXQ_DISPATCH_DT(dt, T, ...)                                            \
    do {                                                                      \
        if ((dt) == HXQ_F32) { constexpr int T = HXQ_F32; __VA_ARGS__; }       \
        else if ((dt) == HXQ_BF16) { constexpr int T = HXQ_BF16; __VA_ARGS__; } \
        else { constexpr int T = HXQ_F16; __VA_ARGS__; }                       \
    } while (0)

extern "C" int hxq_add_rmsnorm(float *x, const void *delta, int32_t delta_dtype,
                               const float *weight, float eps, int64_t rows, int64_t hidden,
                               void *out, int32_t out_dtype, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && weight && out, "x, weight and out are required");
    HXQ_REQUIRE(fdt(out_dtype) && (!delta || fdt(delta_dtype)), "bad dtype");
    HXQ_REQUIRE(rows > 0 && hidden > 0 && rows < (int64_t{1} << 31) &&
                    hidden <= (int64_t)kDecThreads * kNormPer, "bad sizes (hidden <= 4096)");
    const dim3 grid(static_cast<uint32_t>(rows));
    HXQ_DISPATCH_DT(delta ? delta_dtype : HXQ_F32, DD, HXQ_DISPATCH_DT(out_dtype, OD,
        hipLaunchKernelGGL((add_rmsnorm_kernel<DD, OD>), grid, dim3(kDecThreads), 0, stream, x,
                           delta, weight, eps, static_cast<int32_t>(hidden), out)));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_rope_kv_append(const float *qkv, const int32_t *pos, int32_t n_heads,
                                  int32_t n_kv_heads, int32_t head_dim, float theta, float *q_out,
                                  void *k_cache, void *v_cache, int32_t cache_dtype,
                                  int32_t max_seq, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(qkv && pos && q_out && k_cache && v_cache, "all pointers are required");
    HXQ_REQUIRE(fdt(cache_dtype), "bad cache dtype");
    HXQ_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && head_dim > 0 &&
                    head_dim % 2 == 0 && max_seq > 0, "bad sizes");
    const int total = (n_heads + n_kv_heads) * head_dim / 2 + n_kv_heads * head_dim;
    const dim3 grid((total + kDecThreads - 1) / kDecThreads);
    HXQ_DISPATCH_DT(cache_dtype, CD,
        hipLaunchKernelGGL((rope_append_kernel<CD>), grid, dim3(kDecThreads), 0, stream, qkv, pos,
                           n_heads, n_kv_heads, head_dim, theta, q_out, k_cache, v_cache,
                           max_seq));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_attn_decode(const float *q, const void *k_cache, const void *v_cache,
                               int32_t cache_dtype, const int32_t *pos, int32_t n_heads,
                               int32_t n_kv_heads, int32_t head_dim, int32_t max_seq, void *out,
                               int32_t out_dtype, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(q && k_cache && v_cache && pos && out, "all pointers are required");
    HXQ_REQUIRE(fdt(cache_dtype) && fdt(out_dtype), "bad dtype");
    HXQ_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 &&
                    head_dim == kAttnD && max_seq > 0, "head_dim must be 128");
    HXQ_REQUIRE(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0, "k_cache must be 16-byte aligned");
    const size_t shm = sizeof(float) * max_seq;
    HXQ_REQUIRE(shm <= 64 * 1024, "max_seq too large for the LDS score buffer");
    HXQ_DISPATCH_DT(cache_dtype, CD, HXQ_DISPATCH_DT(out_dtype, OD,
        hipLaunchKernelGGL((attn_decode_kernel<CD, OD, false>), dim3(n_heads), dim3(kDecThreads),
                           shm, stream, q, k_cache, v_cache, pos, n_heads, n_kv_heads, max_seq,
                           out, 0.f)));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_attn_rope_decode(const float *qkv, const int32_t *pos, int32_t n_heads,
                                    int32_t n_kv_heads, int32_t head_dim, float theta,
                                    void *k_cache, void *v_cache, int32_t cache_dtype,
                                    int32_t max_seq, void *out, int32_t out_dtype,
                                    hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(qkv && k_cache && v_cache && pos && out, "all pointers are required");
    HXQ_REQUIRE(fdt(cache_dtype) && fdt(out_dtype), "bad dtype");
    HXQ_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 &&
                    head_dim == kAttnD && max_seq > 0, "head_dim must be 128");
    HXQ_REQUIRE(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0, "k_cache must be 16-byte aligned");
    const size_t shm = sizeof(float) * max_seq;
    HXQ_REQUIRE(shm <= 64 * 1024, "max_seq too large for the LDS score buffer");
    HXQ_DISPATCH_DT(cache_dtype, CD, HXQ_DISPATCH_DT(out_dtype, OD,
        hipLaunchKernelGGL((attn_decode_kernel<CD, OD, true>), dim3(n_heads), dim3(kDecThreads),
                           shm, stream, qkv, k_cache, v_cache, pos, n_heads, n_kv_heads, max_seq,
                           out, theta)));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_silu_mul(const float *gate, const float *up, int64_t n, void *out,
                            int32_t out_dtype, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(gate && up && out && n > 0, "bad arguments");
    HXQ_REQUIRE(fdt(out_dtype), "bad dtype");
    HXQ_DISPATCH_DT(out_dtype, OD,
        hipLaunchKernelGGL((silu_mul_kernel<OD>), dim3((n + kDecThreads - 1) / kDecThreads),
                           dim3(kDecThreads), 0, stream, gate, up, n, out));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_argmax(const float *logits, int64_t n, int32_t *out_id, int32_t *pos,
                          void *workspace, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(logits && out_id && workspace && n > 0 && n < (int64_t{1} << 31),
                "bad arguments");
    float *pv = static_cast<float *>(workspace);
    int32_t *pi = reinterpret_cast<int32_t *>(pv + kArgBlocks);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks), dim3(kDecThreads), 0, stream,
                       logits, static_cast<int32_t>(n), pv, pi);
    HXQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kDecThreads), 0, stream, pv, pi, out_id,
                       pos);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_dense_gemv_bf16(const uint16_t *weight, const void *x, int32_t x_dtype,
                                   int64_t rows, int64_t in_features, float *y,
                                   hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(weight && x && y, "all pointers are required");
    HXQ_REQUIRE(fdt(x_dtype), "bad dtype");
    HXQ_REQUIRE(rows > 0 && rows < (int64_t{1} << 31) && in_features > 0 &&
                    in_features % 8 == 0 && in_features <= 16384,
                "in_features must be a multiple of 8, at most 16384");
    HXQ_REQUIRE(reinterpret_cast<uintptr_t>(weight) % 16 == 0, "weight must be 16-byte aligned");
    const int64_t rpb = (kDecThreads / kWave) * kDenseRowsPerWave;
    const dim3 grid(static_cast<uint32_t>((rows + rpb - 1) / rpb));
    const size_t shm = sizeof(float) * in_features;
    HXQ_DISPATCH_DT(x_dtype, XD,
        hipLaunchKernelGGL((dense_gemv_bf16_kernel<XD>), grid, dim3(kDecThreads), shm, stream,
                           weight, x, rows, static_cast<int32_t>(in_features), y));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}
