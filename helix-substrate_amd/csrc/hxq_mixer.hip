// Mamba2 mixer kernels around the selective scan: the causal depthwise conv1d
// + SiLU that splits in_proj's output into the scan inputs, the dt transform,
// and the gated RMSNorm in front of out_proj.  Prefill and single-token forms.
//
// Follows the reference mixer _chunked_scan_forward (helix_substrate/
// mamba_scan_chunked.py:239-387): split of in_proj's output into
// [d_mlp, d_mlp, gate, xBC, dt] (:256-261), causal conv1d over xBC with left
// zero padding and activation (:296-303), split xBC into x / B / C
// (:306-310), dt = clamp(softplus(dt + dt_bias), time_step_min) (:356-357),
// decode-step conv through a rolling conv_state (:269-282), and
// norm(y, gate) (:384) = weight * (y * silu(gate)) * rsqrt(mean(.^2) + eps)
// (transformers' gated RMSNorm, models/mamba2/modeling_mamba2.py:111-120).
// Arithmetic is fp32; each output is rounded once to its storage type.
#include "hxq_common.h"

namespace hxq {

constexpr int kConvT = 16;       // time steps per prefill conv block
constexpr int kConvTB = 4;       // time steps whose inputs one round requests together
constexpr int kMaxConvW = 8;     // supported conv widths 1..8

struct ConvArgs {
    const void *proj;        // [batch, seqlen, proj_width]
    const float *w;          // [conv_dim, width]
    const float *bias;       // [conv_dim] or null
    const float *dt_bias;    // [heads] or null
    void *x;                 // [batch, seqlen, d_inner]
    void *B;                 // [batch, seqlen, ngroups*state]
    void *C;
    float *dt;               // [batch, seqlen, heads]
    float *conv_state;       // [batch, conv_dim, width] or null (prefill: written)
    float dt_min, dt_max;
    int32_t batch, seqlen, proj_width, xbc_off, dt_off, d_inner, gn, heads, width;
    int32_t proj_dt, out_dt;
};

__device__ __forceinline__ float ld16or32(const void *p, int64_t i, int dt) {
    if (dt == HXQ_F32) return static_cast<const float *>(p)[i];
    const uint16_t v = static_cast<const uint16_t *>(p)[i];
    return dt == HXQ_BF16 ? bf16_to_f32(v) : f16_to_f32(v);
}

__device__ __forceinline__ void st16or32(void *p, int64_t i, int dt, float v) {
    if (dt == HXQ_F32) static_cast<float *>(p)[i] = v;
    else if (dt == HXQ_BF16) static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
    else static_cast<uint16_t *>(p)[i] = f32_to_f16(v);
}

__device__ __forceinline__ float silu(float v) { return v / (1.f + expf(-v)); }

// torch.nn.functional.softplus (beta 1, threshold 20)
__device__ __forceinline__ float softplus(float v) { return v > 20.f ? v : log1pf(expf(v)); }

__device__ __forceinline__ float dt_transform(float raw, const ConvArgs &a, int h) {
    float v = raw + (a.dt_bias ? a.dt_bias[h] : 0.f);
    v = softplus(v);
    return fminf(fmaxf(v, a.dt_min), a.dt_max);
}

__device__ __forceinline__ void store_xbc(const ConvArgs &a, int64_t bt, int c, float v) {
    if (c < a.d_inner) st16or32(a.x, bt * a.d_inner + c, a.out_dt, v);
    else if (c < a.d_inner + a.gn) st16or32(a.B, bt * a.gn + (c - a.d_inner), a.out_dt, v);
    else st16or32(a.C, bt * a.gn + (c - a.d_inner - a.gn), a.out_dt, v);
}

// Prefill: thread = channel (conv_dim channels, then `heads` dt channels);
// a block walks kConvT time steps keeping a sliding window of inputs in
// registers, so every input is read once per block.
__global__ __launch_bounds__(256) void conv_split_kernel(const ConvArgs a) {
    const int conv_dim = a.d_inner + 2 * a.gn;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int t0 = blockIdx.y * kConvT;
    const int b = blockIdx.z;
    if (c >= conv_dim + a.heads) return;
    const int t1 = min(t0 + kConvT, a.seqlen);
    const int64_t row0 = (int64_t)b * a.seqlen;
    if (c >= conv_dim) {
        const int h = c - conv_dim;
        for (int t = t0; t < t1; ++t)
            a.dt[(row0 + t) * a.heads + h] =
                dt_transform(ld16or32(a.proj, (row0 + t) * a.proj_width + a.dt_off + h, a.proj_dt), a, h);
        return;
    }
    const int W = a.width;
    float w[kMaxConvW], win[kMaxConvW];
#pragma unroll
    for (int k = 0; k < kMaxConvW; ++k) {
        w[k] = k < W ? a.w[(int64_t)c * W + k] : 0.f;
        win[k] = 0.f;
    }
    const float bias = a.bias ? a.bias[c] : 0.f;
    const float wlast = a.w[(int64_t)c * W + W - 1];  // tap of the current input
    const int64_t col = a.xbc_off + c;
    // window slots 0..W-2 hold inputs t-W+1 .. t-1 (zero before t = 0)
#pragma unroll
    for (int k = 0; k < kMaxConvW - 1; ++k) {
        const int tt = t0 - (W - 1) + k;
        if (k < W - 1 && tt >= 0) win[k] = ld16or32(a.proj, (row0 + tt) * a.proj_width + col, a.proj_dt);
    }
    for (int t = t0; t < t1; ++t) {
        const float cur = ld16or32(a.proj, (row0 + t) * a.proj_width + col, a.proj_dt);
        float acc = bias;
#pragma unroll
        for (int k = 0; k < kMaxConvW; ++k) {
            if (k < W - 1) acc = fmaf(w[k], win[k], acc);
        }
        acc = fmaf(wlast, cur, acc);
        store_xbc(a, row0 + t, c, silu(acc));
#pragma unroll
        for (int k = 0; k < kMaxConvW - 1; ++k) {
            if (k < W - 2) win[k] = win[k + 1];
        }
        if (W >= 2) {
            // slot W-2 takes the current input
#pragma unroll
            for (int k = 0; k < kMaxConvW - 1; ++k)
                if (k == W - 2) win[k] = cur;
        }
    }
    // conv_state after the last step: the last W raw inputs (zero before t=0)
    if (a.conv_state && t1 == a.seqlen) {
        float *cs = a.conv_state + ((int64_t)b * conv_dim + c) * W;
        for (int k = 0; k < W; ++k) {
            const int tt = a.seqlen - W + k;
            cs[k] = tt >= 0 ? ld16or32(a.proj, (row0 + tt) * a.proj_width + col, a.proj_dt) : 0.f;
        }
    }
}

// Prefill, 16-bit proj and outputs (the Mamba2 shapes: channel counts and
// offsets multiples of 8): a thread owns 8 consecutive channels, reads each
// time step's 8 inputs as one 16-byte load and writes the 8 outputs as one
// 16-byte store; the W-1 previous inputs of its channels stay in registers
// (W <= 4).  dt channels keep the scalar kernel (a second launch).
template <int W, bool BF16>
__global__ __launch_bounds__(256) void conv_split_vec_kernel(const ConvArgs a) {
    const int conv_dim = a.d_inner + 2 * a.gn;
    const int cg = blockIdx.x * 256 + threadIdx.x;  // channel group: channels 8 cg .. 8 cg + 7
    const int c0 = 8 * cg;
    if (c0 >= conv_dim) return;
    const int t0 = blockIdx.y * kConvT;
    const int b = blockIdx.z;
    const int t1 = min(t0 + kConvT, a.seqlen);
    const int64_t row0 = (int64_t)b * a.seqlen;
    float w[8][W], bias[8], win[W > 1 ? W - 1 : 1][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int k = 0; k < W; ++k) w[j][k] = a.w[(int64_t)(c0 + j) * W + k];
        bias[j] = a.bias ? a.bias[c0 + j] : 0.f;
    }
    const uint16_t *proj = static_cast<const uint16_t *>(a.proj);
    auto load8 = [&](int64_t t, float (&v)[8]) {
        const u32x4 q = *reinterpret_cast<const u32x4 *>(proj + (row0 + t) * a.proj_width + a.xbc_off + c0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint16_t h = static_cast<uint16_t>(q[j >> 1] >> (16 * (j & 1)));
            v[j] = BF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
    };
    // window slot k holds input t - (W - 1) + k (zero before t = 0)
#pragma unroll
    for (int k = 0; k < W - 1; ++k) {
        const int tt = t0 - (W - 1) + k;
        if (tt >= 0) load8(tt, win[k]);
        else {
#pragma unroll
            for (int j = 0; j < 8; ++j) win[k][j] = 0.f;
        }
    }
    // destination: x, B or C (a group of 8 never straddles them)
    uint16_t *dst;
    int64_t dstride, doff;
    if (c0 < a.d_inner) { dst = static_cast<uint16_t *>(a.x); dstride = a.d_inner; doff = c0; }
    else if (c0 < a.d_inner + a.gn) { dst = static_cast<uint16_t *>(a.B); dstride = a.gn; doff = c0 - a.d_inner; }
    else { dst = static_cast<uint16_t *>(a.C); dstride = a.gn; doff = c0 - a.d_inner - a.gn; }
    const bool obf = a.out_dt == HXQ_BF16;
    // kConvTB time steps per round: their inputs are all requested before the
    // first is used (one memory round trip per round, not per step)
    for (int tb = t0; tb < t1; tb += kConvTB) {
        u32x4 qin[kConvTB];
#pragma unroll
        for (int i = 0; i < kConvTB; ++i) {
            const int t = min(tb + i, t1 - 1);  // past t1: a repeat of a loaded row, unused
            qin[i] = *reinterpret_cast<const u32x4 *>(proj + (row0 + t) * a.proj_width + a.xbc_off + c0);
        }
#pragma unroll
        for (int i = 0; i < kConvTB; ++i) {
            const int t = tb + i;
            if (t >= t1) break;
            float cur[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint16_t h = static_cast<uint16_t>(qin[i][j >> 1] >> (16 * (j & 1)));
                cur[j] = BF16 ? bf16_to_f32(h) : f16_to_f32(h);
            }
            uint32_t o[4];
#pragma unroll
            for (int j2 = 0; j2 < 4; ++j2) {
                float r[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int j = 2 * j2 + e;
                    float acc = bias[j];
#pragma unroll
                    for (int k = 0; k < W - 1; ++k) acc = fmaf(w[j][k], win[k][j], acc);
                    acc = fmaf(w[j][W - 1], cur[j], acc);
                    r[e] = silu(acc);
                }
                o[j2] = obf ? (uint32_t(f32_to_bf16(r[0])) | (uint32_t(f32_to_bf16(r[1])) << 16))
                            : (uint32_t(f32_to_f16(r[0])) | (uint32_t(f32_to_f16(r[1])) << 16));
            }
            *reinterpret_cast<u32x4 *>(dst + (row0 + t) * dstride + doff) = u32x4{o[0], o[1], o[2], o[3]};
#pragma unroll
            for (int k = 0; k + 1 < W - 1; ++k)
#pragma unroll
                for (int j = 0; j < 8; ++j) win[k][j] = win[k + 1][j];
            if constexpr (W > 1) {
#pragma unroll
                for (int j = 0; j < 8; ++j) win[W - 2][j] = cur[j];
            }
        }
    }
    // conv_state after the last step: the last W raw inputs (zero before t=0)
    if (a.conv_state && t1 == a.seqlen) {
#pragma unroll
        for (int k = 0; k < W; ++k) {
            const int tt = a.seqlen - W + k;
            float v[8];
            if (tt >= 0) load8(tt, v);
            else {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) a.conv_state[((int64_t)b * conv_dim + c0 + j) * W + k] = v[j];
        }
    }
}

// dt channels only (the vector conv kernel covers x/B/C)
__global__ __launch_bounds__(256) void dt_kernel(const ConvArgs a) {
    const int64_t i = blockIdx.x * 256ll + threadIdx.x;  // (row, head)
    const int64_t n = (int64_t)a.batch * a.seqlen * a.heads;
    if (i >= n) return;
    const int64_t row = i / a.heads;
    const int h = static_cast<int>(i % a.heads);
    a.dt[i] = dt_transform(ld16or32(a.proj, row * a.proj_width + a.dt_off + h, a.proj_dt), a, h);
}

// Decode: one token per batch row; conv_state [b, conv_dim, W] rolls left and
// takes the new input in its last slot, then y = silu(sum(state * w) + bias).
__global__ __launch_bounds__(256) void conv_step_kernel(const ConvArgs a) {
    const int conv_dim = a.d_inner + 2 * a.gn;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= conv_dim + a.heads) return;
    if (c >= conv_dim) {
        const int h = c - conv_dim;
        a.dt[(int64_t)b * a.heads + h] =
            dt_transform(ld16or32(a.proj, (int64_t)b * a.proj_width + a.dt_off + h, a.proj_dt), a, h);
        return;
    }
    const int W = a.width;
    float *cs = a.conv_state + ((int64_t)b * conv_dim + c) * W;
    const float cur = ld16or32(a.proj, (int64_t)b * a.proj_width + a.xbc_off + c, a.proj_dt);
    float acc = a.bias ? a.bias[c] : 0.f;
    for (int k = 0; k < W - 1; ++k) {
        const float v = cs[k + 1];
        cs[k] = v;
        acc = fmaf(a.w[(int64_t)c * W + k], v, acc);
    }
    cs[W - 1] = cur;
    acc = fmaf(a.w[(int64_t)c * W + W - 1], cur, acc);
    store_xbc(a, b, c, silu(acc));
}

// Gated RMSNorm: one block per row; h = y * silu(gate), out = weight * h *
// rsqrt(mean(h^2 over the row's group) + eps).  group = width for the
// single-group norm.
template <int YDT, int GDT, int ODT>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const void *y, const void *gate,
                                                            int64_t gate_stride, const float *w,
                                                            float eps, int32_t width,
                                                            int32_t group, void *out) {
    __shared__ float red[256 / kWave];
    const int64_t r = blockIdx.x;
    const int ngrp = width / group;
    const int tid = threadIdx.x;
    for (int gi = 0; gi < ngrp; ++gi) {
        const int c0 = gi * group;
        float ss = 0.f;
        for (int i = tid; i < group; i += 256) {
            const float h = load_act<YDT>(y, r * width + c0 + i) *
                            silu(load_act<GDT>(gate, r * gate_stride + c0 + i));
            ss = fmaf(h, h, ss);
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid / 64] = ss;
        __syncthreads();
        const float tot = red[0] + red[1] + red[2] + red[3];
        __syncthreads();
        const float inv = rsqrtf(tot / group + eps);
        for (int i = tid; i < group; i += 256) {
            const float h = load_act<YDT>(y, r * width + c0 + i) *
                            silu(load_act<GDT>(gate, r * gate_stride + c0 + i));
            store_act<ODT>(out, r * width + c0 + i, w[c0 + i] * (h * inv));
        }
    }
}

// One row per block with group == width == 256 EPT: a thread holds EPT
// elements in registers (chunks of 8 at stride 256 x 8), one read of y and
// gate, 16-byte accesses.
template <int YDT, int GDT, int ODT, int EPT>
__global__ __launch_bounds__(256) void gated_rmsnorm_vec_kernel(const void *y, const void *gate,
                                                                int64_t gate_stride, const float *w,
                                                                float eps, void *out) {
    constexpr int NC = EPT / 8;
    constexpr int width = 256 * EPT;
    __shared__ float red[256 / kWave];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    float h[NC][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int e0 = 8 * (tid + 256 * j);
        float yv[8], gv[8];
        if constexpr (YDT == HXQ_F32) {
            const float4 a0 = *reinterpret_cast<const float4 *>(static_cast<const float *>(y) + r * width + e0);
            const float4 a1 = *reinterpret_cast<const float4 *>(static_cast<const float *>(y) + r * width + e0 + 4);
            yv[0] = a0.x; yv[1] = a0.y; yv[2] = a0.z; yv[3] = a0.w;
            yv[4] = a1.x; yv[5] = a1.y; yv[6] = a1.z; yv[7] = a1.w;
        } else {
            const u32x4 q = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(y) + r * width + e0);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t v = static_cast<uint16_t>(q[e >> 1] >> (16 * (e & 1)));
                yv[e] = YDT == HXQ_BF16 ? bf16_to_f32(v) : f16_to_f32(v);
            }
        }
        if constexpr (GDT == HXQ_F32) {
            const float *gp = static_cast<const float *>(gate) + r * gate_stride + e0;
            const float4 a0 = *reinterpret_cast<const float4 *>(gp);
            const float4 a1 = *reinterpret_cast<const float4 *>(gp + 4);
            gv[0] = a0.x; gv[1] = a0.y; gv[2] = a0.z; gv[3] = a0.w;
            gv[4] = a1.x; gv[5] = a1.y; gv[6] = a1.z; gv[7] = a1.w;
        } else {
            const u32x4 q = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(gate) + r * gate_stride + e0);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t v = static_cast<uint16_t>(q[e >> 1] >> (16 * (e & 1)));
                gv[e] = GDT == HXQ_BF16 ? bf16_to_f32(v) : f16_to_f32(v);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h[j][e] = yv[e] * silu(gv[e]);
            ss = fmaf(h[j][e], h[j][e], ss);
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid / 64] = ss;
    __syncthreads();
    const float inv = rsqrtf((red[0] + red[1] + red[2] + red[3]) / width + eps);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int e0 = 8 * (tid + 256 * j);
        const float4 w0 = *reinterpret_cast<const float4 *>(w + e0);
        const float4 w1 = *reinterpret_cast<const float4 *>(w + e0 + 4);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = wv[e] * (h[j][e] * inv);
        if constexpr (ODT == HXQ_F32) {
            float *op = static_cast<float *>(out) + r * width + e0;
            *reinterpret_cast<float4 *>(op) = make_float4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<float4 *>(op + 4) = make_float4(o[4], o[5], o[6], o[7]);
        } else {
            uint32_t q[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t lo = ODT == HXQ_BF16 ? f32_to_bf16(o[2 * e]) : f32_to_f16(o[2 * e]);
                const uint16_t hi = ODT == HXQ_BF16 ? f32_to_bf16(o[2 * e + 1]) : f32_to_f16(o[2 * e + 1]);
                q[e] = uint32_t(lo) | (uint32_t(hi) << 16);
            }
            *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(out) + r * width + e0) = u32x4{q[0], q[1], q[2], q[3]};
        }
    }
}

template <int YDT, int GDT>
static void launch_norm_o(int odt, dim3 grid, hipStream_t s, const void *y, const void *gate,
                          int64_t gs, const float *w, float eps, int32_t width, int32_t group,
                          void *out) {
    // one group per row, 256 x {8, 16, 32} wide, 16-byte aligned rows: the register kernel
    const int ys = YDT == HXQ_F32 ? 4 : 2, gsz = GDT == HXQ_F32 ? 4 : 2, os = odt == HXQ_F32 ? 4 : 2;
    const bool aligned = ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(gate) |
                           reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(w)) & 15u) == 0 &&
                         (int64_t{width} * ys) % 16 == 0 && (gs * gsz) % 16 == 0 &&
                         (int64_t{width} * os) % 16 == 0;
    if (group == width && aligned && (width == 2048 || width == 4096 || width == 8192)) {
#define HXQ_NORM_VEC(EPT)                                                                          \
        if (odt == HXQ_F32)                                                                         \
            hipLaunchKernelGGL((gated_rmsnorm_vec_kernel<YDT, GDT, HXQ_F32, EPT>), grid, dim3(256), 0, s, y, gate, gs, w, eps, out); \
        else if (odt == HXQ_BF16)                                                                   \
            hipLaunchKernelGGL((gated_rmsnorm_vec_kernel<YDT, GDT, HXQ_BF16, EPT>), grid, dim3(256), 0, s, y, gate, gs, w, eps, out); \
        else                                                                                        \
            hipLaunchKernelGGL((gated_rmsnorm_vec_kernel<YDT, GDT, HXQ_F16, EPT>), grid, dim3(256), 0, s, y, gate, gs, w, eps, out);
        if (width == 2048) { HXQ_NORM_VEC(8) }
        else if (width == 4096) { HXQ_NORM_VEC(16) }
        else { HXQ_NORM_VEC(32) }
#undef HXQ_NORM_VEC
        return;
    }
    if (odt == HXQ_F32)
        hipLaunchKernelGGL((gated_rmsnorm_kernel<YDT, GDT, HXQ_F32>), grid, dim3(256), 0, s, y,
                           gate, gs, w, eps, width, group, out);
    else if (odt == HXQ_BF16)
        hipLaunchKernelGGL((gated_rmsnorm_kernel<YDT, GDT, HXQ_BF16>), grid, dim3(256), 0, s, y,
                           gate, gs, w, eps, width, group, out);
    else
        hipLaunchKernelGGL((gated_rmsnorm_kernel<YDT, GDT, HXQ_F16>), grid, dim3(256), 0, s, y,
                           gate, gs, w, eps, width, group, out);
}

template <int YDT>
static void launch_norm_g(int gdt, int odt, dim3 grid, hipStream_t s, const void *y,
                          const void *gate, int64_t gs, const float *w, float eps, int32_t width,
                          int32_t group, void *out) {
    if (gdt == HXQ_F32) launch_norm_o<YDT, HXQ_F32>(odt, grid, s, y, gate, gs, w, eps, width, group, out);
    else if (gdt == HXQ_BF16) launch_norm_o<YDT, HXQ_BF16>(odt, grid, s, y, gate, gs, w, eps, width, group, out);
    else launch_norm_o<YDT, HXQ_F16>(odt, grid, s, y, gate, gs, w, eps, width, group, out);
}

static bool dt_ok(int32_t d) { return d == HXQ_F32 || d == HXQ_BF16 || d == HXQ_F16; }

static int check_conv(const void *proj, int32_t proj_dtype, const float *conv_w,
                      int64_t batch, int64_t seqlen, int64_t d_mlp, int64_t d_inner,
                      int64_t ngroups, int64_t state, int64_t heads, int64_t width,
                      int32_t out_dtype, const void *x, const void *B, const void *C,
                      const float *dt) {
    HXQ_REQUIRE(proj && conv_w && x && B && C && dt, "proj, conv_w, x, B, C and dt are required");
    HXQ_REQUIRE(dt_ok(proj_dtype) && dt_ok(out_dtype), "bad dtype");
    HXQ_REQUIRE(batch > 0 && seqlen > 0 && d_inner > 0 && ngroups > 0 && state > 0 && heads > 0 &&
                    d_mlp >= 0, "bad sizes");
    HXQ_REQUIRE(width >= 1 && width <= kMaxConvW, "conv width must be in 1..8");
    const int64_t pw = 2 * d_mlp + 2 * d_inner + 2 * ngroups * state + heads;
    HXQ_REQUIRE(batch * seqlen * pw < (int64_t{1} << 40), "problem too large");
    return HXQ_OK;
}

}  // namespace hxq

using namespace hxq;

extern "C" int hxq_mamba2_conv_split(const void *proj, int32_t proj_dtype, const float *conv_w,
                                     const float *conv_b, const float *dt_bias, float dt_min,
                                     float dt_max, int64_t batch, int64_t seqlen, int64_t d_mlp,
                                     int64_t d_inner, int64_t ngroups, int64_t state,
                                     int64_t heads, int64_t width, void *x, void *B, void *C,
                                     int32_t out_dtype, float *dt, float *conv_state,
                                     hipStream_t stream) {
    clear_error();
    if (int rc = check_conv(proj, proj_dtype, conv_w, batch, seqlen, d_mlp, d_inner, ngroups,
                            state, heads, width, out_dtype, x, B, C, dt))
        return rc;
    ConvArgs a{};
    a.proj = proj; a.w = conv_w; a.bias = conv_b; a.dt_bias = dt_bias;
    a.x = x; a.B = B; a.C = C; a.dt = dt; a.conv_state = conv_state;
    a.dt_min = dt_min; a.dt_max = dt_max;
    a.batch = (int32_t)batch; a.seqlen = (int32_t)seqlen;
    a.proj_width = (int32_t)(2 * d_mlp + 2 * d_inner + 2 * ngroups * state + heads);
    a.xbc_off = (int32_t)(2 * d_mlp + d_inner);
    a.dt_off = (int32_t)(2 * d_mlp + 2 * d_inner + 2 * ngroups * state);
    a.d_inner = (int32_t)d_inner; a.gn = (int32_t)(ngroups * state); a.heads = (int32_t)heads;
    a.width = (int32_t)width; a.proj_dt = proj_dtype; a.out_dt = out_dtype;
    const int channels = a.d_inner + 2 * a.gn + a.heads;
    // 16-bit proj and outputs, channel counts / offsets multiples of 8, 16-byte
    // aligned buffers, W <= 4: the 8-channel vector kernel plus the dt kernel
    const bool vec = proj_dtype != HXQ_F32 && out_dtype == proj_dtype && width <= 4 &&
                     a.proj_width % 8 == 0 && a.xbc_off % 8 == 0 && a.d_inner % 8 == 0 &&
                     a.gn % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(proj) | reinterpret_cast<uintptr_t>(x) |
                       reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) & 15u) == 0;
    if (vec) {
        const int groups = (a.d_inner + 2 * a.gn) / 8;
        const dim3 grid((groups + 255) / 256, (a.seqlen + kConvT - 1) / kConvT, a.batch);
        const bool bf = proj_dtype == HXQ_BF16;
        switch (width) {
            case 1: if (bf) hipLaunchKernelGGL((conv_split_vec_kernel<1, true>), grid, dim3(256), 0, stream, a);
                    else hipLaunchKernelGGL((conv_split_vec_kernel<1, false>), grid, dim3(256), 0, stream, a);
                    break;
            case 2: if (bf) hipLaunchKernelGGL((conv_split_vec_kernel<2, true>), grid, dim3(256), 0, stream, a);
                    else hipLaunchKernelGGL((conv_split_vec_kernel<2, false>), grid, dim3(256), 0, stream, a);
                    break;
            case 3: if (bf) hipLaunchKernelGGL((conv_split_vec_kernel<3, true>), grid, dim3(256), 0, stream, a);
                    else hipLaunchKernelGGL((conv_split_vec_kernel<3, false>), grid, dim3(256), 0, stream, a);
                    break;
            default: if (bf) hipLaunchKernelGGL((conv_split_vec_kernel<4, true>), grid, dim3(256), 0, stream, a);
                     else hipLaunchKernelGGL((conv_split_vec_kernel<4, false>), grid, dim3(256), 0, stream, a);
                     break;
        }
        HXQ_LAUNCH_CHECK();
        const int64_t n = (int64_t)a.batch * a.seqlen * a.heads;
        hipLaunchKernelGGL(dt_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, a);
        HXQ_LAUNCH_CHECK();
        return HXQ_OK;
    }
    const dim3 grid((channels + 255) / 256, (a.seqlen + kConvT - 1) / kConvT, a.batch);
    hipLaunchKernelGGL(conv_split_kernel, grid, dim3(256), 0, stream, a);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_mamba2_conv_step(const void *proj, int32_t proj_dtype, const float *conv_w,
                                    const float *conv_b, const float *dt_bias, float dt_min,
                                    float dt_max, int64_t batch, int64_t d_mlp, int64_t d_inner,
                                    int64_t ngroups, int64_t state, int64_t heads, int64_t width,
                                    float *conv_state, void *x, void *B, void *C,
                                    int32_t out_dtype, float *dt, hipStream_t stream) {
    clear_error();
    if (int rc = check_conv(proj, proj_dtype, conv_w, batch, 1, d_mlp, d_inner, ngroups, state,
                            heads, width, out_dtype, x, B, C, dt))
        return rc;
    HXQ_REQUIRE(conv_state != nullptr, "conv_state is required");
    ConvArgs a{};
    a.proj = proj; a.w = conv_w; a.bias = conv_b; a.dt_bias = dt_bias;
    a.x = x; a.B = B; a.C = C; a.dt = dt; a.conv_state = conv_state;
    a.dt_min = dt_min; a.dt_max = dt_max;
    a.batch = (int32_t)batch; a.seqlen = 1;
    a.proj_width = (int32_t)(2 * d_mlp + 2 * d_inner + 2 * ngroups * state + heads);
    a.xbc_off = (int32_t)(2 * d_mlp + d_inner);
    a.dt_off = (int32_t)(2 * d_mlp + 2 * d_inner + 2 * ngroups * state);
    a.d_inner = (int32_t)d_inner; a.gn = (int32_t)(ngroups * state); a.heads = (int32_t)heads;
    a.width = (int32_t)width; a.proj_dt = proj_dtype; a.out_dt = out_dtype;
    const int channels = a.d_inner + 2 * a.gn + a.heads;
    hipLaunchKernelGGL(conv_step_kernel, dim3((channels + 255) / 256, a.batch), dim3(256), 0,
                       stream, a);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_gated_rmsnorm(const void *y, int32_t y_dtype, const void *gate,
                                 int32_t gate_dtype, int64_t gate_row_stride,
                                 const float *weight, float eps, int64_t rows, int64_t width,
                                 int64_t group_size, void *out, int32_t out_dtype,
                                 hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(y && gate && weight && out, "y, gate, weight and out are required");
    HXQ_REQUIRE(dt_ok(y_dtype) && dt_ok(gate_dtype) && dt_ok(out_dtype), "bad dtype");
    HXQ_REQUIRE(rows > 0 && width > 0 && rows < (int64_t{1} << 31), "bad sizes");
    const int64_t grp = group_size > 0 ? group_size : width;
    HXQ_REQUIRE(width % grp == 0, "group_size must divide width");
    HXQ_REQUIRE(gate_row_stride >= width, "gate_row_stride must be >= width");
    const dim3 grid(static_cast<uint32_t>(rows));
    if (y_dtype == HXQ_F32)
        launch_norm_g<HXQ_F32>(gate_dtype, out_dtype, grid, stream, y, gate, gate_row_stride,
                               weight, eps, (int32_t)width, (int32_t)grp, out);
    else if (y_dtype == HXQ_BF16)
        launch_norm_g<HXQ_BF16>(gate_dtype, out_dtype, grid, stream, y, gate, gate_row_stride,
                                weight, eps, (int32_t)width, (int32_t)grp, out);
    else
        launch_norm_g<HXQ_F16>(gate_dtype, out_dtype, grid, stream, y, gate, gate_row_stride,
                               weight, eps, (int32_t)width, (int32_t)grp, out);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}
