// Mamba/Mamba2 selective scan (fp32 state), chunk-parallel.
//
// Replaces chunked_scan / sequential_scan (helix_substrate/mamba_scan_chunked.py:
// 42-86, 89-213) and triton_scan / triton_mamba_scan_chunk / triton_mamba_decode_step
// (triton_mamba_scan.py:246-416).  Recurrence per (batch b, head h, channel p,
// state n), mamba_scan_chunked.py:66-84:
//     a_t = exp(A[h] * dt[b,t,h])
//     h_t = a_t * h_{t-1} + (dt[b,t,h] * x[b,t,h,p]) * B[b,t,g,n]
//     y_t = sum_n h_t * C[b,t,g,n] + D[h] * x[b,t,h,p]          (g = h / (H/G))
//
// The sequence is cut into chunks of `chunk` steps and scanned in three passes:
//   1. chunk_state : per (b, h, chunk) run the recurrence from a zero state and
//                    store the chunk's end state S_c and its summed log decay
//                    L_c = sum_t A*dt_t;
//   2. state_pass  : per (b, h, p, n), sequentially over chunks,
//                    Hin_0 = h0, Hin_{c+1} = exp(L_c) * Hin_c + S_c
//                    (Hin overwrites S in place; Hin_nchunks is h_final);
//   3. chunk_scan  : per (b, h, chunk) run the recurrence from Hin_c and emit y.
// Every exponent is A*dt <= 0 summed over a chunk, so nothing overflows (the
// reference's b/cumA closed form needs a sequential fallback at strong decay,
// mamba_scan_chunked.py:171-183).
//
// Layout of a scan block: 8 waves = HPB heads x NSPLIT state splits; lane = p
// (head_dim <= 64 per p-block); each lane keeps its N/NSPLIT (<= 32) states in
// VGPRs and reads a step's B/C values into registers before using them.
// Per block of TB = 16 steps, B/C (fp32), x and dt are staged in LDS and B/C
// are read as LDS broadcasts; per-split y partials are summed through LDS in a
// fixed order (deterministic).
#include <algorithm>

#include "hxq_common.h"

namespace hxq {

constexpr int kScanWaves = 8;
constexpr int kScanThreads = kScanWaves * kWave;
constexpr int kTB = 16;  // steps staged per LDS block

struct ScanArgs {
    const void *x;      // [B, L, H, P]
    const void *dt;     // [B, L, H]
    const float *A;     // [H]
    const void *Bm;     // [B, L, G, N]
    const void *Cm;     // [B, L, G, N]
    const float *D;     // [H] or null
    const float *h0;    // [B, H, P, N] or null
    void *y;            // [B, L, H, P]
    float *h_final;     // [B, H, P, N] or null
    float *ws_state;    // [nchunks, B, H, P, N]
    float *ws_decay;    // [nchunks, B, H]
    int32_t batch, seqlen, heads, head_dim, state, ngroups, chunk, nchunks;
    int32_t x_dt, dt_dt, bc_dt, y_dt;
};

__device__ __forceinline__ float ld_any(const void *p, int64_t i, int dt) {
    if (dt == HXQ_F32) return static_cast<const float *>(p)[i];
    const uint16_t v = static_cast<const uint16_t *>(p)[i];
    return dt == HXQ_BF16 ? bf16_to_f32(v) : f16_to_f32(v);
}

// Passes 1 and 3.  SL = states per lane, HPB = heads per block; NSPLIT =
// kScanWaves / HPB state splits, N = SL * NSPLIT.  EMIT_Y selects pass 3.
template <int SL, int HPB, bool EMIT_Y>
__global__ __launch_bounds__(kScanThreads, 4) void scan_chunk_kernel(const ScanArgs a) {
    constexpr int NSPLIT = kScanWaves / HPB;
    const int N = SL * NSPLIT;
    __shared__ float sB[kTB][SL * NSPLIT];
    __shared__ float sC[EMIT_Y ? kTB : 1][SL * NSPLIT];
    __shared__ float sX[kTB][HPB][64];
    __shared__ float sDt[kTB][HPB];
    __shared__ float sY[EMIT_Y ? kTB : 1][NSPLIT][HPB][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int hl = wave % HPB;      // head within the block
    const int ns = wave / HPB;      // state split
    // grid: x = head block * p-blocks, y = chunk, z = batch
    const int pblocks = (a.head_dim + 63) / 64;
    const int hb = blockIdx.x / pblocks, pb = blockIdx.x % pblocks;
    const int c = blockIdx.y, b = blockIdx.z;
    const int h = hb * HPB + hl;
    const int p = pb * 64 + lane;
    const bool p_ok = p < a.head_dim;
    const int H = a.heads, P = a.head_dim, L = a.seqlen;
    const int g_of_block = (hb * HPB) / (H / a.ngroups);  // all heads of a block share a group
    const int t0 = c * a.chunk;
    const int t1 = min(t0 + a.chunk, L);
    const float Ah = a.A[h];
    const float Dh = (EMIT_Y && a.D) ? a.D[h] : 0.f;

    float st[SL];
    const int64_t sbase = (((int64_t)b * H + h) * P + p) * N + ns * SL;  // [B,H,P,N] offset
    if constexpr (EMIT_Y) {
        const float *hin = a.ws_state + (int64_t)c * a.batch * H * P * N;
#pragma unroll
        for (int i = 0; i < SL; ++i) st[i] = p_ok ? hin[sbase + i] : 0.f;
    } else {
#pragma unroll
        for (int i = 0; i < SL; ++i) st[i] = 0.f;
    }
    float lsum = 0.f;  // sum of A*dt over the chunk (pass 1)

    for (int tb = t0; tb < t1; tb += kTB) {
        const int nt = min(kTB, t1 - tb);
        __syncthreads();  // previous block's readers are done
        // stage B (and C) rows: [nt][N]
        for (int e = tid; e < nt * N; e += kScanThreads) {
            const int tt = e / N, n = e % N;
            const int64_t bi = (((int64_t)b * L + tb + tt) * a.ngroups + g_of_block) * N + n;
            sB[tt][n] = ld_any(a.Bm, bi, a.bc_dt);
            if constexpr (EMIT_Y) sC[tt][n] = ld_any(a.Cm, bi, a.bc_dt);
        }
        for (int e = tid; e < nt * HPB * 64; e += kScanThreads) {
            const int tt = e / (HPB * 64), r = e % (HPB * 64);
            const int hh = hb * HPB + r / 64, pp = pb * 64 + r % 64;
            sX[tt][r / 64][r % 64] =
                pp < P ? ld_any(a.x, (((int64_t)b * L + tb + tt) * H + hh) * P + pp, a.x_dt) : 0.f;
        }
        for (int e = tid; e < nt * HPB; e += kScanThreads) {
            const int tt = e / HPB, hh = e % HPB;
            sDt[tt][hh] = ld_any(a.dt, ((int64_t)b * L + tb + tt) * H + hb * HPB + hh, a.dt_dt);
        }
        __syncthreads();
        for (int tt = 0; tt < nt; ++tt) {
            const float dtv = sDt[tt][hl];
            const float ad = Ah * dtv;
            const float da = expf(ad);
            const float xv = sX[tt][hl][lane];
            const float dx = dtv * xv;
            // B (and C) values of a half-slice go to registers before use:
            // one LDS wait per half, and at most 16+16 live values.
            constexpr int HS = SL >= 16 ? 16 : SL;
            const float *Bt = &sB[tt][ns * SL];
            const float *Ct = &sC[EMIT_Y ? tt : 0][ns * SL];
            float yp[4] = {0.f, 0.f, 0.f, 0.f};  // independent partial sums
#pragma unroll
            for (int i0 = 0; i0 < SL; i0 += HS) {
                float bv[HS], cv[EMIT_Y ? HS : 1];
#pragma unroll
                for (int i = 0; i < HS; i += 4) {
                    const float4 b4 = *reinterpret_cast<const float4 *>(Bt + i0 + i);
                    bv[i] = b4.x; bv[i + 1] = b4.y; bv[i + 2] = b4.z; bv[i + 3] = b4.w;
                    if constexpr (EMIT_Y) {
                        const float4 c4 = *reinterpret_cast<const float4 *>(Ct + i0 + i);
                        cv[i] = c4.x; cv[i + 1] = c4.y; cv[i + 2] = c4.z; cv[i + 3] = c4.w;
                    }
                }
#pragma unroll
                for (int i = 0; i < HS; ++i) {
                    st[i0 + i] = fmaf(da, st[i0 + i], dx * bv[i]);
                    if constexpr (EMIT_Y) yp[i & 3] = fmaf(st[i0 + i], cv[i], yp[i & 3]);
                }
            }
            if constexpr (EMIT_Y) sY[tt][ns][hl][lane] = (yp[0] + yp[1]) + (yp[2] + yp[3]);
            else lsum += ad;
        }
        if constexpr (EMIT_Y) {
            __syncthreads();
            for (int e = tid; e < nt * HPB * 64; e += kScanThreads) {
                const int tt = e / (HPB * 64), r = e % (HPB * 64);
                const int hh = r / 64, pp = pb * 64 + r % 64;
                if (pp >= P) continue;
                float v = 0.f;
#pragma unroll
                for (int s = 0; s < NSPLIT; ++s) v += sY[tt][s][hh][r % 64];
                const int hg = hb * HPB + hh;
                v += (a.D ? a.D[hg] : 0.f) * sX[tt][hh][r % 64];
                const int64_t yi = (((int64_t)b * L + tb + tt) * H + hg) * P + pp;
                if (a.y_dt == HXQ_F32) static_cast<float *>(a.y)[yi] = v;
                else if (a.y_dt == HXQ_BF16) static_cast<uint16_t *>(a.y)[yi] = f32_to_bf16(v);
                else static_cast<uint16_t *>(a.y)[yi] = f32_to_f16(v);
            }
        }
    }
    (void)Dh;
    if constexpr (!EMIT_Y) {
        float *out = a.ws_state + (int64_t)c * a.batch * H * P * N;
        if (p_ok) {
#pragma unroll
            for (int i = 0; i < SL; ++i) out[sbase + i] = st[i];
        }
        if (lane == 0 && ns == 0) a.ws_decay[((int64_t)c * a.batch + b) * H + h] = lsum;
    }
}

// Pass 2: Hin_0 = h0, Hin_{c+1} = exp(L_c) Hin_c + S_c, in place; h_final.
__global__ __launch_bounds__(256) void scan_state_pass_kernel(const ScanArgs a) {
    const int64_t per_b = (int64_t)a.heads * a.head_dim * a.state;
    const int64_t total = (int64_t)a.batch * per_b;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int b = static_cast<int>(i / per_b);
    const int h = static_cast<int>((i % per_b) / ((int64_t)a.head_dim * a.state));
    const int64_t stride = total;  // one chunk slab
    float carry = a.h0 ? a.h0[i] : 0.f;
    for (int c = 0; c < a.nchunks; ++c) {
        float *slot = a.ws_state + c * stride + i;
        const float s = *slot;
        *slot = carry;
        const float L = a.ws_decay[((int64_t)c * a.batch + b) * a.heads + h];
        carry = fmaf(expf(L), carry, s);
    }
    if (a.h_final) a.h_final[i] = carry;
}

// Single decode step (triton_mamba_decode_step, triton_mamba_scan.py:312-366):
// h <- exp(A dt) h + dt x B, y = <h, C> + D x; one thread per (b, h, p).
__global__ __launch_bounds__(256) void scan_step_kernel(const ScanArgs a, float *h) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)a.batch * a.heads * a.head_dim;
    if (i >= total) return;
    const int p = static_cast<int>(i % a.head_dim);
    const int hh = static_cast<int>((i / a.head_dim) % a.heads);
    const int b = static_cast<int>(i / ((int64_t)a.head_dim * a.heads));
    const int g = hh / (a.heads / a.ngroups);
    const float dtv = ld_any(a.dt, (int64_t)b * a.heads + hh, a.dt_dt);
    const float da = expf(a.A[hh] * dtv);
    const float xv = ld_any(a.x, i, a.x_dt);
    const float dx = dtv * xv;
    float *hs = h + i * a.state;
    float acc = 0.f;
    for (int n = 0; n < a.state; ++n) {
        const int64_t bi = ((int64_t)b * a.ngroups + g) * a.state + n;
        const float v = fmaf(da, hs[n], dx * ld_any(a.Bm, bi, a.bc_dt));
        hs[n] = v;
        acc = fmaf(v, ld_any(a.Cm, bi, a.bc_dt), acc);
    }
    acc += (a.D ? a.D[hh] : 0.f) * xv;
    if (a.y_dt == HXQ_F32) static_cast<float *>(a.y)[i] = acc;
    else if (a.y_dt == HXQ_BF16) static_cast<uint16_t *>(a.y)[i] = f32_to_bf16(acc);
    else static_cast<uint16_t *>(a.y)[i] = f32_to_f16(acc);
}

template <int SL, int HPB>
static int launch_chunks(const ScanArgs &a, hipStream_t stream) {
    const int pblocks = (a.head_dim + 63) / 64;
    const dim3 grid((a.heads / HPB) * pblocks, a.nchunks, a.batch);
    hipLaunchKernelGGL((scan_chunk_kernel<SL, HPB, false>), grid, dim3(kScanThreads), 0, stream, a);
    HXQ_LAUNCH_CHECK();
    const int64_t total = (int64_t)a.batch * a.heads * a.head_dim * a.state;
    hipLaunchKernelGGL(scan_state_pass_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a);
    HXQ_LAUNCH_CHECK();
    hipLaunchKernelGGL((scan_chunk_kernel<SL, HPB, true>), grid, dim3(kScanThreads), 0, stream, a);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

static int valid_dtype(int32_t d) { return d == HXQ_F32 || d == HXQ_BF16 || d == HXQ_F16; }

}  // namespace hxq

using namespace hxq;

extern "C" int64_t hxq_ssm_scan_workspace_bytes(int64_t batch, int64_t seqlen, int64_t heads,
                                               int64_t head_dim, int64_t state, int64_t chunk) {
    if (batch <= 0 || seqlen <= 0 || heads <= 0 || head_dim <= 0 || state <= 0 || chunk <= 0)
        return -1;
    const int64_t nchunks = (seqlen + chunk - 1) / chunk;
    return nchunks * batch * heads * (head_dim * state + 1) * (int64_t)sizeof(float) + 256;
}

extern "C" int hxq_ssm_chunk_scan(const void *x, int32_t x_dtype, const void *dt,
                                  int32_t dt_dtype, const float *A, const void *B, const void *C,
                                  int32_t bc_dtype, const float *D, const float *h0, void *y,
                                  int32_t y_dtype, float *h_final, int64_t batch, int64_t seqlen,
                                  int64_t heads, int64_t head_dim, int64_t state, int64_t ngroups,
                                  int64_t chunk, void *workspace, int64_t workspace_bytes,
                                  hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && dt && A && B && C && y && workspace, "x, dt, A, B, C, y, workspace are required");
    HXQ_REQUIRE(valid_dtype(x_dtype) && valid_dtype(dt_dtype) && valid_dtype(bc_dtype) &&
                    valid_dtype(y_dtype), "bad dtype code");
    HXQ_REQUIRE(batch > 0 && seqlen > 0 && heads > 0 && head_dim > 0 && state > 0 && chunk > 0,
                "sizes must be positive");
    HXQ_REQUIRE(ngroups > 0 && heads % ngroups == 0, "heads must be a multiple of ngroups");
    HXQ_REQUIRE(state == 16 || state == 32 || state == 64 || state == 128 || state == 256,
                "state size must be 16, 32, 64, 128 or 256");
    const int64_t need = hxq_ssm_scan_workspace_bytes(batch, seqlen, heads, head_dim, state, chunk);
    HXQ_REQUIRE(workspace_bytes >= need, "workspace too small (see hxq_ssm_scan_workspace_bytes)");
    HXQ_REQUIRE(batch * seqlen * heads * head_dim < (int64_t{1} << 40), "problem too large");
    ScanArgs a{};
    a.x = x; a.dt = dt; a.A = A; a.Bm = B; a.Cm = C; a.D = D; a.h0 = h0; a.y = y;
    a.h_final = h_final;
    a.batch = (int32_t)batch; a.seqlen = (int32_t)seqlen; a.heads = (int32_t)heads;
    a.head_dim = (int32_t)head_dim; a.state = (int32_t)state; a.ngroups = (int32_t)ngroups;
    a.chunk = (int32_t)chunk;
    a.nchunks = (int32_t)((seqlen + chunk - 1) / chunk);
    a.x_dt = x_dtype; a.dt_dt = dt_dtype; a.bc_dt = bc_dtype; a.y_dt = y_dtype;
    const uintptr_t wsp = (reinterpret_cast<uintptr_t>(workspace) + 255) & ~uintptr_t(255);
    a.ws_state = reinterpret_cast<float *>(wsp);
    a.ws_decay = a.ws_state + (int64_t)a.nchunks * batch * heads * head_dim * state;
    // A block is 8 waves = HPB heads x (8 / HPB) state splits of SL = state *
    // HPB / 8 states per lane (SL <= 64 VGPRs, a multiple of 4).  All heads of
    // a block must share one B/C group, so HPB divides heads / ngroups; when
    // it cannot, fewer heads per block and narrower splits are used.
    const int64_t hpg = heads / ngroups;
    switch (state) {
        case 256:
            return launch_chunks<32, 1>(a, stream);
        case 128:
            if (hpg % 2 == 0) return launch_chunks<32, 2>(a, stream);
            return launch_chunks<16, 1>(a, stream);
        case 64:
            if (hpg % 4 == 0) return launch_chunks<32, 4>(a, stream);
            return launch_chunks<8, 1>(a, stream);
        case 32:
            if (hpg % 8 == 0) return launch_chunks<32, 8>(a, stream);
            return launch_chunks<4, 1>(a, stream);
        default:
            if (hpg % 8 == 0) return launch_chunks<16, 8>(a, stream);
            HXQ_REQUIRE(hpg % 2 == 0, "state 16 needs an even number of heads per group");
            return launch_chunks<4, 2>(a, stream);
    }
}

extern "C" int hxq_ssm_decode_step(const void *x, int32_t x_dtype, const void *dt,
                                   int32_t dt_dtype, const float *A, const void *B,
                                   const void *C, int32_t bc_dtype, const float *D, float *h,
                                   void *y, int32_t y_dtype, int64_t batch, int64_t heads,
                                   int64_t head_dim, int64_t state, int64_t ngroups,
                                   hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && dt && A && B && C && h && y, "x, dt, A, B, C, h, y are required");
    HXQ_REQUIRE(valid_dtype(x_dtype) && valid_dtype(dt_dtype) && valid_dtype(bc_dtype) &&
                    valid_dtype(y_dtype), "bad dtype code");
    HXQ_REQUIRE(batch > 0 && heads > 0 && head_dim > 0 && state > 0, "sizes must be positive");
    HXQ_REQUIRE(ngroups > 0 && heads % ngroups == 0, "heads must be a multiple of ngroups");
    ScanArgs a{};
    a.x = x; a.dt = dt; a.A = A; a.Bm = B; a.Cm = C; a.D = D; a.y = y;
    a.batch = (int32_t)batch; a.heads = (int32_t)heads; a.head_dim = (int32_t)head_dim;
    a.state = (int32_t)state; a.ngroups = (int32_t)ngroups; a.seqlen = 1; a.chunk = 1;
    a.nchunks = 1;
    a.x_dt = x_dtype; a.dt_dt = dt_dtype; a.bc_dt = bc_dtype; a.y_dt = y_dtype;
    const int64_t total = batch * heads * head_dim;
    hipLaunchKernelGGL(scan_step_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a, h);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}
