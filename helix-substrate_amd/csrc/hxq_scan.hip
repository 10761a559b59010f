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

// ---------------------------------------------------------------------------
// SSD (state-space dual) form on bf16 MFMA, for bf16 x, B and C.
//
// One block per (batch b, head h) walks the sequence in chunks of kQ = 64
// tokens with the state S (P x N, fp32) in MFMA accumulators.  With cs_t the
// inclusive prefix sum of A*dt over the chunk (fp64) and S the state at the
// chunk's start, per chunk:
//   y_t      = sum_{s<=t} exp(cs_t - cs_s) dt_s (C_t . B_s) x_s
//              + exp(cs_t) (C_t . S) + D x_t
//   S_next   = exp(cs_Q) S + sum_s exp(cs_Q - cs_s) dt_s x_s (x) B_s
// which is the recurrence h_t = exp(A dt_t) h_{t-1} + dt_t x_t B_t of the
// sequential scan unrolled over the chunk (mamba_scan_chunked.py:89-213 uses
// the same intra/inter-chunk split).  The four contractions run on
// v_mfma_f32_32x32x16_bf16:
//   (a) CB^T = B C^T         [s, t] over n    (bf16 x bf16: exact products)
//   (b) M  = CB o exp(cs_t - cs_s) dt_s, lower triangle, + D on the diagonal,
//       split M = Mh + Ml into two bf16 (16 mantissa bits kept; x is bf16 and
//       exact)
//   (c) Y  = M x              [t, p] over s    (Mh x + Ml x)
//   (d) Z  = C S^T            [t, p] over n    (S split Sh + Sl)
//   (e) S^T = exp(cs_Q) S^T + B^T X'  [n, p] over s, X' = exp(cs_Q - cs_s) dt_s x_s
//       split X'h + X'l
// so every product is exact or carries a 2^-17 relative split error, with
// fp32 accumulation: well inside the scan's 1e-4 bar.  C and B are staged in
// LDS with n contiguous per row, x with p contiguous, 16-byte chunks
// XOR-swizzled by row so the lanes of a read hit distinct banks; operands
// whose k is s (B^T, x^T) come from those tiles by transposing reads.
// Shapes: head_dim <= 64 (padded to 64), state <= 128 (padded to 32 NT);
// other shapes and other dtypes use the VALU recurrence above.
namespace ssd {

constexpr int kQ = 64;        // tokens per internal chunk
constexpr int kPP = 64;       // padded head_dim
constexpr int kThreads = 256; // 4 waves

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element offset of 16-byte chunk c in row r of an LDS matrix of bf16 rows
// with CPR 16-byte chunks (rows of 16 CPR bytes): the chunk is XORed with the
// row's position among the rows that share the 64 banks.
template <int CPR>
__device__ __forceinline__ int sw(int r, int c) {
    return r * CPR * 8 + ((c ^ ((r * CPR / 16) % CPR)) << 3);
}

__device__ __forceinline__ u32x4 lds16(const uint16_t *p) { return *reinterpret_cast<const u32x4 *>(p); }

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// two fp32 -> packed bf16 pair (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// (a, b) -> packed bf16 hi and lo pairs with hi + lo = value to 16 mantissa bits
__device__ __forceinline__ void split2x2(float a, float b, uint32_t &hi, uint32_t &lo) {
    hi = pk_bf16(a, b);
    lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

// 2^x (v_exp_f32)
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Rows of kPP = 64 bf16 (x in natural order, rows s): 8 chunks, XOR with
// (r / 2) % 8 -- the transposing reads below touch rows r0 + {0..3, 8..11}
// at four consecutive chunks, which this spreads over all 64 banks.
__device__ __forceinline__ int swx(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 7)) << 3); }

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: in each group of 16 lanes, result lane 4q + c gets as
// element e the element c of the 8 bytes addressed by lane 4e + q.
__device__ __forceinline__ u32x2 lds_tr(const uint16_t *p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4 *)(p));
    return __builtin_bit_cast(u32x2, v);
}

// Accumulator tile -> MFMA operand.  An accumulator holds, in lane (c, h),
// the values at k = 8 (r / 4) + 4 h + r % 4 (r = 0..15) of column c; an A or
// B operand of a 16-wide k step ks2 wants k = 16 ks2 + 8 h + 0..7 of the same
// column.  Lane h = 0 has k 0..3 and 8..11 of each step, lane h = 1 has 4..7
// and 12..15: v_permlane32_swap of the two 4-value groups gives each lane the
// other half's group.  The values are split into bf16 hi + lo (16 mantissa
// bits); op[ks2][0] is hi, op[ks2][1] lo.
__device__ __forceinline__ void acc_to_op(const f32x16 &m, u32x4 (&op)[2][2]) {
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
        const int q0 = 2 * ks2, q1 = 2 * ks2 + 1;
        uint32_t xh0, xl0, xh1, xl1, yh0, yl0, yh1, yl1;
        split2x2(m[4 * q0], m[4 * q0 + 1], xh0, xl0);
        split2x2(m[4 * q0 + 2], m[4 * q0 + 3], xh1, xl1);
        split2x2(m[4 * q1], m[4 * q1 + 1], yh0, yl0);
        split2x2(m[4 * q1 + 2], m[4 * q1 + 3], yh1, yl1);
        const auto h0 = __builtin_amdgcn_permlane32_swap(xh0, yh0, false, false);
        const auto h1 = __builtin_amdgcn_permlane32_swap(xh1, yh1, false, false);
        const auto l0 = __builtin_amdgcn_permlane32_swap(xl0, yl0, false, false);
        const auto l1 = __builtin_amdgcn_permlane32_swap(xl1, yl1, false, false);
        op[ks2][0] = u32x4{h0[0], h1[0], h0[1], h1[1]};
        op[ks2][1] = u32x4{l0[0], l1[0], l0[1], l1[1]};
    }
}

// The SSD chunk form, two 4-wave blocks per CU (70.5 KB of LDS at state 128).
// Wave w owns output tile (t-tile w/2, p-tile w%2) of (c) and (d) and state
// tiles (p-tile w%2, n-tiles of half the state) of (e).  Where the operands live:
//  - the three decay-masked M tiles (t, s) = (0, 0), (1, 0), (1, 1) are built
//    once each, by waves 0, 2, 3 (wave 1 computes the next chunk's decay
//    terms instead), with D added on the diagonal so that (c)'s product
//    carries y's D x term, and handed to (c) in B-operand form through LDS;
//  - the state stays in the (e) waves' accumulators and becomes (d)'s A
//    operand in registers (v_permlane32_swap), each wave contracting its own
//    n tiles for both t tiles and handing the other t tile's partial to its
//    partner through LDS;
//  - B^T and x^T operands come from the s-major B and x tiles through
//    transposing LDS reads (ds_read_b64_tr_b16), so no transposed copies are
//    stored; X' = w x is formed where (e) reads x^T.
// The next chunk's inputs are loaded into registers right after the current
// chunk is stored to LDS.  Three barriers per chunk.
template <int NT>  // state tiles of 32 (NP = 32 NT)
__global__ __launch_bounds__(kThreads, 2) void ssd_kernel(const ScanArgs a) {
    constexpr int NP = 32 * NT;
    constexpr int CN = NP / 8;   // 16-byte chunks per row of n
    __shared__ __attribute__((aligned(16))) uint16_t sC[kQ * NP];
    __shared__ __attribute__((aligned(16))) uint16_t sB[kQ * NP];
    __shared__ __attribute__((aligned(16))) uint16_t sX[kQ * kPP];
    // (d) partials handed between the two waves of a p tile: [pj][t tile][r][lane]
    __shared__ __attribute__((aligned(16))) float sZ[2][2][16][64];
    // M tiles (t, s) = (0, 0), (1, 0), (1, 1) in (c)'s B-operand form, each built
    // by one wave: [tile][k step][hi, lo][lane]
    __shared__ __attribute__((aligned(16))) u32x4 sM[3][2][2][64];
    __shared__ __attribute__((aligned(16))) double scs2[2][kQ];
    __shared__ __attribute__((aligned(16))) float sdt2[2][kQ], swt2[2][kQ];
    __shared__ __attribute__((aligned(16))) float sec2[2][kQ];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ml = lane & 31, hh = lane >> 5;
    const int b = blockIdx.x / a.heads, h = blockIdx.x % a.heads;
    const int H = a.heads, P = a.head_dim, N = a.state, L = a.seqlen;
    const int g = h / (H / a.ngroups);
    const float Ah = a.A[h];
    const float Dh = a.D ? a.D[h] : 0.f;
    const int ti = wave >> 1, pj = wave & 1;  // (c)/(d) output tile; (e) p tile
    // (e) state tiles: p tile pj, n tiles [nj0, nj0 + nst) (NT = 1: waves 2, 3 hold none)
    const int nst = NT == 4 ? 2 : 1;
    const int nj0 = NT == 4 ? 2 * ti : ti;
    const bool has_s = NT >= 2 || wave < 2;
    const int sp = 32 * pj + ml;
    const int64_t y_bytes = (int64_t)a.batch * L * H * P * (a.y_dt == HXQ_F32 ? 4 : 2);
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, y_bytes);
    constexpr uint32_t kYOob = 0xfffffff0u;

    // ---- chunk inputs: B and C rows of two tokens and x rows, 16 bytes a lane ----
    constexpr uint32_t kOob = 0xfffffff0u;
    const int dtb = a.dt_dt == HXQ_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (int64_t)a.batch * L * H * P * 2);
    const __amdgpu_buffer_rsrc_t br = make_rsrc(a.Bm, (int64_t)a.batch * L * a.ngroups * N * 2);
    const __amdgpu_buffer_rsrc_t cr = make_rsrc(a.Cm, (int64_t)a.batch * L * a.ngroups * N * 2);
    const __amdgpu_buffer_rsrc_t dr = make_rsrc(a.dt, (int64_t)a.batch * L * H * dtb);
    constexpr int BC_ITEMS = (kQ / 2) * CN;
    constexpr int BC_PER = (BC_ITEMS + kThreads - 1) / kThreads;
    u32x4 rB[BC_PER][2], rC[BC_PER][2];
    u32x4 rX[2];
    auto load_chunk = [&](int t0) {
#pragma unroll
        for (int i = 0; i < BC_PER; ++i) {
            const int item = tid + kThreads * i;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int t = t0 + 2 * (item / CN) + e, c = item % CN;
                const bool ok = item < BC_ITEMS && t < L && 8 * c < N;
                const uint32_t o = ok ? static_cast<uint32_t>(((((int64_t)b * L + t) * a.ngroups + g) * N + 8 * c) * 2) : kOob;
                rB[i][e] = buf_load16(br, o);
                rC[i][e] = buf_load16(cr, o);
            }
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = t0 + 2 * (tid >> 3) + e, c = tid & 7;
            const bool ok = t < L && 8 * c < P;
            rX[e] = buf_load16(xr, ok ? static_cast<uint32_t>(((((int64_t)b * L + t) * H + h) * P + 8 * c) * 2) : kOob);
        }
    };
    auto load_dt = [&](int t0) -> uint32_t {
        const int t = t0 + lane;
        const uint32_t o = t < L ? static_cast<uint32_t>((((int64_t)b * L + t) * H + h) * dtb) : kOob;
        return dtb == 4 ? __builtin_amdgcn_raw_buffer_load_b32(dr, o, 0, 0)
                        : static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(dr, o, 0, 0));
    };
    auto dt_value = [&](uint32_t raw) -> float {
        return a.dt_dt == HXQ_F32 ? __uint_as_float(raw)
             : a.dt_dt == HXQ_BF16 ? bf16_to_f32(static_cast<uint16_t>(raw)) : f16_to_f32(static_cast<uint16_t>(raw));
    };
    auto decay_terms = [&](float dtv, int buf) {
        double cs = static_cast<double>(Ah * dtv);
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(cs, off, 64);
            if (lane >= off) cs += o;
        }
        cs *= 1.4426950408889634;  // log2(e)
        const double csq = __shfl(cs, 63, 64);
        scs2[buf][lane] = cs;
        sdt2[buf][lane] = dtv;
        swt2[buf][lane] = exp2_fast(static_cast<float>(csq - cs)) * dtv;
        sec2[buf][lane] = exp2_fast(static_cast<float>(cs));
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int i = 0; i < BC_PER; ++i) {
            const int item = tid + kThreads * i;
            if (item >= BC_ITEMS) continue;
            const int u = item / CN, c = item % CN;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                *reinterpret_cast<u32x4 *>(sB + sw<CN>(2 * u + e, c)) = rB[i][e];
                *reinterpret_cast<u32x4 *>(sC + sw<CN>(2 * u + e, c)) = rC[i][e];
            }
        }
#pragma unroll
        for (int e = 0; e < 2; ++e)
            *reinterpret_cast<u32x4 *>(sX + swx(2 * (tid >> 3) + e, tid & 7)) = rX[e];
    };
    // Operands with k = s read from the s-major tiles by transposing reads:
    // lane 16G + 4e + q addresses row s = 16 ks + 8 (G / 2) + 4 half + e and
    // column 16 (G % 2) + 4q of its 32-wide tile, so that lane l receives
    // column l % 32 at s = 16 ks + 8 (l / 32) + 4 half + 0..3.
    const int tr_s = 8 * ((lane >> 4) >> 1) + ((lane >> 2) & 3);
    const int tr_m = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto x_op = [&](int ks) -> u32x4 {  // x^T: p = 32 pj + l % 32
        const int c = (32 * pj + tr_m) >> 3, o = tr_m & 7;
        const u32x2 lo = lds_tr(sX + swx(16 * ks + tr_s, c) + o);
        const u32x2 hi = lds_tr(sX + swx(16 * ks + tr_s + 4, c) + o);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    auto bt_op = [&](int ks, int nt) -> u32x4 {  // B^T: n = 32 nt + l % 32
        const int n = 32 * nt + tr_m;
        const u32x2 lo = lds_tr(sB + sw<CN>(16 * ks + tr_s, n >> 3) + (n & 7));
        const u32x2 hi = lds_tr(sB + sw<CN>(16 * ks + tr_s + 4, n >> 3) + (n & 7));
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };

    // ---- state: Sacc[j][r] = S[p = 32 pj + ml][n = 32(nj0 + j) + 8(r/4) + 4hh + r%4]
    // h0 / h_final through buffer resources: elements outside (p < P, n < N)
    // take an offset past the range (reads give 0, writes are dropped), so no
    // per-element lane masks stay live across the chunk loop
    const int64_t st_bytes = (int64_t)a.batch * H * P * N * 4;
    const __amdgpu_buffer_rsrc_t h0r = make_rsrc(a.h0, a.h0 ? st_bytes : 0);
    const __amdgpu_buffer_rsrc_t hfr = make_rsrc(a.h_final, a.h_final ? st_bytes : 0);
    auto st_off = [&](int j, int r) -> uint32_t {
        const int n = 32 * (nj0 + j) + 8 * (r >> 2) + 4 * hh + (r & 3);
        return (has_s && j < nst && sp < P && n < N)
                   ? static_cast<uint32_t>(((((int64_t)b * H + h) * P + sp) * N + n) * 4) : kOob;
    };
    f32x16 Sacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            Sacc[j][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(h0r, st_off(j, r), 0, 0));

    const int nch = (L + kQ - 1) / kQ;
    load_chunk(0);
    uint32_t rdt = load_dt(0);
    if (wave == 1) decay_terms(dt_value(rdt), 0);
    rdt = load_dt(kQ);
    for (int ch = 0; ch < nch; ++ch) {
        const int t0 = ch * kQ;
        const int db = ch & 1;
        const double *scs = scs2[db];
        const float *sdt = sdt2[db], *swt = swt2[db], *sec = sec2[db];
        lds_barrier();  // the previous chunk's readers of the inputs and partials are done
        store_chunk();
        // the next chunk's inputs: issued a whole chunk ahead of their store
        if (ch + 1 < nch) load_chunk(t0 + kQ);
        lds_barrier();
        if (wave == 1 && ch + 1 < nch) {
            decay_terms(dt_value(rdt), db ^ 1);
            rdt = load_dt(t0 + 2 * kQ);
        }

        // (a)+(b): M tile (mt, ms) of this wave -- waves 0, 2, 3 build (0, 0),
        // (1, 0), (1, 1); wave 1 builds none and computes the decay terms --
        // with D on the diagonal (y's D x term rides in (c)'s product)
        if (wave != 1) {
            const int mt = wave >> 1, ms = wave == 2 ? 0 : mt;
            const int t = 32 * mt + ml;
            // t made opaque per chunk: the 16 lane masks below are then formed
            // in VALU here instead of being hoisted into loop-long SGPRs
            int tq = t;
            asm volatile("" : "+v"(tq));
            const double cst = scs[t];
            f32x16 cb;
#pragma unroll
            for (int r = 0; r < 16; ++r) cb[r] = 0.f;
#pragma unroll
            for (int ks = 0; ks < NP / 16; ++ks) {
                const u32x4 bv = lds16(sB + sw<CN>(32 * ms + ml, 2 * ks + hh));
                const u32x4 cv = lds16(sC + sw<CN>(32 * mt + ml, 2 * ks + hh));
                cb = mfma(bv, cv, cb);
            }
            // cb[4q + e]: s = 32 ms + 8q + 4hh + e of column t; the four s of a q
            // are consecutive, so their cs and dt come in 16-byte reads
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int sb = 32 * ms + 8 * q + 4 * hh;
                const f64x2 c01 = *reinterpret_cast<const f64x2 *>(scs + sb);
                const f64x2 c23 = *reinterpret_cast<const f64x2 *>(scs + sb + 2);
                const f32x4 d4 = *reinterpret_cast<const f32x4 *>(sdt + sb);
                const double cs4[4] = {c01[0], c01[1], c23[0], c23[1]};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int s = sb + e;
                    const float v = cb[4 * q + e] * exp2_fast(static_cast<float>(cst - cs4[e])) * d4[e];
                    cb[4 * q + e] = s < tq ? v : (s == tq ? v + Dh : 0.f);
                }
            }
            u32x4 mop[2][2];
            acc_to_op(cb, mop);
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int hl = 0; hl < 2; ++hl) sM[mt + ms][k2][hl][lane] = mop[k2][hl];
        }
        const int t = 32 * ti + ml;

        // (d): Z^T partials over this wave's n tiles, for its own t tile (kept)
        // and the partner's (handed over through LDS)
        f32x16 zown, zoth;
#pragma unroll
        for (int r = 0; r < 16; ++r) zown[r] = zoth[r] = 0.f;
        if (has_s) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (j >= nst) break;
                u32x4 sop[2][2];
                acc_to_op(Sacc[j], sop);
#pragma unroll
                for (int ks2 = 0; ks2 < 2; ++ks2) {
                    const int c = 4 * (nj0 + j) + 2 * ks2 + hh;  // 16-byte chunk of n
                    const u32x4 cvo = lds16(sC + sw<CN>(32 * ti + ml, c));
                    const u32x4 cvp = lds16(sC + sw<CN>(32 * (ti ^ 1) + ml, c));
                    zown = mfma(sop[ks2][0], cvo, zown);
                    zoth = mfma(sop[ks2][0], cvp, zoth);
                    zown = mfma(sop[ks2][1], cvo, zown);
                    zoth = mfma(sop[ks2][1], cvp, zoth);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) sZ[pj][ti ^ 1][r][lane] = zoth[r];
        // the next chunk's inputs: issued once P1's operands are dead (their
        // registers are free), landing while (c) and (e) run
        lds_barrier();

        // (c) Y^T = x^T M^T over s <= end of t tile ti; y = Y + exp(cs_t) Z + D x
        {
            f32x16 yv, zv = zown;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                yv[r] = 0.f;
                zv[r] += sZ[pj][ti][r][lane];
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if (ks >= 2 * (ti + 1)) break;
                const u32x4 xa = x_op(ks);
                yv = mfma(xa, sM[ti + (ks >> 1)][ks & 1][0][lane], yv);
                yv = mfma(xa, sM[ti + (ks >> 1)][ks & 1][1][lane], yv);
            }
            const float et = sec[t];
            const bool t_ok = t0 + t < L;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int p0 = 32 * pj + 8 * q + 4 * hh;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = yv[4 * q + e] + et * zv[4 * q + e];
                const bool ok = t_ok && p0 < P;
                const uint32_t yo = static_cast<uint32_t>((((int64_t)b * L + t0 + t) * H + h) * P + p0);
                if (a.y_dt == HXQ_F32) {
                    __builtin_amdgcn_raw_buffer_store_b128(
                        u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                              __float_as_uint(v[3])},
                        yr, ok ? yo * 4u : kYOob, 0, 0);
                } else {
                    u32x2 w;
                    if (a.y_dt == HXQ_BF16) {
                        w = u32x2{pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3])};
                    } else {
                        w = u32x2{uint32_t(f32_to_f16(v[0])) | (uint32_t(f32_to_f16(v[1])) << 16),
                                  uint32_t(f32_to_f16(v[2])) | (uint32_t(f32_to_f16(v[3])) << 16)};
                    }
                    __builtin_amdgcn_raw_buffer_store_b64(w, yr, ok ? yo * 2u : kYOob, 0, 0);
                }
            }
        }

        // (e) S = exp(cs_Q) S + X'^T B, X'[s][p] = w_s x[s][p] formed from x^T
        if (has_s) {
            const float eq = exp2_fast(static_cast<float>(scs[kQ - 1]));
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (j >= nst) break;
#pragma unroll
                for (int r = 0; r < 16; ++r) Sacc[j][r] *= eq;
            }
#pragma unroll
            for (int ks = 0; ks < kQ / 16; ++ks) {
                const u32x4 xx = x_op(ks);
                const int s0 = 16 * ks + 8 * hh;
                const f32x4 w0 = *reinterpret_cast<const f32x4 *>(swt + s0);
                const f32x4 w1 = *reinterpret_cast<const f32x4 *>(swt + s0 + 4);
                const float w8[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
                u32x4 xh, xl;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const float x0 = __uint_as_float(xx[d] << 16) * w8[2 * d];
                    const float x1 = __uint_as_float(xx[d] & 0xffff0000u) * w8[2 * d + 1];
                    uint32_t hv, lv;
                    split2x2(x0, x1, hv, lv);
                    xh[d] = hv;
                    xl[d] = lv;
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (j >= nst) break;
                    const u32x4 bt = bt_op(ks, nj0 + j);
                    Sacc[j] = mfma(bt, xh, Sacc[j]);
                    Sacc[j] = mfma(bt, xl, Sacc[j]);
                }
            }
        }
    }
    if (a.h_final) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Sacc[j][r]), hfr, st_off(j, r), 0, 0);
    }
}

}  // namespace ssd

// The SSD kernel's shapes and dtypes: bf16 x/B/C, head_dim <= 64, state <= 128.
static bool ssd_eligible(const ScanArgs &a) {
    const int64_t y_bytes = (int64_t)a.batch * a.seqlen * a.heads * a.head_dim * (a.y_dt == HXQ_F32 ? 4 : 2);
    const int64_t bc_bytes = (int64_t)a.batch * a.seqlen * a.ngroups * a.state * 2;
    return a.x_dt == HXQ_BF16 && a.bc_dt == HXQ_BF16 && a.head_dim <= ssd::kPP && a.state <= 128 &&
           a.head_dim % 8 == 0 && a.state % 8 == 0 && y_bytes < (int64_t{1} << 31) &&
           bc_bytes < (int64_t{1} << 31);
}

static int launch_ssd(const ScanArgs &a, hipStream_t stream) {
    const dim3 grid(a.batch * a.heads);
    if (a.state <= 32) hipLaunchKernelGGL(ssd::ssd_kernel<1>, grid, dim3(ssd::kThreads), 0, stream, a);
    else if (a.state <= 64) hipLaunchKernelGGL(ssd::ssd_kernel<2>, grid, dim3(ssd::kThreads), 0, stream, a);
    else hipLaunchKernelGGL(ssd::ssd_kernel<4>, grid, dim3(ssd::kThreads), 0, stream, a);
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
    // bf16 x/B/C with head_dim <= 64 and state <= 128: the SSD form on MFMA
    // (no workspace); otherwise the three-pass VALU recurrence
    if (ssd_eligible(a)) return launch_ssd(a, stream);
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
