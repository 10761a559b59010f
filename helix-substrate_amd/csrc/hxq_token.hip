// Persistent batch-1 decode step: ONE cooperative launch runs a whole token of
// a Qwen2-shaped decoder whose q/k/v/o/gate/up/down projections are HXQ
// matrices -- every layer's norm + q/k/v GEMV, RoPE + KV append + GQA
// attention, o GEMV, norm + gate/up GEMV with the SiLU product, down GEMV,
// then the final norm, the tied bf16 LM head and the greedy argmax.
//
// Why: at batch 1 the multi-launch step pays a fixed cost per launch (launch
// gap, first-data round trip, tail) that is larger than the data time of most
// projections.  Here the grid stays resident (one 16-wave block per CU) and
// the stages are separated by grid barriers; the compressed weights of the
// NEXT stage do not depend on the barrier, so every block issues their loads
// (index rows, affine factors, codebook, CSR row pointers) right after
// arriving and before waiting: HBM streams while the grid synchronises.
//
// Grid barrier (per-block arrival flags):
//   arrive: each wave waits for its own stores (s_waitcnt 0), workgroup
//           barrier, thread 0 stores flag[block] = target (coherent store);
//   wait:   wave 0 of every block polls all flags (or only its producers'
//           flags) until each reached target -- one cross-XCD hop.  Every
//           wait gives up after 1 s of wall clock or when the error word is
//           set, and the kernel then returns, so every wave ends even if the
//           grid cannot synchronise.  (The release word in the workspace is
//           cleared but no longer used.)
// Data that crosses blocks inside a launch (residual stream, q/k/v, attention
// output, o, SiLU product, down output, argmax partials) is written with
// coherent stores (sc1) and read with coherent loads (sc1), so no L2
// write-back or invalidate is needed at the barriers (each XCD has its own
// L2).  Weights, norms and the KV cache rows of earlier positions are read
// with ordinary loads (written before the launch).
//
// GEMV stages follow hxq_gemv.hip's scheme (16-byte index loads per lane, the
// 256-entry codebook replicated 64x in LDS, affine factored out of the sum,
// sidecar as an epilogue in CSR order, fixed summation order): rows of a
// stage are split over the blocks, the 16 waves of a block split into S
// K-slices x row lanes.  Gate and up rows j are computed by the same block
// (waves 0-7 gate, 8-15 up, each with its own LDS codebook) so the block
// writes act[j] = bf16(silu(g) * u) directly.
//
// Math: transformers' Qwen2 (models/qwen2/modeling_qwen2.py): RMSNorm
// (:247-253), rotate_half RoPE (:105-135), eager GQA attention (:138-170),
// residuals (:269-300), MLP down(act(gate) * up).  Residual stream fp32,
// activations entering the projections bf16, KV cache bf16.
#include <cfloat>
#include <cstring>
#include <vector>

#include "hxq_common.h"

namespace hxq {
namespace tok {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;      // 16
constexpr int CPS = 1;                        // 1024-column chunks per wave slice
constexpr int RB = 4;                         // rows per load batch
constexpr int NREP = 64;                      // codebook replicas in LDS
constexpr int kTbl = 256 * NREP;              // floats per codebook table (64 KB)
constexpr int kTPW = kTbl / (4 * kThreads);   // float4 table writes per thread (4)
constexpr int kChunk = 1024;
constexpr int kRedCap = 512;                  // row x slice partials per segment
constexpr int kEnt = 512;                     // sidecar entries per segment staged in LDS
constexpr int kRps = 1028;                    // CSR row pointers per segment staged in LDS
constexpr int kHeadDim = 128;
constexpr int kVStage = 3584;                  // float offset of attention's staged V rows in LDS
constexpr int kMaxSeq = 1024;
static_assert(kMaxSeq + 3 * kHeadDim + kWaves * kHeadDim + 2 * kWaves + 1 <= kVStage,
              "attention scratch overlaps the staged V rows");
constexpr int kLmRB = 1;                      // LM-head rows per load batch
constexpr int kLmBuf = 2;                     // LM-head load batches in flight per wave
constexpr int kLmPol = 2;                     // LM-head row loads: nt (read once per token)
constexpr int kLmStage = 64;                  // float offset of the block's logits in LDS
constexpr uint32_t kOob = 0x80000000u;        // buffer offset past any range: reads 0
constexpr int kCoh = 16;                      // cache policy sc1: coherent across XCDs
constexpr int kVmcnt0 = 0x0F70;               // s_waitcnt vmcnt(0) (expcnt, lgkmcnt untouched)
constexpr uint64_t kTimeoutTicks = 100000000ull;  // 1 s of the 100 MHz wall clock

enum { kQ = 0, kK = 1, kV = 2, kO = 3, kG = 4, kU = 5, kD = 6 };

// wave-uniform values forced into scalar registers
__device__ __forceinline__ uint64_t ufl64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
template <typename T>
__device__ __forceinline__ T *uptr(T *p) {
    return reinterpret_cast<T *>(ufl64(reinterpret_cast<uint64_t>(p)));
}


struct Mat {
    const uint8_t *idx;
    const float *cb;
    const float *gs;
    const float *go;
    const int32_t *rp;
    const int32_t *col;
    const float *delta;
    const float *bias;
    int64_t out;
};

// The launch's tables (plan, layers) are written by the host before the
// launch and nothing changes them during it: they are read with kload
// (hxq_common.h), scalar loads whose fields land in scalar registers and count
// in lgkmcnt only -- no vector-memory wait (which would also wait for the
// previous stage's output stores) precedes a stage.

// A matrix descriptor read from the layer table into scalar registers.
__device__ __forceinline__ Mat umat(const Mat &m) { return kload(m); }

struct Layer {
    Mat m[7];
    const float *in_norm;
    const float *post_norm;
    uint16_t *kc;
    uint16_t *vc;
};

struct Plan {
    int32_t hidden, n_layers, n_heads, n_kv, inter, vocab, max_seq, group, nblocks;
    float eps, theta;
    int32_t qkv_b1, qkv_b2;            // blocks [qkv_b0,b1) q, [b1,b2) k, [b2,nb) v
    int32_t s_qkv, s_o, s_gu, s_down;  // K slices per wave group
    int32_t lds_red;                   // float offset of the red/ent area in LDS
    int32_t o_b0;                      // first block of the o stage (blocks before it run attention)
    int32_t qkv_b0, pad_;              // first block of the q/k/v stage (likewise)
    const uint16_t *embed;
    const float *final_norm;
    int32_t *tok;
    int32_t *pos;
    float *logits;
    const Layer *layers;
    // Data that crosses blocks: one slot per layer (every address written
    // once per launch), in flag-in-data words (ll_* below): fp32 values as
    // two words, bf16 values as one, each word tagged with the producing
    // stage's epoch.  Producers store with sc1 (write-through); consumers
    // poll with sc1 loads until every word they need carries the epoch, so
    // no grid barrier separates the stages of a layer.
    //   res[l]  residual entering layer l (l = 1..L; layer 0 embeds)
    //   ra[l]   residual after layer l's attention block input add
    //   qkv[l], attn[l], o[l], act[l], dn[l]
    uint32_t *res, *ra, *qkv, *o, *dn;
    float *part_v;
    uint32_t *attn, *act;
    int32_t ls_hid, ls_qkv, ls_attn, ls_act;  // slot strides (32-bit words)
    int32_t *part_i;
    uint32_t *flags, *release;
    int32_t *err;
};

// Buffer resource with base and size forced into scalar registers (the
// values are wave-uniform; without this the compiler may not prove it and
// wraps every load in a per-lane loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t urs(const void *base, int64_t bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    const uint32_t n = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bytes));
    return make_rsrc(reinterpret_cast<const void *>((static_cast<uint64_t>(hi) << 32) | lo), n);
}

// ---------------------------------------------------------------------------
// coherent accesses
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 coh_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoh);
}
__device__ __forceinline__ void coh_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCoh);
}
__device__ __forceinline__ float coh_loadf(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t coh_loadi(const int32_t *p) {
    return __hip_atomic_load(const_cast<int32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_storef(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_storei(int32_t *p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_store_u32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_store_bf16(uint16_t *base, int64_t n, int64_t i, float v) {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), urs(base, n * 2),
                                          static_cast<uint32_t>(i * 2), 0, kCoh);
}
__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// ---------------------------------------------------------------------------
// flag-in-data words
// ---------------------------------------------------------------------------
// A word holds 16 data bits in its high half and the producing stage's epoch
// (never 0: zeroed memory is never valid) in its low half.  fp32 values are
// two words (high, low 16 bits), bf16 values one.  Each word is validated on
// its own, so no store wider than 32 bits needs to be single-copy atomic.
__device__ __forceinline__ uint32_t ll_epoch(uint32_t target) { return (target & 0x7fffu) | 0x8000u; }
__device__ __forceinline__ bool ll_ok(uint32_t w, uint32_t e) { return (w & 0xffffu) == e; }
__device__ __forceinline__ float ll_f32(uint32_t hi, uint32_t lo) {
    return __uint_as_float((hi & 0xffff0000u) | (lo >> 16));
}
__device__ __forceinline__ float ll_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t ll_hi(float v, uint32_t e) { return (__float_as_uint(v) & 0xffff0000u) | e; }
__device__ __forceinline__ uint32_t ll_lo(float v, uint32_t e) { return (__float_as_uint(v) << 16) | e; }
__device__ __forceinline__ uint32_t ll_bf16w(float v, uint32_t e) {
    return (static_cast<uint32_t>(f32_to_bf16(v)) << 16) | e;
}
// Coherent word stores through a buffer resource whose base is the output
// array (byte offsets).  Buffer stores, not flat ones: a flat access in
// flight makes the compiler wait for every outstanding load at the next
// wait, which would serialise the following stage's weight stream.
constexpr int64_t kAnyBytes = 0x7fffffff;  // output arrays are < 2 GiB
// two words at byte offset off (8-byte aligned), one store
__device__ __forceinline__ void ll_store2(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t a, uint32_t b) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{a, b}, r, off, 0, kCoh);
}
__device__ __forceinline__ void ll_store1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t a) {
    __builtin_amdgcn_raw_buffer_store_b32(a, r, off, 0, kCoh);
}
__device__ __forceinline__ uint2 coh_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCoh);
    return make_uint2(v[0], v[1]);
}

// Wave64 reductions via DPP (no lane-address registers); the result is
// read from lane 63 into a scalar register, i.e. every lane gets it.
__device__ __forceinline__ float wave_sum_all(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_lane63(v)), 63));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max(float v) {
    const int s = __builtin_amdgcn_update_dpp(__float_as_int(-FLT_MAX), __float_as_int(v), CTRL,
                                              ROW_MASK, 0xf, false);
    return fmaxf(v, __int_as_float(s));
}

__device__ __forceinline__ float wave_max_all(float v) {
    v = dpp_max<0xb1, 0xf>(v);
    v = dpp_max<0x4e, 0xf>(v);
    v = dpp_max<0x141, 0xf>(v);
    v = dpp_max<0x140, 0xf>(v);
    v = dpp_max<0x142, 0xa>(v);
    v = dpp_max<0x143, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// The kWaves (16) per-wave values at a (16-byte aligned LDS), read with four
// 16-byte loads in flight; sum in index order / maximum.
__device__ __forceinline__ void lds16(const float *a, float (&v)[kWaves]) {
#pragma unroll
    for (int i = 0; i < kWaves / 4; ++i) {
        const float4 f = reinterpret_cast<const float4 *>(a)[i];
        v[4 * i] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
}
__device__ __forceinline__ float sum16(const float *a) {
    float v[kWaves];
    lds16(a, v);
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t += v[i];
    return t;
}


// Redefines a value with an empty asm so the compiler recomputes whatever
// derives from it instead of keeping it live from an earlier stage.
__device__ __forceinline__ int fresh_s(int v) {
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ int fresh_v(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// ---------------------------------------------------------------------------
// grid barrier
// ---------------------------------------------------------------------------
__device__ __forceinline__ void arrive(const Plan &P, uint32_t target) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(P.flags + blockIdx.x, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool gave_up(const Plan &P, uint64_t t0) {
    const int32_t e = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (e != 0 || wall_clock64() - t0 > kTimeoutTicks) {
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_store(P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // complete before this path rejoins the stream code (see ll_store2)
        __builtin_amdgcn_s_waitcnt(0);
        return true;
    }
    return false;
}

// Grid barrier, one hop: wave 0 of every block polls all blocks' flags
// (one coherent 16-byte load per lane per 256 blocks) until each reached
// `target`.  Returns false when the grid could not synchronise (the caller
// returns).
__device__ __forceinline__ bool wait_all(const Plan &P, uint32_t target, int *sh) {
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        int ok = 1;
        const uint64_t t0 = wall_clock64();
        const int nb = P.nblocks;
        const __amdgpu_buffer_rsrc_t fr = urs(P.flags, static_cast<int64_t>(nb) * 4);
        while (true) {
            int done = 1;
            for (int i0 = 0; i0 < nb; i0 += 4 * kWave) {
                const u32x4 f = coh_load16(fr, static_cast<uint32_t>(i0 + 4 * lane) * 4u);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = i0 + 4 * lane + j;
                    done &= (i >= nb) || static_cast<int32_t>(f[j] - target) >= 0;
                }
            }
            if (__all(done)) break;
            if (gave_up(P, t0)) { ok = 0; break; }
        }
        if (lane == 0) *sh = ok;
    }
    __syncthreads();
    return *sh != 0;
}

// Waits until the producer blocks of this block's input reached `target`:
// the blocks in up to three ranges [a, b) (one hop: no release word).
// Wave 0 polls; returns false when it gave up.
__device__ __forceinline__ bool wait_blocks(const Plan &P, uint32_t target, int *sh, int a0,
                                            int b0, int a1, int b1, int a2, int b2) {
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        const int n0 = b0 - a0, n1 = b1 - a1, n = n0 + n1 + (b2 - a2);
        int ok = 1;
        const uint64_t t0 = wall_clock64();
        while (true) {
            int done = 1;
            for (int i = lane; i < n; i += kWave) {
                const int blk = i < n0 ? a0 + i : i < n0 + n1 ? a1 + i - n0 : a2 + i - n0 - n1;
                const uint32_t f = __hip_atomic_load(P.flags + blk, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                done &= static_cast<int32_t>(f - target) >= 0;
            }
            if (__all(done)) break;
            if (gave_up(P, t0)) { ok = 0; break; }
        }
        if (lane == 0) *sh = ok;
    }
    __syncthreads();
    return *sh != 0;
}

// Block (of nbm, rows split as out*b/nbm) holding row r.
__device__ __forceinline__ int block_of_row(uint32_t out, uint32_t nbm, uint32_t r) {
    uint32_t b = r * nbm / out;
    while (b + 1 < nbm && out * (b + 1) / nbm <= r) ++b;
    while (b > 0 && out * b / nbm > r) --b;
    return static_cast<int>(b);
}

// ---------------------------------------------------------------------------
// GEMV stages
// ---------------------------------------------------------------------------
struct Batch {
    u32x4 q[RB][CPS];
    float sc[RB][CPS];
    float of[RB][CPS];
};

// Loads issued before a stage's barrier: the codebook values this thread
// writes into the LDS tables, the block's CSR range (per segment) and the
// first batch of this wave's rows.  One batch (about 16 MB over the GPU)
// covers the barrier and activation latency; a deeper prefetch fills the
// HBM queues and delays the barrier's own flag traffic behind it.  The
// second batch is issued right after the stage's activation loads.
struct Pre {
    Batch bt[2];
    float cbv[2][kTPW];
    int32_t b0[2], b1[2];
};

// One wave's share of a matrix segment: rows [lo, lo+n) of the block, waves
// split into S K-slices x RG row lanes.
struct Seg {
    int64_t lo, n, n_mine;
    int s_id, rg, RG, S, c_lo, nc;
};

// A stage as seen by one block: one matrix (q/k/v by block, o, down) or the
// gate/up pair (segment = wave / 8).
struct Geo {
    Mat m0, m1;
    int nseg;
    int seg;       // this wave's segment
    int64_t lo, n;
    int32_t K;
    int64_t y_off; // output offset of the block's matrix (q/k/v rows in qkv)
    Seg g;
};

__device__ __forceinline__ Seg make_seg(int64_t lo, int64_t n, int w, int nw, int S, int nchunks) {
    Seg g;
    g.lo = lo;
    g.n = n;
    g.S = S;
    g.RG = nw / S;
    g.s_id = w % S;
    g.rg = w / S;
    g.c_lo = g.s_id * nchunks / S;
    g.nc = (g.s_id + 1) * nchunks / S - g.c_lo;
    g.n_mine = (g.rg < g.RG && n > g.rg) ? (n - g.rg + g.RG - 1) / g.RG : 0;
    return g;
}

__device__ __forceinline__ int nchunks_of(int32_t K) { return (K + kChunk - 1) / kChunk; }

// Pass p of wave w in a two-pass stage (K above kWaves chunks): slice
// w + kWaves * p is chunk w + kWaves * p alone, over every row of the block
// (S = nchunks slices in all; a slice past the last chunk has no rows).
__device__ __forceinline__ Seg make_seg_pass(int64_t lo, int64_t n, int w, int p, int nchunks) {
    Seg g;
    g.lo = lo;
    g.n = n;
    g.S = nchunks;
    g.RG = 1;
    g.rg = 0;
    g.s_id = w + kWaves * p;
    g.c_lo = g.s_id;
    g.nc = g.s_id < nchunks ? 1 : 0;
    g.n_mine = g.nc ? n : 0;
    return g;
}

__device__ __forceinline__ Geo geo_qkv(const Plan &P, const Layer &L, int wave) {
    Geo G;
    const int b = blockIdx.x, nb = P.nblocks;
    const int mi = b < P.qkv_b1 ? 0 : b < P.qkv_b2 ? 1 : 2;
    const int bs = mi == 0 ? P.qkv_b0 : mi == 1 ? P.qkv_b1 : P.qkv_b2;
    const int be = mi == 0 ? P.qkv_b1 : mi == 1 ? P.qkv_b2 : nb;
    G.m0 = G.m1 = umat(L.m[mi]);
    G.nseg = 1;
    G.seg = 0;
    const int64_t out = G.m0.out;
    G.lo = static_cast<uint32_t>(out) * static_cast<uint32_t>(b - bs) / static_cast<uint32_t>(be - bs);
    G.n = static_cast<uint32_t>(out) * static_cast<uint32_t>(b - bs + 1) / static_cast<uint32_t>(be - bs) - G.lo;
    G.K = P.hidden;
    G.y_off = mi == 0 ? 0 : mi == 1 ? int64_t{P.n_heads} * kHeadDim
                                    : int64_t{P.n_heads + P.n_kv} * kHeadDim;
    G.g = make_seg(G.lo, G.n, wave, kWaves, P.s_qkv, nchunks_of(G.K));
    return G;
}

// rows of matrix mi spread over blocks [b0, nblocks)
__device__ __forceinline__ Geo geo_plain(const Plan &P, const Layer &L, int mi, int32_t K, int S,
                                         int wave, int b0 = 0) {
    Geo G;
    const int b = static_cast<int>(blockIdx.x) - b0, nb = P.nblocks - b0;
    G.m0 = G.m1 = umat(L.m[mi]);
    G.nseg = 1;
    G.seg = 0;
    const int64_t out = G.m0.out;
    G.lo = static_cast<uint32_t>(out) * static_cast<uint32_t>(b) / static_cast<uint32_t>(nb);
    G.n = static_cast<uint32_t>(out) * static_cast<uint32_t>(b + 1) / static_cast<uint32_t>(nb) - G.lo;
    G.K = K;
    G.y_off = 0;
    G.g = make_seg(G.lo, G.n, wave, kWaves, S, nchunks_of(K));
    return G;
}

__device__ __forceinline__ Geo geo_pair(const Plan &P, const Layer &L, int wave) {
    Geo G;
    const int b = blockIdx.x, nb = P.nblocks;
    G.m0 = umat(L.m[kG]);
    G.m1 = umat(L.m[kU]);
    G.nseg = 2;
    G.seg = wave / (kWaves / 2);
    const int64_t out = P.inter;
    G.lo = static_cast<uint32_t>(out) * static_cast<uint32_t>(b) / static_cast<uint32_t>(nb);
    G.n = static_cast<uint32_t>(out) * static_cast<uint32_t>(b + 1) / static_cast<uint32_t>(nb) - G.lo;
    G.K = P.hidden;
    G.y_off = 0;
    G.g = make_seg(G.lo, G.n, wave % (kWaves / 2), kWaves / 2, P.s_gu, nchunks_of(G.K));
    return G;
}

// Issues the index words and affine factors of rows [t0, t0 + RB) of the
// wave's share.  Every load is issued on every path -- rows and chunks
// outside the share get an out-of-range offset (no traffic, zeros) -- so the
// number of loads in flight never depends on a branch and the waits before
// each batch's use count exactly the loads issued after it.  Without affine
// factors both factor buffers have no records: scales and offsets read 0,
// and row_dot adds `nonaff` (1) to the scale.
__device__ __forceinline__ void load_batch(const Mat &M, const Seg &g, int32_t K, int32_t group,
                                           int64_t t0, int lane, Batch &b) {
    const bool affine = M.gs != nullptr;
    const uint32_t gsz = group > 0 ? static_cast<uint32_t>(group) : 1u;
    const uint32_t ngroups = affine ? static_cast<uint32_t>(K) / gsz : 0u;
    const __amdgpu_buffer_rsrc_t qr = urs(M.idx, M.out * K);
    const __amdgpu_buffer_rsrc_t sr = urs(M.gs, affine ? M.out * ngroups * 4 : 0);
    const __amdgpu_buffer_rsrc_t orr = urs(M.go, affine ? M.out * ngroups * 4 : 0);
    const int32_t nm = static_cast<int32_t>(g.n_mine);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int32_t t = static_cast<int32_t>(t0) + r;
        const bool mine = t < nm;
        const uint32_t row = static_cast<uint32_t>(g.lo + g.rg) + static_cast<uint32_t>(t * g.RG);
#pragma unroll
        for (int ci = 0; ci < CPS; ++ci) {
            const uint32_t k0 = static_cast<uint32_t>((g.c_lo + ci) * kChunk + lane * 16);
            const bool ok = mine && ci < g.nc && k0 < static_cast<uint32_t>(K);
            const uint32_t g4 = (row * ngroups + k0 / gsz) * 4u;
            b.q[r][ci] = buf_load16(qr, ok ? row * static_cast<uint32_t>(K) + k0 : kOob);
            b.sc[r][ci] = buf_loadf(sr, ok ? g4 : kOob);
            b.of[r][ci] = buf_loadf(orr, ok ? g4 : kOob);
        }
    }
}

// Everything a stage needs that does not depend on the barrier.
__device__ __forceinline__ void prefetch(const Geo &G, int32_t group, int tid, Pre &p,
                                         bool with_batch = true, int buf = 0) {
    const int lane = tid & 63;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (s >= G.nseg) break;
        const Mat &M = s ? G.m1 : G.m0;
        const __amdgpu_buffer_rsrc_t cr = urs(M.cb, 256 * 4);
#pragma unroll
        for (int k = 0; k < kTPW; ++k) {
            const uint32_t f = tid + k * kThreads;  // float4 slot of the table
            p.cbv[s][k] = buf_loadf(cr, (f * 4u / NREP) * 4u);
        }
        // the block's CSR range: scalar loads (read-only table), no vector wait
        const bool has_sc = M.rp != nullptr;
        p.b0[s] = has_sc ? kload(M.rp[G.lo]) : 0;
        p.b1[s] = has_sc ? kload(M.rp[G.lo + G.n]) : 0;
    }
    __builtin_amdgcn_sched_barrier(0);  // small loads first: they return first
    const Mat &Mw = G.seg ? G.m1 : G.m0;
    if (with_batch) load_batch(Mw, G.g, G.K, group, 0, lane, p.bt[buf]);
}

// Codebook lookup of byte B of the packed index word w.  Tables start at LDS
// address 0 (the kernel has no static LDS; checked at launch start), table t
// at t * 65536 bytes, entry j replica r at byte 256 j + 4 r.  One v_perm
// builds the whole byte address {0, t, w.byte[B], 4 * lane} from
// lane_seg = (t << 16) | (4 * lane).
template <int B>
__device__ __forceinline__ float tok_lookup(uint32_t lane_seg, uint32_t w) {
    constexpr uint32_t sel = (12u << 24) | (6u << 16) | (static_cast<uint32_t>(B) << 8) | 4u;
    const uint32_t addr = __builtin_amdgcn_perm(lane_seg, w, sel);
    return *reinterpret_cast<lds_cfloat *>(static_cast<uintptr_t>(addr));
}

__device__ __forceinline__ float row_dot(uint32_t lane_seg, const Batch &b, int r,
                                         const float (&xv)[CPS][16], const float (&xs)[CPS],
                                         float nonaff) {
    float acc = 0.f;
#pragma unroll
    for (int ci = 0; ci < CPS; ++ci) {
        float part = 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t w = b.q[r][ci][d];
            const float c0 = tok_lookup<0>(lane_seg, w);
            const float c1 = tok_lookup<1>(lane_seg, w);
            const float c2 = tok_lookup<2>(lane_seg, w);
            const float c3 = tok_lookup<3>(lane_seg, w);
            part = fmaf(xv[ci][4 * d + 0], c0, part);
            part = fmaf(xv[ci][4 * d + 1], c1, part);
            part = fmaf(xv[ci][4 * d + 2], c2, part);
            part = fmaf(xv[ci][4 * d + 3], c3, part);
        }
        acc = fmaf(part, b.sc[r][ci] + nonaff, acc);
        acc = fmaf(b.of[r][ci], xs[ci], acc);
    }
    return acc;
}

// Activation sources of a GEMV stage (flag-in-data slots, polled until
// every word carries its producer's epoch: eb for base / xb, ed for delta).
//   XNORM: r = base + delta (fp32 words; delta may be null) or the bf16
//          embedding row emb (plain); x = bf16(w * r * rsqrt(mean(r^2) +
//          eps)); block 0 stores r to res_out with epoch eo.
//   XBF16: x = bf16 words.
enum { XNORM = 0, XBF16 = 1 };

struct XSrc {
    const uint32_t *base;
    const uint32_t *delta;
    const uint16_t *emb;
    const float *w;
    uint32_t *res_out;
    int32_t res_blk;  // the block that stores res_out
    const uint32_t *xb;
    uint32_t eb, ed, eo;
};

// Poll iterations between checks of the error word / clock.
constexpr int kPollCheck = 16;

// Builds the stage's activation vector in LDS xl (fp32 [K]) block-wide --
// each thread handles 4 (XNORM) or 8 (XBF16) consecutive elements, so few
// registers are live next to the prefetched batches -- then loads the wave's
// slice into xv / xs (zeros outside it).  `part` is 16 floats of LDS scratch.
template <int HC, int XM, typename After>
__device__ __forceinline__ void load_x(const Plan &P, const XSrc &X, const Geo &G, int tid,
                                       int lane, float *xl, float *part, float (&xv)[CPS][16],
                                       float (&xs)[CPS], After after) {
    const int32_t K = G.K;
    const int t = tid;
    if constexpr (XM == XNORM) {
        // K <= 4096: one float4 per thread
        const bool mine = t * 4 < K;
        const uint32_t o4 = mine ? static_cast<uint32_t>(t) * 16u : kOob;
        // the norm weights are constant: issued ahead of the poll, so they
        // have landed when the activations have
        const u32x4 w = buf_load16(urs(X.w, static_cast<int64_t>(K) * 4), o4);
        float r[4];
        if (X.emb) {
            const __amdgpu_buffer_rsrc_t er = urs(X.emb, static_cast<int64_t>(K) * 2);
            const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(er, mine ? t * 8u : kOob, 0, 0);
            const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(er, mine ? t * 8u + 4u : kOob, 0, 0);
            r[0] = __uint_as_float(lo << 16);
            r[1] = __uint_as_float(lo & 0xffff0000u);
            r[2] = __uint_as_float(hi << 16);
            r[3] = __uint_as_float(hi & 0xffff0000u);
        } else {
            // 4 values = 8 words = two 16-byte pieces per buffer
            const __amdgpu_buffer_rsrc_t br = urs(X.base, static_cast<int64_t>(K) * 8);
            const __amdgpu_buffer_rsrc_t dr = urs(X.delta, X.delta ? static_cast<int64_t>(K) * 8 : 0);
            const uint32_t o8 = mine ? static_cast<uint32_t>(t) * 32u : kOob;
            const bool has_d = X.delta != nullptr;
            u32x4 a0, a1, d0, d1;
            // loads return in order: a poll issued now would come back only
            // after the prefetched batch, with data sampled now -- so wait
            // for the batch first and sample later
            __builtin_amdgcn_s_waitcnt(kVmcnt0);
            // pins the norm-weight load above the poll (the compiler would
            // otherwise sink it to its use, a round trip after the poll)
            asm volatile("" ::"v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]));
            const uint64_t t0 = wall_clock64();
            for (int it = 1;; ++it) {
                a0 = coh_load16(br, o8);
                a1 = coh_load16(br, o8 + 16u);
                d0 = coh_load16(dr, o8);
                d1 = coh_load16(dr, o8 + 16u);
                bool ok = true;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ok = ok && ll_ok(a0[j], X.eb) && ll_ok(a1[j], X.eb) &&
                         (!has_d || (ll_ok(d0[j], X.ed) && ll_ok(d1[j], X.ed)));
                if (__all(ok || !mine)) break;
                if (it % kPollCheck == 0 && gave_up(P, t0)) break;
            }
            r[0] = ll_f32(a0[0], a0[1]) + ll_f32(d0[0], d0[1]);
            r[1] = ll_f32(a0[2], a0[3]) + ll_f32(d0[2], d0[3]);
            r[2] = ll_f32(a1[0], a1[1]) + ll_f32(d1[0], d1[1]);
            r[3] = ll_f32(a1[2], a1[3]) + ll_f32(d1[2], d1[3]);
        }
        if (X.res_out && static_cast<int>(blockIdx.x) == X.res_blk && mine) {
            const __amdgpu_buffer_rsrc_t rr = urs(X.res_out, static_cast<int64_t>(K) * 8);
            const u32x4 v0{ll_hi(r[0], X.eo), ll_lo(r[0], X.eo), ll_hi(r[1], X.eo), ll_lo(r[1], X.eo)};
            const u32x4 v1{ll_hi(r[2], X.eo), ll_lo(r[2], X.eo), ll_hi(r[3], X.eo), ll_lo(r[3], X.eo)};
            coh_store16(rr, static_cast<uint32_t>(t) * 32u, v0);
            coh_store16(rr, static_cast<uint32_t>(t) * 32u + 16u, v1);
        }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = fmaf(r[j], r[j], ss);
        ss = wave_sum_all(ss);
        if (lane == 0) part[t / kWave] = ss;
        lds_barrier();
        const float tot = sum16(part);
        const float inv = rsqrtf(tot / K + P.eps);
        if (mine)
            *reinterpret_cast<float4 *>(xl + 4 * t) =
                make_float4(bf16r(__uint_as_float(w[0]) * (r[0] * inv)),
                            bf16r(__uint_as_float(w[1]) * (r[1] * inv)),
                            bf16r(__uint_as_float(w[2]) * (r[2] * inv)),
                            bf16r(__uint_as_float(w[3]) * (r[3] * inv)));
    } else {
        // K <= XP * 8192: at most XP pieces of 8 values (8 words, 32 bytes) per thread
        constexpr int XP = HC == 4 ? 3 : 2;
        const __amdgpu_buffer_rsrc_t xr = urs(X.xb, static_cast<int64_t>(K) * 4);
        u32x4 w[XP][2];
        bool have[XP];
#pragma unroll
        for (int j = 0; j < XP; ++j) have[j] = (t + j * kThreads) * 8 < K;
        __builtin_amdgcn_s_waitcnt(kVmcnt0);  // sample after the prefetched batch (see above)
        const uint64_t t0 = wall_clock64();
        for (int it = 1;; ++it) {
            bool ok = true;
#pragma unroll
            for (int j = 0; j < XP; ++j) {
                const uint32_t off = have[j] ? static_cast<uint32_t>(t + j * kThreads) * 32u : kOob;
                w[j][0] = coh_load16(xr, off);
                w[j][1] = coh_load16(xr, off + 16u);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ok = ok && (!have[j] || (ll_ok(w[j][0][e], X.eb) && ll_ok(w[j][1][e], X.eb)));
            }
            if (__all(ok)) break;
            if (it % kPollCheck == 0 && gave_up(P, t0)) break;
        }
#pragma unroll
        for (int j = 0; j < XP; ++j) {
            const int i = t + j * kThreads;
            if (have[j]) {
                float4 *dst = reinterpret_cast<float4 *>(xl + 8 * i);
                dst[0] = make_float4(ll_bf16(w[j][0][0]), ll_bf16(w[j][0][1]), ll_bf16(w[j][0][2]),
                                     ll_bf16(w[j][0][3]));
                dst[1] = make_float4(ll_bf16(w[j][1][0]), ll_bf16(w[j][1][1]), ll_bf16(w[j][1][2]),
                                     ll_bf16(w[j][1][3]));
            }
        }
    }
    lds_barrier();  // xl complete
    // Every wave has polled and the activation is in LDS: the stream's next
    // loads go out now.  Issued by a wave that finished polling early, they
    // would queue ahead of the other waves' polls (a CU returns vector loads
    // in issue order); issued before the norm, their issue (the memory
    // pipeline takes a batch only as fast as it drains) would hold the norm.
    __builtin_amdgcn_sched_barrier(0);
    after();
    __builtin_amdgcn_sched_barrier(0);
    const Seg &g = G.g;
#pragma unroll
    for (int ci = 0; ci < CPS; ++ci) {
        const int k0 = (g.c_lo + ci) * kChunk + lane * 16;
        const bool ok = ci < g.nc && k0 < K;
        float t2 = 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float4 f = ok ? reinterpret_cast<const float4 *>(xl + k0)[v] : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[ci][4 * v] = f.x;
            xv[ci][4 * v + 1] = f.y;
            xv[ci][4 * v + 2] = f.z;
            xv[ci][4 * v + 3] = f.w;
            t2 += (f.x + f.y) + (f.z + f.w);
        }
        xs[ci] = t2;
    }
}

// Outputs of a GEMV stage (flag-in-data words with epoch ey, coherent):
//   YF32: fp32 y[y_off + row] for the block's matrix;
//   YACT: pair stage, bf16 act[row] = silu(gate) * up.
enum { YF32 = 0, YACT = 1 };

// Lanes per row of the final pass: the most (up to 16) that keep every row
// of the block within one 1024-thread pass.
__device__ __forceinline__ int final_lanes(int64_t n) {
    int L = 16;
    while (L > 1 && n * L > kThreads) L >>= 1;
    return L;
}

// Lane q's share of row r: slices q, q + L, ... and sidecar entries j0 + q,
// j0 + q + L, ... (the caller reduces over the row's L lanes, then adds the
// bias).  Entries past the LDS-staged ones (rare) are read from memory.
__device__ __forceinline__ float row_part(const Mat &M, int r, int q, int L, int S, const float *red,
                                          int32_t j0, int32_t j1, int32_t b0, const float *ent,
                                          const float *xl) {
    float v = 0.f;
    for (int s = q; s < S; s += L) v += red[r * S + s];
    if (M.rp) {
        for (int32_t j = j0 + q; j < j1; j += L) {
            const int32_t e = j - b0;
            float p = ent[min(e, kEnt - 1)];
            if (e >= kEnt) {
                const float d = buf_loadf(urs(M.delta, kAnyBytes), static_cast<uint32_t>(j) * 4u);
                const int32_t c = buf_loadi(urs(M.col, kAnyBytes), static_cast<uint32_t>(j) * 4u);
                p = xl[c] * d;
            }
            v += p;
        }
    }
    return v;
}

// Sum over the aligned group of L lanes (L a power of two up to 16), in a
// fixed order: every lane of the wave takes part.
__device__ __forceinline__ float group_sum(float v, int L) { return lane_group_sum(v, L); }

struct NoNext {
    __device__ void operator()() const {}
};

// B0: the buffer holding the stage's first batch; PRE1: the second batch
// is loaded after the poll (without it the stage has at most one batch per
// wave, and the other buffer belongs to the next stage's prefetch).
// next(): issued when the stream is done (both buffers free) -- the next
// stage's first batch, which then lands during this stage's final pass and
// the next stage's wait instead of after the next stage begins.
// NP = 2: the stage's K has more than kWaves chunks; G.g is pass 0 of
// make_seg_pass and each wave streams the block's rows once per pass (its
// second chunk's activations are reloaded from LDS between the passes).
template <int HC, int XM, int YM, int B0 = 0, bool PRE1 = true, int NP = 1, typename Next = NoNext>
__device__ __forceinline__ void run_gemv(const Plan &P, const Geo &G, Pre &pf, const XSrc &X,
                                         uint32_t *y, uint32_t ey, float *smem, int tid, int lane,
                                         Next next = Next{}) {
    const int32_t K = G.K, group = P.group;
    float *xl = smem + (G.nseg == 2 ? 2 * kTbl : kTbl);
    float *red = smem + P.lds_red;                           // [2][kRedCap]
    float *ent = red + 2 * kRedCap;                          // [2][kEnt]
    int32_t *rps = reinterpret_cast<int32_t *>(ent + 2 * kEnt);  // [2][kRps]
    float *misc = reinterpret_cast<float *>(rps + 2 * kRps);
    const int t = tid;
    // Issue every other load the stage needs before its stream: the CSR row
    // pointers and biases of the block's rows and its sidecar entries.  They
    // queue behind the prefetched batches (which the stream needs first
    // anyway); row pointers and sidecar products go to LDS, so few registers
    // stay live during the stream.
    const int fl = final_lanes(G.n);  // lanes per row of the final pass
    int32_t rpv[2] = {0, 0}, ecol[2] = {0, 0}, nent[2] = {0, 0};
    float edl[2] = {0.f, 0.f}, bias[2] = {0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (s >= G.nseg) break;
        const Mat &M = s ? G.m1 : G.m0;
        const __amdgpu_buffer_rsrc_t rr = urs(M.rp, M.rp ? (M.out + 1) * 4 : 0);
        rpv[s] = buf_loadi(rr, t <= G.n ? static_cast<uint32_t>((G.lo + t) * 4) : kOob);
        const __amdgpu_buffer_rsrc_t br = urs(M.bias, M.bias ? M.out * 4 : 0);
        // the final pass's lane 0 of row t / L adds the bias
        bias[s] = buf_loadf(br, t % fl == 0 && t / fl < G.n ? static_cast<uint32_t>((G.lo + t / fl) * 4) : kOob);
        const int32_t b0 = __builtin_amdgcn_readfirstlane(pf.b0[s]);
        const int32_t b1 = __builtin_amdgcn_readfirstlane(pf.b1[s]);
        nent[s] = M.rp ? b1 - b0 : 0;
        const bool mine = t < min(nent[s], kEnt);
        const __amdgpu_buffer_rsrc_t colr = urs(M.col, M.rp ? static_cast<int64_t>(b1) * 4 : 0);
        const __amdgpu_buffer_rsrc_t dlr = urs(M.delta, M.rp ? static_cast<int64_t>(b1) * 4 : 0);
        const uint32_t e4 = mine ? (static_cast<uint32_t>(b0) + t) * 4u : kOob;
        ecol[s] = buf_loadi(colr, e4);
        edl[s] = buf_loadf(dlr, e4);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (s >= G.nseg) break;
        float *tb = smem + s * kTbl;
#pragma unroll
        for (int k = 0; k < kTPW; ++k)
            reinterpret_cast<float4 *>(tb)[t + k * kThreads] =
                make_float4(pf.cbv[s][k], pf.cbv[s][k], pf.cbv[s][k], pf.cbv[s][k]);
    }
    float xv[CPS][16], xs[CPS];
    const Mat &Mw = G.seg ? G.m1 : G.m0;
    load_x<HC, XM>(P, X, G, t, lane, xl, misc + 16, xv, xs,  // ends with a barrier: xl ready
                   [&] {
                       if constexpr (PRE1) load_batch(Mw, G.g, K, group, RB, lane, pf.bt[1 - B0]);
                   });
    // the loads above have landed by now (they were issued before x's)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (s >= G.nseg) break;
        if (t <= G.n) rps[s * kRps + t] = rpv[s];
        if (t < min(nent[s], kEnt)) ent[s * kEnt + t] = xl[ecol[s]] * edl[s];
    }

    // stream the wave's rows (two batches already in flight)
    const Seg &g = G.g;
    float *redw = red + G.seg * kRedCap;
    const uint32_t lane_seg = (static_cast<uint32_t>(G.seg) << 16) | (static_cast<uint32_t>(lane) * 4u);
    const float nonaff = Mw.gs != nullptr ? 0.f : 1.f;
    const int32_t n_mine = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(g.n_mine));
    // Items of the stream: pass 0's rows padded to whole batch pairs (the two
    // batches in flight at the start are pass 0's), then pass 1's rows.  A
    // wave with no pass-0 rows has none in pass 1 either (its slices are
    // chunks w and w + kWaves).
    const Seg g1 = NP == 2 ? make_seg_pass(G.lo, G.n, __builtin_amdgcn_readfirstlane(t >> 6), 1,
                                           nchunks_of(K))
                           : g;
    const int32_t n0p = NP == 2 ? (n_mine + 2 * RB - 1) / (2 * RB) * (2 * RB) : n_mine;
    const int32_t n_all = NP == 2 ? n0p + __builtin_amdgcn_readfirstlane(static_cast<int32_t>(g1.n_mine))
                                  : n_mine;
    // the batch of items [t0, t0 + RB): every load issued on both passes
    // (the pass only selects scalar fields)
    auto load_item = [&](int32_t t0, Batch &b) {
        const bool p1 = NP == 2 && t0 >= n0p;
        Seg gs = g;
        gs.lo = p1 ? g1.lo : g.lo;
        gs.rg = p1 ? g1.rg : g.rg;
        gs.RG = p1 ? g1.RG : g.RG;
        gs.c_lo = p1 ? g1.c_lo : g.c_lo;
        gs.nc = p1 ? g1.nc : g.nc;
        gs.n_mine = p1 ? g1.n_mine : g.n_mine;
        load_batch(Mw, gs, K, group, p1 ? t0 - n0p : t0, lane, b);
    };
    auto compute = [&](int32_t t0, const Batch &b) {
        const bool p1 = NP == 2 && t0 >= n0p;
        if constexpr (NP == 2) {
            if (t0 == n0p) {
                // pass 1: this wave's second chunk of the activation
                const int k0 = g1.c_lo * kChunk + lane * 16;
                const bool ok = g1.nc > 0 && k0 < K;
                float t2 = 0.f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float4 f = ok ? reinterpret_cast<const float4 *>(xl + k0)[v]
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
                    xv[0][4 * v] = f.x;
                    xv[0][4 * v + 1] = f.y;
                    xv[0][4 * v + 2] = f.z;
                    xv[0][4 * v + 3] = f.w;
                    t2 += (f.x + f.y) + (f.z + f.w);
                }
                xs[0] = t2;
            }
        }
        const int32_t lt = p1 ? t0 - n0p : t0;
        const int32_t nm = p1 ? static_cast<int32_t>(g1.n_mine) : n_mine;
        const int32_t s_id = p1 ? g1.s_id : g.s_id;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int32_t tt = lt + r;
            if (tt < nm) {
                const float v = wave_sum_lane63(row_dot(lane_seg, b, r, xv, xs, nonaff));
                if (lane == kWave - 1) redw[(g.rg + tt * g.RG) * g.S + s_id] = v;
            }
            __builtin_amdgcn_sched_barrier(0);  // one row's lookups in flight at a time
        }
    };
    // The stream ends with no load in flight, so nothing after it (the final
    // pass, the next stage) waits on a load that lands in a reused register
    // -- such a wait would also wait for this stage's output stores.
    for (int32_t i0 = 0; i0 < n_all; i0 += 2 * RB) {
        compute(i0, pf.bt[B0]);
        if (!PRE1 || i0 + RB >= n_all) break;
        load_item(i0 + 2 * RB, pf.bt[B0]);
        __builtin_amdgcn_sched_barrier(0);
        compute(i0 + RB, pf.bt[1 - B0]);
        if (i0 + 2 * RB >= n_all) break;
        load_item(i0 + 3 * RB, pf.bt[1 - B0]);
        __builtin_amdgcn_sched_barrier(0);
    }
    next();
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();  // red and ent complete

    // final pass: fl lanes per row of the block (rows r = t / fl < n)
    if (t < ((G.n * fl + kWave - 1) & ~(kWave - 1))) {  // whole waves: the lane sums shuffle
        const int r = t / fl, q = t % fl;
        const bool live = r < G.n;
        const int rr = live ? r : 0;
        const int S = g.S;
        float v0 = live ? row_part(G.m0, rr, q, fl, S, red, rps[rr], rps[rr + 1], rps[0], ent, xl) : 0.f;
        v0 = group_sum(v0, fl) + bias[0];
        const int64_t row = G.lo + r;
        if constexpr (YM == YF32) {
            if (live && q == 0)
                ll_store2(urs(y, kAnyBytes), static_cast<uint32_t>(G.y_off + row) * 8u, ll_hi(v0, ey),
                          ll_lo(v0, ey));
        } else {
            float v1 = live ? row_part(G.m1, rr, q, fl, S, red + kRedCap, rps[kRps + rr],
                                       rps[kRps + rr + 1], rps[kRps], ent + kEnt, xl)
                            : 0.f;
            v1 = group_sum(v1, fl) + bias[1];
            if (live && q == 0)
                ll_store1(urs(y, kAnyBytes), static_cast<uint32_t>(row) * 4u,
                          ll_bf16w(v0 / (1.f + expf(-v0)) * v1, ey));
        }
    }
    // the next stage rebuilds the tables and xl in LDS: every thread is past
    // this stage's reads first (stores stay in flight: LDS-only barrier)
    lds_barrier();
}

// ---------------------------------------------------------------------------
// attention (one block per query head)
// ---------------------------------------------------------------------------
// Block-wide maximum / sum through red (kWaves floats that no wave reads
// between the previous barrier and this call: one barrier per reduction).
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / kWave] = v;
    lds_barrier();
    float w[kWaves];
    lds16(red, w);
    float t = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t = fmaxf(t, w[i]);
    return t;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / kWave] = v;
    lds_barrier();
    return sum16(red);
}


// Rotation of element pair (i, i + D/2) by the angle table entry cs = (cos, sin).
__device__ __forceinline__ void rope_rot(float x1, float x2, float2 cs, float &o1, float &o2) {
    o1 = x1 * cs.x - x2 * cs.y;
    o2 = x2 * cs.x + x1 * cs.y;
}

// cos / sin of pos * theta^(-2i/D), i < D/2: the same for every layer of a
// token, so attention blocks compute them once per launch into LDS.
__device__ __forceinline__ void rope_table(const Plan &P, int pos, float2 *tab) {
    if (threadIdx.x < kHeadDim / 2) {
        const int i = threadIdx.x;
        const float inv_freq = powf(P.theta, -2.f * i / kHeadDim);
        float sn, cs;
        sincosf(static_cast<float>(pos) * inv_freq, &sn, &cs);
        tab[i] = make_float2(cs, sn);
    }
}

// One block per query head: softmax(q . k_t * D^-1/2, t <= pos) . v_t over
// the head's KV group (head h reads kv head h / (n_heads / n_kv)).
//   The cache rows of earlier positions do not depend on this token: the
//   key rows (quad t / 4 holds positions t / 4 + 256 k, each thread a
//   32-dim quarter) and each wave's first eight value rows are loaded BEFORE
//   waiting for the q/k/v producers, so they arrive while the block waits;
//   later value rows go to LDS by buffer-to-LDS loads.  Then q and the new
//   key are rotated (angle table in LDS), the new key/value are stored into
//   the caches by the first head of each group, scores are one position per
//   quad (two quad DPP adds), softmax by block reductions (one barrier
//   each), and the output is summed by wave over positions (lane = 2 dims)
//   and across waves in LDS.
__device__ __forceinline__ bool attention(const Plan &P, const Layer &L, const uint32_t *qkv, uint32_t eq,
                          uint32_t *attn, uint32_t ea, int h,
                          int pos, float *smem, const float2 *rope) {
    constexpr int D = kHeadDim;
    float *sc = smem;                     // [kMaxSeq]
    float *qs = sc + kMaxSeq;             // [D]
    float *kn = qs + D;                   // [D]
    float *vn = kn + D;                   // [D]
    float *part = vn + D;                 // [kWaves][D]
    float *red = part + kWaves * D;       // [kWaves] block maximum
    float *red2 = red + kWaves;           // [kWaves] block sum
    float *spos = red2 + kWaves;          // [1] score of position pos
    const int grp = P.n_heads / P.n_kv;
    const int kvh = h / grp;
    const int n = pos + 1;
    // ids redefined here, so that the compiler derives the per-position
    // masks below in this stage instead of hoisting them out of the layer
    // loop (masks kept live across the loop spill)
    const int t = fresh_v(static_cast<int>(threadIdx.x));
    const int lane = t & 63, wave = fresh_s(__builtin_amdgcn_readfirstlane(t / kWave));
    const int64_t row = static_cast<int64_t>(P.n_kv) * D;  // cache elements between positions
    const uint16_t *kc = kload(L.kc), *vcache = kload(L.vc);
    // earlier positions' cache rows
    const __amdgpu_buffer_rsrc_t kr = urs(kc, static_cast<int64_t>(P.max_seq) * row * 2);
    const __amdgpu_buffer_rsrc_t vr = urs(vcache, static_cast<int64_t>(P.max_seq) * row * 2);
    // key rows: the four threads of quad t / 4 hold positions t / 4 + kThreads / 4 * k
    // (k < 4), thread t % 4 a quarter of each row (dims 32 (t % 4) + 0..31)
    constexpr int kQP = kThreads / 4;  // positions per quad round
    u32x4 kw[kMaxSeq / kQP][4];
    {
        const int qd = t & 3;
#pragma unroll
        for (int k = 0; k < kMaxSeq / kQP; ++k) {
            const int pk = (t >> 2) + kQP * k;
            const uint32_t base = static_cast<uint32_t>((pk * row + static_cast<int64_t>(kvh) * D + 32 * qd) * 2);
#pragma unroll
            for (int c = 0; c < 4; ++c) kw[k][c] = buf_load16(kr, pk < pos ? base + 16u * c : kOob);
        }
    }
    uint32_t vw[8];
    const uint32_t voff = static_cast<uint32_t>((static_cast<int64_t>(kvh) * D + 2 * lane) * 2);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int tt = wave + u * kWaves;
        vw[u] = __builtin_amdgcn_raw_buffer_load_b32(
            vr, tt < pos ? static_cast<uint32_t>(tt * row * 2) + voff : kOob, 0, 0);
    }
    // V rows of positions [8 * kWaves, vend) go straight to LDS (buffer loads
    // into LDS: no registers), four 256-byte rows per wave instruction, into
    // the LDS the GEMV stages use for tables (free during attention); later
    // positions are read from memory in the accumulation loop.
    uint32_t *vst = reinterpret_cast<uint32_t *>(smem + kVStage);
    const int vcap = ((P.lds_red - kVStage) / (D / 2)) & ~3;  // whole 4-row instructions fit
    const int vbeg = 8 * kWaves;
    const int vend = pos > vbeg ? min(pos, vbeg + vcap) : vbeg;
    for (int q = wave; 4 * q < vend - vbeg; q += kWaves) {
        const int r = vbeg + 4 * q + lane / 16;
        const uint32_t go = r < vend ? static_cast<uint32_t>((static_cast<int64_t>(r) * row +
                                                               static_cast<int64_t>(kvh) * D) * 2) +
                                           16u * static_cast<uint32_t>(lane % 16)
                                     : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            vr, (__attribute__((address_space(3))) void *)(vst + 4 * q * (D / 2)), 16,
            go, 0, 0, 0);
    }
    // this token's q, k, v (flag-in-data words of the q/k/v stage, epoch eq):
    // threads [0, D/2) take q[t], q[t + D/2], k[t], k[t + D/2]; threads
    // [D/2, D/2 + D) take v[t - D/2]
    const int64_t qe = static_cast<int64_t>(h) * D, ke = static_cast<int64_t>(P.n_heads + kvh) * D;
    const int64_t ve = static_cast<int64_t>(P.n_heads + P.n_kv + kvh) * D;
    float qv0 = 0.f, qv1 = 0.f, kv0 = 0.f, kv1 = 0.f, vv = 0.f;
    {
        const __amdgpu_buffer_rsrc_t qr =
            urs(qkv, static_cast<int64_t>(P.n_heads + 2 * P.n_kv) * D * 8);
        const bool qk = t < D / 2, vt = t >= D / 2 && t < D / 2 + D;
        const uint32_t o0 = qk ? static_cast<uint32_t>(qe + t) * 8u : vt ? static_cast<uint32_t>(ve + t - D / 2) * 8u : kOob;
        const uint32_t o1 = qk ? static_cast<uint32_t>(qe + t + D / 2) * 8u : kOob;
        const uint32_t o2 = qk ? static_cast<uint32_t>(ke + t) * 8u : kOob;
        const uint32_t o3 = qk ? static_cast<uint32_t>(ke + t + D / 2) * 8u : kOob;
        uint2 w0, w1, w2, w3;
        __builtin_amdgcn_s_waitcnt(kVmcnt0);  // sample after the K/V preloads land
        const uint64_t t0 = wall_clock64();
        for (int it = 1;; ++it) {
            w0 = coh_load8(qr, o0);
            w1 = coh_load8(qr, o1);
            w2 = coh_load8(qr, o2);
            w3 = coh_load8(qr, o3);
            const bool ok = !(qk || vt) ||
                            (ll_ok(w0.x, eq) && ll_ok(w0.y, eq) &&
                             (vt || (ll_ok(w1.x, eq) && ll_ok(w1.y, eq) && ll_ok(w2.x, eq) &&
                                     ll_ok(w2.y, eq) && ll_ok(w3.x, eq) && ll_ok(w3.y, eq))));
            if (__all(ok)) break;
            if (it % kPollCheck == 0 && gave_up(P, t0)) break;
        }
        if (qk) {
            qv0 = ll_f32(w0.x, w0.y);
            qv1 = ll_f32(w1.x, w1.y);
            kv0 = ll_f32(w2.x, w2.y);
            kv1 = ll_f32(w3.x, w3.y);
        } else {
            vv = ll_f32(w0.x, w0.y);
        }
    }
    const bool writer = h % grp == 0;
    const float scale = rsqrtf(static_cast<float>(D));
    if (t < D / 2) {  // wave 0
        const float2 cs = rope[t];
        float a, b;
        rope_rot(qv0, qv1, cs, a, b);
        const float q0 = a * scale, q1 = b * scale;
        qs[t] = q0;
        qs[t + D / 2] = q1;
        rope_rot(kv0, kv1, cs, a, b);
        const int64_t base = static_cast<int64_t>(pos) * row + static_cast<int64_t>(kvh) * D;
        if (writer) {  // buffer stores (a flat store in flight would make every later LDS wait
                       // of this stage also wait for it)
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(a), kr, static_cast<uint32_t>((base + t) * 2), 0, 0);
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(b), kr,
                                                  static_cast<uint32_t>((base + t + D / 2) * 2), 0, 0);
        }
        kn[t] = bf16r(a);
        kn[t + D / 2] = bf16r(b);
        // this position's score, reduced across the wave
        const float sp = wave_sum_all(fmaf(q0, bf16r(a), q1 * bf16r(b)));
        if (t == 0) *spos = sp;
    } else if (t < D / 2 + D) {
        const int j = t - D / 2;
        const float v = vv;
        if (writer)
            __builtin_amdgcn_raw_buffer_store_b16(
                f32_to_bf16(v), vr,
                static_cast<uint32_t>((static_cast<int64_t>(pos) * row + static_cast<int64_t>(kvh) * D + j) * 2), 0, 0);
        vn[j] = bf16r(v);
    }
    lds_barrier();  // LDS only: the cache stores are read by later launches
    float mx = -FLT_MAX;
    {
        // scores: each quad sums its position's four quarter dot products
        // (two quad DPP adds); q's quarter is read 16 values at a time, four
        // 16-byte LDS reads in flight per round
        const int qd = t & 3;
        const float sp = *spos;
#pragma unroll
        for (int k = 0; k < kMaxSeq / kQP; ++k) {
            if (kQP * k < n) {  // block-uniform
                const int pk = (t >> 2) + kQP * k;
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int c0 = 0; c0 < 4; c0 += 2) {
                    float4 qv[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) qv[i] = reinterpret_cast<const float4 *>(qs)[8 * qd + 2 * c0 + i];
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const float q8[8] = {qv[2 * c].x, qv[2 * c].y, qv[2 * c].z, qv[2 * c].w,
                                             qv[2 * c + 1].x, qv[2 * c + 1].y, qv[2 * c + 1].z, qv[2 * c + 1].w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            s0 = fmaf(q8[2 * e], __uint_as_float(kw[k][c0 + c][e] << 16), s0);
                            s1 = fmaf(q8[2 * e + 1], __uint_as_float(kw[k][c0 + c][e] & 0xffff0000u), s1);
                        }
                    }
                }
                float sq = s0 + s1;
                sq += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sq), 0xb1, 0xf, 0xf, false));
                sq += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sq), 0x4e, 0xf, 0xf, false));
                if (pk == pos) sq = sp;
                if (pk < n) {
                    if (qd == 0) sc[pk] = sq;
                    mx = fmaxf(mx, sq);
                }
            }
        }
    }
    mx = block_max(mx, red);
    float sum = 0.f;
    if (t < n) {
        const float p = expf(sc[t] - mx);
        sc[t] = p;
        sum = p;
    }
    sum = block_sum(sum, red2);
    const float inv = 1.f / sum;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // first eight positions of the wave: preloaded
        const int tt = wave + u * kWaves;
        const float p = tt < pos ? sc[tt] : 0.f;
        a0 = fmaf(p, __uint_as_float(vw[u] << 16), a0);
        a1 = fmaf(p, __uint_as_float(vw[u] & 0xffff0000u), a1);
    }
    // Positions [vbeg, vend) from the V rows staged in LDS, then [vend, pos)
    // from memory, each in increasing order (the same accumulation order as
    // one loop).  Two loops, so that no register of the LDS loop is also the
    // target of a buffer load: otherwise the compiler waits vmcnt(0) before
    // the LDS reads, which on this target also waits for the K/V stores above.
    for (int t0 = wave + vbeg; t0 < vend; t0 += 8 * kWaves) {
        uint32_t w[8];
        float p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int tt = t0 + u * kWaves;
            const bool ok = tt < vend;
            w[u] = vst[(ok ? tt - vbeg : 0) * (D / 2) + lane];
            p[u] = ok ? sc[tt] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            a0 = fmaf(p[u], __uint_as_float(w[u] << 16), a0);
            a1 = fmaf(p[u], __uint_as_float(w[u] & 0xffff0000u), a1);
        }
    }
    for (int t0 = vend + ((wave - vend) % kWaves + kWaves) % kWaves; t0 < pos; t0 += 8 * kWaves) {
        uint32_t w[8];
        float p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int tt = t0 + u * kWaves;
            const bool ok = tt < pos;
            w[u] = __builtin_amdgcn_raw_buffer_load_b32(
                vr, ok ? static_cast<uint32_t>(tt * row * 2) + voff : kOob, 0, 0);
            p[u] = ok ? sc[tt] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            a0 = fmaf(p[u], __uint_as_float(w[u] << 16), a0);
            a1 = fmaf(p[u], __uint_as_float(w[u] & 0xffff0000u), a1);
        }
    }
    if (wave == pos % kWaves) {  // position pos: value from LDS
        a0 = fmaf(sc[pos], vn[2 * lane], a0);
        a1 = fmaf(sc[pos], vn[2 * lane + 1], a1);
    }
    part[wave * D + 2 * lane] = a0;
    part[wave * D + 2 * lane + 1] = a1;
    lds_barrier();
    if (t < D / 2) {
        const int d = 2 * t;
        float2 pw[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) pw[w] = *reinterpret_cast<const float2 *>(part + w * D + d);
        float v0 = 0.f, v1 = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            v0 += pw[w].x;
            v1 += pw[w].y;
        }
        ll_store2(urs(attn, kAnyBytes), static_cast<uint32_t>(h * D + d) * 4u, ll_bf16w(v0 * inv, ea),
                  ll_bf16w(v1 * inv, ea));
    }
    return true;
}

// ---------------------------------------------------------------------------
// LM head: final norm, tied bf16 embedding rows, per-block argmax
// ---------------------------------------------------------------------------
template <int HC>
struct LmPre {
    u32x4 w[kLmBuf][kLmRB][2 * HC];  // 16-byte loads (8 weights) per lane and row
};

// Row t of wave w in block b is ((t * nblocks + b) * 16 + w): at any moment
// the whole grid reads one compact window of the table, which keeps the DRAM
// row buffers open (one contiguous range per block would give 256 streams
// spread over the whole table).
__device__ __forceinline__ int64_t lm_row(const Plan &P, int wave, int64_t t) {
    return (t * P.nblocks + static_cast<int>(blockIdx.x)) * kWaves + wave;
}

template <int HC>
__device__ __forceinline__ void lm_load(const Plan &P, int wave, int lane, int64_t t0,
                                        u32x4 (&w)[kLmRB][2 * HC]) {
    const int32_t K = P.hidden;
    const __amdgpu_buffer_rsrc_t er = urs(P.embed, static_cast<int64_t>(P.vocab) * K * 2);
#pragma unroll
    for (int r = 0; r < kLmRB; ++r) {
        const int64_t row = lm_row(P, wave, t0 + r);
        const bool mine = row < P.vocab;
        const uint32_t rowb = static_cast<uint32_t>(row * K * 2);
#pragma unroll
        for (int c = 0; c < 2 * HC; ++c) {
            const uint32_t col = c * 512 + lane * 8;
            w[r][c] = __builtin_amdgcn_raw_buffer_load_b128(
                er, mine && col < static_cast<uint32_t>(K) ? rowb + col * 2 : kOob, 0, kLmPol);
        }
    }
}

template <int HC>
__device__ void lm_head(const Plan &P, LmPre<HC> &pf, float *smem, int wave, int lane) {
    const int32_t K = P.hidden;
    const int b = blockIdx.x;
    // h = bf16(final_norm * r * inv), r = xa + dn; lane holds columns c*512 + lane*8 + j
    float hx[2 * HC][8];
    float ss = 0.f;
    const int64_t lL = P.n_layers;
    // flag-in-data words (complete: every block arrived after its last stage)
    const __amdgpu_buffer_rsrc_t ar = urs(P.res + lL * P.ls_hid, static_cast<int64_t>(K) * 8);
    const __amdgpu_buffer_rsrc_t dr = urs(P.dn + (lL - 1) * P.ls_hid, static_cast<int64_t>(K) * 8);
    const __amdgpu_buffer_rsrc_t wr = urs(P.final_norm, static_cast<int64_t>(K) * 4);
#pragma unroll
    for (int c = 0; c < 2 * HC; ++c) {
        const uint32_t col = c * 512 + lane * 8;
        const bool ok = col < static_cast<uint32_t>(K);
        u32x4 a[4], d[4];  // all eight loads in flight together
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            a[v] = coh_load16(ar, ok ? col * 8 + 16u * v : kOob);
            d[v] = coh_load16(dr, ok ? col * 8 + 16u * v : kOob);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            hx[c][2 * v] = ll_f32(a[v][0], a[v][1]) + ll_f32(d[v][0], d[v][1]);
            hx[c][2 * v + 1] = ll_f32(a[v][2], a[v][3]) + ll_f32(d[v][2], d[v][3]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(hx[c][j], hx[c][j], ss);
    }
    ss = wave_sum_all(ss);
    const float inv = rsqrtf(ss / K + P.eps);
    u32x4 nw[2 * HC][2];  // the norm weights: every load issued before the first use
#pragma unroll
    for (int c = 0; c < 2 * HC; ++c) {
        const uint32_t col = c * 512 + lane * 8;
        const bool ok = col < static_cast<uint32_t>(K);
#pragma unroll
        for (int v = 0; v < 2; ++v) nw[c][v] = buf_load16(wr, ok ? col * 4 + 16u * v : kOob);
    }
#pragma unroll
    for (int c = 0; c < 2 * HC; ++c) {
        const bool ok = c * 512 + lane * 8 < K;
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                hx[c][4 * v + j] = ok ? bf16r(__uint_as_float(nw[c][v][j]) * (hx[c][4 * v + j] * inv)) : 0.f;
    }
    float best = -FLT_MAX;
    int bi = 0x7fffffff;
    const int64_t step = static_cast<int64_t>(P.nblocks) * kWaves;  // rows per t
    const int64_t first = static_cast<int64_t>(b) * kWaves + wave;   // row at t = 0
    const int64_t n_mine = P.vocab > first ? (P.vocab - first + step - 1) / step : 0;
    // the block's logits collect in LDS and leave in one coalesced pass after
    // the stream: a store inside the stream would sit in the same in-order
    // counter as the row loads
    float *lg = smem + kLmStage;
    auto compute = [&](int64_t t0, const u32x4 (&w)[kLmRB][2 * HC]) {
#pragma unroll
        for (int r = 0; r < kLmRB; ++r) {
            const int64_t t = t0 + r;
            if (t < n_mine) {
                float acc = 0.f;
#pragma unroll
                for (int c = 0; c < 2 * HC; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc = fmaf(__uint_as_float(w[r][c][e] << 16), hx[c][2 * e], acc);
                        acc = fmaf(__uint_as_float(w[r][c][e] & 0xffff0000u), hx[c][2 * e + 1], acc);
                    }
                const float v = wave_sum_lane63(acc);
                if (lane == kWave - 1) {
                    lg[t * kWaves + wave] = v;
                    if (v > best) { best = v; bi = static_cast<int>(first + t * step); }
                }
            }
        }
    };
    // no early exits: batches past the range load nothing (out-of-range
    // offsets), so each batch waits only for its own loads
    for (int64_t i0 = 0; i0 < n_mine; i0 += kLmBuf * kLmRB) {
#pragma unroll
        for (int s = 0; s < kLmBuf; ++s) {
            compute(i0 + s * kLmRB, pf.w[s]);
            lm_load<HC>(P, wave, lane, i0 + (kLmBuf + s) * kLmRB, pf.w[s]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float *bv = smem;
    int *bix = reinterpret_cast<int *>(smem + kWaves);
    if (lane == kWave - 1) {
        bv[wave] = best;
        bix[wave] = bi;
    }
    __syncthreads();
    // wave 0 has the most rows; lg[t * 16 + w] is row lm_row(w, t)
    const int64_t n_stage = (P.vocab > b * kWaves ? (P.vocab - b * kWaves + step - 1) / step : 0) * kWaves;
    const __amdgpu_buffer_rsrc_t lr = urs(P.logits, static_cast<int64_t>(P.vocab) * 4);
    for (int i = threadIdx.x; i < n_stage; i += blockDim.x) {
        const int64_t row = lm_row(P, i % kWaves, i / kWaves);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lg[i]), lr,
                                              row < P.vocab ? static_cast<uint32_t>(row) * 4u : kOob, 0, 0);
    }
    if (threadIdx.x == 0) {
        float v = -FLT_MAX;
        int i = 0x7fffffff;
        for (int w = 0; w < kWaves; ++w)
            if (bv[w] > v || (bv[w] == v && bix[w] < i)) { v = bv[w]; i = bix[w]; }
        coh_storef(P.part_v + b, v);
        coh_storei(P.part_i + b, i);
    }
}

__device__ void final_argmax(const Plan &P, float *smem) {
    float v = -FLT_MAX;
    int i = 0x7fffffff;
    if (static_cast<int>(threadIdx.x) < P.nblocks) {
        v = P.part_v[threadIdx.x];
        i = P.part_i[threadIdx.x];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(v, m, kWave);
        const int oi = __shfl_xor(i, m, kWave);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
    float *bv = smem;
    int *bix = reinterpret_cast<int *>(smem + kWaves);
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x / kWave] = v;
        bix[threadIdx.x / kWave] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < kWaves; ++w)
            if (bv[w] > v || (bv[w] == v && bix[w] < i)) { v = bv[w]; i = bix[w]; }
        *P.tok = i;
        *P.pos += 1;  // next decode position
    }
}

// ---------------------------------------------------------------------------
// the token kernel
// ---------------------------------------------------------------------------
// One layer: five stages whose outputs are flag-in-data words tagged with
// the stage's epoch (ll_epoch of the running stage count `target`); each
// stage's readers poll for their producers' epochs, so no grid barrier runs
// inside the layer.  Every stage issues its compressed-weight loads first.
template <int HC>
__device__ __forceinline__ bool do_layer(const Plan &P, int l, int pos, uint32_t &target,
                                         float *smem, const float2 *rope, int wave0, int tok,
                                         Pre &pf) {
    const Layer &L = P.layers[l];
    const uint32_t t0 = target;  // the previous layer's last stage (its down output)
    const uint32_t e1 = ll_epoch(t0 + 1), e2 = ll_epoch(t0 + 2), e3 = ll_epoch(t0 + 3);
    const uint32_t e4 = ll_epoch(t0 + 4), e5 = ll_epoch(t0 + 5);
    target = t0 + 5;
    // Each stage starts from fresh copies of the thread / wave ids, so values
    // derived from them are recomputed per stage rather than kept live.
    int tid = fresh_v(static_cast<int>(threadIdx.x)), wave = fresh_s(wave0), lane = tid & 63;
    // 1. r = x + delta -> ra; q/k/v = W norm(r), on blocks [qkv_b0,
    // nblocks): with qkv_b0 = n_heads the attention blocks start attention
    // (loading this layer's K/V cache rows) at once, so those loads stream
    // while the q/k/v projection runs instead of after it
    if (static_cast<int>(blockIdx.x) >= P.qkv_b0) {
        const Geo G = geo_qkv(P, L, wave);
        // after layer 0 the previous layer's down stage loaded the first batch
        prefetch(G, P.group, tid, pf, l == 0);
        XSrc X{};
        X.base = P.res + static_cast<int64_t>(l) * P.ls_hid;
        X.delta = l == 0 ? nullptr : P.dn + static_cast<int64_t>(l - 1) * P.ls_hid;
        X.emb = l == 0 ? P.embed + static_cast<int64_t>(tok) * P.hidden : nullptr;
        X.w = kload(L.in_norm);
        X.res_out = P.ra + static_cast<int64_t>(l) * P.ls_hid;
        X.res_blk = P.qkv_b0;
        X.eb = ll_epoch(t0 - 1);  // res[l]: the previous layer's stage 4
        X.ed = ll_epoch(t0);      // dn[l-1]: the previous layer's stage 5
        X.eo = e1;
        run_gemv<HC, XNORM, YF32>(P, G, pf, X, P.qkv + static_cast<int64_t>(l) * P.ls_qkv, e1, smem,
                                  tid, lane);
    }
    tid = fresh_v(tid), wave = fresh_s(wave), lane = tid & 63;
    // 2. attention (block h = query head h); the other blocks go straight on
    // to the o stage's prefetch
    if (static_cast<int>(blockIdx.x) < P.n_heads) {
        attention(P, L, P.qkv + static_cast<int64_t>(l) * P.ls_qkv, e1,
                  P.attn + static_cast<int64_t>(l) * P.ls_attn, e2, blockIdx.x, pos, smem, rope);
        lds_barrier();  // attention's LDS is reused by the next stage
    }
    // 3. o = W_o attn, on blocks [o_b0, nblocks): with o_b0 = n_heads the
    // attention blocks, which finish attention after everyone else has
    // started o, skip it and go on to the gate/up stage, instead of being
    // the last o producers every layer
    if (static_cast<int>(blockIdx.x) >= P.o_b0) {
        // The o weights (at most one batch per wave: the host checks) go to
        // bt[1]; the gate/up stage's first batch goes to bt[0] now, so it
        // streams while o waits for attention rather than after o.
        const Geo Go = geo_plain(P, L, kO, P.n_heads * kHeadDim, P.s_o, wave, P.o_b0);
        prefetch(Go, P.group, tid, pf, true, 1);
        {
            const Geo Gp = geo_pair(P, L, wave);
            load_batch(Gp.seg ? Gp.m1 : Gp.m0, Gp.g, Gp.K, P.group, 0, lane, pf.bt[0]);
        }
        tid = fresh_v(tid), lane = tid & 63;
        XSrc X{};
        X.xb = P.attn + static_cast<int64_t>(l) * P.ls_attn;
        X.eb = e2;
        run_gemv<HC, XBF16, YF32, 1, false>(P, Go, pf, X, P.o + static_cast<int64_t>(l) * P.ls_hid,
                                            e3, smem, tid, lane);
    } else {
        // attention blocks: the gate/up stage's first batch (written as the
        // other branch of the o stage, so no earlier batch stays live across
        // attention)
        const Geo Gp = geo_pair(P, L, wave);
        load_batch(Gp.seg ? Gp.m1 : Gp.m0, Gp.g, Gp.K, P.group, 0, lane, pf.bt[0]);
    }
    {
        tid = fresh_v(tid), wave = fresh_s(wave), lane = tid & 63;
        const Geo Gp = geo_pair(P, L, wave);
        prefetch(Gp, P.group, tid, pf, false);  // first batch: loaded above
        // 4. r = ra + o -> res[l+1]; act = silu(W_g norm(r)) * (W_u norm(r))
        XSrc X{};
        X.base = P.ra + static_cast<int64_t>(l) * P.ls_hid;
        X.delta = P.o + static_cast<int64_t>(l) * P.ls_hid;
        X.w = kload(L.post_norm);
        X.res_out = P.res + static_cast<int64_t>(l + 1) * P.ls_hid;
        X.res_blk = 0;
        X.eb = e1;
        X.ed = e3;
        X.eo = e4;
        run_gemv<HC, XNORM, YACT>(P, Gp, pf, X, P.act + static_cast<int64_t>(l) * P.ls_act, e4, smem,
                                  tid, lane);
    }
    {
        tid = fresh_v(tid), wave = fresh_s(wave), lane = tid & 63;
        // hidden above 2048 (HC 4): intermediate may exceed kWaves chunks, so
        // the down stage streams its rows in two chunk passes
        constexpr int NPD = HC == 4 ? 2 : 1;
        Geo Gd = geo_plain(P, L, kD, P.inter, P.s_down, wave);
        if constexpr (NPD == 2) Gd.g = make_seg_pass(Gd.lo, Gd.n, wave, 0, nchunks_of(P.inter));
        prefetch(Gd, P.group, tid, pf);
        // 5. dn = W_d act
        XSrc X{};
        X.xb = P.act + static_cast<int64_t>(l) * P.ls_act;
        X.eb = e4;
        run_gemv<HC, XBF16, YF32, 0, true, NPD>(P, Gd, pf, X, P.dn + static_cast<int64_t>(l) * P.ls_hid,
                                                e5, smem, tid, lane, [&] {
                                      if (l + 1 < P.n_layers &&
                                          static_cast<int>(blockIdx.x) >= P.qkv_b0) {
                                          const Geo G1 = geo_qkv(P, P.layers[l + 1], wave);
                                          load_batch(G1.m0, G1.g, G1.K, P.group, 0, lane, pf.bt[0]);
                                      }
                                  });
    }
    return true;
}

template <int HC>
__global__ __launch_bounds__(kThreads, 1) void token_kernel(const Plan *__restrict__ plan,
                                                             int32_t step, int32_t *out_ids) {
    extern __shared__ float smem[];
    const Plan &P = *plan;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int *sh = reinterpret_cast<int *>(smem + P.lds_red + 2 * kRedCap + 2 * kEnt + 2 * kRps);
    uint32_t target = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(P.flags + blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int pos = __builtin_amdgcn_readfirstlane(*P.pos);
    const int tok = __builtin_amdgcn_readfirstlane(*P.tok);
    if (lds_offset_of(smem) != 0) {  // the table lookups address LDS from 0
        if (threadIdx.x == 0) __hip_atomic_store(P.err, 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (pos < 0 || pos >= P.max_seq || tok < 0 || tok >= P.vocab) {
        // the host keeps pos < max_seq; a bad state ends the launch everywhere
        if (threadIdx.x == 0) __hip_atomic_store(P.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && out_ids) out_ids[step] = tok;
    float2 *rope = reinterpret_cast<float2 *>(smem + P.lds_red + 2 * kRedCap + 2 * kEnt + 2 * kRps + 64);
    if (static_cast<int>(blockIdx.x) < P.n_heads) rope_table(P, pos, rope);  // read after barriers
    // Nothing of the prologue stays in flight into the layer loop: a load
    // pending at the loop entry would make the compiler wait at the top of
    // every layer, and that wait would also cover the previous layer's
    // output stores.
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    Pre pf;  // weight batches; a stage may load the next stage's first batch
#pragma clang loop unroll(disable)
    for (int l = 0; l < P.n_layers; ++l)
        if (!do_layer<HC>(P, l, pos, target, smem, rope, wave, tok, pf)) return;
    // the last layer's outputs are complete everywhere once every block has
    // arrived (arriving waits for the block's stores)
    arrive(P, target);
    {
        LmPre<HC> lpf;
#pragma unroll
        for (int s = 0; s < kLmBuf; ++s) lm_load<HC>(P, wave, lane, s * kLmRB, lpf.w[s]);
        if (!wait_all(P, target, sh)) return;
        lm_head<HC>(P, lpf, smem, wave, lane);
    }
    arrive(P, ++target);
    if (!wait_all(P, target, sh)) return;
    if (blockIdx.x == 0) final_argmax(P, smem);
}

__global__ void clear_sync_kernel(uint32_t *flags, int32_t n, uint32_t *release, int32_t *err) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) flags[i] = 0;
    if (threadIdx.x == 0) {
        *release = 0;
        *err = 0;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct Layout {
    int64_t plan, layers, res, ra, qkv, o, dn, part_v, part_i, attn, act, flags, release, err, total;
    int32_t s_hid, s_qkv, s_attn, s_act;  // slot strides in 32-bit words (256-byte multiples)
};

static int64_t align256(int64_t v) { return (v + 255) & ~int64_t{255}; }

static Layout layout_of(const hxq_decoder *d, int nb) {
    Layout L{};
    int64_t off = 0;
    auto take = [&](int64_t bytes) { const int64_t o = off; off = align256(off + bytes); return o; };
    const int64_t nl = d->n_layers;
    // slots in flag-in-data words: fp32 values two words, bf16 values one
    L.s_hid = static_cast<int32_t>(align256(8LL * d->hidden) / 4);
    L.s_qkv = static_cast<int32_t>(align256(8LL * (d->n_heads + 2 * d->n_kv_heads) * kHeadDim) / 4);
    L.s_attn = static_cast<int32_t>(align256(4LL * d->n_heads * kHeadDim) / 4);
    L.s_act = static_cast<int32_t>(align256(4LL * d->intermediate) / 4);
    L.plan = take(sizeof(Plan));
    L.layers = take(static_cast<int64_t>(sizeof(Layer)) * nl);
    L.res = take(4LL * L.s_hid * (nl + 1));
    L.ra = take(4LL * L.s_hid * nl);
    L.qkv = take(4LL * L.s_qkv * nl);
    L.o = take(4LL * L.s_hid * nl);
    L.dn = take(4LL * L.s_hid * nl);
    L.part_v = take(4LL * nb);
    L.part_i = take(4LL * nb);
    L.attn = take(4LL * L.s_attn * nl);
    L.act = take(4LL * L.s_act * nl);
    L.flags = take(4LL * nb);
    L.release = take(256);
    L.err = take(256);
    L.total = off;
    return L;
}

// Slices for a segment of nw waves: every slice at most CPS chunks; fewest
// chunk-rows per wave, then fewest slices.
static int choose_slices(int64_t rows, int nw, int nchunks) {
    int best = -1;
    int64_t best_cost = INT64_MAX;
    for (int S = 1; S <= nw && S <= nchunks; ++S) {
        if ((nchunks + S - 1) / S > CPS) continue;
        const int RG = nw / S;
        const int64_t cost = ((rows + RG - 1) / RG) * ((nchunks + S - 1) / S);
        if (cost < best_cost) { best_cost = cost; best = S; }
    }
    return best;
}

static int lds_red_offset(const hxq_decoder *d) {
    const int kmax = std::max({d->hidden, d->n_heads * kHeadDim, d->intermediate});
    const int a = 2 * kTbl + ((d->hidden + 3) & ~3);
    const int b = kTbl + ((kmax + 3) & ~3);
    return std::max(a, b);
}

static size_t lds_bytes(const hxq_decoder *d) {
    return sizeof(float) * (static_cast<size_t>(lds_red_offset(d)) + 2 * kRedCap + 2 * kEnt + 2 * kRps +
                             64 + kHeadDim);
}

static int hc_of(const hxq_decoder *d) { return d->hidden <= 1024 ? 1 : d->hidden <= 2048 ? 2 : 4; }

}  // namespace tok
}  // namespace hxq

using namespace hxq;
using namespace hxq::tok;

static int check_mat(const hxq_matrix &m, int64_t out, int64_t in, int32_t group, const char *name) {
    if (!m.indices || !m.codebook) {
        set_error(std::string("hxq_decoder_init: ") + name + ": indices and codebook are required");
        return HXQ_ERR_INVALID_ARG;
    }
    if (m.out_features != out) {
        set_error(std::string("hxq_decoder_init: ") + name + ": out_features " +
                  std::to_string(m.out_features) + ", expected " + std::to_string(out));
        return HXQ_ERR_INVALID_ARG;
    }
    if ((m.group_scale == nullptr) != (m.group_offset == nullptr) ||
        (m.group_scale && (group <= 0 || group % 16 != 0 || in % group != 0))) {
        set_error(std::string("hxq_decoder_init: ") + name + ": bad affine / group_size");
        return HXQ_ERR_INVALID_ARG;
    }
    if ((m.sc_row_ptr == nullptr) != (m.sc_col == nullptr) ||
        (m.sc_row_ptr == nullptr) != (m.sc_delta == nullptr)) {
        set_error(std::string("hxq_decoder_init: ") + name + ": sidecar arrays must be all set or all NULL");
        return HXQ_ERR_INVALID_ARG;
    }
    if (out * in >= (int64_t{1} << 31)) {
        set_error(std::string("hxq_decoder_init: ") + name + ": matrix too large");
        return HXQ_ERR_INVALID_ARG;
    }
    return HXQ_OK;
}

static int validate(const hxq_decoder *d, int nb) {
    HXQ_REQUIRE(d && d->layers && d->embed && d->final_norm && d->token && d->pos && d->logits,
                "descriptor pointers are required");
    // two codebook tables plus the hidden-wide activation row must fit the
    // 160 KB of LDS next to the staging areas: hidden 3584 is the largest
    // multiple of 512 that does
    HXQ_REQUIRE(d->hidden >= 512 && d->hidden <= 3584 && d->hidden % 512 == 0,
                "hidden must be 512..3584, a multiple of 512");
    HXQ_REQUIRE(d->head_dim == kHeadDim, "head_dim must be 128");
    HXQ_REQUIRE(d->n_layers >= 1 && d->n_heads >= 1 && d->n_kv_heads >= 1 &&
                    d->n_heads % d->n_kv_heads == 0 && d->n_heads <= nb,
                "bad head counts");
    HXQ_REQUIRE(d->n_heads * kHeadDim <= CPS * kChunk * kWaves, "too many heads");
    // one chunk per wave and stage; above hidden 2048 the down stage takes two
    // chunk passes (the activation load covers 3 x 8192 values)
    const int64_t max_inter = hc_of(d) == 4 ? 3 * 8 * kThreads : CPS * kChunk * kWaves;
    HXQ_REQUIRE(d->intermediate >= 16 && d->intermediate % 16 == 0 && d->intermediate <= max_inter,
                "intermediate must be a multiple of 16, at most 16384 (24576 above hidden 2048)");
    HXQ_REQUIRE(d->max_seq >= 1 && d->max_seq <= kMaxSeq, "max_seq must be 1..1024");
    HXQ_REQUIRE(d->vocab >= 1 && static_cast<int64_t>(d->vocab) * d->hidden * 2 < (int64_t{1} << 32),
                "vocab too large");
    HXQ_REQUIRE(lds_bytes(d) <= 160 * 1024, "LDS budget exceeded (intermediate too large)");
    const int64_t H = d->hidden, I = d->intermediate, QD = int64_t{d->n_heads} * kHeadDim,
                  KD = int64_t{d->n_kv_heads} * kHeadDim;
    for (int l = 0; l < d->n_layers; ++l) {
        const hxq_decoder_layer &L = d->layers[l];
        HXQ_REQUIRE(L.in_norm && L.post_norm && L.k_cache && L.v_cache, "layer norms and caches are required");
        HXQ_REQUIRE(reinterpret_cast<uintptr_t>(L.k_cache) % 16 == 0, "k_cache must be 16-byte aligned");
        if (int rc = check_mat(L.q, QD, H, d->group_size, "q")) return rc;
        if (int rc = check_mat(L.k, KD, H, d->group_size, "k")) return rc;
        if (int rc = check_mat(L.v, KD, H, d->group_size, "v")) return rc;
        if (int rc = check_mat(L.o, H, QD, d->group_size, "o")) return rc;
        if (int rc = check_mat(L.gate, I, H, d->group_size, "gate")) return rc;
        if (int rc = check_mat(L.up, I, H, d->group_size, "up")) return rc;
        if (int rc = check_mat(L.down, H, I, d->group_size, "down")) return rc;
    }
    return HXQ_OK;
}

static Mat mat_of(const hxq_matrix &m) {
    Mat r;
    r.idx = m.indices;
    r.cb = m.codebook;
    r.gs = m.group_scale;
    r.go = m.group_offset;
    r.rp = m.sc_row_ptr;
    r.col = m.sc_col;
    r.delta = m.sc_delta;
    r.bias = m.bias;
    r.out = m.out_features;
    return r;
}

extern "C" int64_t hxq_decoder_workspace_bytes(const hxq_decoder *d) {
    clear_error();
    if (!d) return -1;
    return layout_of(d, device_cu_count()).total;
}

extern "C" int hxq_decoder_init(const hxq_decoder *d, void *workspace, int64_t workspace_bytes,
                                hipStream_t stream) {
    clear_error();
    const int nb = device_cu_count();
    if (int rc = validate(d, nb)) return rc;
    const Layout lay = layout_of(d, nb);
    HXQ_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small");
    HXQ_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
    char *ws = static_cast<char *>(workspace);

    // The attention blocks [0, n_heads) skip the q/k/v and o stages when the
    // other blocks are the large majority (they would finish last).
    const int att_b0 = nb - d->n_heads >= 3 * nb / 4 ? d->n_heads : 0;
    // q/k/v block split in proportion to rows (every matrix at least one block)
    const int nbq = nb - att_b0;
    const int64_t rq = int64_t{d->n_heads} * kHeadDim, rk = int64_t{d->n_kv_heads} * kHeadDim;
    const int64_t rt = rq + 2 * rk;
    int bq = static_cast<int>((nbq * rq + rt / 2) / rt);
    int bk = static_cast<int>((nbq * rk + rt / 2) / rt);
    bq = std::max(1, std::min(bq, nbq - 2));
    bk = std::max(1, std::min(bk, nbq - bq - 1));
    const int bv = nbq - bq - bk;
    const int nch_h = (d->hidden + kChunk - 1) / kChunk;
    const int nch_o = (d->n_heads * kHeadDim + kChunk - 1) / kChunk;
    const int nch_i = (d->intermediate + kChunk - 1) / kChunk;
    const int64_t rows_qkv = std::max({(rq + bq - 1) / bq, (rk + bk - 1) / bk, (rk + bv - 1) / bv});
    const int o_b0 = att_b0;
    const int64_t rows_o = (d->hidden + (nb - o_b0) - 1) / (nb - o_b0);
    const int64_t rows_gu = (d->intermediate + nb - 1) / nb;
    const int64_t rows_d = (d->hidden + nb - 1) / nb;
    HXQ_REQUIRE((d->vocab + nb * kWaves - 1) / (nb * kWaves) * kWaves + kLmStage <= lds_red_offset(d),
                "vocab too large for the block count");
    Plan P{};
    P.hidden = d->hidden;
    P.n_layers = d->n_layers;
    P.n_heads = d->n_heads;
    P.n_kv = d->n_kv_heads;
    P.inter = d->intermediate;
    P.vocab = d->vocab;
    P.max_seq = d->max_seq;
    P.group = d->group_size > 0 ? d->group_size : 16;
    P.nblocks = nb;
    P.eps = d->rms_eps;
    P.theta = d->rope_theta;
    P.o_b0 = o_b0;
    P.qkv_b0 = att_b0;
    P.qkv_b1 = att_b0 + bq;
    P.qkv_b2 = att_b0 + bq + bk;
    P.s_qkv = choose_slices(rows_qkv, kWaves, nch_h);
    P.s_o = choose_slices(rows_o, kWaves, nch_o);
    P.s_gu = choose_slices(rows_gu, kWaves / 2, nch_h);
    P.s_down = hc_of(d) == 4 ? nch_i : choose_slices(rows_d, kWaves, nch_i);
    HXQ_REQUIRE(P.s_qkv > 0 && P.s_o > 0 && P.s_gu > 0 && P.s_down > 0, "no slice split fits");
    HXQ_REQUIRE((rows_o + kWaves / P.s_o - 1) / (kWaves / P.s_o) <= RB,
                "o stage needs more than one batch per wave");
    HXQ_REQUIRE(rows_qkv <= kThreads && rows_o <= kThreads && rows_gu <= kThreads &&
                    rows_qkv * P.s_qkv <= kRedCap && rows_o * P.s_o <= kRedCap &&
                    rows_gu * P.s_gu <= kRedCap && rows_d * P.s_down <= kRedCap,
                "too many rows per block for this GPU");
    P.lds_red = lds_red_offset(d);
    P.embed = d->embed;
    P.final_norm = d->final_norm;
    P.tok = d->token;
    P.pos = d->pos;
    P.logits = d->logits;
    P.layers = reinterpret_cast<const Layer *>(ws + lay.layers);
    P.res = reinterpret_cast<uint32_t *>(ws + lay.res);
    P.ra = reinterpret_cast<uint32_t *>(ws + lay.ra);
    P.qkv = reinterpret_cast<uint32_t *>(ws + lay.qkv);
    P.o = reinterpret_cast<uint32_t *>(ws + lay.o);
    P.dn = reinterpret_cast<uint32_t *>(ws + lay.dn);
    P.part_v = reinterpret_cast<float *>(ws + lay.part_v);
    P.part_i = reinterpret_cast<int32_t *>(ws + lay.part_i);
    P.attn = reinterpret_cast<uint32_t *>(ws + lay.attn);
    P.act = reinterpret_cast<uint32_t *>(ws + lay.act);
    P.ls_hid = lay.s_hid;
    P.ls_qkv = lay.s_qkv;
    P.ls_attn = lay.s_attn;
    P.ls_act = lay.s_act;
    P.flags = reinterpret_cast<uint32_t *>(ws + lay.flags);
    P.release = reinterpret_cast<uint32_t *>(ws + lay.release);
    P.err = reinterpret_cast<int32_t *>(ws + lay.err);

    std::vector<Layer> layers(d->n_layers);
    for (int l = 0; l < d->n_layers; ++l) {
        const hxq_decoder_layer &s = d->layers[l];
        Layer &L = layers[l];
        L.m[kQ] = mat_of(s.q);
        L.m[kK] = mat_of(s.k);
        L.m[kV] = mat_of(s.v);
        L.m[kO] = mat_of(s.o);
        L.m[kG] = mat_of(s.gate);
        L.m[kU] = mat_of(s.up);
        L.m[kD] = mat_of(s.down);
        L.in_norm = s.in_norm;
        L.post_norm = s.post_norm;
        L.kc = s.k_cache;
        L.vc = s.v_cache;
    }
    HXQ_HIP_TRY(hipMemcpyAsync(ws + lay.plan, &P, sizeof(Plan), hipMemcpyHostToDevice, stream));
    HXQ_HIP_TRY(hipMemcpyAsync(ws + lay.layers, layers.data(), sizeof(Layer) * layers.size(),
                               hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(clear_sync_kernel, dim3(1), dim3(256), 0, stream, P.flags, nb, P.release, P.err);
    HXQ_LAUNCH_CHECK();
    HXQ_HIP_TRY(hipStreamSynchronize(stream));  // host staging buffers go out of scope
    return HXQ_OK;
}

template <int HC>
static int launch_steps(const hxq_decoder *d, void *workspace, int32_t n_steps, int32_t *out_ids,
                        hipStream_t stream) {
    const size_t lds = lds_bytes(d);
    const void *fn = reinterpret_cast<const void *>(&token_kernel<HC>);
    HXQ_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    int occ = 0;
    HXQ_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, token_kernel<HC>, kThreads, lds));
    HXQ_REQUIRE(occ >= 1, "the token kernel does not fit on a compute unit");
    const Plan *plan = reinterpret_cast<const Plan *>(workspace);
    const int nb = device_cu_count();
    for (int32_t s = 0; s < n_steps; ++s) {
        int32_t step = s;
        void *args[] = {&plan, &step, &out_ids};
        HXQ_HIP_TRY(hipLaunchCooperativeKernel(fn, dim3(nb), dim3(kThreads), args, lds, stream));
    }
    return HXQ_OK;
}

extern "C" int hxq_decoder_step(const hxq_decoder *d, void *workspace, int32_t n_steps,
                                int32_t *out_ids, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(d && workspace && n_steps >= 0, "bad arguments");
    HXQ_REQUIRE(d->hidden >= 512 && d->hidden <= 3584, "hidden must be 512..3584");
    if (hc_of(d) == 1) return launch_steps<1>(d, workspace, n_steps, out_ids, stream);
    if (hc_of(d) == 2) return launch_steps<2>(d, workspace, n_steps, out_ids, stream);
    return launch_steps<4>(d, workspace, n_steps, out_ids, stream);
}

extern "C" int hxq_decoder_error(const void *workspace, const hxq_decoder *d, int32_t *err_out,
                                 hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(workspace && d && err_out, "bad arguments");
    const Layout lay = layout_of(d, device_cu_count());
    HXQ_HIP_TRY(hipMemcpyAsync(err_out, static_cast<const char *>(workspace) + lay.err, 4,
                               hipMemcpyDeviceToHost, stream));
    HXQ_HIP_TRY(hipStreamSynchronize(stream));
    return HXQ_OK;
}
