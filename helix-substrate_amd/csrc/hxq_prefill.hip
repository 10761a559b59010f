// HXQ prefill GEMM, register-dequant design: Y[M, OUT] = X[M, K] @ W^T with
// W held in one of the HXQ index formats (uint8 or uint16 codebook indices,
// uint16 or 12-bit pair-codebook indices, 6-bit affine levels; + per-group
// affine, + sidecar) and never written anywhere in dense form.
//
// Replaces fused_vq_matmul's N > 1 path (helix_substrate/triton_vq_matmul.py:
// 249-334 _vq_gather_matmul_tiled_kernel, 634-661 dispatch, 693-698 sidecar
// scatter_add, 724-725 bias), the pair-codebook tiled kernel
// (triton_vq2d_matmul.py:73-160) and the default materialise-then-BLAS
// _forward_buffered (helix_linear.py:556-634).
//
// Block: 512 threads = 8 waves (two per SIMD), output tile BM x 256 (BM 256
// or 128), K step 64.  Wave w owns the 32 output columns [n0 + 32w, +32) for
// all BM rows: BM/32 accumulator tiles of v_mfma_f32_32x32x16_{bf16,f16}
// (fp32).  Per K step:
//   * A (X rows, 16-bit) is staged through LDS once per block and read by
//     all eight waves (16-byte chunks XOR-swizzled by (row / 2) % 8 for the
//     64 banks: conflict-free);
//   * B (the wave's 32 W rows x 64 k) is dequantised straight into the MFMA
//     operand registers by the wave that uses it -- nothing of W goes to LDS
//     and no wave waits on another for its weights.  The MFMA lane layout
//     gives lane (c = lane % 32, h = lane / 32) the k range [8h, 8h+8) of a
//     16-wide k substep; the kernel permutes k identically for A and B so
//     that lane h of substep s covers physical k = 32h + 8s .. +8, i.e. a
//     lane's B data for the whole step is the contiguous index bytes of
//     weights [32h, 32h + 32) of its row.  uint8 lookups go to a codebook
//     replicated 64x in LDS (lane l reads replica l: no bank conflicts; the
//     byte address {0, 0, idx, 4l} is one v_perm_b32); uint16 and pair
//     codebooks are one 4096-entry table; 6-bit levels need none.  The
//     affine is one FMA, fl(c * scale + offset), for 16-bit operands (the
//     form of the reference's GPU kernel, triton_affine_group_matmul.py:99;
//     rounded to 16 bits right after) and fl(fl(c * scale) + offset), the
//     reference's PyTorch order, for fp32 activations; then
//     v_cvt_pk_bf16_f32 / f16;
//   * B of step s+1 is built while the MFMAs of step s run (substep by
//     substep), index loads run two steps ahead and X loads one, one barrier
//     per step.
// Sidecar: the entries of each group of 64 output rows are given sorted by
// column, with a pointer per K step.  Per step a wave loads the 64 entries
// from its group's pointer, one per lane; those of the step and of its rows
// are found by a ballot and each is applied by one indexed register write in
// its owning lane (v_readlane for the entry, an SGPR-indexed move for the
// operand register) -- no per-lane cursors and no divergent loops.
// Results are written once per element (split-K: fp32 partials reduced in
// order by a second kernel): deterministic.
#include "hxq_prefill.h"
#include <algorithm>
#include <type_traits>

#include "hxq_common.h"

namespace hxq {
namespace pg {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBN = 256;       // output columns per block
constexpr int kBK = 64;        // K per step
constexpr int kNrep = 64;      // codebook replicas (one per lane)
constexpr int kXcds = 8;
constexpr int kGroupRows = 8;  // tile-order group height (X row tiles)
#ifndef HXQ_PREFILL_NJ
#define HXQ_PREFILL_NJ 1
#endif
constexpr int kNJ = HXQ_PREFILL_NJ;  // 32-column subtiles per wave

struct Args {
    const uint16_t *x;       // [M, K] bf16 / fp16
    const uint8_t *idx;      // index data, rows of K * (bits per weight) / 8 bytes
    const float *cb;         // [256] (uint8), [n_codes] (uint16), [n_codes, 2] (pairs)
    const float2 *ga;        // [K/G, OUT] {scale, offset} or null
    const int32_t *sc_ptr;   // [ceil(OUT/64) * K/64 + 1] step pointers, or null
    const uint32_t *sc_key;  // (col << 6) | (row % 64), sorted within each 64-row group
    const float *sc_val;
    const float *bias;       // [OUT] or null
    void *y;                 // [M, OUT]
    float *part;             // split-K partials [ksplit, ntiles, BM, 256] (ksplit > 1)
    int32_t M, OUT, K, group, y_dtype, ksplit, ks_per, n_codes;
    // affine groups per row (ceil(K / group): K may be padded past the last
    // group); group % 64 != 0: each lane finds its own group; group % 32 != 0:
    // a lane's 32 weights span two groups (one per 16)
    int32_t ngroups, g_lane, g16;
    int32_t tiles_x, tiles_y;   // the whole tile grid
    int32_t t0, ntiles;         // this launch: tiles [t0, t0 + ntiles) of the order
    int32_t tiles_per_xcd;      // of this launch
    int32_t vec_out;         // 16-bit y, 16-byte aligned rows, no split: LDS-transposed stores
    // Grouped (expert) launches: output rows are the sorted assignment list,
    // expert e owning rows [seg[e], seg[e+1]); X row of output row r is
    // rows[r] (rows null: r) of x_rows; output columns [0, out_split) come
    // from bank 0 (idx .. sc_val above), [out_split, OUT) from bank 1; each
    // bank stacks its experts at the strides below (elements of each array).
    const int32_t *rows;
    const int32_t *seg;
    int32_t n_exp, out_split, x_rows, grp_tiles_x, grp_per_xcd;
    int64_t idx_es, cb_es, ga_es, scp_es;
    const uint8_t *idx1;
    const float *cb1;
    const float2 *ga1;
    const int32_t *sc_ptr1;
    const uint32_t *sc_key1;
    const float *sc_val1;
};

// Row tile rt of a grouped launch: the expert e whose segment holds it, its
// first sorted row and the segment end.  Every wave computes it alike (lanes
// cover experts e, e + 64, ...; a wave scan of the per-expert tile counts).
__device__ __forceinline__ bool grouped_tile(const Args &g, int bm, int rt, int &e, int &row0,
                                             int &rend) {
    const int lane = threadIdx.x & 63;
    int base = 0;
    for (int c0 = 0; c0 < g.n_exp; c0 += 64) {
        const int ee = c0 + lane;
        const int a = ee < g.n_exp ? g.seg[ee] : 0;
        const int b = ee < g.n_exp ? g.seg[ee + 1] : 0;
        const int nt = (b - a + bm - 1) / bm;
        // inclusive scan of nt over the wave by DPP (row_shr 1, 2, 4, 8 within
        // rows, then row_bcast:15 / :31 across them): no LDS round trips
        int inc = nt;
        inc += __builtin_amdgcn_update_dpp(0, inc, 0x111, 0xf, 0xf, false);
        inc += __builtin_amdgcn_update_dpp(0, inc, 0x112, 0xf, 0xf, false);
        inc += __builtin_amdgcn_update_dpp(0, inc, 0x114, 0xf, 0xf, false);
        inc += __builtin_amdgcn_update_dpp(0, inc, 0x118, 0xf, 0xf, false);
        inc += __builtin_amdgcn_update_dpp(0, inc, 0x142, 0xa, 0xf, false);
        inc += __builtin_amdgcn_update_dpp(0, inc, 0x143, 0xc, 0xf, false);
        const int tot = __builtin_amdgcn_readlane(inc, 63);
        if (rt < base + tot) {
            const unsigned long long m = __ballot(base + inc > rt);
            const int L = __builtin_amdgcn_readfirstlane(__builtin_ctzll(m));
            // wave-uniform results, in scalar registers (they form buffer bases)
            e = c0 + L;
            row0 = __builtin_amdgcn_readlane(a, L) + (rt - base - __builtin_amdgcn_readlane(inc - nt, L)) * bm;
            rend = __builtin_amdgcn_readlane(b, L);
            return true;
        }
        base += tot;
    }
    return false;
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

template <bool BF16>
__device__ __forceinline__ uint32_t to16(float v) { return pack2<BF16>(v, 0.f) & 0xffffu; }

// Element offset of 16-byte chunk c (0..7) of LDS row r (64 elements, 128 B).
// gfx950's LDS has 64 banks and serves 16 lanes of a 16-byte access per
// clock: two consecutive rows fill the 64 banks, so the chunk is XORed with
// (r / 2) % 8 -- any 16 consecutive rows then map one chunk index to 16
// distinct (row parity, slot) pairs, conflict-free (XOR with r % 8 leaves
// rows r and r + 8 on the same banks: measured 155 vs 220 B/clk per CU).
__device__ __forceinline__ int swz(int r, int c) { return r * kBK + ((c ^ ((r >> 1) & 7)) << 3); }

// Tile order: blocks are dealt round-robin to the XCDs (block b runs on XCD
// b % 8); XCD x takes the contiguous run [x * per, (x + 1) * per) of an order
// that walks groups of kGroupRows row tiles column by column, so the blocks
// one XCD runs together share X row tiles and W column tiles in its L2.
__device__ __forceinline__ void order_tile(int t, int tiles_x, int tiles_y, int &tx, int &ty) {
    const int grp = t / (kGroupRows * tiles_x);
    const int r0 = grp * kGroupRows;
    const int gr = min(kGroupRows, tiles_y - r0);
    const int w = t - grp * kGroupRows * tiles_x;
    tx = w / gr;
    ty = r0 + w % gr;
}

// Block b of a launch over tiles [t0, t0 + ntiles): tile index tl within the
// launch and its grid position (false for the padding blocks).
__device__ __forceinline__ bool tile_of(const Args &g, int b, int &tl, int &tx, int &ty) {
    tl = (b % kXcds) * g.tiles_per_xcd + b / kXcds;
    if (tl >= g.ntiles) return false;
    order_tile(g.t0 + tl, g.tiles_x, g.tiles_y, tx, ty);
    return true;
}

// NJ: 32-column subtiles per wave (2: four waves of 64 columns, one wave per
// SIMD; 1: eight waves of 32 columns, two waves per SIMD).
template <int NJ>
struct BVec { typedef u32x32 type; };
template <>
struct BVec<1> { typedef u32x16 type; };

// Index formats (HXQ_FMT_*): index bytes per 32 weights (one lane's share of
// a row per K step) and whether the lookup table is a pair codebook.
__host__ __device__ constexpr int fmt_b32(int f) {
    return f == HXQ_FMT_SCALAR_U16 ? 64 : (f == HXQ_FMT_VQ2_P12 || f == HXQ_FMT_AF6) ? 24 : 32;
}

// Activation types: XT 0 = fp16, 1 = bf16 (v_mfma_f32_32x32x16_{f16,bf16},
// B packed as 16-bit pairs), 2 = fp32 (v_mfma_f32_32x32x2_f32, fp32 B: the
// fp32 path keeps fp32 arithmetic end to end).
// GM, the affine group layout: 0 group % 64 == 0 (one group per K step);
// 1 group % 32 == 0 (each lane finds its own group); 2 group % 16 == 0 (a
// lane's 32 weights span two groups: a second set of factors per row).  The
// per-lane forms cost registers, so the common layout keeps its own build.
template <int BM, int XT, bool AFFINE, int NJ, int FMT, bool GRP = false, int GM = 0>
// 64-row tiles (80 KB of LDS) run two blocks per CU: four waves per SIMD
__global__ __launch_bounds__(kBN / (32 * NJ) * 64, BM == 64 ? 4 : 1) void prefill_kernel(const Args g) {
    constexpr bool F32 = XT == 2;
    constexpr bool BF16 = XT == 1;
    static_assert(!F32 || (NJ == 1 && BM == 128), "fp32 activations: 128-row tiles, NJ = 1");
    constexpr int kThreads = kBN / (32 * NJ) * 64;
    constexpr int TM = BM / 32;           // accumulator tiles along M per wave
    constexpr int XB = F32 ? 4 : 2;       // bytes per X element
    constexpr int XCH = kBK * XB / 16;    // 16-byte chunks per X row and step
    constexpr int XP = BM * XCH / kThreads; // 16-byte X chunks per thread per step
    // B operand registers: 16-bit pairs (16 per 32 columns) or fp32 (32)
    typedef typename std::conditional<F32, u32x32, typename BVec<NJ>::type>::type BV;
    constexpr int B32 = fmt_b32(FMT);     // index bytes per lane, row and step
    constexpr int NQ = B32 == 64 ? 4 : 2; // 16-byte (12-byte for 24) index loads per row
    constexpr bool PAIR = FMT == HXQ_FMT_VQ2_U16 || FMT == HXQ_FMT_VQ2_P12;
    // uint8: 256 entries x 64 replicas; uint16 scalar: 4096 floats; pairs:
    // 4096 float2; 6-bit levels: no table (the region is sized for the largest)
    constexpr int kTblBytes = 256 * kNrep * 4;
    constexpr int kABytes = BM * kBK * XB;
    // the table first, so it sits at LDS address 0 (lookups need no base add)
    __shared__ __attribute__((aligned(16))) char smem[kTblBytes + 2 * kABytes];
    float *tbl = reinterpret_cast<float *>(smem);
    uint16_t *sA0 = reinterpret_cast<uint16_t *>(smem + kTblBytes);
    float *sAf0 = reinterpret_cast<float *>(smem + kTblBytes);

    int tl, tx, ty = 0;
    // this block's rows, their bound, and its weight bank (output columns
    // [wbase, wbase + wout) are rows [0, wout) of the bank's matrix)
    int r0, mlim, wbase = 0, wout = g.OUT;
    const uint8_t *gidx = g.idx;
    const float *gcb = g.cb;
    const float2 *gga = g.ga;
    const int32_t *gscp = g.sc_ptr;
    const uint32_t *gkey = g.sc_key;
    const float *gval = g.sc_val;
    if constexpr (GRP) {
        // row tile rt runs on XCD rt % 8 with all its column tiles (they share
        // its X rows in that XCD's L2); blocks are dispatched in order, so the
        // real tiles (row tiles below the routing's count) go first on every XCD
        const int j = blockIdx.x / kXcds;
        const int rt = static_cast<int>(blockIdx.x % kXcds) + kXcds * (j / g.grp_tiles_x);
        tx = j % g.grp_tiles_x;
        tl = rt * g.grp_tiles_x + tx;
        int e, row0, rend;
        if (!grouped_tile(g, BM, rt, e, row0, rend)) return;  // block-uniform
        r0 = row0;
        mlim = rend;
        const bool b1 = tx * kBN >= g.out_split;
        wbase = b1 ? g.out_split : 0;
        wout = b1 ? g.OUT - g.out_split : g.out_split;
        gidx = (b1 ? g.idx1 : g.idx) + e * g.idx_es;
        gcb = (b1 ? g.cb1 : g.cb) + e * g.cb_es;
        const float2 *ga = b1 ? g.ga1 : g.ga;
        gga = ga ? ga + e * g.ga_es : nullptr;
        const int32_t *sp = b1 ? g.sc_ptr1 : g.sc_ptr;
        gscp = sp ? sp + e * g.scp_es : nullptr;
        gkey = b1 ? g.sc_key1 : g.sc_key;
        gval = b1 ? g.sc_val1 : g.sc_val;
    } else {
        if (!tile_of(g, blockIdx.x, tl, tx, ty)) return;  // block-uniform
        r0 = ty * BM;
        mlim = g.M;
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ml = lane & 31, hh = lane >> 5;
    const int K = g.K;
    const int n0 = tx * kBN;
    const int nw = n0 + 32 * NJ * wave;      // first output column of this wave
    const int nwr = nw - wbase;              // its first row of the bank's matrix
    const int kb = blockIdx.y * g.ks_per;    // first K step of this block's range
    const int nk = min(K / kBK - kb, g.ks_per);
    constexpr uint32_t kOob = 0x80000000u;

    if (lds_offset_of(tbl) != 0) return;  // never taken: no other LDS in this kernel

    // ---- global sources ----------------------------------------------------------
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, (int64_t)(GRP ? g.x_rows : g.M) * K * XB);
    const int64_t row_bytes = (int64_t)K / 32 * B32;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(gidx, (int64_t)wout * row_bytes);
    const int ngroups = AFFINE ? g.ngroups : 1;
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(gga, AFFINE ? (int64_t)ngroups * wout * 8 : 0);
    // X: thread t copies chunk t % XCH of rows t / XCH + (threads / XCH) p
    const int xc = tid % XCH;
    uint32_t x_off[XP];
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        const int r = r0 + tid / XCH + (kThreads / XCH) * p;
        const int xrow = GRP && g.rows && r < mlim ? g.rows[r] : r;
        x_off[p] = r < mlim ? static_cast<uint32_t>((xrow * K + xc * (16 / XB)) * XB) : kOob;
    }
    // W rows of this lane: nw + 32j + ml
    uint32_t q_off[NJ];
    uint32_t a_off[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = nwr + 32 * j + ml;
        q_off[j] = n < wout ? static_cast<uint32_t>(n * row_bytes + B32 * hh) : kOob;
        a_off[j] = n < wout ? static_cast<uint32_t>(n * 8) : kOob;
    }

    // ---- sidecar: the entries of each K step, one per lane ----------------------
    // sc_ptr[G * nsteps + t] is the first entry of 64-row group G whose column
    // lies in K step t or later (the groups' lists are concatenated, so the
    // pointer one past a group's last step starts the next group).  Per step,
    // a wave loads 64 entries from that pointer: those before the step's end
    // column are the step's.  Pointers are loaded two steps before their
    // entries and entries one step before their use, all unconditionally (the
    // loads past a range read 0 and are masked when used), so that no wait
    // on a fresh load enters the pipeline.  Steps with more than 64 entries
    // in a group read the rest directly (correct, slower).
    const bool has_sc = gscp != nullptr && nwr < wout;
    const int nsteps = K / kBK;
    const int sgrp = nwr >> 6;
    const int sp0 = sgrp * nsteps + kb;  // pointer of this block's first step
    const int e_hi = has_sc ? gscp[(sgrp + 1) * nsteps] : 0;  // end of the group's list
    const __amdgpu_buffer_rsrc_t pr =
        make_rsrc(gscp, has_sc ? int64_t{4} * ((wout + 63) / 64 * nsteps + 1) : 0);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(gkey, int64_t{4} * e_hi);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(gval, int64_t{4} * e_hi);
    // this wave's rows within its 64-row sidecar group: [rlo, rlo + 32 NJ)
    const uint32_t rlo = static_cast<uint32_t>(nwr & 63);
    uint32_t ps[2];  // pointer of step t, loaded by load_step(t - 2) (buffer t & 1)
    uint32_t sk[2];  // keys and values of step t (buffer t & 1)
    float sv[2];
    int sb[2];       // the list index of lane 0's entry in sk/sv
    auto load_ptr = [&](int t, int buf) {
        ps[buf] = __builtin_amdgcn_raw_buffer_load_b32(
            pr, (has_sc && t < nk) ? static_cast<uint32_t>(sp0 + t) * 4u : kOob, 0, 0);
    };
    auto load_entries = [&](int t, int buf) {
        sb[buf] = __builtin_amdgcn_readfirstlane(static_cast<int>(ps[buf]));
        const uint32_t o = (has_sc && t < nk) ? static_cast<uint32_t>(sb[buf] + lane) * 4u : kOob;
        sk[buf] = __builtin_amdgcn_raw_buffer_load_b32(kr, o, 0, 0);
        sv[buf] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vr, o, 0, 0));
        load_ptr(t + 2, buf);
    };

    u32x4 xv[XP];      // X of the next step, on its way to LDS
    u32x4 qv[2][NQ * NJ]; // index bytes of row j: qv[.][NQ j .. NQ j + NQ)
    float2 av[2][NJ];     // {scale, offset} per j (weights 0..15 of the lane's 32)
    constexpr bool G16 = GM == 2;
    float2 av2[G16 ? 2 : 1][NJ];  // GM 2: ... of weights 16..31
    auto load_x = [&](int s) {
        const bool live = s < nk;
        const uint32_t k0 = static_cast<uint32_t>((kb + (live ? s : 0)) * kBK);
#pragma unroll
        for (int p = 0; p < XP; ++p)
            xv[p] = buf_load16(xr, (x_off[p] == kOob || !live) ? kOob : x_off[p] + k0 * XB);
    };
    auto load_step = [&](int s, int buf) {
        const bool live = s < nk;
        const uint32_t k0 = static_cast<uint32_t>((kb + (live ? s : 0)) * kBK);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const uint32_t o = (q_off[j] == kOob || !live) ? kOob : q_off[j] + k0 / 32u * B32;
#pragma unroll
            for (int h = 0; h < NQ; ++h) {
                if constexpr (B32 == 24) {  // two 12-byte loads
                    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
                    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(qr, o == kOob ? kOob : o + 12u * h, 0, 0);
                    qv[buf][NQ * j + h] = u32x4{v[0], v[1], v[2], 0u};
                } else {
                    qv[buf][NQ * j + h] = buf_load16(qr, o == kOob ? kOob : o + 16u * h);
                }
            }
        }
        if constexpr (AFFINE) {
            // the lane's weights are physical k0 + 32 hh + [0, 32): one group
            // for the whole step when group % 64 == 0 (uniform), else per lane
            const uint32_t G = static_cast<uint32_t>(g.group);
            const uint32_t row8 = static_cast<uint32_t>(wout) * 8u;
            const uint32_t ga = GM == 0 ? k0 / G : (k0 + 32u * hh) / G;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const uint32_t o = (a_off[j] == kOob || !live) ? kOob : a_off[j] + ga * row8;
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(ar, o, 0, 0);
                av[buf][j] = make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
            }
            if constexpr (G16) {
                const uint32_t gb = (k0 + 32u * hh + 16u) / G;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const uint32_t o = (a_off[j] == kOob || !live) ? kOob : a_off[j] + gb * row8;
                    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(ar, o, 0, 0);
                    av2[buf][j] = make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
                }
            }
        }
        load_entries(s, buf);
    };
    // rows r and r + (threads / XCH) p share the swizzle: one base address,
    // the other rows at immediate offsets.  16-bit rows (128 B, 8 chunks):
    // chunk ^ (r / 2) % 8; fp32 rows (256 B = the 64 banks, 16 chunks):
    // chunk ^ r % 16, so 16 lanes reading one logical chunk of 16 rows hit
    // 16 distinct chunks
    const int x_lds = F32 ? (tid / XCH) * kBK + ((xc ^ ((tid / XCH) & 15)) << 2) : swz(tid >> 3, xc);
    auto store_x = [&](int buf) {
        if constexpr (F32) {
            float *sA = sAf0 + buf * (BM * kBK) + x_lds;
#pragma unroll
            for (int p = 0; p < XP; ++p)
                *reinterpret_cast<u32x4 *>(sA + (kThreads / XCH) * p * kBK) = xv[p];
        } else {
            uint16_t *sA = sA0 + buf * (BM * kBK) + x_lds;
#pragma unroll
            for (int p = 0; p < XP; ++p)
                *reinterpret_cast<u32x4 *>(sA + (kThreads / XCH) * p * kBK) = xv[p];
        }
    };

    // ---- lookup table ------------------------------------------------------------
    if constexpr (FMT == HXQ_FMT_SCALAR) {
        // 64 replicas, conflict-free float4 writes
#pragma unroll
        for (int q = 0; q < 4096 / kThreads; ++q) {
            const int slot = tid + kThreads * q;  // float4 slot: entry slot / 16
            const float c = gcb[slot >> 4];
            *reinterpret_cast<float4 *>(tbl + 4 * slot) = make_float4(c, c, c, c);
        }
    } else if constexpr (FMT == HXQ_FMT_SCALAR_U16) {
        for (int j = tid; j < kPairCodes; j += kThreads) tbl[j] = j < g.n_codes ? gcb[j] : 0.f;
    } else if constexpr (PAIR) {
        float2 *t2 = reinterpret_cast<float2 *>(tbl);
        for (int j = tid; j < kPairCodes; j += kThreads)
            t2[j] = j < g.n_codes ? make_float2(gcb[2 * j], gcb[2 * j + 1]) : make_float2(0.f, 0.f);
    }

    // ---- dequantise B into operand registers, one k substep at a time ----------
    // b[16j + 4s + t] holds bf16 pairs (weights 8s + 2t, 8s + 2t + 1 of the
    // lane's 32) of W row nw + 32j + ml: the B operand of substep s, subtile j
    const uint32_t lane_off = static_cast<uint32_t>(lane) * 4u;
    // bits [bit, bit + width) of the little-endian 192-bit stream of a 24-byte chunk
    auto field24 = [&](const u32x4 &q0, const u32x4 &q1, int bit, int width) -> uint32_t {
        const uint32_t d[6] = {q0[0], q0[1], q0[2], q1[0], q1[1], q1[2]};
        const int wi = bit >> 5, sh = bit & 31;
        const uint32_t v = sh + width <= 32 ? d[wi] >> sh : __builtin_amdgcn_alignbit(d[wi + 1], d[wi], sh);
        return v & ((1u << width) - 1u);
    };
    auto dequant_sub = [&](int buf, int s, BV &b) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            // substep s holds weights 8s .. 8s+7: the first 16 for s < 2
            const float sc = AFFINE ? (G16 && s >= 2 ? av2[G16 ? buf : 0][j].x : av[buf][j].x) : 1.f;
            const float of = AFFINE ? (G16 && s >= 2 ? av2[G16 ? buf : 0][j].y : av[buf][j].y) : 0.f;
            if constexpr (FMT == HXQ_FMT_SCALAR_U16) {
                // weights 8s .. 8s+7: the 16 bytes of load s, eight uint16 indices
                const u32x4 q = qv[buf][NQ * j + s];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float v0 = tbl[q[t] & (kPairCodes - 1u)];
                    float v1 = tbl[(q[t] >> 16) & (kPairCodes - 1u)];
                    if constexpr (AFFINE) {
                        v0 = affine_fma(v0, sc, of);
                        v1 = affine_fma(v1, sc, of);
                    }
                    b[16 * j + 4 * s + t] = pack2<BF16>(v0, v1);
                }
                continue;
            } else if constexpr (FMT == HXQ_FMT_VQ2_U16) {
                // pairs 4s .. 4s+3: dwords 2s, 2s+1 of the 32 bytes
                const float2 *t2 = reinterpret_cast<const float2 *>(tbl);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t w = qv[buf][NQ * j + (s >> 1)][2 * (s & 1) + (t >> 1)];
                    const float2 c = t2[(w >> (16 * (t & 1))) & (kPairCodes - 1u)];
                    b[16 * j + 4 * s + t] = pack2<BF16>(c.x, c.y);
                }
                continue;
            } else if constexpr (FMT == HXQ_FMT_VQ2_P12) {
                // pairs 4s .. 4s+3: 12-bit fields at bit 48s + 12t
                const float2 *t2 = reinterpret_cast<const float2 *>(tbl);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float2 c = t2[field24(qv[buf][NQ * j], qv[buf][NQ * j + 1], 48 * s + 12 * t, 12)];
                    b[16 * j + 4 * s + t] = pack2<BF16>(c.x, c.y);
                }
                continue;
            } else if constexpr (FMT == HXQ_FMT_AF6) {
                // levels 8s .. 8s+7: 6-bit fields at bit 48s + 6f
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float v0 = static_cast<float>(field24(qv[buf][NQ * j], qv[buf][NQ * j + 1], 48 * s + 12 * t, 6));
                    const float v1 = static_cast<float>(field24(qv[buf][NQ * j], qv[buf][NQ * j + 1], 48 * s + 12 * t + 6, 6));
                    b[16 * j + 4 * s + t] = pack2<BF16>(affine_fma(v0, sc, of), affine_fma(v1, sc, of));
                }
                continue;
            }
#pragma unroll
            for (int dd = 0; dd < 2; ++dd) {
                const int d = 2 * s + dd;  // index dword (4 weights)
                const uint32_t w = qv[buf][2 * j + (d >> 2)][d & 3];
                float v0 = tbl_lookup0<kNrep, 0>(lane_off, w);
                float v1 = tbl_lookup0<kNrep, 1>(lane_off, w);
                float v2 = tbl_lookup0<kNrep, 2>(lane_off, w);
                float v3 = tbl_lookup0<kNrep, 3>(lane_off, w);
                if constexpr (AFFINE) {
                    v0 = affine_fma(v0, sc, of);
                    v1 = affine_fma(v1, sc, of);
                    v2 = affine_fma(v2, sc, of);
                    v3 = affine_fma(v3, sc, of);
                }
                b[16 * j + 2 * d] = pack2<BF16>(v0, v1);
                b[16 * j + 2 * d + 1] = pack2<BF16>(v2, v3);
            }
        }
    };
    // fp32 B: b[w] holds weight w of the lane's 32 (row nw + ml); group q
    // (weights 4q .. 4q+3) feeds MFMA substeps 4q .. 4q+3
    auto dequant_f32 = [&](int buf, int q, BV &b) {
        if constexpr (F32) {
        const float sc = AFFINE ? (G16 && q >= 4 ? av2[G16 ? buf : 0][0].x : av[buf][0].x) : 1.f;
        const float of = AFFINE ? (G16 && q >= 4 ? av2[G16 ? buf : 0][0].y : av[buf][0].y) : 0.f;
        float v[4];
        if constexpr (FMT == HXQ_FMT_SCALAR) {
            const uint32_t w = qv[buf][q >> 2][q & 3];
            v[0] = tbl_lookup0<kNrep, 0>(lane_off, w);
            v[1] = tbl_lookup0<kNrep, 1>(lane_off, w);
            v[2] = tbl_lookup0<kNrep, 2>(lane_off, w);
            v[3] = tbl_lookup0<kNrep, 3>(lane_off, w);
        } else if constexpr (FMT == HXQ_FMT_SCALAR_U16) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t w = qv[buf][(2 * q + t) >> 2][(2 * q + t) & 3];
                v[2 * t] = tbl[w & (kPairCodes - 1u)];
                v[2 * t + 1] = tbl[(w >> 16) & (kPairCodes - 1u)];
            }
        } else if constexpr (FMT == HXQ_FMT_VQ2_U16) {
            const float2 *t2 = reinterpret_cast<const float2 *>(tbl);
            const uint32_t w = qv[buf][q >> 2][q & 3];
            const float2 c0 = t2[w & (kPairCodes - 1u)];
            const float2 c1 = t2[(w >> 16) & (kPairCodes - 1u)];
            v[0] = c0.x; v[1] = c0.y; v[2] = c1.x; v[3] = c1.y;
        } else if constexpr (FMT == HXQ_FMT_VQ2_P12) {
            const float2 *t2 = reinterpret_cast<const float2 *>(tbl);
            const float2 c0 = t2[field24(qv[buf][0], qv[buf][1], 24 * q, 12)];
            const float2 c1 = t2[field24(qv[buf][0], qv[buf][1], 24 * q + 12, 12)];
            v[0] = c0.x; v[1] = c0.y; v[2] = c1.x; v[3] = c1.y;
        } else {  // 6-bit levels
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = static_cast<float>(field24(qv[buf][0], qv[buf][1], 24 * q + 6 * t, 6));
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) b[4 * q + t] = __float_as_uint(AFFINE ? affine_exact(v[t], sc, of) : v[t]);
        }
    };
    // Replace sidecar entries in b: the lanes set in m hold (key, value) pairs
    // of step columns [k1, k1 + 64) and this wave's rows.
    auto apply = [&](uint32_t key_v, float val_v, unsigned long long m, uint32_t k1, BV &b) {
        while (m) {
            const int src = __builtin_ctzll(m);
            m &= m - 1;
            const uint32_t key = __builtin_amdgcn_readlane(key_v, src);
            const float val = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(val_v), src));
            const uint32_t col = (key >> 6) - k1;  // 0..63
            const uint32_t row = (key & 63u) - rlo; // row within this wave
            const int owner = static_cast<int>((row & 31u) + 32u * (col >> 5));
            if constexpr (F32) {
                const int reg = __builtin_amdgcn_readfirstlane(static_cast<int>(col & 31u));
                b[reg] = lane == owner ? __float_as_uint(val) : b[reg];
            } else {
                const int reg = __builtin_amdgcn_readfirstlane(static_cast<int>(16u * (row >> 5) + ((col & 31u) >> 1)));
                const uint32_t v16 = to16<BF16>(val);
                const uint32_t hi = col & 1u;
                const uint32_t old = b[reg];
                const uint32_t upd = hi ? ((old & 0xffffu) | (v16 << 16)) : ((old & 0xffff0000u) | v16);
                b[reg] = lane == owner ? upd : old;
            }
        }
    };
    // The sidecar entries of step s (buffer buf) into b.
    auto patch = [&](int s, int buf, BV &b) {
        if (!has_sc || s >= nk) return;  // (the pipeline's last refill is past the range)
        const uint32_t k1 = static_cast<uint32_t>((kb + s) * kBK);
        const uint32_t khi = (k1 + kBK) << 6;
        const uint32_t nrow = static_cast<uint32_t>(32 * NJ);
        const uint32_t key = sk[buf];
        apply(key, sv[buf], __ballot(sb[buf] + lane < e_hi && key < khi && (key & 63u) - rlo < nrow), k1, b);
        if (sb[buf] + 64 < e_hi && __builtin_amdgcn_readlane(key, 63) < khi) {
            // more than 64 entries in this step: the rest straight from the list
            for (int ob = sb[buf] + 64; ob < e_hi; ob += 64) {
                const int e = ob + lane;
                const uint32_t k2 = e < e_hi ? gkey[e] : 0xffffffffu;
                const float v2 = e < e_hi ? gval[e] : 0.f;
                apply(k2, v2, __ballot(k2 < khi && (k2 & 63u) - rlo < nrow), k1, b);
                if (__builtin_amdgcn_readlane(k2, 63) >= khi) break;
            }
        }
    };

    // ---- accumulators -----------------------------------------------------------
    f32x16 acc[TM][NJ];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // One step: the MFMAs of B(k) (in b, A from LDS buffer abuf), each k
    // substep's operand registers refilled with B(k+1) from index buffer qbuf
    // as soon as its MFMAs are issued.  The A rows 32i + ml of one substep
    // share a swizzle: one base address per substep, rows at immediate offsets.
    const int a_sw = (ml >> 1) & 7;
    auto mfma_step = [&](int abuf, int qbuf, BV &b) {
        if constexpr (F32) {
            // 8 groups of 4 k substeps: one 16-byte A read per row tile (the 4
            // k of the group), 4 MFMAs per row tile, then B(k+1) of the group
            const float *sA = sAf0 + abuf * (BM * kBK) + ml * kBK;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float *as = sA + (((8 * hh + q) ^ (ml & 15)) << 2);
                float4 a[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const float4 *>(as + 32 * i * kBK);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float bv = __uint_as_float(b[4 * q + e]);
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const float av_ = e == 0 ? a[i].x : e == 1 ? a[i].y : e == 2 ? a[i].z : a[i].w;
                        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av_, bv, acc[i][0], 0, 0, 0);
                    }
                }
                if (qbuf >= 0) dequant_f32(qbuf, q, b);
            }
            return;
        }
        const uint16_t *sA = sA0 + abuf * (BM * kBK) + ml * kBK;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u32x4 bj[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                bj[j] = u32x4{b[16 * j + 4 * s], b[16 * j + 4 * s + 1], b[16 * j + 4 * s + 2],
                              b[16 * j + 4 * s + 3]};
            const uint16_t *as = sA + (((4 * hh + s) ^ a_sw) << 3);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const u32x4 a = *reinterpret_cast<const u32x4 *>(as + 32 * i * kBK);
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    if constexpr (BF16)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, bj[j]), acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, bj[j]), acc[i][j], 0, 0, 0);
                }
            }
            if (qbuf >= 0) dequant_sub(qbuf, s, b);
        }
    };

    // ---- pipeline ---------------------------------------------------------------
    // index, affine and sidecar loads two steps ahead; X one step ahead, its
    // registers written to LDS at the end of the step before its use (16 fewer
    // live registers than a second X buffer; X rows are mostly L2 hits); B of
    // step s+1 replaces B of step s substep by substep; one barrier per step.
    load_ptr(0, 0);
    load_ptr(1, 1);
    load_x(0);
    load_step(0, 0);
    load_step(1, 1);
    store_x(0);                 // waits for X(0)
    load_x(1);
    __syncthreads();            // table and A(0) visible
    BV b;
    if constexpr (F32) {
#pragma unroll
        for (int q = 0; q < 8; ++q) dequant_f32(0, q, b);  // B(0)
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) dequant_sub(0, s, b);  // B(0)
    }
    patch(0, 0, b);
    load_step(2, 0);
    int ks = 0;
    for (; ks + 1 < nk; ks += 2) {
        // step ks: A in LDS buffer 0, B(ks) in b, idx(ks+1) in buffer 1, X(ks+1) in xv
        mfma_step(0, 1, b);     // b <- B(ks+1)
        patch(ks + 1, 1, b);
        load_step(ks + 3, 1);
        store_x(1);
        load_x(ks + 2);
        lds_barrier();
        // step ks + 1: A in buffer 1, idx(ks+2) in buffer 0, X(ks+2) in xv
        mfma_step(1, 0, b);     // b <- B(ks+2)
        patch(ks + 2, 0, b);
        load_step(ks + 4, 0);
        store_x(0);
        load_x(ks + 3);
        lds_barrier();
    }
    if (ks < nk) mfma_step(0, -1, b);  // odd step count: the last step (A in buffer 0)

    // ---- epilogue: acc[i][j][r] = C[32i + 8(r/4) + 4h + r%4][nw + 32j + ml] ----
    const bool split = g.ksplit > 1;
    if (g.vec_out) {
        // 16-bit outputs through LDS: each wave transposes its BM x 64 tile in a
        // private region (the A buffers and the table are dead now), then
        // stores rows in 16-byte pieces (eight lanes cover a 128-byte row run)
        __syncthreads();
        constexpr int CW = 32 * NJ;  // columns per wave
        uint16_t *cw = reinterpret_cast<uint16_t *>(smem) + wave * (BM * CW);
        // 16-byte chunk q of row mr: 128-byte rows (NJ = 2) take the A-tile
        // swizzle; 64-byte rows (NJ = 1) are conflict-free as they are
        auto cofs = [&](int mr, int q) { return NJ == 2 ? swz(mr, q) : mr * CW + 8 * q; };
        const bool obf = g.y_dtype == HXQ_BF16;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = 32 * j + ml;
            const float bv = (g.bias && nw + c < g.OUT) ? g.bias[nw + c] : 0.f;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int mr = 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
                    const float v = acc[i][j][r] + bv;
                    cw[cofs(mr, c >> 3) + (c & 7)] =
                        static_cast<uint16_t>(obf ? to16<true>(v) : to16<false>(v));
                }
        }
        // same-wave LDS traffic is ordered: no barrier between the two passes
        uint16_t *yb = static_cast<uint16_t *>(g.y);
        constexpr int QPR = CW / 8;  // 16-byte chunks per row
#pragma unroll 4
        for (int t = 0; t < BM * QPR / 64; ++t) {
            const int id = t * 64 + lane;
            const int mr = id / QPR, q = id % QPR;
            const int m = r0 + mr, n = nw + 8 * q;
            const u32x4 v = *reinterpret_cast<const u32x4 *>(cw + cofs(mr, q));
            if (m < mlim && n < g.OUT)
                *reinterpret_cast<u32x4 *>(yb + (int64_t)m * g.OUT + n) = v;
        }
        return;
    }
    if (split) {
        // this range's partial tile, compact [BM][256]; the reduce adds the
        // ranges in order and maps the tile back to Y
        float *dst = g.part + ((int64_t)blockIdx.y * g.ntiles + tl) * (BM * kBN);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = nw - n0 + 32 * j + ml;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    dst[(32 * i + 8 * (r >> 2) + 4 * hh + (r & 3)) * kBN + c] = acc[i][j][r];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = nw + 32 * j + ml;
        if (n >= g.OUT) continue;
        const float bv = g.bias ? g.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = r0 + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
                if (m >= mlim) continue;
                const int64_t o = (int64_t)m * g.OUT + n;
                const float v = acc[i][j][r] + bv;
                if (g.y_dtype == HXQ_F32) static_cast<float *>(g.y)[o] = v;
                else if (g.y_dtype == HXQ_BF16) static_cast<uint16_t *>(g.y)[o] = static_cast<uint16_t>(to16<true>(v));
                else static_cast<uint16_t *>(g.y)[o] = static_cast<uint16_t>(to16<false>(v));
            }
    }
}

// Ordered split-K reduction of a launch's compact partial tiles:
// y[m, n] = sum over ranges (in order) + bias, for the tiles' in-range elements.
// Four consecutive outputs of one tile row per thread: the ks partials of
// each are loaded together (16-byte loads, all requested before the first
// is used) and summed in range order, as one element at a time would; y
// takes 8- or 16-byte stores when vec (out % 4 == 0 and y 16-byte aligned),
// element stores at the edge of the matrix.
constexpr int kRedKs = 8;  // the plan splits K at most 8 ways
__global__ __launch_bounds__(256) void prefill_reduce_kernel(const float *__restrict__ part,
                                                             int32_t ksplit, int32_t ntiles,
                                                             int32_t t0, int32_t tiles_x,
                                                             int32_t tiles_y, int32_t bm,
                                                             int32_t M, int32_t out,
                                                             const float *bias, void *y,
                                                             int32_t y_dtype, int32_t vec) {
    const int64_t per = (int64_t)bm * kBN;
    const int64_t i = (blockIdx.x * 256ll + threadIdx.x) * 4;
    if (i >= per * ntiles) return;
    const int tl = static_cast<int>(i / per);
    const int e = static_cast<int>(i - (int64_t)tl * per);
    int tx, ty;
    order_tile(t0 + tl, tiles_x, tiles_y, tx, ty);
    const int m = ty * bm + e / kBN, n = tx * kBN + e % kBN;
    if (m >= M || n >= out) return;
    const int64_t stride = per * ntiles;
    float4 pv[kRedKs];
#pragma unroll
    for (int s = 0; s < kRedKs; ++s)
        if (s < ksplit) pv[s] = *reinterpret_cast<const float4 *>(part + s * stride + i);
    float v[4] = {pv[0].x, pv[0].y, pv[0].z, pv[0].w};
#pragma unroll
    for (int s = 1; s < kRedKs; ++s)
        if (s < ksplit) {
            v[0] += pv[s].x;
            v[1] += pv[s].y;
            v[2] += pv[s].z;
            v[3] += pv[s].w;
        }
    const int nv = min(4, out - n);
    if (bias)
        for (int j = 0; j < nv; ++j) v[j] += bias[n + j];
    const int64_t o = (int64_t)m * out + n;
    if (vec && nv == 4) {
        if (y_dtype == HXQ_F32) {
            *reinterpret_cast<float4 *>(static_cast<float *>(y) + o) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            const bool b16 = y_dtype == HXQ_BF16;
            auto h = [&](float x) { return static_cast<uint32_t>(b16 ? f32_to_bf16(x) : f32_to_f16(x)); };
            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + o) =
                make_uint2(h(v[0]) | (h(v[1]) << 16), h(v[2]) | (h(v[3]) << 16));
        }
        return;
    }
    for (int j = 0; j < nv; ++j) {
        if (y_dtype == HXQ_F32) static_cast<float *>(y)[o + j] = v[j];
        else if (y_dtype == HXQ_BF16) static_cast<uint16_t *>(y)[o + j] = f32_to_bf16(v[j]);
        else static_cast<uint16_t *>(y)[o + j] = f32_to_f16(v[j]);
    }
}

// One launch of the plan: tiles [t0, t0 + n) of the order, K split ks ways.
struct Launch {
    int t0, n, ks, ks_per;
};

struct Plan {
    int bm, tiles_x, tiles_y, nl;
    Launch l[2];
    int64_t ws_bytes;  // largest partial buffer of a split launch
};

// K split of a tile grid: when the tiles cover fewer than all CUs, up to 8
// ranges of >= 4 steps (fp32 partials + an ordered reduce).
static int split_of(int64_t tiles, int nk, int cus) {
    return tiles < cus ? static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({8, cus / tiles, nk / 4})))
                       : 1;
}

static Launch launch_of(int t0, int n, int ks, int nk) {
    Launch l{t0, n, 1, nk};
    if (ks >= 2) {
        l.ks_per = (nk + ks - 1) / ks;
        l.ks = (nk + l.ks_per - 1) / l.ks_per;
    }
    return l;
}

// Row tile 256 (half the dequantisation per flop of 128) when its tiles,
// times their K split, keep more than half the CUs busy; otherwise 128.
// Measured on config-2 shapes: kv (2 column tiles) takes 128 at M <= 2048,
// every other shape 256 down to M = 512.  One block runs per CU, so a grid
// of several rounds whose last round would fill under half the CUs runs
// that tail as a second launch with K split across the idle CUs.
// bm_max 128: formats whose 256-row kernel would not fit the register file.
Plan plan(int64_t m, int64_t out, int64_t in, int cus, int bm_max = 256) {
    Plan p{};
    p.tiles_x = static_cast<int>((out + kBN - 1) / kBN);
    const int nk = static_cast<int>(in / kBK);
    const int64_t t256 = p.tiles_x * ((m + 255) / 256);
    p.bm = bm_max == 256 && t256 * split_of(t256, nk, cus) * 2 > cus ? 256 : 128;
    p.tiles_y = static_cast<int>((m + p.bm - 1) / p.bm);
    const int tiles = p.tiles_x * p.tiles_y;
    const int rem = tiles % cus;
    if (tiles < cus) {
        p.nl = 1;
        p.l[0] = launch_of(0, tiles, split_of(tiles, nk, cus), nk);
    } else if (rem > 0 && 2 * rem < cus && nk >= 8) {
        p.nl = 2;
        p.l[0] = launch_of(0, tiles - rem, 1, nk);
        p.l[1] = launch_of(tiles - rem, rem, split_of(rem, nk, cus), nk);
    } else {
        p.nl = 1;
        p.l[0] = launch_of(0, tiles, 1, nk);
    }
    p.ws_bytes = 0;
    for (int i = 0; i < p.nl; ++i)
        if (p.l[i].ks > 1)
            p.ws_bytes = std::max<int64_t>(p.ws_bytes, int64_t{4} * p.l[i].ks * p.l[i].n * p.bm * kBN);
    return p;
}

bool grouped_ok(const hxq_expert_bank *b, int64_t out, int64_t in, int32_t group) {
    return b && b->indices && b->codebook && in % kBK == 0 && in < (int64_t{1} << 26) &&
           (!b->group_affine || (group >= kBK && group % kBK == 0 && in % group == 0)) &&
           (!b->sc_row_ptr || (b->sc_grp_ptr && b->sc_grp_key && b->sc_grp_val)) &&
           out * in < (int64_t{1} << 31) &&
           (!b->group_affine || (in / group) * out * 8 < (int64_t{1} << 31));
}

#ifndef GRP_BM64_MAX
#define GRP_BM64_MAX 96
#endif
int grouped_gemm(const GroupedReq &r, hipStream_t stream) {
    HXQ_REQUIRE(r.x && r.seg && r.bank0 && r.y, "x, expert_offsets, bank and y are required");
    HXQ_REQUIRE(r.x_dtype == HXQ_BF16 || r.x_dtype == HXQ_F16 || r.x_dtype == HXQ_F32,
                "x must be fp32, bf16 or fp16");
    HXQ_REQUIRE(r.y_dtype >= HXQ_F32 && r.y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(r.n_exp >= 1 && r.n_exp <= 256, "n_experts must be in 1..256");
    HXQ_REQUIRE(r.n_assign > 0 && r.x_rows > 0 && r.out0 > 0 && r.in > 0, "empty problem");
    HXQ_REQUIRE(r.rows || r.x_rows >= r.n_assign, "without sorted_rows x holds n_assign rows");
    HXQ_REQUIRE(grouped_ok(r.bank0, r.out0, r.in, r.group), "bank not eligible for the grouped kernel");
    HXQ_REQUIRE(!r.bank1 || (r.out1 > 0 && r.out0 % kBN == 0 && grouped_ok(r.bank1, r.out1, r.in, r.group) &&
                             (r.bank0->group_affine != nullptr) == (r.bank1->group_affine != nullptr)),
                "the second bank needs out0 % 256 == 0 and the same affine layout");
    const int64_t out = r.out0 + (r.bank1 ? r.out1 : 0);
    HXQ_REQUIRE(r.x_rows * r.in * (r.x_dtype == HXQ_F32 ? 4 : 2) < (int64_t{1} << 31) &&
                    r.n_assign * out * 4 < (int64_t{1} << 31),
                "problem too large for 32-bit offsets");
    HXQ_REQUIRE((reinterpret_cast<uintptr_t>(r.x) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(r.bank0->indices) & 15u) == 0 &&
                    (!r.bank1 || (reinterpret_cast<uintptr_t>(r.bank1->indices) & 15u) == 0),
                "x and indices must be 16-byte aligned");
    Args a{};
    a.x = static_cast<const uint16_t *>(r.x);
    a.y = r.y;
    a.M = static_cast<int32_t>(r.n_assign);
    a.OUT = static_cast<int32_t>(out);
    a.K = static_cast<int32_t>(r.in);
    const bool aff = r.bank0->group_affine != nullptr;
    a.group = aff ? r.group : kBK;
    a.ngroups = static_cast<int32_t>(r.in / a.group);
    a.y_dtype = r.y_dtype;
    a.ksplit = 1;
    a.ks_per = static_cast<int32_t>(r.in / kBK);
    a.n_codes = 256;
    a.rows = r.rows;
    a.seg = r.seg;
    a.n_exp = r.n_exp;
    a.out_split = static_cast<int32_t>(r.bank1 ? r.out0 : out);
    a.x_rows = static_cast<int32_t>(r.x_rows);
    // 16-bit outputs leave through the LDS-transposed 16-byte row stores
    a.vec_out = r.y_dtype != HXQ_F32 && out % 8 == 0 && (reinterpret_cast<uintptr_t>(r.y) & 15u) == 0;
    auto bank = [&](const hxq_expert_bank *b, const uint8_t *&idx, const float *&cb, const float2 *&ga,
                    const int32_t *&sp, const uint32_t *&key, const float *&val) {
        idx = b->indices;
        cb = b->codebook;
        ga = reinterpret_cast<const float2 *>(b->group_affine);
        sp = b->sc_row_ptr ? b->sc_grp_ptr : nullptr;
        key = b->sc_grp_key;
        val = b->sc_grp_val;
    };
    bank(r.bank0, a.idx, a.cb, a.ga, a.sc_ptr, a.sc_key, a.sc_val);
    if (r.bank1) bank(r.bank1, a.idx1, a.cb1, a.ga1, a.sc_ptr1, a.sc_key1, a.sc_val1);
    else bank(r.bank0, a.idx1, a.cb1, a.ga1, a.sc_ptr1, a.sc_key1, a.sc_val1);
    // both banks have the same per-expert shape (out0 == out1 when paired)
    const int64_t wo = r.out0;
    HXQ_REQUIRE(!r.bank1 || r.out1 == r.out0, "paired banks must have the same shape");
    a.idx_es = wo * r.in;
    a.cb_es = 256;
    a.ga_es = aff ? (r.in / a.group) * wo : 0;
    a.scp_es = (wo + 63) / 64 * (r.in / kBK) + 1;
    // 256-row tiles when the experts average more than 192 rows, 128 above 96, else 64
    // (fp32 activations: 128-row tiles always, the fp32 A tile doubles the LDS)
    const int64_t mean_rows = r.n_assign / r.n_exp;
    const bool f32 = r.x_dtype == HXQ_F32;
    const int bm = f32 ? 128 : mean_rows > 192 ? 256 : mean_rows > GRP_BM64_MAX ? 128 : 64;
    a.grp_tiles_x = static_cast<int32_t>((out + kBN - 1) / kBN);
    const int64_t row_tiles = (r.n_assign + bm - 1) / bm + r.n_exp;  // upper bound over any routing
    a.grp_per_xcd = static_cast<int32_t>((row_tiles + kXcds - 1) / kXcds * a.grp_tiles_x);
    const dim3 grid(static_cast<uint32_t>(a.grp_per_xcd) * kXcds);
    const bool bf16 = r.x_dtype == HXQ_BF16;
#define HXQ_PG_GRP(BM_, BF_, AF_) \
    hipLaunchKernelGGL((prefill_kernel<BM_, BF_, AF_, kNJ, HXQ_FMT_SCALAR, true>), grid, \
                       dim3(kBN / (32 * kNJ) * 64), 0, stream, a)
    if (f32) {
        if (aff) HXQ_PG_GRP(128, 2, true); else HXQ_PG_GRP(128, 2, false);
    } else if (bm == 256) {
        if (bf16) { if (aff) HXQ_PG_GRP(256, 1, true); else HXQ_PG_GRP(256, 1, false); }
        else { if (aff) HXQ_PG_GRP(256, 0, true); else HXQ_PG_GRP(256, 0, false); }
    } else if (bm == 64) {
        if (bf16) { if (aff) HXQ_PG_GRP(64, 1, true); else HXQ_PG_GRP(64, 1, false); }
        else { if (aff) HXQ_PG_GRP(64, 0, true); else HXQ_PG_GRP(64, 0, false); }
    } else {
        if (bf16) { if (aff) HXQ_PG_GRP(128, 1, true); else HXQ_PG_GRP(128, 1, false); }
        else { if (aff) HXQ_PG_GRP(128, 0, true); else HXQ_PG_GRP(128, 0, false); }
    }
#undef HXQ_PG_GRP
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

}  // namespace pg
}  // namespace hxq

using namespace hxq;

extern "C" int64_t hxq_prefill_gemm_workspace_bytes(int64_t m_rows, int64_t out_features,
                                                    int64_t in_features) {
    if (m_rows <= 0 || out_features <= 0 || in_features <= 0 || in_features % pg::kBK) return 0;
    // the largest over the row-tile heights a format may use
    const int cus = device_cu_count();
    return std::max(pg::plan(m_rows, out_features, in_features, cus).ws_bytes,
                    pg::plan(m_rows, out_features, in_features, cus, 128).ws_bytes);
}

extern "C" int hxq_prefill_gemm(const void *x, int32_t x_dtype, int32_t format,
                                const uint8_t *indices, const float *codebook, int32_t n_codes,
                                const float *group_affine, int32_t group_size,
                                const int32_t *sc_grp_ptr,
                                const uint32_t *sc_grp_key, const float *sc_grp_val,
                                const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                                int64_t out_features, int64_t in_features, void *workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(format >= HXQ_FMT_SCALAR && format <= HXQ_FMT_SCALAR_U16, "unknown index format");
    HXQ_REQUIRE(x && indices && y && (codebook || format == HXQ_FMT_AF6),
                "x, indices, codebook and y are required");
    HXQ_REQUIRE(x_dtype == HXQ_BF16 || x_dtype == HXQ_F16 || x_dtype == HXQ_F32,
                "x_dtype must be fp32, bf16 or fp16");
    HXQ_REQUIRE(format == HXQ_FMT_SCALAR || format == HXQ_FMT_AF6 ||
                    (n_codes >= 1 && n_codes <= kPairCodes),
                "uint16 and pair codebooks need 1..4096 entries");
    HXQ_REQUIRE(format != HXQ_FMT_AF6 || group_affine, "6-bit levels need the group affine");
    HXQ_REQUIRE(!(format == HXQ_FMT_VQ2_U16 || format == HXQ_FMT_VQ2_P12) || !group_affine,
                "pair codebooks take no group affine");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(m_rows > 0 && out_features > 0 && in_features > 0, "empty problem");
    HXQ_REQUIRE(in_features % pg::kBK == 0, "in_features must be a multiple of 64");
    HXQ_REQUIRE(in_features < (int64_t{1} << 26), "in_features must be below 2^26");
    HXQ_REQUIRE(m_rows * in_features * (x_dtype == HXQ_F32 ? 4 : 2) < (int64_t{1} << 31) &&
                    out_features * (in_features / 32 * pg::fmt_b32(format)) < (int64_t{1} << 31),
                "problem too large for 32-bit offsets");
    HXQ_REQUIRE(!group_affine || (group_size >= 16 && group_size % 16 == 0),
                "group_size must be a positive multiple of 16");
    const int64_t ngroups = group_affine ? (in_features + group_size - 1) / group_size : 1;
    HXQ_REQUIRE(!group_affine || ngroups * out_features * 8 < (int64_t{1} << 31),
                "affine factors too large for 32-bit offsets");
    HXQ_REQUIRE(!sc_grp_ptr || (sc_grp_key && sc_grp_val),
                "the sidecar needs sc_grp_ptr, sc_grp_key and sc_grp_val");
    HXQ_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(indices) & 15u) == 0,
                "x and indices must be 16-byte aligned");
    // uint16 scalar indices with the affine need more registers than the
    // 256-row tile leaves: 128-row tiles
    // fp32 activations: 128-row tiles (the fp32 A tile doubles the LDS)
    const bool u16_aff = format == HXQ_FMT_SCALAR_U16 && group_affine != nullptr;
    const bool f32 = x_dtype == HXQ_F32;
    const pg::Plan p = pg::plan(m_rows, out_features, in_features, device_cu_count(),
                                (u16_aff || f32) ? 128 : 256);
    pg::Args a{};
    a.x = static_cast<const uint16_t *>(x);
    a.idx = indices;
    a.cb = codebook;
    a.n_codes = n_codes;
    a.ga = reinterpret_cast<const float2 *>(group_affine);
    a.sc_ptr = sc_grp_ptr;
    a.sc_key = sc_grp_key;
    a.sc_val = sc_grp_val;
    a.bias = bias;
    a.y = y;
    a.M = static_cast<int32_t>(m_rows);
    a.OUT = static_cast<int32_t>(out_features);
    a.K = static_cast<int32_t>(in_features);
    a.group = group_affine ? group_size : pg::kBK;
    a.ngroups = static_cast<int32_t>(ngroups);
    a.g_lane = a.group % pg::kBK != 0;
    a.g16 = a.group % 32 != 0;
    a.y_dtype = y_dtype;
    a.tiles_x = p.tiles_x;
    a.tiles_y = p.tiles_y;
    if (p.ws_bytes > 0) {
        HXQ_REQUIRE(workspace != nullptr && workspace_bytes >= p.ws_bytes,
                    "workspace too small (hxq_prefill_gemm_workspace_bytes)");
        HXQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0,
                    "workspace must be 16-byte aligned");
        a.part = static_cast<float *>(workspace);
    }
    const bool bf16 = x_dtype == HXQ_BF16;
    const bool aff = group_affine != nullptr;
    const bool vec = y_dtype != HXQ_F32 && out_features % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    for (int li = 0; li < p.nl; ++li) {
        const pg::Launch &L = p.l[li];
        a.t0 = L.t0;
        a.ntiles = L.n;
        a.ksplit = L.ks;
        a.ks_per = L.ks_per;
        a.tiles_per_xcd = (L.n + pg::kXcds - 1) / pg::kXcds;
        a.vec_out = L.ks == 1 && vec;
        const dim3 grid(a.tiles_per_xcd * pg::kXcds, L.ks);
#define HXQ_PG_LAUNCH(BM_, BF_, AF_, F_)                                                      \
        do {                                                                                  \
            if ((AF_) && a.g16)                                                               \
                hipLaunchKernelGGL((pg::prefill_kernel<BM_, BF_, AF_, pg::kNJ, F_, false, 2>), \
                                   grid, dim3(pg::kBN / (32 * pg::kNJ) * 64), 0, stream, a);  \
            else if ((AF_) && a.g_lane)                                                       \
                hipLaunchKernelGGL((pg::prefill_kernel<BM_, BF_, AF_, pg::kNJ, F_, false, 1>), \
                                   grid, dim3(pg::kBN / (32 * pg::kNJ) * 64), 0, stream, a);  \
            else                                                                              \
                hipLaunchKernelGGL((pg::prefill_kernel<BM_, BF_, AF_, pg::kNJ, F_>), grid,     \
                                   dim3(pg::kBN / (32 * pg::kNJ) * 64), 0, stream, a);        \
        } while (0)
#define HXQ_PG_FMT(BM_, BF_)                                                                  \
        switch (format) {                                                                      \
            case HXQ_FMT_SCALAR:                                                               \
                if (aff) HXQ_PG_LAUNCH(BM_, BF_, true, HXQ_FMT_SCALAR);                        \
                else HXQ_PG_LAUNCH(BM_, BF_, false, HXQ_FMT_SCALAR);                           \
                break;                                                                         \
            case HXQ_FMT_SCALAR_U16:                                                           \
                if (aff) HXQ_PG_LAUNCH(128, BF_, true, HXQ_FMT_SCALAR_U16);                    \
                else HXQ_PG_LAUNCH(BM_, BF_, false, HXQ_FMT_SCALAR_U16);                       \
                break;                                                                         \
            case HXQ_FMT_VQ2_U16: HXQ_PG_LAUNCH(BM_, BF_, false, HXQ_FMT_VQ2_U16); break;       \
            case HXQ_FMT_VQ2_P12: HXQ_PG_LAUNCH(BM_, BF_, false, HXQ_FMT_VQ2_P12); break;       \
            default: HXQ_PG_LAUNCH(BM_, BF_, true, HXQ_FMT_AF6); break;                        \
        }
        if (p.bm == 256) {
            if (bf16) { HXQ_PG_FMT(256, 1) } else { HXQ_PG_FMT(256, 0) }
        } else if (f32) {
            HXQ_PG_FMT(128, 2)
        } else {
            if (bf16) { HXQ_PG_FMT(128, 1) } else { HXQ_PG_FMT(128, 0) }
        }
#undef HXQ_PG_FMT
#undef HXQ_PG_LAUNCH
        HXQ_LAUNCH_CHECK();
        if (L.ks > 1) {
            HXQ_REQUIRE(L.ks <= pg::kRedKs, "K split above the reduce's limit");
            const int64_t n = int64_t{1} * L.n * p.bm * pg::kBN / 4;  // four outputs per thread
            const int32_t vec = a.OUT % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
            hipLaunchKernelGGL(pg::prefill_reduce_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)),
                               dim3(256), 0, stream, a.part, L.ks, L.n, L.t0, p.tiles_x, p.tiles_y,
                               p.bm, a.M, a.OUT, bias, y, y_dtype, vec);
            HXQ_LAUNCH_CHECK();
        }
    }
    return HXQ_OK;
}
