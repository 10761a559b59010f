// HXQ prefill GEMM: Y[M, OUT] = X[M, K] @ W^T, W dequantised into LDS and fed
// to bf16/fp16 MFMA (v_mfma_f32_32x32x16_{bf16,f16}) with fp32 accumulation,
// plus its grouped form for mixture-of-experts FFNs (rows of X gathered per
// expert, one expert's HXQ matrix per row tile).
//
// Replaces fused_vq_matmul's N > 1 path (helix_substrate/triton_vq_matmul.py:
// 634-661 _vq_gather_matmul_tiled_kernel, 693-698 scatter_add sidecar, 724-725
// bias) and the default _forward_buffered materialise-then-BLAS path
// (helix_linear.py:556-634).
//
// Block: 768 threads = 12 waves, block tile BM x 256 (BM = 64 or 128), K-step
// 64, split by role.  Waves 0-3 consume: each owns BM x 64 outputs
// ((BM/32) x 2 MFMA 32x32 tiles) and only issues MFMAs on LDS operands.
// Waves 4-11 produce: per K-step they copy the X tile (16-bit) into LDS, rows
// XOR-swizzled in 16-byte chunks so the MFMA operand reads (8 lanes x 16 B
// per row group) hit all banks, and build the W tile: thread t owns 16
// columns of 2 W rows and
//   * turns its 64 indices into weights: codebook lookup (LDS, 32 replicas;
//     16 in pair mode) -> fma(cb, scale, offset) -> v_cvt_pk_bf16_f32 ->
//     LDS, then REPLACES sidecar entries of the step (the block's CSR
//     entries are staged in LDS once);
//   * issues the global loads two steps ahead.
// The hardware places wave w on SIMD w % 4, so each SIMD runs one consumer
// and two producers: dequantisation (VALU, LDS lookups, whose latency two
// producer waves hide) overlaps the MFMAs.  LDS is double-buffered with one
// barrier per step.
// Results are written once per output element: deterministic.
//
// Grouped mode (MoE): `seg` holds the expert segments [E+1] of a sorted
// assignment list; row tile y maps to (expert, rows) by a prefix over
// ceil(count_e / BM); X rows are gathered through `rows` (or taken in order),
// the weight pointers step by the per-expert strides, and outputs land in
// sorted order.  Pair mode computes gate rows (tile rows 0..127) and up rows
// (128..255) of the same 128 features and writes silu(gate) * up.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "hxq_common.h"
#include "hxq_prefill.h"

namespace hxq {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kConsumers = 4;                   // MFMA waves
constexpr int kProducers = 8;                   // dequantising waves
constexpr int kGemmThreads = (kConsumers + kProducers) * 64;
constexpr int kPT = kProducers * 64;            // producer threads
constexpr int kPRows = 256 / (kPT / 4);         // W rows per producer thread (2)
constexpr int kBK = 64;        // K per step
constexpr int kBN = 256;       // tile rows of W (output features) per block
constexpr int kScCap = 8192;   // sidecar entries staged in LDS per block

// One HXQ weight set.  For a bank of experts every array is the per-expert
// arrays stacked along a leading expert axis.
struct WSet {
    const uint8_t *idx;   // [E, OUT, K]
    const float *cb;      // [E, 256]
    const float *ga;      // [E, K/G, OUT, 2] {scale, offset} or null
    const int32_t *rp;    // [E, OUT+1] absolute offsets into col/val, or null
    const int32_t *col;
    const float *val;     // replacement values
};

struct GemmArgs {
    const uint16_t *x;    // [x_rows, K] bf16/fp16
    const int32_t *rows;  // grouped: x row of each sorted assignment (null = in order)
    const int32_t *seg;   // grouped: [E+1] segment offsets (null = dense)
    WSet w[2];            // w[1]: up matrix of a SwiGLU pair
    const float *bias;    // [OUT] or null (dense only)
    void *y;              // [M, OUT]
    int32_t M, OUT, K, group, y_dtype, n_experts, x_rows, pad_;
    int32_t tiles_x, tiles_y, tiles_per_xcd, pad2_;  // dense: tile grid, XCD share
    float *part;          // dense split-K: fp32 partials [ksplit, M, OUT] (ksplit > 1)
    int32_t ksplit, ks_per;  // dense: K-step ranges (blockIdx.y = range), steps per range
};

// Dense tile order.  Blocks are dealt round-robin to the XCDs (block b runs on
// XCD b % kXcds), each with its own L2.  Tile t = (b % kXcds) * per + b / kXcds
// gives every XCD a contiguous run of the order, and the order walks groups of
// kGroupRows row tiles column by column, so the ~32 blocks one XCD runs at a
// time cover about 8 X row tiles x 4 W column tiles: each tile is fetched into
// that L2 once and reused by the blocks beside it, instead of every block
// fetching a W tile no other block on its XCD reads.  Returns false for the
// padding blocks past the last tile.
constexpr int kXcds = 8;
constexpr int kGroupRows = 8;
__device__ __forceinline__ bool dense_tile(const GemmArgs &g, int b, int &tx, int &ty) {
    const int t = (b % kXcds) * g.tiles_per_xcd + b / kXcds;
    if (t >= g.tiles_x * g.tiles_y) return false;
    const int grp = t / (kGroupRows * g.tiles_x);
    const int r0 = grp * kGroupRows;
    const int gr = min(kGroupRows, g.tiles_y - r0);  // rows in this group
    const int w = t - grp * kGroupRows * g.tiles_x;
    tx = w / gr;
    ty = r0 + w % gr;
    return true;
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

template <bool BF16>
__device__ __forceinline__ uint16_t to16(float v) {
    return static_cast<uint16_t>(pack2<BF16>(v, 0.f) & 0xffffu);
}

// Element offset of 16-byte chunk c (0..7) of LDS row r (64 elements, 128 B).
// gfx950's LDS has 64 banks and serves 16 lanes of a 16-byte access per
// clock: two consecutive rows fill the 64 banks, so the chunk is XORed with
// (r / 2) % 8 -- any 16 consecutive rows then map one chunk index to 16
// distinct (row parity, slot) pairs, conflict-free (XOR with r % 8 leaves
// rows r and r + 8 on the same banks: measured 155 vs 220 B/clk per CU).
__device__ __forceinline__ int swz(int r, int c) { return r * kBK + ((c ^ ((r >> 1) & 7)) << 3); }

// Global data of one K-step for one producer thread, held in registers until
// written to LDS.  Producer thread t owns W rows (t/4) + 128i (i = 0, 1), 16
// indices each (columns 16*(t%4) .. +16 of the step): four lanes cover one
// row's 64 bytes, so a load instruction touches 16 rows, not 64.
template <int BM>
struct GemmStage {
    u32x4 q[kPRows];              // 16 indices of each of the thread's W rows
    float2 so[1];                 // {scale, offset} of row qc's group (shared in the quad)
    u32x4 a[BM * 8 / kPT];        // X: chunk t%8 of rows t/8 + (kPT/8) p
};

template <int BM, bool BF16, bool AFFINE, bool GROUPED, bool PAIR>
__global__ __launch_bounds__(kGemmThreads, 3) void gemm_kernel(const GemmArgs g) {
    static_assert(!PAIR || GROUPED, "pair mode is a grouped-GEMM epilogue");
    static_assert(BM == 64 || BM == 128, "row tile");
    constexpr int TM = BM / 32;      // consumer wave tile BM x 64: TM x TN MFMA tiles
    constexpr int TN = 2;
    constexpr int NT = PAIR ? 2 : 1; // codebook tables
    // Codebook replicas: 32 per table keep lookups bank-conflict-free (the two
    // half-waves use the same 32 banks in different cycles); a SwiGLU pair
    // needs two tables and keeps 16 replicas to fit the 160 KB of LDS.
    constexpr int NREP = PAIR ? 16 : 32;
    constexpr int kTblBytes = NT * 256 * NREP * 4;
    constexpr int kABytes = 2 * BM * kBK * 2;
    constexpr int kBBytes = 2 * kBN * kBK * 2;
    // sidecar entries of the block's rows, staged once: {col u16, value u16}
    constexpr int kScBytes = kScCap * 4;
    static_assert(kTblBytes + kABytes + kBBytes + kScBytes <= 160 * 1024, "LDS budget");
    // table first: its LDS offset is 0, so lookups need no base add
    __shared__ __attribute__((aligned(16))) char smem[kTblBytes + kABytes + kBBytes + kScBytes];
    float (*tbl)[256 * NREP] = reinterpret_cast<float (*)[256 * NREP]>(smem);
    uint16_t (*sA)[BM * kBK] = reinterpret_cast<uint16_t (*)[BM * kBK]>(smem + kTblBytes);
    uint16_t (*sB)[kBN * kBK] = reinterpret_cast<uint16_t (*)[kBN * kBK]>(smem + kTblBytes + kABytes);
    uint32_t *sSc = reinterpret_cast<uint32_t *>(smem + kTblBytes + kABytes + kBBytes);
    int *s_tile = reinterpret_cast<int *>(&sA[0][0]);  // read before sA is first written

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    // Waves 0-3 consume (MFMA on the staged tiles), waves 4-11 produce (load,
    // dequantise, write LDS); the hardware places wave w on SIMD w % 4, so
    // every SIMD runs one consumer next to two producers and their VALU and
    // MFMA work overlap.
    const bool producer = wave >= kConsumers;
    const int cw = wave & 3;               // consumer: 64-column block of the tile
    const int pt = tid - kConsumers * 64;  // producer thread 0..kPT-1
    const int K = g.K;
    // dense split-K: this block runs K-steps [kb, kb + nk) of the tile
    const int kb = GROUPED ? 0 : static_cast<int>(blockIdx.y) * g.ks_per;
    const int nk = GROUPED ? K / kBK : min(K / kBK - kb, g.ks_per);

    // ---- row tile -> (expert, first row, end row) --------------------------
    int e = 0, r0, r1;
    if constexpr (GROUPED) {
        if (wave == 0) {
            const int by = blockIdx.y;
            int base = 0, fe = -1, fr0 = 0, fr1 = 0;
            for (int e0 = 0; e0 < g.n_experts; e0 += 64) {
                const int ee = e0 + lane;
                int lo = 0, cnt = 0;
                if (ee < g.n_experts) {
                    lo = g.seg[ee];
                    cnt = g.seg[ee + 1] - lo;
                }
                const int t = (cnt + BM - 1) / BM;
                int incl = t;
#pragma unroll
                for (int d = 1; d < 64; d <<= 1) {
                    const int v = __shfl_up(incl, d, kWave);
                    if (lane >= d) incl += v;
                }
                const int excl = base + incl - t;
                if (t > 0 && by >= excl && by < excl + t) {
                    fe = ee;
                    fr0 = lo + (by - excl) * BM;
                    fr1 = min(fr0 + BM, lo + cnt);
                }
                base += __shfl(incl, 63, kWave);
            }
            // at most one lane matched
            const unsigned long long hit = __ballot(fe >= 0);
            if (lane == 0) s_tile[0] = -1;
            if (hit) {
                const int src = __builtin_ctzll(hit);
                const int be = __shfl(fe, src, kWave), b0 = __shfl(fr0, src, kWave),
                          b1 = __shfl(fr1, src, kWave);
                if (lane == 0) {
                    s_tile[0] = be;
                    s_tile[1] = b0;
                    s_tile[2] = b1;
                }
            }
        }
        __syncthreads();
        e = s_tile[0];
        r0 = s_tile[1];
        r1 = s_tile[2];
        __syncthreads();  // s_tile lives in sA: everyone has read it
        if (e < 0) return;  // block-uniform: no tile for this block index
    }
    int tile_x = blockIdx.x;
    if constexpr (!GROUPED) {
        int ty;
        if (!dense_tile(g, blockIdx.x, tile_x, ty)) return;  // block-uniform
        r0 = ty * BM;
        r1 = min(r0 + BM, g.M);
    }
    const int64_t eo = static_cast<int64_t>(e);
    const int n0 = tile_x * (PAIR ? kBN / 2 : kBN);
    const int ngroups = AFFINE ? K / g.group : 1;

    // codebook replicas: entry j at [j * NREP + r]; thread t fills entry t/2
    // of each table, NREP/2 replicas
    if (tid < 512) {
        const int j = tid >> 1;
#pragma unroll
        for (int p = 0; p < NT; ++p) {
            const float c = g.w[p].cb[eo * 256 + j];
            float4 *d = reinterpret_cast<float4 *>(&tbl[p][j * NREP + (tid & 1) * (NREP / 2)]);
#pragma unroll
            for (int q = 0; q < NREP / 8; ++q) d[q] = make_float4(c, c, c, c);
        }
    }

    // ---- sidecar: the block's CSR entries (per part a contiguous range) ----
    // Staged into LDS as {col, 16-bit value} so the producers' per-step cursor
    // reads LDS and never waits on global loads behind the prefetched stages.
    // A block with more than kScCap entries (or K > 65535) reads them from
    // global memory instead (same results, slower).
    constexpr int RPP = PAIR ? kBN / 2 : kBN;  // rows per part
    int sc_lo[NT], sc_base[NT], sc_total = 0;
#pragma unroll
    for (int p = 0; p < NT; ++p) {
        sc_base[p] = sc_total;
        sc_lo[p] = 0;
        if (g.w[p].rp != nullptr) {
            const int32_t *rpp = g.w[p].rp + eo * (g.OUT + 1);
            sc_lo[p] = rpp[n0];
            sc_total += rpp[min(n0 + RPP, g.OUT)] - sc_lo[p];
        }
    }
    const bool sc_in_lds = sc_total <= kScCap && K <= 0xffff;
    if (sc_in_lds) {
        for (int i = tid; i < sc_total; i += kGemmThreads) {
            const int p = (NT == 2 && i >= sc_base[NT - 1]) ? 1 : 0;
            const int j = sc_lo[p] + (i - sc_base[p]);
            const int32_t col = p ? g.w[NT - 1].col[j] : g.w[0].col[j];
            const float v = p ? g.w[NT - 1].val[j] : g.w[0].val[j];
            sSc[i] = static_cast<uint32_t>(col) | (static_cast<uint32_t>(to16<BF16>(v)) << 16);
        }
    }

    // ---- producers: load two steps ahead, fill the LDS buffer the consumers
    // read next; one barrier per step (the consumers' loop below hits the
    // same barriers) -------------------------------------------------------
    if (producer) {
        // ---- producer state: W rows (pt/4) + 64i, X chunk pt % 8 ----------------
        const int qc = pt & 3;                  // 16-index chunk of the step
        const int qr0 = pt >> 2;                // first W row of this thread (tile row)
        // rows qr0 + 128i; in pair mode rows 0..127 come from matrix 0 (gate) and
        // 128..255 from matrix 1 (up): part = i
        auto tile_row = [&](int i) { return qr0 + 128 * i; };
        auto mat_row = [&](int i) { return n0 + (PAIR ? (tile_row(i) & 127) : tile_row(i)); };
        auto part_of = [&](int i) { return PAIR ? i : 0; };

        constexpr uint32_t kOob = 0x80000000u;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, (int64_t)g.x_rows * K * 2);
        __amdgpu_buffer_rsrc_t qr[NT];
    #pragma unroll
        for (int p = 0; p < NT; ++p) qr[p] = make_rsrc(g.w[p].idx + eo * g.OUT * K, (int64_t)g.OUT * K);

        // X: producer thread pt copies chunk pt % 8 of rows pt/8 + (kPT/8) p
        constexpr int kXP = BM * 8 / kPT;
        const int a_cc = pt & 7;
        uint32_t a_off[kXP];
    #pragma unroll
        for (int p = 0; p < kXP; ++p) {
            const int r = r0 + (pt >> 3) + (kPT / 8) * p;
            int src = r;
            if constexpr (GROUPED) {
                if (producer && r < r1 && g.rows) src = g.rows[r];
            }
            a_off[p] = (producer && r < r1 && src >= 0 && src < g.x_rows)
                           ? (uint32_t)(src * K + a_cc * 8) * 2u : kOob;
        }
        uint32_t q_off[kPRows];
    #pragma unroll
        for (int i = 0; i < kPRows; ++i) {
            const bool ok = producer && mat_row(i) < g.OUT;
            q_off[i] = ok ? (uint32_t)(mat_row(i) * K + qc * 16) : kOob;
        }
        // affine factors: this lane fetches those of its row qc (see load_stage)
        const float *ga_mine = nullptr;
        if constexpr (AFFINE) {
            const int ri = qc & (kPRows - 1);
            ga_mine = ((PAIR && ri == 1) ? g.w[NT - 1].ga : g.w[0].ga) + eo * ngroups * g.OUT * 2 +
                      (int64_t)(mat_row(ri) < g.OUT ? mat_row(ri) : 0) * 2;
        }

        // sidecar cursors of the thread's 4 rows (each covers its 16 columns);
        // sc_nc holds the column of the next entry (or a sentinel past any K), so
        // a step without entries costs one register compare per row
        int32_t sc_cur[kPRows], sc_end[kPRows], sc_nc[kPRows];
    #pragma unroll
        for (int i = 0; i < kPRows; ++i) {
            sc_cur[i] = 0;
            sc_end[i] = 0;
            const int p = part_of(i);
            const int32_t *rpb = p ? g.w[NT - 1].rp : g.w[0].rp;
            if (rpb != nullptr && producer && mat_row(i) < g.OUT) {
                const int32_t *rp = rpb + eo * (g.OUT + 1);
                sc_cur[i] = rp[mat_row(i)];
                sc_end[i] = rp[mat_row(i) + 1];
                if (sc_in_lds) {
                    const int shift = sc_base[p] - sc_lo[p];
                    sc_cur[i] += shift;
                    sc_end[i] += shift;
                }
            }
        }
        auto sc_col_of = [&](int i, int j) -> int32_t {
            if (sc_in_lds) return static_cast<int32_t>(sSc[j] & 0xffffu);
            return part_of(i) ? g.w[NT - 1].col[j] : g.w[0].col[j];
        };

        // Loads are issued unconditionally (steps past the end read at kOob, which
        // the buffer range check turns into zeros without memory traffic): a
        // conditional prefetch would make the compiler's wait counting assume the
        // prefetch absent and wait for it at the next use of the older stage.
        auto load_stage = [&](int ks, GemmStage<BM> &st) {
            const bool live = ks < nk;
            const uint32_t k0 = (kb + (live ? ks : 0)) * kBK;
    #pragma unroll
            for (int p = 0; p < kXP; ++p)
                st.a[p] = buf_load16(xr, (a_off[p] == kOob || !live) ? kOob : a_off[p] + k0 * 2);
    #pragma unroll
            for (int i = 0; i < kPRows; ++i)
                st.q[i] = buf_load16(qr[part_of(i)], (q_off[i] == kOob || !live) ? kOob : q_off[i] + k0);
            if constexpr (AFFINE) {
                // the 4 lanes of a quad share their 4 rows: lane qc loads row qc's
                // factors, a quad broadcast (DPP) hands them to the others
                // (always a valid address: rows past OUT read row 0, whose value
                // only reaches outputs the epilogue drops)
                st.so[0] = *reinterpret_cast<const float2 *>(ga_mine + (int64_t)(k0 / g.group) * g.OUT * 2);
            } else {
                st.so[0] = make_float2(1.f, 0.f);
            }
        };

        // row i's factors from quad lane i (DPP quad_perm [i,i,i,i])
        auto quad_bcast = [&](float2 v, float2 (&out)[kPRows]) {
            if constexpr (AFFINE) {
                const int x = __float_as_int(v.x), y = __float_as_int(v.y);
                out[0] = make_float2(__int_as_float(__builtin_amdgcn_mov_dpp(x, 0x00, 0xf, 0xf, false)),
                                     __int_as_float(__builtin_amdgcn_mov_dpp(y, 0x00, 0xf, 0xf, false)));
                out[1] = make_float2(__int_as_float(__builtin_amdgcn_mov_dpp(x, 0x55, 0xf, 0xf, false)),
                                     __int_as_float(__builtin_amdgcn_mov_dpp(y, 0x55, 0xf, 0xf, false)));
            } else {
    #pragma unroll
                for (int i = 0; i < kPRows; ++i) out[i] = make_float2(1.f, 0.f);
            }
        };
        const uint32_t lane_off = (lane & (NREP - 1)) * 4u;
        auto lookup = [&](int p, uint32_t w, int b) -> float {
            constexpr int kShift = NREP == 32 ? 7 : 6;  // log2(NREP * 4)
            const char *tb = reinterpret_cast<const char *>(&tbl[p][0]);
            return *reinterpret_cast<const float *>(tb + lane_off + (((w >> (8 * b)) & 0xffu) << kShift));
        };

        auto write_stage = [&](int ks, const GemmStage<BM> &st, int buf, auto sc_lds) {
            constexpr bool SC_LDS = decltype(sc_lds)::value;
    #pragma unroll
            for (int p = 0; p < kXP; ++p)
                *reinterpret_cast<u32x4 *>(&sA[buf][swz((pt >> 3) + (kPT / 8) * p, a_cc)]) = st.a[p];
            float2 so[kPRows];
            quad_bcast(st.so[0], so);
            // each row: 16 indices -> 2 chunks of 8 16-bit weights
    #pragma unroll
            for (int i = 0; i < kPRows; ++i)
    #pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint32_t pk[4];
    #pragma unroll
                    for (int dd = 0; dd < 2; ++dd) {
                        const uint32_t w = st.q[i][h * 2 + dd];
                        float v[4];
    #pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const float c = lookup(part_of(i), w, b);
                            v[b] = AFFINE ? affine_fma(c, so[i].x, so[i].y) : c;
                        }
                        pk[dd * 2] = pack2<BF16>(v[0], v[1]);
                        pk[dd * 2 + 1] = pack2<BF16>(v[2], v[3]);
                    }
                    *reinterpret_cast<u32x4 *>(&sB[buf][swz(tile_row(i), qc * 2 + h)]) =
                        u32x4{pk[0], pk[1], pk[2], pk[3]};
                }
            // sidecar: replace entries with column in this thread's [lo, lo + 16)
            const int k0 = (kb + ks) * kBK, lo = k0 + qc * 16, hi = lo + 16;
            uint16_t *brow = &sB[buf][0];
    #pragma unroll
            for (int i = 0; i < kPRows; ++i) {
                while (sc_nc[i] < hi) {
                    const int j = sc_cur[i];
                    if (sc_nc[i] >= lo) {
                        const int kc = sc_nc[i] - k0;
                        uint16_t v16;
                        if constexpr (SC_LDS) v16 = static_cast<uint16_t>(sSc[j] >> 16);
                        else v16 = to16<BF16>(part_of(i) ? g.w[NT - 1].val[j] : g.w[0].val[j]);
                        brow[swz(tile_row(i), kc >> 3) + (kc & 7)] = v16;
                    }
                    sc_cur[i] = j + 1;
                    sc_nc[i] = j + 1 < sc_end[i] ? sc_col_of(i, j + 1) : 0x7fffffff;
                }
            }
        };

        auto run = [&](auto sc_lds) {
            GemmStage<BM> s0, s1;
            load_stage(0, s0);
            load_stage(1, s1);
            __syncthreads();  // codebook tables and staged sidecar visible
#pragma unroll
            for (int i = 0; i < kPRows; ++i)
                sc_nc[i] = sc_cur[i] < sc_end[i] ? sc_col_of(i, sc_cur[i]) : 0x7fffffff;
            write_stage(0, s0, 0, sc_lds);
            lds_barrier();
            int ks = 0;
            for (; ks + 1 < nk; ks += 2) {
                load_stage(ks + 2, s0);
                write_stage(ks + 1, s1, 1, sc_lds);
                lds_barrier();
                load_stage(ks + 3, s1);
                if (ks + 2 < nk) write_stage(ks + 2, s0, 0, sc_lds);
                lds_barrier();
            }
            if (ks < nk) lds_barrier();  // odd step count: the consumers' last step
        };
        if (sc_in_lds) run(std::true_type{});
        else run(std::false_type{});
        if constexpr (PAIR) __syncthreads();  // the consumers' gate/up hand-over
        return;
    }

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // consumer: one K-step of MFMAs on LDS buffer `buf` (k permuted within the
    // step identically for X and W: lane half h takes chunks 2kk + h)
    auto mfma_step = [&](int buf) {
        const int hsel = lane >> 5;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            u32x4 bv[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bv[j] = *reinterpret_cast<const u32x4 *>(
                    &sB[buf][swz(cw * 64 + j * 32 + (lane & 31), kk * 2 + hsel)]);
            // one X operand at a time keeps the live operand registers at 3 x 4
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const u32x4 av = *reinterpret_cast<const u32x4 *>(
                    &sA[buf][swz(i * 32 + (lane & 31), kk * 2 + hsel)]);
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (BF16)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv[j]),
                            acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv[j]),
                            acc[i][j], 0, 0, 0);
                }
            }
        }
    };

    // ---- consumers: MFMAs on the current buffer --------------------------------
    __syncthreads();
    lds_barrier();
    int ks = 0;
    for (; ks + 1 < nk; ks += 2) {
        mfma_step(0);
        lds_barrier();
        mfma_step(1);
        lds_barrier();
    }
    if (ks < nk) {
        mfma_step(0);
        lds_barrier();
    }

    // ---- epilogue (consumers): acc[i][j][r] = C[8*(r/4) + 4*(lane/32) + r%4][lane%32]
    const int nrows = r1 - r0;
    if constexpr (PAIR) {
        // consumer waves 2, 3 hold the up rows of the features waves 0, 1 hold
        // as gate rows, in the same lane/register positions: hand them over
        // through LDS (the B buffers are free now).
        float *xch = reinterpret_cast<float *>(&sB[0][0]);
        constexpr int PER = TM * TN * 16;
        if (cw >= 2) {
            float *d = xch + ((cw - 2) * PER) * 64 + lane;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) d[((i * TN + j) * 16 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (cw < 2) {
            const float *u = xch + (cw * PER) * 64 + lane;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + cw * 64 + j * 32 + (lane & 31);
                if (n >= g.OUT) continue;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                        if (m < nrows) {
                            const float gt = acc[i][j][r];
                            const float up = u[((i * TN + j) * 16 + r) * 64];
                            const float hv = gt / (1.f + expf(-gt)) * up;
                            const int64_t o = (int64_t)(r0 + m) * g.OUT + n;
                            static_cast<uint16_t *>(g.y)[o] = to16<BF16>(hv);
                        }
                    }
            }
        }
        return;
    } else if (!GROUPED && g.ksplit > 1) {
        // split-K: this range's fp32 partial; the reduce kernel adds the
        // ranges in order, then the bias
        float *part = g.part + static_cast<int64_t>(blockIdx.y) * g.M * g.OUT;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + cw * 64 + j * 32 + (lane & 31);
            if (n >= g.OUT) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                    if (m < nrows) part[(int64_t)(r0 + m) * g.OUT + n] = acc[i][j][r];
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + cw * 64 + j * 32 + (lane & 31);
            if (n >= g.OUT) continue;
            const float bv = g.bias ? g.bias[n] : 0.f;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                    if (m < nrows) {
                        const float v = acc[i][j][r] + bv;
                        const int64_t o = (int64_t)(r0 + m) * g.OUT + n;
                        if (g.y_dtype == HXQ_F32) static_cast<float *>(g.y)[o] = v;
                        else static_cast<uint16_t *>(g.y)[o] = g.y_dtype == HXQ_BF16
                                                                    ? to16<true>(v) : to16<false>(v);
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------
// MoE routing: softmax over experts, top-k (ties -> lower expert id), and the
// expert-sorted assignment lists.
// ---------------------------------------------------------------------------
// Wave64 reductions on DPP (row shuffles, row mirrors and row broadcasts:
// VALU operations, where a __shfl_xor is an LDS permute with its round trip);
// every lane receives the result.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_fmax(float v) {
    const int s = __builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), CTRL,
                                              ROW_MASK, 0xf, false);
    return fmaxf(v, __int_as_float(s));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_imin(int v) {
    const int s = __builtin_amdgcn_update_dpp(0x7fffffff, v, CTRL, ROW_MASK, 0xf, false);
    return min(v, s);
}
__device__ __forceinline__ float wave_fmax_all(float v) {
    v = dpp_fmax<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_fmax<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_fmax<0x141, 0xf>(v);  // row_half_mirror
    v = dpp_fmax<0x140, 0xf>(v);  // row_mirror
    v = dpp_fmax<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_fmax<0x143, 0xc>(v);  // row_bcast:31: lane 63 holds the maximum
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ int wave_imin_all(int v) {
    v = dpp_imin<0xb1, 0xf>(v);
    v = dpp_imin<0x4e, 0xf>(v);
    v = dpp_imin<0x141, 0xf>(v);
    v = dpp_imin<0x140, 0xf>(v);
    v = dpp_imin<0x142, 0xa>(v);
    v = dpp_imin<0x143, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

// One wave per token; lane l holds logits l, l + 64, ... (E <= 256).  The
// softmax denominator and each of the k picks are wave reductions: a pick is
// the wave maximum of the lanes' best values, then the lowest expert id among
// the lanes holding it (ties -> lower expert id).
__global__ __launch_bounds__(256) void moe_topk_kernel(const float *logits, int32_t T, int32_t E,
                                                       int32_t k, int32_t renorm, int32_t *ids,
                                                       float *wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + threadIdx.x / 64;
    if (t >= T) return;  // wave-uniform
    const float *l = logits + (int64_t)t * E;
    float v[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < E ? l[e] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_fmax_all(mx);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < E) sum += expf(v[j] - mx);
    sum = wave_sum(sum);
    float picked = 0.f, my_w = 0.f;
    int my_id = 0;
    // entries already picked, one bit per j: skipped by later picks, so an
    // expert is never picked twice even when fewer than k logits are finite
    // (the remaining picks are then the lowest unpicked ids at -inf, weight 0)
    uint32_t taken = 0;
    for (int s = 0; s < k; ++s) {
        // best (value, id) of this lane among its unpicked entries; ties -> lower id
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            if (e < E && !(taken >> j & 1u) && (v[j] > bv || (v[j] == bv && e < bi))) {
                bv = v[j];
                bi = e;
            }
        }
        const float wv = wave_fmax_all(bv);
        const int wi = wave_imin_all(bv == wv ? bi : 0x7fffffff);
        // mark the pick in its owner lane
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j == wi) taken |= 1u << j;
        const float p = expf(wv - mx) / sum;
        picked += p;
        if (lane == s) { my_id = wi; my_w = p; }
    }
    // lanes 0..k-1 hold the picks in order (k <= 64)
    if (lane < k) {
        ids[(int64_t)t * k + lane] = my_id;
        wts[(int64_t)t * k + lane] = renorm ? my_w / picked : my_w;
    }
}

// Count and place the assignments of expert blockIdx.x (its offset is the
// number of assignments to lower experts, counted in the same pass over the
// list).  4 waves split the assignment list into contiguous quarters;
// positions follow assignment order (token-major), so they are deterministic.
// A wave reads its quarter kSortU rounds of 64 ids at a time, all requested
// before the first is used (one round trip per 512 ids, not per 64).
constexpr int kSortU = 8;
__global__ __launch_bounds__(256) void moe_sort_kernel(const int32_t *ids, int64_t n_assign,
                                                       int32_t E, int32_t k, int32_t *counts,
                                                       int32_t *offsets, int32_t *sorted_rows,
                                                       int32_t *assign_pos) {
    __shared__ int wsum[4], psum[4];
    const int e = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t per = ((n_assign + 255) / 256) * 64;  // multiple of 64
    const int64_t a0 = wave * per, a1 = min(a0 + per, n_assign);
    // one pass counts this expert's assignments and those of lower experts
    // (the expert's global offset), so no second launch waits for all counts
    int cnt = 0, lt = 0;
    for (int64_t a = a0; a < a1; a += 64 * kSortU) {
        int v[kSortU];
#pragma unroll
        for (int u = 0; u < kSortU; ++u) {
            const int64_t aa = a + 64 * u + lane;
            v[u] = ids[aa < a1 ? aa : a0];  // in range: a0 < a1 here
        }
#pragma unroll
        for (int u = 0; u < kSortU; ++u) {
            const bool in = a + 64 * u + lane < a1;
            cnt += __popcll(__ballot(in && v[u] == e));
            lt += __popcll(__ballot(in && v[u] < e));
        }
    }
    if (lane == 0) {
        psum[wave] = lt;
        wsum[wave] = cnt;
    }
    __syncthreads();
    const int off = psum[0] + psum[1] + psum[2] + psum[3];
    const int tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    int base = off;
    for (int w = 0; w < wave; ++w) base += wsum[w];
    if (threadIdx.x == 0) {
        counts[e] = tot;
        offsets[e] = off;
        if (e == E - 1) offsets[E] = off + tot;
    }
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int64_t a = a0; a < a1; a += 64 * kSortU) {
        int v[kSortU];
#pragma unroll
        for (int u = 0; u < kSortU; ++u) {
            const int64_t aa = a + 64 * u + lane;
            v[u] = ids[aa < a1 ? aa : a0];
        }
#pragma unroll
        for (int u = 0; u < kSortU; ++u) {
            const int64_t aa = a + 64 * u + lane;
            const bool hit = aa < a1 && v[u] == e;
            const unsigned long long mask = __ballot(hit);
            if (hit) {
                const int pos = base + __popcll(mask & below);
                sorted_rows[pos] = static_cast<int32_t>(aa / k);
                assign_pos[aa] = pos;
            }
            base += __popcll(mask);
        }
    }
}

// y[t, :] = sum_s w[t, s] * O[assign_pos[t*k + s], :], slots in order.

// H[r, j] = silu(GU[r, j]) * GU[r, I + j] (GU [rows, 2I] in x's 16-bit type,
// as the projections' outputs are), rounded to x's 16-bit type: the SwiGLU
// product of the paired gate/up grouped launch.
template <bool BF16>
// 8 values per thread, 16-byte accesses (inter % 8 == 0, rows * inter < 2^31:
// the host checks both); silu(g) = g * rcp(1 + exp(-g)) (hardware exp and
// reciprocal, ~1 ulp each: far inside the 16-bit rounding of the result)
__global__ __launch_bounds__(256) void moe_silu_mul_kernel(const uint16_t *__restrict__ gu, int64_t rows,
                                                          int32_t inter, uint16_t *__restrict__ h) {
    const int32_t cpr = inter >> 3;
    const int32_t n = static_cast<int32_t>(rows) * cpr;
    auto f = [](uint32_t b) { return BF16 ? bf16_to_f32(static_cast<uint16_t>(b)) : f16_to_f32(static_cast<uint16_t>(b)); };
    auto silu_mul = [&](uint32_t g16, uint32_t u16) -> uint32_t {
        const float gv = f(g16);
        const float v = gv * __builtin_amdgcn_rcpf(1.f + __expf(-gv)) * f(u16);
        return BF16 ? f32_to_bf16(v) : f32_to_f16(v);
    };
    for (int32_t i = static_cast<int32_t>(blockIdx.x * 256 + threadIdx.x); i < n;
         i += static_cast<int32_t>(gridDim.x * 256)) {
        const int32_t r = i / cpr;
        const int32_t c = (i - r * cpr) * 8;
        const uint4 g = *reinterpret_cast<const uint4 *>(gu + static_cast<int64_t>(r) * 2 * inter + c);
        const uint4 u = *reinterpret_cast<const uint4 *>(gu + static_cast<int64_t>(r) * 2 * inter + inter + c);
        const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            o[k] = silu_mul(gw[k] & 0xffffu, uw[k] & 0xffffu) | (silu_mul(gw[k] >> 16, uw[k] >> 16) << 16);
        *reinterpret_cast<uint4 *>(h + static_cast<int64_t>(r) * inter + c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}
// fp32 activations: h = silu(g) * u in fp32, [rows, 2 * inter] -> [rows, inter]
__global__ __launch_bounds__(256) void moe_silu_mul_f32_kernel(const float *__restrict__ gu, int64_t rows,
                                                              int32_t inter, float *__restrict__ h) {
    const int64_t n = rows * inter;
    for (int64_t i = (int64_t{blockIdx.x} * 256 + threadIdx.x) * 4; i < n; i += int64_t{gridDim.x} * 1024) {
        const int64_t r = i / inter;
        const int32_t c = static_cast<int32_t>(i - r * inter);
        const float4 g = *reinterpret_cast<const float4 *>(gu + r * 2 * inter + c);
        const float4 u = *reinterpret_cast<const float4 *>(gu + r * 2 * inter + inter + c);
        auto f = [](float a, float b) { return a / (1.f + expf(-a)) * b; };
        *reinterpret_cast<float4 *>(h + i) = make_float4(f(g.x, u.x), f(g.y, u.y), f(g.z, u.z), f(g.w, u.w));
    }
}
// V consecutive columns per thread (V = 4 when hidden % 4 == 0: 16-byte
// loads of fp32 O, 8-byte loads of 16-bit O); each column's slots are added
// in order, in fp32, either way.
template <int OT, int YDT, int V>
__global__ __launch_bounds__(256) void moe_combine_kernel(const void *Ov, const float *wts,
                                                          const int32_t *pos, int32_t k,
                                                          int32_t hidden, void *y) {
    const int t = blockIdx.y;
    const int c = (blockIdx.x * 256 + threadIdx.x) * V;
    if (c >= hidden) return;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;
    for (int s = 0; s < k; ++s) {
        const int64_t a = (int64_t)t * k + s;
        const float w = wts[a];
        const int64_t oi = (int64_t)pos[a] * hidden + c;
        if constexpr (OT == HXQ_F32) {
            const float *o = static_cast<const float *>(Ov) + oi;
            if constexpr (V == 4) {
                const float4 f = *reinterpret_cast<const float4 *>(o);
                acc[0] = fmaf(w, f.x, acc[0]);
                acc[1] = fmaf(w, f.y, acc[1]);
                acc[2] = fmaf(w, f.z, acc[2]);
                acc[3] = fmaf(w, f.w, acc[3]);
            } else {
                acc[0] = fmaf(w, o[0], acc[0]);
            }
        } else {
            const uint16_t *o = static_cast<const uint16_t *>(Ov) + oi;
            auto f = [](uint32_t b) {
                return OT == HXQ_BF16 ? bf16_to_f32(static_cast<uint16_t>(b)) : f16_to_f32(static_cast<uint16_t>(b));
            };
            if constexpr (V == 4) {
                const uint2 q = *reinterpret_cast<const uint2 *>(o);
                acc[0] = fmaf(w, f(q.x & 0xffffu), acc[0]);
                acc[1] = fmaf(w, f(q.x >> 16), acc[1]);
                acc[2] = fmaf(w, f(q.y & 0xffffu), acc[2]);
                acc[3] = fmaf(w, f(q.y >> 16), acc[3]);
            } else {
                acc[0] = fmaf(w, f(o[0]), acc[0]);
            }
        }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) store_act<YDT>(y, (int64_t)t * hidden + c + v, acc[v]);
}

// y = sum over the split-K ranges in range order (+ bias), in y's dtype.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part,
                                                            int32_t ksplit, int64_t mn,
                                                            int32_t out, const float *bias,
                                                            void *y, int32_t y_dtype) {
    const int64_t i = blockIdx.x * 256ll + threadIdx.x;
    if (i >= mn) return;
    float v = part[i];
    for (int s = 1; s < ksplit; ++s) v += part[s * mn + i];
    if (bias) v += bias[i % out];
    if (y_dtype == HXQ_F32) static_cast<float *>(y)[i] = v;
    else static_cast<uint16_t *>(y)[i] = y_dtype == HXQ_BF16 ? to16<true>(v) : to16<false>(v);
}

// ga[g][o] = {scale[o][g], offset[o][g]}: the GEMM's affine layout, so a
// block's rows for one group are contiguous.
__global__ __launch_bounds__(256) void affine_pack_kernel(const float *gs, const float *go,
                                                          int32_t out, int32_t ng, float2 *ga) {
    const int64_t i = blockIdx.x * 256ll + threadIdx.x;  // = o * ng + g
    if (i >= (int64_t)out * ng) return;
    const int o = static_cast<int>(i / ng), gi = static_cast<int>(i % ng);
    ga[(int64_t)gi * out + o] = make_float2(gs[i], go[i]);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <int BM, bool BF16, bool GROUPED, bool PAIR>
static int gemm_launch(GemmArgs &a, int grid_x, int grid_y, hipStream_t stream) {
    dim3 grid(grid_x, grid_y);
    if constexpr (!GROUPED) {
        // one dimension: the kernel maps blocks to tiles XCD by XCD
        a.tiles_x = grid_x;
        a.tiles_y = grid_y;
        a.tiles_per_xcd = (grid_x * grid_y + kXcds - 1) / kXcds;
        grid = dim3(a.tiles_per_xcd * kXcds, a.ksplit > 1 ? a.ksplit : 1);
    }
    if (a.w[0].ga)
        hipLaunchKernelGGL((gemm_kernel<BM, BF16, true, GROUPED, PAIR>), grid, dim3(kGemmThreads),
                           0, stream, a);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, BF16, false, GROUPED, PAIR>), grid, dim3(kGemmThreads),
                           0, stream, a);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

static int check_bank(const hxq_expert_bank *b, const char *what, int64_t out, int64_t in,
                      int32_t group) {
    HXQ_REQUIRE(b && b->indices && b->codebook, std::string(what) + ": indices and codebook required");
    HXQ_REQUIRE(!b->group_affine || (group >= kBK && group % kBK == 0 && in % group == 0),
                std::string(what) + ": group_size must be a multiple of 64 dividing in_features");
    HXQ_REQUIRE(!b->sc_row_ptr || (b->sc_col && b->sc_val),
                std::string(what) + ": sidecar CSR needs row_ptr, col and val");
    HXQ_REQUIRE(out * in < (int64_t{1} << 31), std::string(what) + ": matrix too large");
    HXQ_REQUIRE(!b->group_affine || (in / group) * out * 8 < (int64_t{1} << 31),
                std::string(what) + ": affine factors too large for 32-bit offsets");
    return HXQ_OK;
}

static WSet wset_of(const hxq_expert_bank *b) {
    return WSet{b->indices, b->codebook, b->group_affine, b->sc_row_ptr, b->sc_col, b->sc_val};
}

// Grouped launch over a sorted assignment list: BM 128 when the mean rows per
// expert exceed 64, else 64.
template <bool PAIR>
static int grouped_launch(GemmArgs &a, int64_t n_assign, bool bf16, hipStream_t stream) {
    const int64_t mean = n_assign / std::max<int32_t>(a.n_experts, 1);
    const int bn = PAIR ? kBN / 2 : kBN;
    const int gx = static_cast<int>((a.OUT + bn - 1) / bn);
    if (mean > 64) {
        const int gy = static_cast<int>((n_assign + 127) / 128 + a.n_experts);
        return bf16 ? gemm_launch<128, true, true, PAIR>(a, gx, gy, stream)
                    : gemm_launch<128, false, true, PAIR>(a, gx, gy, stream);
    }
    const int gy = static_cast<int>((n_assign + 63) / 64 + a.n_experts);
    return bf16 ? gemm_launch<64, true, true, PAIR>(a, gx, gy, stream)
                : gemm_launch<64, false, true, PAIR>(a, gx, gy, stream);
}

}  // namespace hxq

using namespace hxq;

namespace {
// Dense split-K plan: when the output tiles fill under half of the 256 CUs,
// split K into up to 8 ranges of at least 4 steps (fp32 partials + an ordered
// reduce); otherwise one range.
struct SplitPlan {
    int ksplit, ks_per;
};
SplitPlan split_plan(int64_t m_rows, int64_t out_features, int64_t in_features) {
    const int64_t tiles = ((out_features + kBN - 1) / kBN) * ((m_rows + 127) / 128);
    const int nk = static_cast<int>(in_features / kBK);
    int ks = 1;
    if (tiles < 128) ks = static_cast<int>(std::min<int64_t>({8, 256 / tiles, nk / 4}));
    if (ks < 2) return {1, nk};
    const int per = (nk + ks - 1) / ks;
    return {(nk + per - 1) / per, per};
}
}  // namespace

static int gemm_dense(const void *x, int32_t x_dtype, const uint8_t *indices,
                      const float *codebook, const float *group_affine, int32_t group_size,
                      const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                      const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                      int64_t out_features, int64_t in_features, void *workspace,
                      int64_t workspace_bytes, hipStream_t stream);

extern "C" int64_t hxq_gemm_workspace_bytes(int64_t m_rows, int64_t out_features,
                                            int64_t in_features) {
    if (m_rows <= 0 || out_features <= 0 || in_features <= 0 || in_features % kBK) return 0;
    const SplitPlan sp = split_plan(m_rows, out_features, in_features);
    return sp.ksplit > 1 ? int64_t{4} * sp.ksplit * m_rows * out_features : 0;
}

extern "C" int hxq_gemm(const void *x, int32_t x_dtype, const uint8_t *indices,
                        const float *codebook, const float *group_affine, int32_t group_size,
                        const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                        const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                        int64_t out_features, int64_t in_features, hipStream_t stream) {
    return hxq_gemm_ws(x, x_dtype, indices, codebook, group_affine, group_size, sc_row_ptr,
                       sc_col, sc_val, bias, y, y_dtype, m_rows, out_features, in_features,
                       nullptr, 0, stream);
}

extern "C" int hxq_gemm_ws(const void *x, int32_t x_dtype, const uint8_t *indices,
                           const float *codebook, const float *group_affine, int32_t group_size,
                           const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                           const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                           int64_t out_features, int64_t in_features, void *workspace,
                           int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    return gemm_dense(x, x_dtype, indices, codebook, group_affine, group_size, sc_row_ptr, sc_col,
                      sc_val, bias, y, y_dtype, m_rows, out_features, in_features, workspace,
                      workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// hxq_gemm_noalloc: hxq_gemm_ws with the split-K partials in a static device
// array instead of a caller workspace, for callers that cannot allocate.
// The array is a file-scope __device__ symbol: every GPU the library runs on
// holds its own copy (kGemmScratchBytes) until the process ends.  Host code
// never passes the symbol itself (a host-side stand-in, not a device
// address): the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and only that pointer reaches kernels.
// The partials are fully overwritten by every call that uses them, so nothing
// needs clearing; calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
constexpr int64_t kGemmScratchBytes = int64_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kGemmScratchBytes];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices] = {};

// Device address of this device's scratch array (nullptr + error on failure).
void *scratch_of_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
        set_error("hxq_gemm_noalloc: no usable current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error(std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int64_t hxq_gemm_noalloc_max_bytes(void) { return kGemmScratchBytes; }

extern "C" int hxq_gemm_noalloc(const void *x, int32_t x_dtype, const uint8_t *indices,
                                const float *codebook, const float *group_affine,
                                int32_t group_size, const int32_t *sc_row_ptr,
                                const int32_t *sc_col, const float *sc_val, const float *bias,
                                void *y, int32_t y_dtype, int64_t m_rows, int64_t out_features,
                                int64_t in_features, hipStream_t stream) {
    clear_error();
    const int64_t need = hxq_gemm_workspace_bytes(m_rows, out_features, in_features);
    HXQ_REQUIRE(need <= kGemmScratchBytes,
                "hxq_gemm_noalloc: this shape's split-K partials need " + std::to_string(need) +
                    " bytes, more than the static " + std::to_string(kGemmScratchBytes) +
                    "-byte scratch (use hxq_gemm_ws with a workspace)");
    void *ws = nullptr;
    if (need > 0) {
        ws = scratch_of_current_device();
        if (ws == nullptr) return HXQ_ERR_HIP;
    }
    return gemm_dense(x, x_dtype, indices, codebook, group_affine, group_size, sc_row_ptr, sc_col,
                      sc_val, bias, y, y_dtype, m_rows, out_features, in_features, ws, need,
                      stream);
}

static int gemm_dense(const void *x, int32_t x_dtype, const uint8_t *indices,
                      const float *codebook, const float *group_affine, int32_t group_size,
                      const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                      const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                      int64_t out_features, int64_t in_features, void *workspace,
                      int64_t workspace_bytes, hipStream_t stream) {
    HXQ_REQUIRE(x && indices && codebook && y, "x, indices, codebook and y are required");
    HXQ_REQUIRE(x_dtype == HXQ_BF16 || x_dtype == HXQ_F16,
                "the MFMA GEMM takes bf16 or fp16 activations (fp32 goes through hxq_gemv)");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(m_rows > 0 && out_features > 0 && in_features > 0, "empty problem");
    HXQ_REQUIRE(in_features % kBK == 0, "in_features must be a multiple of 64");
    HXQ_REQUIRE(m_rows * in_features * 2 < (int64_t{1} << 31) &&
                    out_features * in_features < (int64_t{1} << 31),
                "problem too large for 32-bit offsets");
    const hxq_expert_bank bank{indices, codebook, group_affine, sc_row_ptr, sc_col, sc_val};
    if (int rc = check_bank(&bank, "weights", out_features, in_features, group_size)) return rc;
    GemmArgs a{};
    a.x = static_cast<const uint16_t *>(x);
    a.w[0] = wset_of(&bank);
    a.w[1] = a.w[0];
    a.bias = bias;
    a.y = y;
    a.M = static_cast<int32_t>(m_rows);
    a.OUT = static_cast<int32_t>(out_features);
    a.K = static_cast<int32_t>(in_features);
    a.group = group_size > 0 ? group_size : kBK;
    a.y_dtype = y_dtype;
    a.n_experts = 1;
    a.x_rows = a.M;
    a.ksplit = 1;
    a.ks_per = a.K / kBK;
    const int64_t need = hxq_gemm_workspace_bytes(m_rows, out_features, in_features);
    if (workspace != nullptr && need > 0) {
        HXQ_REQUIRE(workspace_bytes >= need, "workspace too small (hxq_gemm_workspace_bytes)");
        const SplitPlan sp = split_plan(m_rows, out_features, in_features);
        a.ksplit = sp.ksplit;
        a.ks_per = sp.ks_per;
        a.part = static_cast<float *>(workspace);
    }
    const int gx = static_cast<int>((out_features + kBN - 1) / kBN);
    const bool bf16 = x_dtype == HXQ_BF16;
    const int gy = static_cast<int>((m_rows + 127) / 128);
    const int rc = bf16 ? gemm_launch<128, true, false, false>(a, gx, gy, stream)
                        : gemm_launch<128, false, false, false>(a, gx, gy, stream);
    if (rc != HXQ_OK || a.ksplit == 1) return rc;
    const int64_t mn = m_rows * out_features;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<uint32_t>((mn + 255) / 256)),
                       dim3(256), 0, stream, a.part, a.ksplit, mn, a.OUT, bias, y, y_dtype);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_affine_pack(const float *group_scale, const float *group_offset,
                               int64_t out_features, int64_t n_groups, float *group_affine,
                               hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(group_scale && group_offset && group_affine, "all pointers are required");
    HXQ_REQUIRE(out_features > 0 && n_groups > 0 && out_features * n_groups < (int64_t{1} << 31),
                "bad sizes");
    const int64_t n = out_features * n_groups;
    hipLaunchKernelGGL(affine_pack_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                       group_scale, group_offset, (int32_t)out_features, (int32_t)n_groups,
                       reinterpret_cast<float2 *>(group_affine));
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_moe_route(const float *logits, int64_t n_tokens, int32_t n_experts,
                             int32_t top_k, int32_t renormalize, int32_t *topk_ids,
                             float *topk_weights, int32_t *expert_counts,
                             int32_t *expert_offsets, int32_t *sorted_rows, int32_t *assign_pos,
                             hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(logits && topk_ids && topk_weights && expert_counts && expert_offsets &&
                    sorted_rows && assign_pos, "all pointers are required");
    HXQ_REQUIRE(n_tokens > 0 && n_tokens * top_k < (int64_t{1} << 31), "bad n_tokens");
    HXQ_REQUIRE(n_experts >= 1 && n_experts <= 256, "n_experts must be in 1..256");
    HXQ_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= 64, "top_k must be in 1..min(n_experts, 64)");
    const int64_t n_assign = n_tokens * top_k;
    hipLaunchKernelGGL(moe_topk_kernel, dim3((n_tokens + 3) / 4), dim3(256), 0, stream,
                       logits, static_cast<int32_t>(n_tokens), n_experts, top_k, renormalize,
                       topk_ids, topk_weights);
    HXQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(moe_sort_kernel, dim3(n_experts), dim3(256), 0, stream, topk_ids, n_assign,
                       n_experts, top_k, expert_counts, expert_offsets, sorted_rows, assign_pos);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_moe_grouped_gemm(const void *x, int32_t x_dtype, int64_t x_rows,
                                    const int32_t *sorted_rows, const int32_t *expert_offsets,
                                    int64_t n_assign, int32_t n_experts,
                                    const hxq_expert_bank *bank, int32_t group_size, void *y,
                                    int32_t y_dtype, int64_t out_features, int64_t in_features,
                                    hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && expert_offsets && y, "x, expert_offsets and y are required");
    HXQ_REQUIRE(x_dtype == HXQ_BF16 || x_dtype == HXQ_F16, "x must be bf16 or fp16");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(n_experts >= 1 && n_experts <= 256, "n_experts must be in 1..256");
    HXQ_REQUIRE(n_assign > 0 && x_rows > 0 && out_features > 0 && in_features > 0, "empty problem");
    HXQ_REQUIRE(in_features % kBK == 0, "in_features must be a multiple of 64");
    HXQ_REQUIRE(x_rows * in_features * 2 < (int64_t{1} << 31), "x too large for 32-bit offsets");
    HXQ_REQUIRE(sorted_rows || x_rows >= n_assign, "without sorted_rows x holds n_assign rows");
    if (int rc = check_bank(bank, "bank", out_features, in_features, group_size)) return rc;
    if (pg::grouped_ok(bank, out_features, in_features, group_size)) {
        pg::GroupedReq r{};
        r.x = x;
        r.x_dtype = x_dtype;
        r.x_rows = x_rows;
        r.rows = sorted_rows;
        r.seg = expert_offsets;
        r.n_exp = n_experts;
        r.n_assign = n_assign;
        r.bank0 = bank;
        r.out0 = out_features;
        r.in = in_features;
        r.group = group_size;
        r.y = y;
        r.y_dtype = y_dtype;
        return pg::grouped_gemm(r, stream);
    }
    GemmArgs a{};
    a.x = static_cast<const uint16_t *>(x);
    a.rows = sorted_rows;
    a.seg = expert_offsets;
    a.w[0] = wset_of(bank);
    a.w[1] = a.w[0];
    a.y = y;
    a.M = static_cast<int32_t>(n_assign);
    a.OUT = static_cast<int32_t>(out_features);
    a.K = static_cast<int32_t>(in_features);
    a.group = group_size > 0 ? group_size : kBK;
    a.y_dtype = y_dtype;
    a.n_experts = n_experts;
    a.x_rows = static_cast<int32_t>(x_rows);
    return grouped_launch<false>(a, n_assign, x_dtype == HXQ_BF16, stream);
}

extern "C" int64_t hxq_moe_ffn_workspace_bytes(int64_t n_tokens, int64_t hidden,
                                               int64_t intermediate, int32_t top_k) {
    if (n_tokens <= 0 || hidden <= 0 || intermediate <= 0 || top_k <= 0) return -1;
    const int64_t na = n_tokens * top_k;
    // sized for fp32 activations (16-bit ones use the first half of H and GU)
    const int64_t h_bytes = ((na * intermediate * 4 + 255) / 256) * 256;
    const int64_t o_bytes = ((na * hidden * 4 + 255) / 256) * 256;
    // + the gate|up outputs of the register-dequant path
    return h_bytes + o_bytes + na * 2 * intermediate * 4 + 256;
}

extern "C" int hxq_moe_ffn(const void *x, int32_t x_dtype, int64_t n_tokens, int64_t hidden,
                           int64_t intermediate, int32_t n_experts, int32_t top_k,
                           const float *topk_weights, const int32_t *expert_offsets,
                           const int32_t *sorted_rows, const int32_t *assign_pos,
                           const hxq_expert_bank *gate, const hxq_expert_bank *up,
                           const hxq_expert_bank *down, int32_t group_size, void *workspace,
                           int64_t workspace_bytes, void *y, int32_t y_dtype,
                           hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && topk_weights && expert_offsets && sorted_rows && assign_pos && y &&
                    workspace, "all pointers are required");
    HXQ_REQUIRE(x_dtype == HXQ_BF16 || x_dtype == HXQ_F16 || x_dtype == HXQ_F32,
                "x must be fp32, bf16 or fp16");
    HXQ_REQUIRE(y_dtype >= HXQ_F32 && y_dtype <= HXQ_F16, "bad y_dtype");
    HXQ_REQUIRE(n_experts >= 1 && n_experts <= 256, "n_experts must be in 1..256");
    HXQ_REQUIRE(top_k >= 1 && top_k <= n_experts, "top_k must be in 1..n_experts");
    HXQ_REQUIRE(n_tokens > 0 && hidden > 0 && intermediate > 0, "empty problem");
    HXQ_REQUIRE(hidden % kBK == 0 && intermediate % kBK == 0,
                "hidden and intermediate must be multiples of 64");
    const int64_t na = n_tokens * top_k;
    HXQ_REQUIRE(na * std::max(hidden, intermediate) * 4 < (int64_t{1} << 31) &&
                    n_tokens * hidden * 4 < (int64_t{1} << 31),
                "problem too large for 32-bit offsets");
    const int64_t need = hxq_moe_ffn_workspace_bytes(n_tokens, hidden, intermediate, top_k);
    HXQ_REQUIRE(workspace_bytes >= need, "workspace too small (hxq_moe_ffn_workspace_bytes)");
    HXQ_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-B aligned");
    if (int rc = check_bank(gate, "gate", intermediate, hidden, group_size)) return rc;
    if (int rc = check_bank(up, "up", intermediate, hidden, group_size)) return rc;
    if (int rc = check_bank(down, "down", hidden, intermediate, group_size)) return rc;
    HXQ_REQUIRE((gate->group_affine != nullptr) == (up->group_affine != nullptr),
                "gate and up must agree on the affine");
    const bool bf16 = x_dtype == HXQ_BF16;
    const bool f32 = x_dtype == HXQ_F32;
    // H and GU hold x's type (fp32 activations: fp32 throughout)
    uint16_t *H = static_cast<uint16_t *>(workspace);
    float *O = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                         ((na * intermediate * 4 + 255) / 256) * 256);
    uint16_t *GU = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(O) + ((na * hidden * 4 + 255) / 256) * 256);
    const bool reg = pg::grouped_ok(gate, intermediate, hidden, group_size) &&
                     pg::grouped_ok(up, intermediate, hidden, group_size) &&
                     pg::grouped_ok(down, hidden, intermediate, group_size) && intermediate % 256 == 0;
    // expert outputs O: x's 16-bit type on the register-dequant path (the
    // reference's experts return x's type too), fp32 otherwise
    const int32_t o_dt = reg && !f32 ? x_dtype : HXQ_F32;
    HXQ_REQUIRE(reg || !f32, "fp32 activations need the register-dequant grouped kernel "
                             "(uint8 indices, group_size a multiple of 64, intermediate a multiple of 256)");
    if (reg) {
        // 1) GU = [X_e Wg_e^T | X_e Wu_e^T] (one grouped launch, x's 16-bit type), H = silu(G) * U
        pg::GroupedReq r{};
        r.x = x;
        r.x_dtype = x_dtype;
        r.x_rows = n_tokens;
        r.rows = sorted_rows;
        r.seg = expert_offsets;
        r.n_exp = n_experts;
        r.n_assign = na;
        r.bank0 = gate;
        r.bank1 = up;
        r.out0 = intermediate;
        r.out1 = intermediate;
        r.in = hidden;
        r.group = group_size;
        r.y = GU;
        r.y_dtype = x_dtype;
        if (int rc = pg::grouped_gemm(r, stream)) return rc;
        const int64_t n4 = na * intermediate / (f32 ? 4 : 8);  // values per thread: 4 (fp32), 8
        const dim3 sg(static_cast<uint32_t>(std::min<int64_t>((n4 + 255) / 256, 4096)));
        if (f32)
            hipLaunchKernelGGL(moe_silu_mul_f32_kernel, sg, dim3(256), 0, stream,
                               reinterpret_cast<const float *>(GU), na,
                               static_cast<int32_t>(intermediate), reinterpret_cast<float *>(H));
        else if (bf16)
            hipLaunchKernelGGL(moe_silu_mul_kernel<true>, sg, dim3(256), 0, stream, GU, na,
                               static_cast<int32_t>(intermediate), H);
        else
            hipLaunchKernelGGL(moe_silu_mul_kernel<false>, sg, dim3(256), 0, stream, GU, na,
                               static_cast<int32_t>(intermediate), H);
        HXQ_LAUNCH_CHECK();
        // 2) O = H_e Wd_e^T (sorted order; x's type: the combine sums in fp32)
        pg::GroupedReq d{};
        d.x = H;
        d.x_dtype = x_dtype;
        d.x_rows = na;
        d.rows = nullptr;
        d.seg = expert_offsets;
        d.n_exp = n_experts;
        d.n_assign = na;
        d.bank0 = down;
        d.out0 = hidden;
        d.in = intermediate;
        d.group = group_size;
        d.y = O;
        d.y_dtype = o_dt;
        if (int rc = pg::grouped_gemm(d, stream)) return rc;
    }
    if (!reg) {
        // 1) H = silu(X_e Wg_e^T) * (X_e Wu_e^T), rows in expert-sorted order
        GemmArgs a{};
        a.x = static_cast<const uint16_t *>(x);
        a.rows = sorted_rows;
        a.seg = expert_offsets;
        a.w[0] = wset_of(gate);
        a.w[1] = wset_of(up);
        a.y = H;
        a.M = static_cast<int32_t>(na);
        a.OUT = static_cast<int32_t>(intermediate);
        a.K = static_cast<int32_t>(hidden);
        a.group = group_size > 0 ? group_size : kBK;
        a.y_dtype = x_dtype;
        a.n_experts = n_experts;
        a.x_rows = static_cast<int32_t>(n_tokens);
        if (int rc = grouped_launch<true>(a, na, bf16, stream)) return rc;
        // 2) O = H_e Wd_e^T (fp32, sorted order)
        GemmArgs d{};
        d.x = H;
        d.rows = nullptr;
        d.seg = expert_offsets;
        d.w[0] = wset_of(down);
        d.w[1] = d.w[0];
        d.y = O;
        d.M = static_cast<int32_t>(na);
        d.OUT = static_cast<int32_t>(hidden);
        d.K = static_cast<int32_t>(intermediate);
        d.group = a.group;
        d.y_dtype = HXQ_F32;
        d.n_experts = n_experts;
        d.x_rows = static_cast<int32_t>(na);
        if (int rc = grouped_launch<false>(d, na, bf16, stream)) return rc;
    }
    // 3) y[t] = sum_s w[t,s] O[pos(t,s)]
    const bool v4 = hidden % 4 == 0;
    const dim3 grid((hidden + (v4 ? 1023 : 255)) / (v4 ? 1024 : 256), n_tokens);
#define HXQ_COMBINE(OT, YDT)                                                                 \
    do {                                                                                      \
        if (v4)                                                                               \
            hipLaunchKernelGGL((moe_combine_kernel<OT, YDT, 4>), grid, dim3(256), 0, stream, O, \
                               topk_weights, assign_pos, top_k, static_cast<int32_t>(hidden), y); \
        else                                                                                  \
            hipLaunchKernelGGL((moe_combine_kernel<OT, YDT, 1>), grid, dim3(256), 0, stream, O, \
                               topk_weights, assign_pos, top_k, static_cast<int32_t>(hidden), y); \
    } while (0)
#define HXQ_COMBINE_Y(OT)                                                                    \
    do {                                                                                      \
        if (y_dtype == HXQ_F32) HXQ_COMBINE(OT, HXQ_F32);                                     \
        else if (y_dtype == HXQ_BF16) HXQ_COMBINE(OT, HXQ_BF16);                              \
        else HXQ_COMBINE(OT, HXQ_F16);                                                        \
    } while (0)
    if (o_dt == HXQ_F32) HXQ_COMBINE_Y(HXQ_F32);
    else if (o_dt == HXQ_BF16) HXQ_COMBINE_Y(HXQ_BF16);
    else HXQ_COMBINE_Y(HXQ_F16);
#undef HXQ_COMBINE_Y
#undef HXQ_COMBINE
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}
