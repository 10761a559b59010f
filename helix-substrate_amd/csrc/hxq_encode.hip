// CDNAv3 encoder on the GPU: 1-D k-means codebook, nearest-codebook
// assignment and percentile outliers (the sidecar), and the pair-codebook
// (vector_dim 2) k-means steps, with the reference's CPU results reproduced
// bit for bit.
//
// Reference (helix_substrate/hxq_encoder.py:107-177 _simple_kmeans,
// hxq_writer_v3.py:427-470 _build_kmeans_codebook / _chunked_assign,
// generate_sidecars_v3.py:18-40 find_outliers_percentile) computes with
// numpy; the arithmetic restated here is numpy's:
//   * assignment: argmin_j |fl(x - c_j)| in fp32, first index on ties, NaN
//     distances win (numpy argmin returns the first NaN);
//   * cluster mean: np.mean of the members in index order = fp32 sum over
//     consecutive 8192-element blocks, each block summed pairwise (blocks of
//     <= 128 with eight running sums, larger ones split at n/2 rounded down
//     to a multiple of 8), divided by the count in fp32;
//   * percentiles: numpy's 'linear' method on the sorted data (virtual index
//     (n-1) q, lerp a + (b-a) t for t < 1/2 else b - (b-a)(1-t)); fp64 for
//     the k-means initialisation (an array of percentiles), fp32 for the
//     sidecar thresholds (a scalar percentile of fp32 data);
//   * convergence: max |new - old| (fp32) < rtol * (c_last - c_first).
// Every reduction is integer or follows that fixed order: results are
// deterministic and independent of the launch shape.
#include <cfloat>
#include <cmath>

#include "hxq_common.h"

namespace hxq {
namespace enc {

constexpr int kThreads = 256;
constexpr int kMaxK = 256;     // scalar codebooks with uint8 indices
constexpr int kMaxKW = 4096;   // wide scalar codebooks (uint16 indices)

// fp32 -> uint32 whose unsigned order is numpy's sort order (NaN last).
__device__ __forceinline__ uint32_t sort_key(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
    if (k == 0xffffffffu) return __uint_as_float(0x7fc00000u);
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// ---------------------------------------------------------------------------
// nearest codebook entry
// ---------------------------------------------------------------------------
__device__ __forceinline__ float absdiff(float x, float c) {
#pragma clang fp contract(off)
    return fabsf(x - c);
}

// General scan: first index of the minimum; a NaN distance is a minimum.
__device__ __forceinline__ int nearest_scan(float x, const float *cb, int k) {
    int best = 0;
    float bd = absdiff(x, cb[0]);
    if (bd != bd) return 0;
    for (int j = 1; j < k; ++j) {
        const float d = absdiff(x, cb[j]);
        if (d != d) return j;
        if (d < bd) { bd = d; best = j; }
    }
    return best;
}

// Sorted (non-decreasing, no NaN) codebook: the distances fall then rise
// with j, so the minimum is at the last entry <= x or the first entry > x,
// and the first index holding the minimum value is found by a second
// binary search over the falling part.
__device__ __forceinline__ int nearest_sorted(float x, const float *cb, int k) {
    if (x != x) return 0;
    // hi = first j with cb[j] > x (k if none)
    int lo = 0, hi = k;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (cb[mid] > x) hi = mid; else lo = mid + 1;
    }
    const int jr = hi;           // first entry > x
    const int jl = hi - 1;       // last entry <= x
    float dmin;
    if (jl < 0) return 0;        // every entry > x: distances rise from j = 0
    dmin = absdiff(x, cb[jl]);
    const bool right_wins = jr < k && absdiff(x, cb[jr]) < dmin;
    if (right_wins) return jr;
    // first j <= jl with |x - cb[j]| == dmin (distances non-increasing on [0, jl])
    int a = 0, b = jl;
    while (a < b) {
        const int mid = (a + b) >> 1;
        if (absdiff(x, cb[mid]) <= dmin) b = mid; else a = mid + 1;
    }
    return a;
}

// Codebook staged in LDS; `sorted` decided by the block (uniform).
__device__ __forceinline__ bool stage_codebook(const float *cb, int k, float *s_cb, int *s_flag) {
    if (threadIdx.x == 0) *s_flag = 1;
    __syncthreads();
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
        const float v = cb[j];
        s_cb[j] = v;
        // finite and non-decreasing: the binary-search path applies
        if (!isfinite(v) || (j + 1 < k && !(v <= cb[j + 1]))) *s_flag = 0;
    }
    __syncthreads();
    return *s_flag != 0;
}

template <typename IT, int KM>
__global__ __launch_bounds__(kThreads) void assign_kernel(const float *x, int64_t n, const float *cb,
                                                          int k, IT *idx) {
    __shared__ float s_cb[KM];
    __shared__ int s_flag;
    const bool sorted = stage_codebook(cb, k, s_cb, &s_flag);
    for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float v = x[i];
        idx[i] = static_cast<IT>(sorted ? nearest_sorted(v, s_cb, k) : nearest_scan(v, s_cb, k));
    }
}

// ---------------------------------------------------------------------------
// bitonic sort of keys (n padded to a power of two with 0xffffffff)
// ---------------------------------------------------------------------------
constexpr int kSortBlock = 2048;  // elements per block in the LDS stages

__global__ __launch_bounds__(kThreads) void keys_kernel(const float *x, int64_t n, int64_t np2,
                                                        uint32_t *keys) {
    for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < np2;
         i += (int64_t)gridDim.x * kThreads)
        keys[i] = i < n ? sort_key(x[i]) : 0xffffffffu;
}

// one global compare-exchange step (k, j >= kSortBlock / 2)
__global__ __launch_bounds__(kThreads) void bitonic_global(uint32_t *keys, int64_t np2, int64_t k,
                                                           int64_t j) {
    for (int64_t t = blockIdx.x * (int64_t)kThreads + threadIdx.x; t < np2 / 2;
         t += (int64_t)gridDim.x * kThreads) {
        const int64_t i = ((t / j) * 2 * j) + (t % j);
        const int64_t p = i + j;
        const bool up = (i & k) == 0;
        const uint32_t a = keys[i], b = keys[p];
        if ((a > b) == up) { keys[i] = b; keys[p] = a; }
    }
}

// all steps j < kSortBlock of stage k (or stages 2..kSortBlock when k == 0), in LDS
__global__ __launch_bounds__(kThreads) void bitonic_local(uint32_t *keys, int64_t k_stage) {
    __shared__ uint32_t s[kSortBlock];
    const int64_t base = blockIdx.x * (int64_t)kSortBlock;
    for (int i = threadIdx.x; i < kSortBlock; i += kThreads) s[i] = keys[base + i];
    __syncthreads();
    const int64_t k_lo = k_stage == 0 ? 2 : k_stage;
    const int64_t k_hi = k_stage == 0 ? kSortBlock : k_stage;
    for (int64_t k = k_lo; k <= k_hi; k <<= 1) {
        for (int j = static_cast<int>(min<int64_t>(k >> 1, kSortBlock >> 1)); j > 0; j >>= 1) {
            for (int t = threadIdx.x; t < kSortBlock / 2; t += kThreads) {
                const int i = ((t / j) * 2 * j) + (t % j);
                const int p = i + j;
                const bool up = ((base + i) & k) == 0;
                const uint32_t a = s[i], b = s[p];
                if ((a > b) == up) { s[i] = b; s[p] = a; }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < kSortBlock; i += kThreads) keys[base + i] = s[i];
}

// ---------------------------------------------------------------------------
// k-means initialisation and bookkeeping
// ---------------------------------------------------------------------------
// distinct values of the sorted keys (NaNs count once, as np.unique)
__global__ void zero_i32_kernel(int32_t *p) { *p = 0; }

__global__ __launch_bounds__(kThreads) void count_unique_kernel(const uint32_t *keys, int64_t n,
                                                                int32_t *count) {
    __shared__ int32_t s;
    if (threadIdx.x == 0) s = 0;
    __syncthreads();
    int32_t c = 0;
    for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        if (i == 0) { ++c; continue; }
        const uint32_t a = keys[i - 1], b = keys[i];
        // +0.0 and -0.0 are equal values
        const bool same = a == b || (key_float(a) == key_float(b));
        c += !same;
    }
    atomicAdd(&s, c);
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(count, s);
}

// centroid j = percentile(data, q_j) with numpy's fp64 'linear' lerp, as fp32
__global__ __launch_bounds__(kMaxK) void kmeans_init_kernel(const uint32_t *keys, int64_t n, const double *q, int k,
                                   float *cb, double rtol, double *abs_tol, int32_t *done,
                                   int32_t *iters) {
#pragma clang fp contract(off)
    // numpy's percentile is NaN for every q once the data holds a NaN
    // (sorted last)
    const bool has_nan = keys[n - 1] == 0xffffffffu;
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
        const double v = static_cast<double>(n - 1) * q[j];
        double r;
        if (has_nan) {
            r = static_cast<double>(key_float(0xffffffffu));
        } else if (v >= static_cast<double>(n - 1)) {
            r = static_cast<double>(key_float(keys[n - 1]));
        } else {
            const int64_t i = static_cast<int64_t>(floor(v));
            const double t = v - static_cast<double>(i);
            const float a = key_float(keys[i]), b = key_float(keys[i + 1]);
            const double d = static_cast<double>(b - a);  // fp32 difference
            r = t >= 0.5 ? static_cast<double>(b) - d * (1.0 - t) : static_cast<double>(a) + d * t;
        }
        cb[j] = static_cast<float>(r);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double range = static_cast<double>(cb[k - 1] - cb[0]);
        if (range < 1e-30) range = 1.0;
        *abs_tol = rtol * range;
        *done = 0;
        *iters = 0;
    }
}

// Lloyd step 1: assignment + per-block cluster counts.  Block b owns the
// contiguous elements [b * per, (b + 1) * per).
template <typename IT, int KM>
__global__ __launch_bounds__(kThreads) void km_assign_kernel(const float *x, int64_t n, int64_t per,
                                                             const float *cb, int k, IT *idx,
                                                             int32_t *blk_counts, const int32_t *done) {
    if (*done) return;
    __shared__ float s_cb[KM];
    __shared__ int s_flag;
    __shared__ int32_t s_cnt[KM];
    for (int j = threadIdx.x; j < KM; j += kThreads) s_cnt[j] = 0;
    const bool sorted = stage_codebook(cb, k, s_cb, &s_flag);
    const int64_t lo = blockIdx.x * per, hi = min(n, lo + per);
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) {
        const float v = x[i];
        const int c = sorted ? nearest_sorted(v, s_cb, k) : nearest_scan(v, s_cb, k);
        idx[i] = static_cast<IT>(c);
        atomicAdd(&s_cnt[c], 1);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < k; j += kThreads) blk_counts[blockIdx.x * (int64_t)k + j] = s_cnt[j];
}

// Lloyd step 2: exclusive offsets, cluster-major then block order (stable)
template <int KM>
__global__ __launch_bounds__(kThreads) void km_offsets_kernel(int32_t *blk_counts, int nblk, int k, int32_t *starts,
                                  int32_t *counts, const int32_t *done) {
    if (*done) return;
    __shared__ int32_t tot[KM];
    for (int j = threadIdx.x; j < k; j += kThreads) {
        int32_t s = 0;
        for (int b = 0; b < nblk; ++b) {
            const int32_t c = blk_counts[(int64_t)b * k + j];
            blk_counts[(int64_t)b * k + j] = s;  // offset within cluster j
            s += c;
        }
        tot[j] = s;
        counts[j] = s;
    }
    __syncthreads();
    const int j = threadIdx.x;
    if (j == 0) {
        int32_t s = 0;
        for (int c = 0; c < k; ++c) { starts[c] = s; s += tot[c]; }
    }
}

// Lloyd step 3: stable scatter of the values into cluster-contiguous order
// (within a cluster, elements keep their index order)
template <typename IT, int KM>
__global__ __launch_bounds__(kThreads) void km_scatter_kernel(const float *x, int64_t n, int64_t per,
                                                              const IT *idx, const int32_t *blk_offs,
                                                              const int32_t *starts, int k, float *out,
                                                              const int32_t *done) {
    if (*done) return;
    constexpr int W = kThreads / kWave;
    __shared__ int32_t base[KM];
    __shared__ int32_t wcnt[W][KM];
    for (int j = threadIdx.x; j < k; j += kThreads)
        base[j] = starts[j] + blk_offs[blockIdx.x * (int64_t)k + j];
    const int lane = threadIdx.x & 63, w = threadIdx.x / kWave;
    const int64_t lo = blockIdx.x * per, hi = min(n, lo + per);
    for (int64_t c0 = lo; c0 < hi; c0 += kThreads) {
        for (int j = threadIdx.x; j < W * KM; j += kThreads) (&wcnt[0][0])[j] = 0;
        __syncthreads();
        const int64_t i = c0 + threadIdx.x;
        const bool ok = i < hi;
        const int c = ok ? idx[i] : -1;
        // rank among earlier lanes of this wave with the same cluster
        int r = 0;
        for (int l = 0; l < kWave; ++l) {
            const int cl = __shfl(c, l, kWave);
            r += (l < lane && cl == c);
        }
        if (ok) atomicAdd(&wcnt[w][c], 1);
        __syncthreads();
        if (ok) {
            int32_t pos = base[c] + r;
            for (int ww = 0; ww < w; ++ww) pos += wcnt[ww][c];
            out[pos] = x[i];
        }
        __syncthreads();
        for (int j = threadIdx.x; j < k; j += kThreads) {
            int32_t s = 0;
            for (int ww = 0; ww < W; ++ww) s += wcnt[ww][j];
            base[j] += s;
        }
        __syncthreads();
    }
}

// numpy's pairwise sum of fp32 (blocks of <= 128: eight running sums)
__device__ float pairwise_leaf(const float *a, int n) {
#pragma clang fp contract(off)
    if (n < 8) {
        float r = 0.f;
        for (int i = 0; i < n; ++i) r += a[i];
        return r;
    }
    float r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int i = 8;
    for (; i < n - (n % 8); i += 8)
        for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
}

// Leaves of numpy's pairwise tree over n <= 8192 elements, left to right:
// ranges of <= 128 elements (nodes above 128 split at n/2 rounded down to a
// multiple of 8, so every leaf has at least 64 elements: at most 128 leaves).
__device__ int pairwise_leaves(int n, int *loff, int *llen) {
    int so[16], sl[16];
    int sp = 1, nl = 0;
    so[0] = 0;
    sl[0] = n;
    while (sp > 0) {
        --sp;
        const int o = so[sp], m = sl[sp];
        if (m <= 128) {
            loff[nl] = o;
            llen[nl] = m;
            ++nl;
            continue;
        }
        int m2 = m / 2;
        m2 -= m2 % 8;
        so[sp] = o + m2;  // right, visited after the left subtree
        sl[sp] = m - m2;
        ++sp;
        so[sp] = o;
        sl[sp] = m2;
        ++sp;
    }
    return nl;
}

// pairwise_sum with the leaf sums given (in leaf order): the same tree and
// the same additions
__device__ float pairwise_combine(int n, const float *lsum) {
#pragma clang fp contract(off)
    if (n <= 128) return lsum[0];
    int len[16], st[16];
    float left[16];
    int sp = 0, li = 0;
    len[0] = n;
    st[0] = 0;
    float ret = 0.f;
    while (sp >= 0) {
        const int m = len[sp];
        if (m <= 128) {
            ret = lsum[li++];
            --sp;
            continue;
        }
        int m2 = m / 2;
        m2 -= m2 % 8;
        if (st[sp] == 0) {
            st[sp] = 1;
            ++sp; len[sp] = m2; st[sp] = 0;
        } else if (st[sp] == 1) {
            left[sp] = ret;
            st[sp] = 2;
            ++sp; len[sp] = m - m2; st[sp] = 0;
        } else {
            ret = left[sp] + ret;
            --sp;
        }
    }
    return ret;
}

// Lloyd step 4a: cluster means, one block per cluster: per 8192-element
// block of the cluster's members, thread 0 lists the pairwise leaves, the
// threads sum one leaf each, thread 0 combines them in tree order; block sums
// are added in order and divided by the count (numpy's np.mean, bit for bit).
// Empty clusters keep their centroid.
__global__ __launch_bounds__(kThreads) void km_sum_kernel(const float *sorted_vals, const int32_t *starts,
                                                          const int32_t *counts, const float *cb,
                                                          float *means, const int32_t *done) {
#pragma clang fp contract(off)
    if (*done) return;
    __shared__ int loff[128], llen[128];
    __shared__ float lsum[128];
    __shared__ int s_nl;
    const int j = blockIdx.x;
    const int32_t c = counts[j];
    if (c == 0) {
        if (threadIdx.x == 0) means[j] = cb[j];
        return;
    }
    const float *a = sorted_vals + starts[j];
    float sum = 0.f;
    for (int32_t s = 0; s < c; s += 8192) {
        const int m = min(8192, c - s);
        if (threadIdx.x == 0) s_nl = pairwise_leaves(m, loff, llen);
        __syncthreads();
        const int nl = s_nl;
        for (int i = threadIdx.x; i < nl; i += kThreads) lsum[i] = pairwise_leaf(a + s + loff[i], llen[i]);
        __syncthreads();
        if (threadIdx.x == 0) {
            const float p = pairwise_combine(m, lsum);
            sum = s == 0 ? p : sum + p;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) means[j] = sum / static_cast<float>(c);
}

// Lloyd step 4b: movement and convergence over the k new means.
template <int KM>
__global__ __launch_bounds__(kThreads) void km_update_kernel(const float *means, int k, float *cb,
                                                          const double *abs_tol, int32_t *done,
                                                          int32_t *iters) {
#pragma clang fp contract(off)
    if (*done) return;
    __shared__ float s_new[KM];
    __shared__ float s_delta[KM];
    __shared__ int s_conv;
    for (int j = threadIdx.x; j < k; j += kThreads) {
        const float v = means[j];
        s_new[j] = v;
        s_delta[j] = fabsf(v - cb[j]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = 0.f;
        bool nan = false;
        for (int c = 0; c < k; ++c) {
            nan |= s_delta[c] != s_delta[c];
            m = fmaxf(m, s_delta[c]);
        }
        // numpy's max propagates NaN; NaN < tol is false: no convergence
        const bool conv = !nan && static_cast<double>(m) < *abs_tol;
        s_conv = conv ? 1 : 0;
        *iters += 1;
        if (conv) *done = 1;
    }
    __syncthreads();
    if (s_conv == 0)
        for (int j = threadIdx.x; j < k; j += kThreads) cb[j] = s_new[j];
}

// ---------------------------------------------------------------------------
// radix select (exact order statistics of up to 4 ranks) and outliers
// ---------------------------------------------------------------------------
constexpr int kSelMax = 4;

struct SelState {
    uint32_t prefix[kSelMax];  // key bits fixed so far
    uint32_t rank[kSelMax];    // rank within the keys matching prefix
    uint32_t hist[kSelMax][256];
    int32_t nan_count;
    int32_t pad_;
};

__global__ __launch_bounds__(kThreads) void select_hist_kernel(const float *x, int64_t n, int m,
                                                               int shift, SelState *st) {
    __shared__ uint32_t h[kSelMax][256];
    for (int i = threadIdx.x; i < kSelMax * 256; i += kThreads) (&h[0][0])[i] = 0;
    __syncthreads();
    uint32_t pre[kSelMax];
    for (int r = 0; r < m; ++r) pre[r] = st->prefix[r];
    const uint32_t hi_mask = shift >= 24 ? 0u : (0xffffffffu << (shift + 8));
    int32_t nans = 0;
    for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const uint32_t key = sort_key(x[i]);
        if (shift == 24 && key == 0xffffffffu) ++nans;
        const uint32_t d = (key >> shift) & 0xffu;
        for (int r = 0; r < m; ++r)
            if ((key & hi_mask) == (pre[r] & hi_mask)) atomicAdd(&h[r][d], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < m * 256; i += kThreads) {
        const uint32_t v = (&h[0][0])[i];
        if (v) atomicAdd(&st->hist[i / 256][i % 256], v);
    }
    if (shift == 24 && nans) atomicAdd(&st->nan_count, nans);
}

__global__ void select_pick_kernel(int m, int shift, SelState *st, float *out) {
    const int r = threadIdx.x;
    if (r < m) {
        uint32_t rank = st->rank[r];
        int d = 0;
        for (; d < 255; ++d) {
            const uint32_t c = st->hist[r][d];
            if (rank < c) break;
            rank -= c;
        }
        st->prefix[r] |= static_cast<uint32_t>(d) << shift;
        st->rank[r] = rank;
        for (int i = 0; i < 256; ++i) st->hist[r][i] = 0;
        if (shift == 0) out[r] = key_float(st->prefix[r]);
    }
}

__global__ void select_init_kernel(const int64_t *ranks, int m, SelState *st) {
    for (int i = threadIdx.x; i < kSelMax * 256; i += blockDim.x) (&st->hist[0][0])[i] = 0;
    if (threadIdx.x < kSelMax) {
        st->prefix[threadIdx.x] = 0;
        st->rank[threadIdx.x] = threadIdx.x < m ? static_cast<uint32_t>(ranks[threadIdx.x]) : 0;
    }
    if (threadIdx.x == 0) st->nan_count = 0;
}

// outliers: x < lo or x > hi, positions ascending (two passes)
__global__ __launch_bounds__(kThreads) void outlier_count_kernel(const float *x, int64_t n, int64_t per,
                                                                 const float *lohi, int32_t *blk) {
    __shared__ int32_t s;
    if (threadIdx.x == 0) s = 0;
    __syncthreads();
    const float lo = lohi[0], hi = lohi[1];
    const int64_t a = blockIdx.x * per, b = min(n, a + per);
    int32_t c = 0;
    for (int64_t i = a + threadIdx.x; i < b; i += kThreads) {
        const float v = x[i];
        c += (v < lo) | (v > hi);
    }
    atomicAdd(&s, c);
    __syncthreads();
    if (threadIdx.x == 0) blk[blockIdx.x] = s;
}

__global__ void outlier_scan_kernel(int32_t *blk, int nblk, int64_t *total) {
    if (threadIdx.x == 0) {
        int64_t s = 0;
        for (int b = 0; b < nblk; ++b) { const int32_t c = blk[b]; blk[b] = static_cast<int32_t>(s); s += c; }
        *total = s;
    }
}

__global__ __launch_bounds__(kThreads) void outlier_write_kernel(const float *x, int64_t n, int64_t per,
                                                                 const float *lohi, const int32_t *blk,
                                                                 int64_t cap, int64_t *pos, float *val) {
    constexpr int W = kThreads / kWave;
    __shared__ int32_t wsum[W];
    __shared__ int32_t base;
    if (threadIdx.x == 0) base = blk[blockIdx.x];
    const float lo = lohi[0], hi = lohi[1];
    const int lane = threadIdx.x & 63, w = threadIdx.x / kWave;
    const int64_t a = blockIdx.x * per, b = min(n, a + per);
    for (int64_t c0 = a; c0 < b; c0 += kThreads) {
        const int64_t i = c0 + threadIdx.x;
        const float v = i < b ? x[i] : 0.f;
        const bool hit = i < b && ((v < lo) | (v > hi));
        const uint64_t mask = __ballot(hit);
        const int r = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0) wsum[w] = __popcll(mask);
        __syncthreads();
        if (hit) {
            int64_t p = base + r;
            for (int ww = 0; ww < w; ++ww) p += wsum[ww];
            if (p < cap) { pos[p] = i; val[p] = v; }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int32_t s = 0;
            for (int ww = 0; ww < W; ++ww) s += wsum[ww];
            base += s;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// per-group affine fit: (s, o) = argmin sum_j (s c_j + o - w_j)^2 over the
// group's elements not in the sidecar, c_j = codebook[idx_j]; fp64 sums in a
// fixed order (lane l of the group's wave adds elements l, l+64, ... in turn,
// then a xor butterfly 32, 16, ..., 1), closed-form solution in fp64, fp32
// results.  Degenerate groups (n < 2 or a zero determinant) keep s = 1 and
// take o = mean(w - c) (0 for an empty group).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void mark_kernel(const int64_t *pos, int64_t m, uint32_t *bits) {
    for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < m;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t p = pos[i];
        atomicOr(&bits[p >> 5], 1u << (p & 31));
    }
}

__global__ __launch_bounds__(kThreads) void zero_u32_kernel(uint32_t *p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads)
        p[i] = 0u;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma clang fp contract(off)
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, kWave);
    return v;
}

template <typename IT, int KM>
__global__ __launch_bounds__(kThreads) void affine_fit_kernel(const float *w, const IT *idx,
                                                              const float *cb, int k, int64_t rows,
                                                              int64_t cols, int group,
                                                              const uint32_t *bits, float *scale,
                                                              float *offset) {
#pragma clang fp contract(off)
    __shared__ float s_cb[KM];
    for (int j = threadIdx.x; j < KM; j += kThreads) s_cb[j] = j < k ? cb[j] : 0.f;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t ngroups = cols / group;
    const int64_t unit = blockIdx.x * (int64_t)(kThreads / kWave) + threadIdx.x / kWave;
    if (unit >= rows * ngroups) return;
    const int64_t r = unit / ngroups, g = unit % ngroups;
    const int64_t base = r * cols + g * group;
    double sc = 0.0, sw = 0.0, scc = 0.0, scw = 0.0, sn = 0.0;
    for (int t = lane; t < group; t += kWave) {
        const int64_t e = base + t;
        const bool skip = bits && ((bits[e >> 5] >> (e & 31)) & 1u);
        if (!skip) {
            // an index past the table (a caller error) reads a zero entry, in bounds
            const double c = static_cast<double>(s_cb[min(static_cast<int>(idx[e]), KM - 1)]);
            const double x = static_cast<double>(w[e]);
            sc = sc + c;
            sw = sw + x;
            scc = scc + c * c;
            scw = scw + c * x;
            sn = sn + 1.0;
        }
    }
    sc = wave_sum_f64(sc);
    sw = wave_sum_f64(sw);
    scc = wave_sum_f64(scc);
    scw = wave_sum_f64(scw);
    sn = wave_sum_f64(sn);
    if (lane == 0) {
        double s = 1.0, o = 0.0;
        const double det = sn * scc - sc * sc;
        if (sn >= 2.0 && det > 0.0) {
            s = (sn * scw - sc * sw) / det;
            o = (sw - s * sc) / sn;
        } else if (sn > 0.0) {
            o = (sw - sc) / sn;
        }
        scale[r * ngroups + g] = static_cast<float>(s);
        offset[r * ngroups + g] = static_cast<float>(o);
    }
}

static int grid_for(int64_t n) {
    const int64_t g = (n + kThreads - 1) / kThreads;
    return static_cast<int>(std::min<int64_t>(std::max<int64_t>(g, 1), 8192));
}

static int64_t next_pow2(int64_t n) {
    int64_t p = kSortBlock;
    while (p < n) p <<= 1;
    return p;
}


// ---------------------------------------------------------------------------
// pair (vector_dim 2) codebook: nearest centroid and centroid update
// ---------------------------------------------------------------------------
// The reference's numpy arithmetic (hxq_encoder.py:280-300):
//   d_j = fl(fl(|x|^2 + |c_j|^2) - 2 x.c_j), |v|^2 = fl(fl(v0*v0) + fl(v1*v1)),
//   x.c = fma(x1, c1, fl(x0*c0)) (what numpy's sgemm gives a K = 2 product),
//   first index of the minimum;  new c_j = fp32(fp64 sum / fp32 count).
// 2 x.c is exact, so fl(t - fl(2 x.c)) is the single rounding fma(-2, x.c, t).
constexpr int kPairMaxK = 4096;
constexpr int kPairThreads = 512;
constexpr int kUpdThreads = 1024;     // one owner thread per cluster id mod 1024
constexpr int kUpdChunk = 1024;       // ids staged in LDS per pass
constexpr int kUpdMaxBlocks = 512;
constexpr int kUpdSlots = kPairMaxK / kUpdThreads;

// {c0, c1, |c|^2, 0} per centroid.
__global__ __launch_bounds__(256) void pair_table_kernel(const float *__restrict__ cb, int k,
                                                         float4 *__restrict__ tab) {
#pragma clang fp contract(off)
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j < k) {
        const float c0 = cb[2 * j], c1 = cb[2 * j + 1];
        tab[j] = make_float4(c0, c1, c0 * c0 + c1 * c1, 0.0f);
    }
}

// V pairs per thread (pair i = block base + threadIdx.x + v * kPairThreads);
// the table is staged once per block in LDS and read as a broadcast.
// MIN: writes dmin[i] = max(min_j d_j, 0) instead of the index (the k-means++
// seeding distance, np.maximum(d, 0).min(axis=1)), for the rows rows[i] of x
// when rows is given (an out-of-range row gives NaN).
template <int V, bool MIN>
__global__ __launch_bounds__(kPairThreads) void pair_assign_kernel(
    const float2 *__restrict__ x, int64_t n, const int64_t *__restrict__ rows, int64_t m,
    const float4 *__restrict__ tab, int k, uint16_t *__restrict__ idx, float *__restrict__ dmin) {
#pragma clang fp contract(off)
    extern __shared__ float4 stab[];
    for (int j = threadIdx.x; j < k; j += kPairThreads) stab[j] = tab[j];
    __syncthreads();
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kPairThreads * V) + threadIdx.x;
    float x0[V], x1[V], xsq[V], best[V];
    int bj[V];
    const float4 c = stab[0];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int64_t i = base + static_cast<int64_t>(v) * kPairThreads;
        int64_t r = i;
        if (MIN && rows != nullptr && i < m) r = rows[i];
        float2 p = make_float2(0.0f, 0.0f);
        if (i < m) p = (r >= 0 && r < n) ? x[r] : make_float2(NAN, NAN);
        x0[v] = p.x;
        x1[v] = p.y;
        xsq[v] = p.x * p.x + p.y * p.y;
        best[v] = fmaf(-2.0f, fmaf(x1[v], c.y, x0[v] * c.x), xsq[v] + c.z);
        bj[v] = 0;
    }
    if constexpr (MIN) {
        for (int j = 1; j < k; ++j) {
            const float4 cj = stab[j];
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const float d = fmaf(-2.0f, fmaf(x1[v], cj.y, x0[v] * cj.x), xsq[v] + cj.z);
                if (d < best[v]) best[v] = d;
            }
        }
    } else {
        // Entries in groups of 8: the group's minimum (fminf skips NaN, as the
        // strict compare does) replaces the best only if strictly smaller, and
        // only then is its first index looked up -- the same (value, first
        // index) as a strict-compare scan, with the index work done on the
        // few groups that improve.  Entries past k read entry k - 1 again; it
        // sits earlier in the same group, so a tie never picks the copy.
        for (int j0 = 1; j0 < k; j0 += 8) {
            float4 cg[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) cg[t] = stab[min(j0 + t, k - 1)];
#pragma unroll
            for (int v = 0; v < V; ++v) {
                float d[8];
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    d[t] = fmaf(-2.0f, fmaf(x1[v], cg[t].y, x0[v] * cg[t].x), xsq[v] + cg[t].z);
                const float g = fminf(fminf(fminf(d[0], d[1]), fminf(d[2], d[3])),
                                      fminf(fminf(d[4], d[5]), fminf(d[6], d[7])));
                if (g < best[v]) {
                    int at = j0 + 7;
#pragma unroll
                    for (int t = 6; t >= 0; --t) at = d[t] == g ? j0 + t : at;
                    best[v] = g;
                    bj[v] = at;
                }
            }
        }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int64_t i = base + static_cast<int64_t>(v) * kPairThreads;
        if (i < m) {
            if (MIN)
                dmin[i] = best[v] >= 0.0f || best[v] != best[v] ? best[v] : 0.0f;
            else
                idx[i] = static_cast<uint16_t>(bj[v]);
        }
    }
}

// fp64 sums and counts per cluster over one block's range of pairs.  Thread
// t = 64 * wave + lane owns the ids with id % 1024 == t and adds their pairs
// in index order, so the partials do not depend on timing.  The ids are
// wave-uniform (read from LDS, made scalar), so the owner test is a scalar
// branch and only the owning lane does vector work.  Block 0 clears
// *max_delta for the finish kernel that follows on the stream.
__global__ __launch_bounds__(kUpdThreads) void pair_partial_kernel(
    const float2 *__restrict__ x, int64_t n, const uint16_t *__restrict__ idx, int k,
    int64_t per_block, double *__restrict__ psum, uint32_t *__restrict__ pcnt,
    float *__restrict__ max_delta) {
    __shared__ uint16_t sidx[kUpdChunk];
    __shared__ float2 sx[kUpdChunk];
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    if (blockIdx.x == 0 && t == 0) *max_delta = 0.0f;
    double s0[kUpdSlots], s1[kUpdSlots];
    uint32_t cnt[kUpdSlots];
#pragma unroll
    for (int s = 0; s < kUpdSlots; ++s) {
        s0[s] = 0.0;
        s1[s] = 0.0;
        cnt[s] = 0;
    }
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t hi = lo + per_block < n ? lo + per_block : n;
    for (int64_t b = lo; b < hi; b += kUpdChunk) {
        const int m = static_cast<int>(hi - b < kUpdChunk ? hi - b : kUpdChunk);
        __syncthreads();
        if (t < m) {
            sidx[t] = idx[b + t];
            sx[t] = x[b + t];
        }
        __syncthreads();
        for (int i = 0; i < m; ++i) {
            const int id = __builtin_amdgcn_readfirstlane(static_cast<int>(sidx[i]));
            if (((id >> 6) & 15) != wave) continue;
            if (lane != (id & 63)) continue;
            const float2 v = sx[i];
            const int slot = id >> 10;
#pragma unroll
            for (int s = 0; s < kUpdSlots; ++s) {
                if (slot == s) {
                    s0[s] += static_cast<double>(v.x);
                    s1[s] += static_cast<double>(v.y);
                    cnt[s] += 1;
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < kUpdSlots; ++s) {
        const int j = s * kUpdThreads + t;
        if (j < k) {
            psum[(2 * static_cast<int64_t>(blockIdx.x)) * k + j] = s0[s];
            psum[(2 * static_cast<int64_t>(blockIdx.x) + 1) * k + j] = s1[s];
            pcnt[static_cast<int64_t>(blockIdx.x) * k + j] = cnt[s];
        }
    }
}

// Adds the block partials in a fixed order (wave w of 16 takes blocks w,
// w + 16, ... in turn; the 16 wave totals are then added in wave order),
// writes the new centroids (empty clusters keep the old one) and raises
// *max_delta to max |new - old| (non-negative floats order as their bits).
__global__ __launch_bounds__(1024) void pair_finish_kernel(
    const double *__restrict__ psum, const uint32_t *__restrict__ pcnt, int nparts, int k,
    const float *__restrict__ old, float *__restrict__ out, float *__restrict__ max_delta) {
    __shared__ double l0[16][64], l1[16][64];
    __shared__ uint32_t lc[16][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane;
    double a0 = 0.0, a1 = 0.0;
    uint32_t c = 0;
    if (j < k) {
        for (int p = w; p < nparts; p += 16) {
            a0 += psum[(2 * static_cast<int64_t>(p)) * k + j];
            a1 += psum[(2 * static_cast<int64_t>(p) + 1) * k + j];
            c += pcnt[static_cast<int64_t>(p) * k + j];
        }
    }
    l0[w][lane] = a0;
    l1[w][lane] = a1;
    lc[w][lane] = c;
    __syncthreads();
    if (w != 0) return;
    float dmax = 0.0f;
    if (j < k) {
        double t0 = 0.0, t1 = 0.0;
        uint32_t tc = 0;
        for (int q = 0; q < 16; ++q) {
            t0 += l0[q][lane];
            t1 += l1[q][lane];
            tc += lc[q][lane];
        }
        const float o0 = old[2 * j], o1 = old[2 * j + 1];
        float n0 = o0, n1 = o1;
        if (tc > 0) {
            const double fc = static_cast<double>(static_cast<float>(tc));
            n0 = static_cast<float>(t0 / fc);
            n1 = static_cast<float>(t1 / fc);
        }
        out[2 * j] = n0;
        out[2 * j + 1] = n1;
        dmax = fmaxf(fabsf(n0 - o0), fabsf(n1 - o1));
    }
    for (int off = 32; off > 0; off >>= 1) dmax = fmaxf(dmax, __shfl_xor(dmax, off));
    if (lane == 0 && dmax > 0.0f)
        atomicMax(reinterpret_cast<unsigned int *>(max_delta), __float_as_uint(dmax));
}

struct PairPlan {
    int64_t per_block;
    int64_t nparts;
};

static PairPlan pair_plan(int64_t n) {
    PairPlan p;
    int64_t per = (n + kUpdMaxBlocks - 1) / kUpdMaxBlocks;
    per = (per + kUpdChunk - 1) / kUpdChunk * kUpdChunk;
    p.per_block = per < kUpdChunk ? kUpdChunk : per;
    p.nparts = n <= 0 ? 1 : (n + p.per_block - 1) / p.per_block;
    return p;
}


}  // namespace enc
}  // namespace hxq

using namespace hxq;
using namespace hxq::enc;

template <typename IT, int KM>
static int assign_nearest_impl(const float *x, int64_t n, const float *codebook, int32_t k,
                               IT *indices, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && codebook && indices, "x, codebook and indices are required");
    HXQ_REQUIRE(n >= 0 && k >= 1 && k <= KM, KM == kMaxK ? "k must be 1..256" : "k must be 1..4096");
    if (n == 0) return HXQ_OK;
    hipLaunchKernelGGL((assign_kernel<IT, KM>), dim3(grid_for(n)), dim3(kThreads), 0, stream, x, n,
                       codebook, k, indices);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_assign_nearest(const float *x, int64_t n, const float *codebook, int32_t k,
                                  uint8_t *indices, hipStream_t stream) {
    return assign_nearest_impl<uint8_t, kMaxK>(x, n, codebook, k, indices, stream);
}

extern "C" int hxq_assign_nearest_wide(const float *x, int64_t n, const float *codebook, int32_t k,
                                       uint16_t *indices, hipStream_t stream) {
    return assign_nearest_impl<uint16_t, kMaxKW>(x, n, codebook, k, indices, stream);
}

extern "C" int64_t hxq_sort_workspace_bytes(int64_t n) {
    return n <= 0 ? 0 : 4 * next_pow2(n);
}

static int sort_keys(const float *x, int64_t n, uint32_t *keys, hipStream_t stream) {
    const int64_t np2 = next_pow2(n);
    hipLaunchKernelGGL(keys_kernel, dim3(grid_for(np2)), dim3(kThreads), 0, stream, x, n, np2, keys);
    HXQ_LAUNCH_CHECK();
    const dim3 lgrid(static_cast<uint32_t>(np2 / kSortBlock));
    hipLaunchKernelGGL(bitonic_local, lgrid, dim3(kThreads), 0, stream, keys, int64_t{0});
    HXQ_LAUNCH_CHECK();
    for (int64_t k = 2 * kSortBlock; k <= np2; k <<= 1) {
        for (int64_t j = k >> 1; j >= kSortBlock; j >>= 1) {
            hipLaunchKernelGGL(bitonic_global, dim3(grid_for(np2 / 2)), dim3(kThreads), 0, stream, keys,
                               np2, k, j);
            HXQ_LAUNCH_CHECK();
        }
        hipLaunchKernelGGL(bitonic_local, lgrid, dim3(kThreads), 0, stream, keys, k);
        HXQ_LAUNCH_CHECK();
    }
    return HXQ_OK;
}

static int64_t align256(int64_t b) { return (b + 255) & ~int64_t{255}; }

// k-means workspace regions, each 256-byte aligned: sort keys, cluster-ordered
// values, per-block counts / offsets, then starts, counts and the fp64
// tolerance + done flag
struct KmLayout {
    int64_t vals, blk, starts, counts, means, tol, done, total;
    explicit KmLayout(int64_t n) {
        const int64_t nblk = (n + 4095) / 4096;
        vals = align256(4 * next_pow2(n));
        blk = vals + align256(4 * n);
        starts = blk + align256(4 * nblk * kMaxKW);
        counts = starts + 4 * kMaxKW;
        means = counts + 4 * kMaxKW;
        tol = means + 4 * kMaxKW;
        done = tol + 8;
        total = align256(done + 8);
    }
};

extern "C" int64_t hxq_kmeans_workspace_bytes(int64_t n) {
    return n <= 0 ? 0 : KmLayout(n).total;
}

extern "C" int hxq_kmeans_init(const float *x, int64_t n, void *workspace, int64_t workspace_bytes,
                               int32_t *n_unique, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && workspace && n_unique && n >= 1, "bad arguments");
    HXQ_REQUIRE(n < (int64_t{1} << 31), "n too large");
    HXQ_REQUIRE(workspace_bytes >= hxq_kmeans_workspace_bytes(n), "workspace too small");
    uint32_t *keys = static_cast<uint32_t *>(workspace);
    if (int rc = sort_keys(x, n, keys, stream)) return rc;
    hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(1), 0, stream, n_unique);
    HXQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(count_unique_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream, keys, n,
                       n_unique);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

template <typename IT, int KM>
static int kmeans_run_impl(const float *x, int64_t n, const double *percentiles01, int32_t k,
                           int32_t max_iters, double rtol, void *workspace, int64_t workspace_bytes,
                           float *codebook, IT *assignments, int32_t *iters, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && percentiles01 && workspace && codebook && assignments && iters, "bad arguments");
    // max_iters == 0 leaves the reference's assignments unbound (an error there)
    HXQ_REQUIRE(n >= 1 && n < (int64_t{1} << 31) && k >= 1 && k <= KM && max_iters >= 1,
                KM == kMaxK ? "bad sizes (n 1..2^31-1, k 1..256, max_iters >= 1)"
                            : "bad sizes (n 1..2^31-1, k 1..4096, max_iters >= 1)");
    HXQ_REQUIRE(workspace_bytes >= hxq_kmeans_workspace_bytes(n), "workspace too small");
    char *ws = static_cast<char *>(workspace);
    const int64_t nblk = (n + 4095) / 4096;
    const KmLayout lay(n);
    uint32_t *keys = reinterpret_cast<uint32_t *>(ws);              // sorted by hxq_kmeans_init
    float *vals = reinterpret_cast<float *>(ws + lay.vals);
    int32_t *blk = reinterpret_cast<int32_t *>(ws + lay.blk);
    int32_t *starts = reinterpret_cast<int32_t *>(ws + lay.starts);
    int32_t *counts = reinterpret_cast<int32_t *>(ws + lay.counts);
    float *means = reinterpret_cast<float *>(ws + lay.means);
    double *abs_tol = reinterpret_cast<double *>(ws + lay.tol);
    int32_t *done = reinterpret_cast<int32_t *>(ws + lay.done);
    hipLaunchKernelGGL(kmeans_init_kernel, dim3(1), dim3(kMaxK), 0, stream, keys, n, percentiles01,
                       k, codebook, rtol, abs_tol, done, iters);
    HXQ_LAUNCH_CHECK();
    const int64_t per = 4096;
    for (int it = 0; it < max_iters; ++it) {
        hipLaunchKernelGGL((km_assign_kernel<IT, KM>), dim3(static_cast<uint32_t>(nblk)), dim3(kThreads),
                           0, stream, x, n, per, codebook, k, assignments, blk, done);
        HXQ_LAUNCH_CHECK();
        hipLaunchKernelGGL(km_offsets_kernel<KM>, dim3(1), dim3(kThreads), 0, stream, blk,
                           static_cast<int>(nblk), k, starts, counts, done);
        HXQ_LAUNCH_CHECK();
        hipLaunchKernelGGL((km_scatter_kernel<IT, KM>), dim3(static_cast<uint32_t>(nblk)), dim3(kThreads),
                           0, stream, x, n, per, assignments, blk, starts, k, vals, done);
        HXQ_LAUNCH_CHECK();
        hipLaunchKernelGGL(km_sum_kernel, dim3(k), dim3(kThreads), 0, stream, vals, starts, counts,
                           codebook, means, done);
        HXQ_LAUNCH_CHECK();
        hipLaunchKernelGGL(km_update_kernel<KM>, dim3(1), dim3(kThreads), 0, stream, means, k, codebook,
                           abs_tol, done, iters);
        HXQ_LAUNCH_CHECK();
    }
    return HXQ_OK;
}

extern "C" int hxq_kmeans_run(const float *x, int64_t n, const double *percentiles01, int32_t k,
                              int32_t max_iters, double rtol, void *workspace,
                              int64_t workspace_bytes, float *codebook, uint8_t *assignments,
                              int32_t *iters, hipStream_t stream) {
    return kmeans_run_impl<uint8_t, kMaxK>(x, n, percentiles01, k, max_iters, rtol, workspace,
                                           workspace_bytes, codebook, assignments, iters, stream);
}

extern "C" int hxq_kmeans_run_wide(const float *x, int64_t n, const double *percentiles01, int32_t k,
                                   int32_t max_iters, double rtol, void *workspace,
                                   int64_t workspace_bytes, float *codebook, uint16_t *assignments,
                                   int32_t *iters, hipStream_t stream) {
    return kmeans_run_impl<uint16_t, kMaxKW>(x, n, percentiles01, k, max_iters, rtol, workspace,
                                             workspace_bytes, codebook, assignments, iters, stream);
}

extern "C" int64_t hxq_select_workspace_bytes(void) { return sizeof(SelState); }

extern "C" int hxq_select_f32(const float *x, int64_t n, const int64_t *ranks, int32_t m,
                              float *values, int32_t *nan_count, void *workspace,
                              int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && ranks && values && workspace, "bad arguments");
    HXQ_REQUIRE(m >= 1 && m <= kSelMax && n >= 1 && n < (int64_t{1} << 32), "bad sizes");
    HXQ_REQUIRE(workspace_bytes >= static_cast<int64_t>(sizeof(SelState)), "workspace too small");
    SelState *st = static_cast<SelState *>(workspace);
    hipLaunchKernelGGL(select_init_kernel, dim3(1), dim3(256), 0, stream, ranks, m, st);
    HXQ_LAUNCH_CHECK();
    const int g = std::min(grid_for(n), 2048);
    for (int shift = 24; shift >= 0; shift -= 8) {
        hipLaunchKernelGGL(select_hist_kernel, dim3(g), dim3(kThreads), 0, stream, x, n, m, shift, st);
        HXQ_LAUNCH_CHECK();
        hipLaunchKernelGGL(select_pick_kernel, dim3(1), dim3(64), 0, stream, m, shift, st, values);
        HXQ_LAUNCH_CHECK();
    }
    if (nan_count)
        HXQ_HIP_TRY(hipMemcpyAsync(nan_count, &st->nan_count, 4, hipMemcpyDeviceToDevice, stream));
    return HXQ_OK;
}

extern "C" int64_t hxq_outliers_workspace_bytes(int64_t n) {
    const int64_t nblk = (n + 65535) / 65536;
    return 4 * std::max<int64_t>(nblk, 1) + 64;
}

extern "C" int hxq_outliers_f32(const float *x, int64_t n, const float *lohi, int64_t capacity,
                                int64_t *positions, float *values, int64_t *count, void *workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && lohi && count && workspace && (capacity == 0 || (positions && values)),
                "bad arguments");
    HXQ_REQUIRE(n >= 1 && capacity >= 0, "bad sizes");
    HXQ_REQUIRE(workspace_bytes >= hxq_outliers_workspace_bytes(n), "workspace too small");
    const int64_t per = 65536;
    const int nblk = static_cast<int>((n + per - 1) / per);
    int32_t *blk = static_cast<int32_t *>(workspace);
    hipLaunchKernelGGL(outlier_count_kernel, dim3(nblk), dim3(kThreads), 0, stream, x, n, per, lohi, blk);
    HXQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(outlier_scan_kernel, dim3(1), dim3(64), 0, stream, blk, nblk, count);
    HXQ_LAUNCH_CHECK();
    if (capacity > 0) {
        hipLaunchKernelGGL(outlier_write_kernel, dim3(nblk), dim3(kThreads), 0, stream, x, n, per, lohi,
                           blk, capacity, positions, values);
        HXQ_LAUNCH_CHECK();
    }
    return HXQ_OK;
}

extern "C" int64_t hxq_affine_fit_workspace_bytes(int64_t rows, int64_t cols) {
    return rows <= 0 || cols <= 0 ? 0 : 4 * ((rows * cols + 31) / 32);
}

template <typename IT, int KM>
static int affine_fit_impl(const float *w, const IT *indices, const float *codebook, int32_t k,
                           int64_t rows, int64_t cols, int32_t group_size,
                           const int64_t *exclude_positions, int64_t n_exclude, void *workspace,
                           int64_t workspace_bytes, float *scale, float *offset, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(w && indices && codebook && scale && offset, "bad arguments");
    HXQ_REQUIRE(k >= 1 && k <= KM && rows >= 1 && cols >= 1,
                KM == kMaxK ? "bad sizes (k 1..256)" : "bad sizes (k 1..4096)");
    HXQ_REQUIRE(group_size >= 1 && cols % group_size == 0, "cols must be a multiple of group_size");
    HXQ_REQUIRE(n_exclude >= 0 && (n_exclude == 0 || exclude_positions), "bad exclusion list");
    uint32_t *bits = nullptr;
    if (n_exclude > 0) {
        HXQ_REQUIRE(workspace && workspace_bytes >= hxq_affine_fit_workspace_bytes(rows, cols),
                    "workspace too small");
        bits = static_cast<uint32_t *>(workspace);
        const int64_t words = (rows * cols + 31) / 32;
        hipLaunchKernelGGL(zero_u32_kernel, dim3(grid_for(words)), dim3(kThreads), 0, stream, bits,
                           words);
        HXQ_LAUNCH_CHECK();
        hipLaunchKernelGGL(mark_kernel, dim3(grid_for(n_exclude)), dim3(kThreads), 0, stream,
                           exclude_positions, n_exclude, bits);
        HXQ_LAUNCH_CHECK();
    }
    const int64_t units = rows * (cols / group_size);
    const int64_t per_block = kThreads / kWave;
    const int64_t blocks = (units + per_block - 1) / per_block;
    HXQ_REQUIRE(blocks < (int64_t{1} << 31), "too many groups");
    hipLaunchKernelGGL((affine_fit_kernel<IT, KM>), dim3(static_cast<uint32_t>(blocks)), dim3(kThreads),
                       0, stream, w, indices, codebook, k, rows, cols, group_size, bits, scale, offset);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_affine_fit(const float *w, const uint8_t *indices, const float *codebook,
                              int32_t k, int64_t rows, int64_t cols, int32_t group_size,
                              const int64_t *exclude_positions, int64_t n_exclude, void *workspace,
                              int64_t workspace_bytes, float *scale, float *offset,
                              hipStream_t stream) {
    return affine_fit_impl<uint8_t, kMaxK>(w, indices, codebook, k, rows, cols, group_size,
                                           exclude_positions, n_exclude, workspace, workspace_bytes,
                                           scale, offset, stream);
}

extern "C" int hxq_affine_fit_wide(const float *w, const uint16_t *indices, const float *codebook,
                                   int32_t k, int64_t rows, int64_t cols, int32_t group_size,
                                   const int64_t *exclude_positions, int64_t n_exclude,
                                   void *workspace, int64_t workspace_bytes, float *scale,
                                   float *offset, hipStream_t stream) {
    return affine_fit_impl<uint16_t, kMaxKW>(w, indices, codebook, k, rows, cols, group_size,
                                             exclude_positions, n_exclude, workspace,
                                             workspace_bytes, scale, offset, stream);
}

extern "C" int64_t hxq_vq2_workspace_bytes(int64_t n, int32_t k) {
    if (n < 0 || k < 1 || k > kPairMaxK) return -1;
    const PairPlan p = pair_plan(n);
    return align256(int64_t{16} * k) + align256(p.nparts * 16 * k) + align256(p.nparts * 4 * k);
}

static int pair_table(const float *codebook, int32_t k, float4 *tab, hipStream_t stream) {
    hipLaunchKernelGGL(pair_table_kernel, dim3((k + 255) / 256), dim3(256), 0, stream, codebook, k,
                       tab);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

template <bool MIN>
static int pair_launch(const float2 *x, int64_t n, const int64_t *rows, int64_t m,
                       const float4 *tab, int32_t k, uint16_t *indices, float *dmin,
                       hipStream_t stream) {
    const size_t lds = static_cast<size_t>(k) * sizeof(float4);
    const int64_t big = (m + kPairThreads * 8 - 1) / (kPairThreads * 8);
    if (big >= 1024) {
        HXQ_REQUIRE(big < (int64_t{1} << 31), "too many pairs");
        hipLaunchKernelGGL((pair_assign_kernel<8, MIN>), dim3(static_cast<uint32_t>(big)),
                           dim3(kPairThreads), lds, stream, x, n, rows, m, tab, k, indices, dmin);
    } else {
        const int64_t g = (m + kPairThreads * 2 - 1) / (kPairThreads * 2);
        hipLaunchKernelGGL((pair_assign_kernel<2, MIN>), dim3(static_cast<uint32_t>(g)),
                           dim3(kPairThreads), lds, stream, x, n, rows, m, tab, k, indices, dmin);
    }
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}

extern "C" int hxq_vq2_assign(const float *x, int64_t n, const float *codebook, int32_t k,
                              uint16_t *indices, void *workspace, int64_t workspace_bytes,
                              hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && codebook && indices && workspace, "x, codebook, indices and workspace are required");
    HXQ_REQUIRE(n >= 0 && k >= 1 && k <= kPairMaxK, "k must be 1..4096");
    HXQ_REQUIRE(workspace_bytes >= int64_t{16} * k, "workspace too small");
    if (n == 0) return HXQ_OK;
    float4 *tab = static_cast<float4 *>(workspace);
    const int rc = pair_table(codebook, k, tab, stream);
    if (rc != HXQ_OK) return rc;
    return pair_launch<false>(reinterpret_cast<const float2 *>(x), n, nullptr, n, tab, k, indices,
                              nullptr, stream);
}

extern "C" int hxq_vq2_min_dist(const float *x, int64_t n, const int64_t *rows, int64_t m,
                                const float *codebook, int32_t k, float *dmin, void *workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && codebook && dmin && workspace, "x, codebook, dmin and workspace are required");
    HXQ_REQUIRE(n >= 0 && m >= 0 && k >= 1 && k <= kPairMaxK, "k must be 1..4096");
    HXQ_REQUIRE(rows != nullptr || m <= n, "without rows, m must be <= n");
    HXQ_REQUIRE(workspace_bytes >= int64_t{16} * k, "workspace too small");
    if (m == 0) return HXQ_OK;
    float4 *tab = static_cast<float4 *>(workspace);
    const int rc = pair_table(codebook, k, tab, stream);
    if (rc != HXQ_OK) return rc;
    return pair_launch<true>(reinterpret_cast<const float2 *>(x), n, rows, m, tab, k, nullptr, dmin,
                             stream);
}

extern "C" int hxq_vq2_update(const float *x, int64_t n, const uint16_t *indices, int32_t k,
                              const float *centroids, float *new_centroids, float *max_delta,
                              void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    HXQ_REQUIRE(x && indices && centroids && new_centroids && max_delta && workspace,
                "x, indices, centroids, new_centroids, max_delta and workspace are required");
    HXQ_REQUIRE(n >= 0 && k >= 1 && k <= kPairMaxK, "k must be 1..4096");
    HXQ_REQUIRE(workspace_bytes >= hxq_vq2_workspace_bytes(n, k), "workspace too small");
    HXQ_REQUIRE(new_centroids != centroids, "new_centroids must not alias centroids");
    const PairPlan p = pair_plan(n);
    char *ws = static_cast<char *>(workspace) + align256(int64_t{16} * k);
    double *psum = reinterpret_cast<double *>(ws);
    uint32_t *pcnt = reinterpret_cast<uint32_t *>(ws + align256(p.nparts * 16 * k));
    hipLaunchKernelGGL(pair_partial_kernel, dim3(static_cast<uint32_t>(p.nparts)),
                       dim3(kUpdThreads), 0, stream, reinterpret_cast<const float2 *>(x), n,
                       indices, k, p.per_block, psum, pcnt, max_delta);
    HXQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(pair_finish_kernel, dim3((k + 63) / 64), dim3(1024), 0, stream, psum, pcnt,
                       static_cast<int>(p.nparts), k, centroids, new_centroids, max_delta);
    HXQ_LAUNCH_CHECK();
    return HXQ_OK;
}
