/*
 * hxq_oracle.c -- CPU restatement of the reference HXQ hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels in helix-substrate_amd/csrc.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * Functions and the reference code each one restates:
 *
 *   hxq_oracle_reconstruct   CDNAv3Reader.reconstruct / reconstruct_block
 *                            (helix_substrate/hxq_reader_v3.py:102-140,142-187):
 *                            W = codebook[idx]; W.flat[pos] = val (replace).
 *                            Plus the per-group affine extension that the
 *                            benchmark configs define (no reference code; the
 *                            op order idx->value*scale then +offset follows
 *                            triton_affine_group_matmul.py:379):
 *                            W[o,k] = fl(fl(cb[idx]*s[o,k/G]) + off[o,k/G]).
 *   hxq_oracle_reconstruct_fma  the same W with the affine as one rounding,
 *                            fl(cb[idx]*s + off) (C99 fmaf, correctly rounded
 *                            in glibc): the form the reference's GPU kernel
 *                            computes (triton_affine_group_matmul.py:99, Triton
 *                            contracts the multiply-add) and the GEMM kernels'
 *                            16-bit operands take before their bf16/fp16
 *                            rounding.
 *   hxq_oracle_linear_f64    x @ W^T (+bias), fp64 accumulation.  The reference
 *                            computes the same contraction with torch matmul
 *                            (helix_linear.py:809-820, triton_vq_matmul.py:521).
 *   hxq_oracle_ssm_scan_f64  sequential_scan (mamba_scan_chunked.py:42-86),
 *                            evaluated in fp64 from fp32 inputs.
 *   hxq_oracle_vq2_assign    the pair (vector_dim 2) nearest-centroid step of
 *                            _vector_kmeans / _chunked_vector_assign
 *                            (hxq_encoder.py:280-289, hxq_writer_v3.py:409-418):
 *                            argmin_j fl(fl(|x|^2 + |c_j|^2) - 2 x.c_j) in fp32,
 *                            |v|^2 = fl(fl(v0*v0) + fl(v1*v1)) (np.sum of the
 *                            squares) and x.c = fma(x1, c1, fl(x0*c0)) (the
 *                            rounding numpy's sgemm gives a K = 2 product);
 *                            first index on ties (np.argmin).
 *   hxq_oracle_vq2_update    the centroid update of the same loop
 *                            (hxq_encoder.py:291-298): fp64 sums in index order
 *                            (np.bincount with weights), counts as fp32, new =
 *                            fp32(sum / count), empty clusters keep the old
 *                            centroid; also max |new - old| (fp32).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; contraction must stay off
 * so the affine step keeps its two roundings).
 */
#include <stdint.h>
#include <stddef.h>
#include <math.h>
#include <string.h>
#include <stdlib.h>

int hxq_oracle_version(void) { return 1; }

/*
 * Reconstruct rows [row_begin, row_end) of W into w_out
 * ([row_end-row_begin, in_features], fp32, row-major).
 *
 * group_scale/group_offset may both be NULL (plain CDNAv3: W = cb[idx]).
 * sc_pos are flat row-major positions into the full [out, in] matrix
 * (the on-disk sidecar.npz layout), sc_val the replacement values.
 */
static int reconstruct_rows(const uint8_t *idx, const float *codebook,
                            const float *group_scale, const float *group_offset,
                            int32_t group_size, const int64_t *sc_pos,
                            const float *sc_val, int64_t nnz,
                            int64_t out_features, int64_t in_features,
                            int64_t row_begin, int64_t row_end, float *w_out, int fused)
{
    if (row_begin < 0 || row_end > out_features || row_begin > row_end)
        return 1;
    const int has_affine = (group_scale != NULL && group_offset != NULL);
    if (has_affine && (group_size <= 0 || in_features % group_size != 0))
        return 1;
    const int64_t n_groups = has_affine ? in_features / group_size : 0;
    for (int64_t o = row_begin; o < row_end; ++o) {
        const uint8_t *irow = idx + o * in_features;
        float *wrow = w_out + (o - row_begin) * in_features;
        for (int64_t k = 0; k < in_features; ++k) {
            float v = codebook[irow[k]];
            if (has_affine) {
                const int64_t g = o * n_groups + k / group_size;
                if (fused) {
                    v = fmaf(v, group_scale[g], group_offset[g]); /* one rounding */
                } else {
                    volatile float t = v * group_scale[g]; /* first rounding */
                    v = t + group_offset[g];               /* second rounding */
                }
            }
            wrow[k] = v;
        }
    }
    /* sidecar replacement, restricted to the row block */
    const int64_t lo = row_begin * in_features, hi = row_end * in_features;
    for (int64_t i = 0; i < nnz; ++i) {
        const int64_t p = sc_pos[i];
        if (p < 0 || p >= out_features * in_features)
            return 2;
        if (p >= lo && p < hi)
            w_out[p - lo] = sc_val[i];
    }
    return 0;
}

int hxq_oracle_reconstruct(const uint8_t *idx, const float *codebook,
                           const float *group_scale, const float *group_offset,
                           int32_t group_size, const int64_t *sc_pos,
                           const float *sc_val, int64_t nnz,
                           int64_t out_features, int64_t in_features,
                           int64_t row_begin, int64_t row_end, float *w_out)
{
    return reconstruct_rows(idx, codebook, group_scale, group_offset, group_size, sc_pos,
                            sc_val, nnz, out_features, in_features, row_begin, row_end,
                            w_out, 0);
}

/* As hxq_oracle_reconstruct, the affine as fl(cb[idx] * s + off). */
int hxq_oracle_reconstruct_fma(const uint8_t *idx, const float *codebook,
                               const float *group_scale, const float *group_offset,
                               int32_t group_size, const int64_t *sc_pos,
                               const float *sc_val, int64_t nnz,
                               int64_t out_features, int64_t in_features,
                               int64_t row_begin, int64_t row_end, float *w_out)
{
    return reconstruct_rows(idx, codebook, group_scale, group_offset, group_size, sc_pos,
                            sc_val, nnz, out_features, in_features, row_begin, row_end,
                            w_out, 1);
}

/* y[m, o] = sum_k x[m, k] * w[o, k] (+ bias[o]); every product and sum in fp64. */
int hxq_oracle_linear_f64(const float *x, int64_t m_rows, const float *w,
                          int64_t out_features, int64_t in_features,
                          const float *bias, double *y)
{
    for (int64_t m = 0; m < m_rows; ++m) {
        const float *xr = x + m * in_features;
        for (int64_t o = 0; o < out_features; ++o) {
            const float *wr = w + o * in_features;
            double acc = 0.0;
            for (int64_t k = 0; k < in_features; ++k)
                acc += (double)xr[k] * (double)wr[k];
            if (bias)
                acc += (double)bias[o];
            y[m * out_features + o] = acc;
        }
    }
    return 0;
}

/*
 * Sequential selective scan, reference layouts (mamba_scan_chunked.py:46-60):
 *   h0   [batch, heads, head_dim, state]     (NULL = zeros)
 *   dt   [batch, seqlen, heads]
 *   A    [heads]                              (negative decay rates)
 *   x    [batch, seqlen, heads, head_dim]
 *   B, C [batch, seqlen, ngroups, state]     head h reads group h / (heads/ngroups)
 *                                             (the reference repeat_interleave,
 *                                             mamba_scan_chunked.py:367-370)
 *   D    [heads]
 * Outputs y [batch, seqlen, heads, head_dim] and h_final [batch, heads,
 * head_dim, state], both fp64.
 *
 * Per step (mamba_scan_chunked.py:66-84):
 *   dA = exp(A*dt);  h = dA*h + (dt*x) (x) B;  y = <h, C> + D*x.
 */
int hxq_oracle_ssm_scan_f64(const float *h0, const float *dt, const float *A,
                            const float *x, const float *B, const float *C,
                            const float *D, int64_t batch, int64_t seqlen,
                            int64_t heads, int64_t head_dim, int64_t state,
                            int64_t ngroups, double *y, double *h_final)
{
    if (ngroups <= 0 || heads % ngroups != 0)
        return 1;
    const int64_t heads_per_group = heads / ngroups;
    const int64_t hsz = batch * heads * head_dim * state;
    for (int64_t i = 0; i < hsz; ++i)
        h_final[i] = h0 ? (double)h0[i] : 0.0;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t t = 0; t < seqlen; ++t) {
            for (int64_t hh = 0; hh < heads; ++hh) {
                const int64_t g = hh / heads_per_group;
                const double dtv = (double)dt[(b * seqlen + t) * heads + hh];
                const double dA = exp((double)A[hh] * dtv);
                const float *Bt = B + ((b * seqlen + t) * ngroups + g) * state;
                const float *Ct = C + ((b * seqlen + t) * ngroups + g) * state;
                for (int64_t p = 0; p < head_dim; ++p) {
                    const double xv = (double)x[((b * seqlen + t) * heads + hh) * head_dim + p];
                    const double dx = dtv * xv;
                    double *hs = h_final + ((b * heads + hh) * head_dim + p) * state;
                    double acc = 0.0;
                    for (int64_t n = 0; n < state; ++n) {
                        hs[n] = dA * hs[n] + dx * (double)Bt[n];
                        acc += hs[n] * (double)Ct[n];
                    }
                    y[((b * seqlen + t) * heads + hh) * head_dim + p] = acc + (double)D[hh] * xv;
                }
            }
        }
    }
    return 0;
}

int hxq_oracle_vq2_assign(const float *x, int64_t n, const float *cb, int32_t k, int32_t *out)
{
    if (n < 0 || k < 1)
        return 1;
    for (int64_t i = 0; i < n; ++i) {
        const float x0 = x[2 * i], x1 = x[2 * i + 1];
        const float xsq = x0 * x0 + x1 * x1;
        float best = 0.0f;
        int32_t bj = 0;
        for (int32_t j = 0; j < k; ++j) {
            const float c0 = cb[2 * j], c1 = cb[2 * j + 1];
            const float csq = c0 * c0 + c1 * c1;
            const float dot = fmaf(x1, c1, x0 * c0);
            const float d = (xsq + csq) - 2.0f * dot;
            if (j == 0 || d < best) {
                best = d;
                bj = j;
            }
        }
        out[i] = bj;
    }
    return 0;
}

int hxq_oracle_vq2_update(const float *x, int64_t n, const int32_t *idx, int32_t k,
                          const float *old, float *out, float *max_delta)
{
    if (n < 0 || k < 1)
        return 1;
    double *sum = (double *)calloc((size_t)k * 2, sizeof(double));
    int64_t *cnt = (int64_t *)calloc((size_t)k, sizeof(int64_t));
    if (!sum || !cnt) {
        free(sum);
        free(cnt);
        return 2;
    }
    for (int64_t i = 0; i < n; ++i) {
        const int32_t j = idx[i];
        if (j < 0 || j >= k) {
            free(sum);
            free(cnt);
            return 3;
        }
        sum[2 * j] += (double)x[2 * i];
        sum[2 * j + 1] += (double)x[2 * i + 1];
        cnt[j] += 1;
    }
    float md = 0.0f;
    for (int32_t j = 0; j < k; ++j) {
        for (int dd = 0; dd < 2; ++dd) {
            const float o = old[2 * j + dd];
            float v = o;
            if (cnt[j] > 0)
                v = (float)(sum[2 * j + dd] / (double)(float)cnt[j]);
            out[2 * j + dd] = v;
            const float dlt = fabsf(v - o);
            if (dlt > md)
                md = dlt;
        }
    }
    *max_delta = md;
    free(sum);
    free(cnt);
    return 0;
}
