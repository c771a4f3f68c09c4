/*
 * CPU oracle for the fused piecewise-linear-embedding path, in C.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never linked into the product.
 *
 * Two entry points:
 *
 *   ple_oracle_forward_f32  -- mirrors the fp32 arithmetic of the reference
 *       forward kernel step for step (bin search csrc/common.cuh:27-63,
 *       frac = (x - e_k) * iw_k at csrc/forward_cuda.cu:223-225, sequential
 *       fp32 prefix of quantised weights at :148-175, fmaf at :269-273,
 *       output rounding at :277-283), so its results are the bit pattern an
 *       IEEE-exact implementation of that kernel must produce.  The optional
 *       bias is added in fp32 after the output rounding, as
 *       src/rtdl_num_embeddings_cuda/module.py:238-239 adds it to x_ple.
 *
 *   ple_oracle_backward_f64 -- dx, dW, db accumulated in double
 *       (csrc/backward_cuda.cu:380-490 for dx with the internal-boundary
 *       term, :170-336 and :889-923 for the bucket/weighted histograms and the
 *       suffix over bins), with the absolute-value sums that scale tolerances.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so the compiler cannot
 * fuse any multiply-add the reference does not fuse).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { Q_F32 = 0, Q_F16 = 1, Q_BF16 = 2 };

static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* float -> bfloat16 -> float, nearest-even; NaN -> quiet NaN. */
static float bf16_round(float v) {
    uint32_t u = f2u(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u2f(0x7fc00000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u2f(u & 0xffff0000u);
}

/* float -> IEEE half -> float, nearest-even, with overflow to inf and
 * half subnormals (quantum 2^-24). */
static float f16_round(float v) {
    uint32_t u = f2u(v);
    uint32_t sign = u & 0x80000000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return v;                      /* inf / nan */
    if (a >= 0x477ff000u) return u2f(sign | 0x7f800000u); /* >= 65520 -> inf */
    if (a < 0x38800000u) {                               /* below 2^-14 */
        double s = (double)u2f(a) * 16777216.0;          /* exact */
        double q = nearbyint(s);                         /* ties to even */
        float r = (float)(q / 16777216.0);
        return sign ? -r : r;
    }
    a = (a + 0xfffu + ((a >> 13) & 1u)) & ~0x1fffu;
    return u2f(sign | a);
}

static inline float quant(float v, int q) {
    if (q == Q_BF16) return bf16_round(v);
    if (q == Q_F16) return f16_round(v);
    return v;
}

/* searchsorted(edges[:n+1], v, right) - 1, clamped to [0, n-1]; NaN -> n-1. */
static int find_bin(float v, const float *e, int n) {
    int lo = 0, hi = n + 1;
    while (lo < hi) {
        int mid = lo + (hi - lo) / 2;
        if (v < e[mid]) hi = mid; else lo = mid + 1;
    }
    int k = lo - 1;
    if (k < 0) k = 0;
    if (k > n - 1) k = n - 1;
    return k;
}

static inline int64_t phys(int k, int n, int64_t bmax) {
    return k == n - 1 ? bmax - 1 : (int64_t)k;
}

float ple_oracle_quantize(float v, int q) { return quant(v, q); }

int ple_oracle_find_bin(float v, const float *edges, int n) { return find_bin(v, edges, n); }

void ple_oracle_forward_f32(const float *x, const float *edges, const float *inv_w,
                            const int32_t *n_bins, const float *weight, const float *bias,
                            int q, int64_t N, int64_t F, int64_t B, int64_t D,
                            float *out, int32_t *idx_out, float *prefix_scratch) {
    /* prefix_scratch: F * B * D floats */
    for (int64_t f = 0; f < F; ++f) {
        int n = n_bins[f];
        for (int64_t j = 0; j < D; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < n; ++k) {
                prefix_scratch[(f * B + k) * D + j] = acc;
                acc += quant(weight[(f * B + phys(k, n, B)) * D + j], q);
            }
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        for (int64_t f = 0; f < F; ++f) {
            int n = n_bins[f];
            const float *e = edges + f * (B + 1);
            float v = x[i * F + f];
            int k = find_bin(v, e, n);
            if (idx_out) idx_out[i * F + f] = k;
            float pos = (v - e[k]) * inv_w[f * B + k];
            float qp = quant(pos, q);
            const float *w = weight + (f * B + phys(k, n, B)) * D;
            const float *p = prefix_scratch + (f * B + k) * D;
            float *o = out + (i * F + f) * D;
            for (int64_t j = 0; j < D; ++j) {
                float r = fmaf(qp, quant(w[j], q), p[j]);
                r = quant(r, q);
                if (bias) r = r + bias[f * D + j];
                o[j] = r;
            }
        }
    }
}

/* g: N*F*D floats (values as the operator sees them); gb: values for db
 * (NULL -> g).  Outputs in double.  idx: int32 logical bins. */
void ple_oracle_backward_f64(const float *g, const float *gb, const float *x,
                             const float *edges, const float *inv_w, const int32_t *n_bins,
                             const float *weight, const int32_t *idx, int q,
                             int64_t N, int64_t F, int64_t B, int64_t D,
                             double *dx, double *dx_abs, double *dw, double *dw_abs,
                             double *db, double *db_abs,
                             double *bucket_scratch, double *weighted_scratch,
                             double *bucket_abs_scratch, double *weighted_abs_scratch) {
    if (!gb) gb = g;
    if (dx) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < N; ++i) {
            for (int64_t f = 0; f < F; ++f) {
                int n = n_bins[f];
                int k = idx[i * F + f];
                const float *gr = g + (i * F + f) * D;
                const float *w = weight + (f * B + phys(k, n, B)) * D;
                double iw = inv_w[f * B + k];
                double s = 0.0, sa = 0.0;
                for (int64_t j = 0; j < D; ++j) {
                    double t = (double)gr[j] * (double)quant(w[j], q);
                    s += t;
                    sa += fabs(t);
                }
                s *= iw;
                sa *= fabs(iw);
                float v = x[i * F + f];
                if (k > 0 && v == edges[f * (B + 1) + k]) {
                    const float *wp = weight + (f * B + k - 1) * D;
                    double iwp = inv_w[f * B + k - 1];
                    double s2 = 0.0, sa2 = 0.0;
                    for (int64_t j = 0; j < D; ++j) {
                        double t = (double)gr[j] * (double)quant(wp[j], q);
                        s2 += t;
                        sa2 += fabs(t);
                    }
                    s += s2 * iwp;
                    sa += sa2 * fabs(iwp);
                }
                dx[i * F + f] = s;
                if (dx_abs) dx_abs[i * F + f] = sa;
            }
        }
    }
    if (!dw && !db) return;
#pragma omp parallel for schedule(dynamic)
    for (int64_t f = 0; f < F; ++f) {
        int n = n_bins[f];
        double *bk = bucket_scratch + f * B * D;
        double *wt = weighted_scratch + f * B * D;
        double *bka = bucket_abs_scratch + f * B * D;
        double *wta = weighted_abs_scratch + f * B * D;
        memset(bk, 0, sizeof(double) * B * D);
        memset(wt, 0, sizeof(double) * B * D);
        memset(bka, 0, sizeof(double) * B * D);
        memset(wta, 0, sizeof(double) * B * D);
        double *dbf = db ? db + f * D : 0;
        double *dbfa = db_abs ? db_abs + f * D : 0;
        if (dbf) memset(dbf, 0, sizeof(double) * D);
        if (dbfa) memset(dbfa, 0, sizeof(double) * D);
        const float *e = edges + f * (B + 1);
        for (int64_t i = 0; i < N; ++i) {
            int k = idx[i * F + f];
            float v = x[i * F + f];
            float pos = (v - e[k]) * inv_w[f * B + k];
            double qp = quant(pos, q);
            const float *gr = g + (i * F + f) * D;
            const float *gbr = gb + (i * F + f) * D;
            for (int64_t j = 0; j < D; ++j) {
                double gv = gr[j];
                bk[k * D + j] += gv;
                bka[k * D + j] += fabs(gv);
                wt[k * D + j] += qp * gv;
                wta[k * D + j] += fabs(qp * gv);
                if (dbf) { dbf[j] += gbr[j]; dbfa[j] += fabs((double)gbr[j]); }
            }
        }
        if (dw) {
            for (int64_t s = 0; s < B * D; ++s) { dw[f * B * D + s] = 0.0; if (dw_abs) dw_abs[f * B * D + s] = 0.0; }
            for (int64_t j = 0; j < D; ++j) {
                double fut = 0.0, futa = 0.0;
                for (int k = n - 1; k >= 0; --k) {
                    int64_t p = phys(k, n, B);
                    dw[(f * B + p) * D + j] = wt[k * D + j] + fut;
                    if (dw_abs) dw_abs[(f * B + p) * D + j] = wta[k * D + j] + futa;
                    fut += bk[k * D + j];
                    futa += bka[k * D + j];
                }
            }
        }
    }
}
