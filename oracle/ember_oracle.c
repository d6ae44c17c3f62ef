/*
 * ember_oracle.c -- CPU restatement of Ember's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file: only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py use it, and only as the checker.  It is built with plain
 * gcc (no HIP) into oracle/liboracle.so by oracle/Makefile.
 *
 * Conventions restated from the reference (paths relative to the reference
 * checkout, pawel002/ember):
 *   - row-major float32 storage, argument order (n, m, k) with m = columns of
 *     B, FP64 accumulation, one cast to float per output:
 *       src/tensor/operators_cpu.c:47-60   (matmul)
 *       src/tensor/operators_cpu.c:62-67   (matmul_batched)
 *       src/tensor/operators_cpu.c:69-76   (transpose)
 *
 * Attention does not exist in the reference.  The functions below define it
 * in the same style (naive loops, FP64 accumulation, integer mask predicate)
 * so that the HIP kernels have a CPU path to agree with:
 *   - scores     s[i][j] = scale * sum_d q[i][d] * k[j][d]      (FP64)
 *   - visibility key j is visible to query i iff j < S and, when causal,
 *                j <= i (top-left aligned, S_q == S_k)
 *   - forward    o[i] = sum_j softmax_j(s[i][.])[j] * v[j];
 *                lse[i] = max_j s[i][j] + ln sum_j exp(s[i][j] - max)
 *   - backward   P = exp(s - lse) recomputed from the *given* lse,
 *                delta[i] = sum_d do[i][d] * o[i][d]  (from the given o),
 *                dV = P^T dO, dP = dO V^T, dS = P * (dP - delta),
 *                dQ = scale * dS K, dK = scale * dS^T Q.
 * Parity pins for these (golden fixtures made from NumPy float64 closed
 * forms, finite differences, the reference's own composed CPU ops, and the
 * invariants of the mask) live in tests/test_oracle.py.
 *
 * Layout: element (b, h, s, d) of q/k/v/dq/dk/dv sits at
 *   b*in_sb + h*in_sh + s*in_ss + d
 * and of o/do at b*out_sb + h*out_sh + s*out_ss + d; lse/delta are dense
 * (B, H, S).  Heads are independent and are spread over OpenMP threads; the
 * arithmetic inside a head is sequential and identical for any thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- GEMM: restates src/tensor/operators_cpu.c:47-76 ---- */

void oracle_matmul(const float *a, const float *b, float *out, int n, int m, int k)
{
    for (int i = 0; i < n; i++) {
        for (int j = 0; j < m; j++) {
            double acc = 0.0;
            for (int l = 0; l < k; l++) acc += (double)a[(size_t)i * k + l] * (double)b[(size_t)l * m + j];
            out[(size_t)i * m + j] = (float)acc;
        }
    }
}

void oracle_matmul_batched(const float *a, const float *b, float *out, int batch, int n, int m, int k)
{
    for (int bi = 0; bi < batch; bi++)
        oracle_matmul(a + (size_t)bi * n * k, b + (size_t)bi * k * m, out + (size_t)bi * n * m, n, m, k);
}

/* Row-blocked variant used for big parity cases: same per-element arithmetic
 * (FP64 sum in l order, one final cast), rows spread over threads. */
void oracle_matmul_mt(const float *a, const float *b, float *out, int n, int m, int k)
{
#pragma omp parallel for schedule(dynamic, 4)
    for (int i = 0; i < n; i++) {
        double *acc = (double *)calloc((size_t)m, sizeof(double));
        for (int l = 0; l < k; l++) {
            const double av = (double)a[(size_t)i * k + l];
            const float *brow = b + (size_t)l * m;
            for (int j = 0; j < m; j++) acc[j] += av * (double)brow[j];
        }
        for (int j = 0; j < m; j++) out[(size_t)i * m + j] = (float)acc[j];
        free(acc);
    }
}

void oracle_transpose(const float *a, float *out, int n, int m)
{
    for (int i = 0; i < n; i++)
        for (int j = 0; j < m; j++) out[(size_t)j * n + i] = a[(size_t)i * m + j];
}

/* ---- attention ---- */

static inline int visible(int64_t i, int64_t j, int causal)
{
    return !causal || j <= i;
}

static double dot_d(const float *x, const float *y, int64_t d)
{
    double acc = 0.0;
    for (int64_t t = 0; t < d; t++) acc += (double)x[t] * (double)y[t];
    return acc;
}

int oracle_attention_fwd(const float *q, const float *k, const float *v, float *o, float *lse,
                         int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                         int64_t in_sb, int64_t in_sh, int64_t in_ss, int64_t out_sb,
                         int64_t out_sh, int64_t out_ss)
{
    if (B < 0 || H < 0 || S < 0 || D <= 0) return 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t bh = 0; bh < B * H; bh++) {
        const int64_t b = bh / H, h = bh % H;
        const float *qh = q + b * in_sb + h * in_sh;
        const float *kh = k + b * in_sb + h * in_sh;
        const float *vh = v + b * in_sb + h * in_sh;
        float *oh = o + b * out_sb + h * out_sh;
        double *s = (double *)malloc((size_t)(S > 0 ? S : 1) * sizeof(double));
        double *acc = (double *)malloc((size_t)D * sizeof(double));
        for (int64_t i = 0; i < S; i++) {
            double mx = -INFINITY;
            for (int64_t j = 0; j < S; j++) {
                if (!visible(i, j, causal)) continue;
                s[j] = (double)scale * dot_d(qh + i * in_ss, kh + j * in_ss, D);
                if (s[j] > mx) mx = s[j];
            }
            double l = 0.0;
            memset(acc, 0, (size_t)D * sizeof(double));
            for (int64_t j = 0; j < S; j++) {
                if (!visible(i, j, causal)) continue;
                const double p = exp(s[j] - mx);
                l += p;
                const float *vj = vh + j * in_ss;
                for (int64_t d = 0; d < D; d++) acc[d] += p * (double)vj[d];
            }
            for (int64_t d = 0; d < D; d++) oh[i * out_ss + d] = (float)(acc[d] / l);
            lse[bh * S + i] = (float)(mx + log(l));
        }
        free(s);
        free(acc);
    }
    return 0;
}

int oracle_attention_bwd(const float *q, const float *k, const float *v, const float *o,
                         const float *lse, const float *d_o, float *dq, float *dk, float *dv,
                         int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                         int64_t in_sb, int64_t in_sh, int64_t in_ss, int64_t out_sb,
                         int64_t out_sh, int64_t out_ss)
{
    if (B < 0 || H < 0 || S < 0 || D <= 0) return 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t bh = 0; bh < B * H; bh++) {
        const int64_t b = bh / H, h = bh % H;
        const float *qh = q + b * in_sb + h * in_sh;
        const float *kh = k + b * in_sb + h * in_sh;
        const float *vh = v + b * in_sb + h * in_sh;
        const float *oh = o + b * out_sb + h * out_sh;
        const float *doh = d_o + b * out_sb + h * out_sh;
        float *dqh = dq + b * in_sb + h * in_sh;
        float *dkh = dk + b * in_sb + h * in_sh;
        float *dvh = dv + b * in_sb + h * in_sh;
        const size_t sd = (size_t)(S > 0 ? S : 1) * (size_t)D;
        double *dk_acc = (double *)calloc(sd, sizeof(double));
        double *dv_acc = (double *)calloc(sd, sizeof(double));
        double *dq_row = (double *)malloc((size_t)D * sizeof(double));
        for (int64_t i = 0; i < S; i++) {
            const float *qi = qh + i * in_ss;
            const float *doi = doh + i * out_ss;
            const double delta = dot_d(doi, oh + i * out_ss, D);
            const double li = (double)lse[bh * S + i];
            memset(dq_row, 0, (size_t)D * sizeof(double));
            for (int64_t j = 0; j < S; j++) {
                if (!visible(i, j, causal)) continue;
                const float *kj = kh + j * in_ss;
                const float *vj = vh + j * in_ss;
                const double p = exp((double)scale * dot_d(qi, kj, D) - li);
                const double dp = dot_d(doi, vj, D);
                const double ds = p * (dp - delta);
                double *dvj = dv_acc + (size_t)j * D;
                double *dkj = dk_acc + (size_t)j * D;
                for (int64_t d = 0; d < D; d++) {
                    dvj[d] += p * (double)doi[d];
                    dkj[d] += ds * (double)qi[d];
                    dq_row[d] += ds * (double)kj[d];
                }
            }
            for (int64_t d = 0; d < D; d++) dqh[i * in_ss + d] = (float)((double)scale * dq_row[d]);
        }
        for (int64_t j = 0; j < S; j++) {
            for (int64_t d = 0; d < D; d++) {
                dkh[j * in_ss + d] = (float)((double)scale * dk_acc[(size_t)j * D + d]);
                dvh[j * in_ss + d] = (float)dv_acc[(size_t)j * D + d];
            }
        }
        free(dk_acc);
        free(dv_acc);
        free(dq_row);
    }
    return 0;
}

/* ---- Adam: restates ember/optim/adam.py:24-45 as Ember executes it ----
 * Every line of adam.py is one fp32 element-wise operator of the reference
 * (src/tensor/operators_cpu.c:8-44 via tensor_api.c), each rounded to fp32;
 * the Python scalars are formed in double and converted to float by the
 * binding ("f", tensor_api.c:213).  Built with -ffp-contract=off, so no
 * multiply-add is fused.  In place on p, m, v. */
void oracle_adam_step(float *p, const float *g, float *m, float *v, int64_t n, double lr,
                      double beta1, double beta2, double eps, int64_t t)
{
    const float b1 = (float)beta1, omb1 = (float)(1.0 - beta1);
    const float b2 = (float)beta2, omb2 = (float)(1.0 - beta2);
    const float bc1 = (float)(1.0 - pow(beta1, (double)t));
    const float bc2 = (float)(1.0 - pow(beta2, (double)t));
    const float flr = (float)lr, feps = (float)eps;
    for (int64_t i = 0; i < n; i++) {
        float mi = m[i] * b1;                 /* m *= beta1                      */
        const float gm = g[i] * omb1;         /* (1 - beta1) * g                 */
        mi = mi + gm;                         /* m += ...                        */
        float vi = v[i] * b2;                 /* v *= beta2                      */
        const float gg = g[i] * g[i];         /* g * g                           */
        const float gv = gg * omb2;           /* (1 - beta2) * (g * g)           */
        vi = vi + gv;                         /* v += ...                        */
        const float mh = mi / bc1;            /* m_hat                           */
        const float vhat = vi / bc2;          /* v_hat                           */
        const float num = mh * flr;           /* lr * m_hat                      */
        const float den = sqrtf(vhat) + feps; /* sqrt(v_hat) + eps               */
        p[i] = p[i] - num / den;              /* p -= num / den                  */
        m[i] = mi;
        v[i] = vi;
    }
}

/* ---- AdamW: restates ember/optim/adamw.py:33-56 as Ember executes it ----
 * adam.py's m, v, m_hat, v_hat (adamw.py:45-52), then
 *   p -= lr * weight_decay * p      (:55; Python forms lr*wd in double first)
 *   p -= lr * m_hat / (sqrt(v_hat) + eps)                             (:56)
 * each an fp32 operator of the reference, scalars rounded to float once. */
void oracle_adamw_step(float *p, const float *g, float *m, float *v, int64_t n, double lr,
                       double beta1, double beta2, double eps, double weight_decay, int64_t t)
{
    const float b1 = (float)beta1, omb1 = (float)(1.0 - beta1);
    const float b2 = (float)beta2, omb2 = (float)(1.0 - beta2);
    const float bc1 = (float)(1.0 - pow(beta1, (double)t));
    const float bc2 = (float)(1.0 - pow(beta2, (double)t));
    const float flr = (float)lr, feps = (float)eps, lrwd = (float)(lr * weight_decay);
    for (int64_t i = 0; i < n; i++) {
        float mi = m[i] * b1;
        const float gm = g[i] * omb1;
        mi = mi + gm;
        float vi = v[i] * b2;
        const float gg = g[i] * g[i];
        const float gv = gg * omb2;
        vi = vi + gv;
        const float mh = mi / bc1;
        const float vhat = vi / bc2;
        const float decay = p[i] * lrwd;      /* (lr * wd) * p                   */
        const float pd = p[i] - decay;        /* p -= ...                        */
        const float num = mh * flr;
        const float den = sqrtf(vhat) + feps;
        p[i] = pd - num / den;
        m[i] = mi;
        v[i] = vi;
    }
}

/* ---- SGD: restates ember/optim/sgd.py:25-35 as Ember executes it ----
 *   v *= momentum;  v += g;  p -= lr * v     (sgd.py:33-35), fp32 each. */
void oracle_sgd_step(float *p, const float *g, float *v, int64_t n, double lr, double momentum)
{
    const float flr = (float)lr, fmom = (float)momentum;
    for (int64_t i = 0; i < n; i++) {
        const float vi = v[i] * fmom + g[i];  /* two roundings: contraction off */
        p[i] = p[i] - vi * flr;
        v[i] = vi;
    }
}

/* ---- LayerNorm (build-defined; Ember has none) ----
 * mean, var (biased) and the backward's row means in FP64, outputs cast to
 * float once, Ember style.  Row-major (rows x d). */
void oracle_layernorm_fwd(const float *x, const float *gamma, const float *beta, float *y,
                          float *mean, float *rstd, int64_t rows, int64_t d, float eps)
{
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * d;
        double s = 0.0;
        for (int64_t c = 0; c < d; c++) s += xr[c];
        const double mu = s / (double)d;
        double q = 0.0;
        for (int64_t c = 0; c < d; c++) q += ((double)xr[c] - mu) * ((double)xr[c] - mu);
        const double rs = 1.0 / sqrt(q / (double)d + (double)eps);
        for (int64_t c = 0; c < d; c++)
            y[r * d + c] = (float)(((double)xr[c] - mu) * rs * (double)gamma[c] + (double)beta[c]);
        mean[r] = (float)mu;
        rstd[r] = (float)rs;
    }
}

/* Backward from the given x and the float mean / rstd the forward stored. */
void oracle_layernorm_bwd(const float *x, const float *gamma, const float *mean, const float *rstd,
                          const float *dy, float *dx, float *dgamma, float *dbeta, int64_t rows,
                          int64_t d)
{
    double *dg = (double *)calloc((size_t)(d > 0 ? d : 1), sizeof(double));
    double *db = (double *)calloc((size_t)(d > 0 ? d : 1), sizeof(double));
    for (int64_t r = 0; r < rows; r++) {
        const double mu = mean[r], rs = rstd[r];
        double m1 = 0.0, m2 = 0.0;
        for (int64_t c = 0; c < d; c++) {
            const double xh = ((double)x[r * d + c] - mu) * rs;
            const double g = (double)dy[r * d + c] * (double)gamma[c];
            m1 += g;
            m2 += g * xh;
            dg[c] += (double)dy[r * d + c] * xh;
            db[c] += (double)dy[r * d + c];
        }
        m1 /= (double)d;
        m2 /= (double)d;
        for (int64_t c = 0; c < d; c++) {
            const double xh = ((double)x[r * d + c] - mu) * rs;
            const double g = (double)dy[r * d + c] * (double)gamma[c];
            dx[r * d + c] = (float)(rs * (g - m1 - xh * m2));
        }
    }
    for (int64_t c = 0; c < d; c++) {
        dgamma[c] = (float)dg[c];
        dbeta[c] = (float)db[c];
    }
    free(dg);
    free(db);
}

/* ---- Ember's GELU (ember/nn/activations.py:56-66), operator by operator ----
 * forward  y  = (x*0.5) * (tanh(x*0.8) + 1)
 * backward dx = dy * ((tanh(x*0.8) + 1) * ((x - y)*0.8 + 0.5))
 * each step one fp32 operation (built with -ffp-contract=off). */
void oracle_gelu_fwd(const float *x, float *y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        const float a = x[i] * 0.5f;
        const float t = tanhf(x[i] * 0.8f) + 1.0f;
        y[i] = a * t;
    }
}

void oracle_gelu_bwd(const float *dy, const float *x, const float *y, float *dx, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        const float t = tanhf(x[i] * 0.8f) + 1.0f;
        const float r = (x[i] - y[i]) * 0.8f + 0.5f;
        dx[i] = dy[i] * (t * r);
    }
}
