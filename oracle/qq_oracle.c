/*
 * qq_oracle.c -- CPU restatement of the LFM2-MoE Q8_0 MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * HIP product path.
 *
 * Build with -ffp-contract=off and no -march flags: every `a + b*c` below
 * must be two IEEE binary64 operations, as in the JavaScript it restates.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   qo_f16_to_f64      exhaustive over all 65,536 bit patterns against numpy's
 *                      IEEE binary16 conversion and the closed form.
 *   qo_matmul_q8_0     exact rational sums (fractions) on tiny shapes, the
 *                      sequential float64 running sum (numpy cumsum) on real
 *                      shapes, one-hot / zero-scale / all-ones closed forms,
 *                      power-of-two linearity, a planted transposed layout.
 *   qo_matmul_f32      same as qo_matmul_q8_0.
 *   qo_silu_inplace    sigma(0)=1/2 exactly, monotonicity, range, Python math.
 *   qo_moe_ffn         top-K against numpy's stable argsort; ties to the lower
 *                      expert; sum of weights = S/(S+1e-6); masked expert =
 *                      expert with zero down scales (bit-exact); all masked =
 *                      hidden unchanged; identical experts; batched = per token.
 *   exp() last ulp     binary64 exp differs between libm and V8's port of fdlibm
 *                      only in rare last-ulp cases; pinned statistically by the
 *                      Node restatement (oracle/moe_ref.js) which runs V8's own
 *                      Math.exp and is compared bit for bit with this file.
 */
#include "qq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define BLK 34

/* src/tensor.js:21-23 -- DataView.getFloat16(off, true). */
double qo_f16_to_f64(uint16_t h)
{
    int s = (h >> 15) & 1;
    int e = (h >> 10) & 0x1f;
    int m = h & 0x3ff;
    double v;
    if (e == 0)
        v = ldexp((double)m, -24);              /* zero / subnormal: m * 2^-24 */
    else if (e == 31)
        v = m ? NAN : INFINITY;
    else
        v = ldexp((double)(1024 + m), e - 25);  /* (1 + m/1024) * 2^(e-15) */
    return s ? -v : v;
}

uint16_t qo_f32_to_f16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u)                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
    if (a >= 0x477ff000u)                       /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {                      /* below 2^-14: subnormal half */
        /* value * 2^24 rounded to nearest even integer */
        float av;
        memcpy(&av, &a, 4);
        double scaled = (double)av * 16777216.0;    /* exact */
        double r = nearbyint(scaled);               /* default mode: RNE */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t e = ((a >> 23) - 127 + 15);
    uint32_t m = a & 0x7fffffu;
    uint32_t hm = m >> 13;
    uint32_t rem = m & 0x1fffu;
    uint32_t hv = (e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u)))
        hv += 1;                                /* carry into exponent is correct */
    return (uint16_t)(sign | hv);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline float rdf32(const uint8_t *p)
{
    float f;
    memcpy(&f, p, 4);   /* little-endian host, like DataView.getFloat32(off, true) */
    return f;
}

/* src/tensor.js:26-53 */
void qo_matmul_q8_0(const uint8_t *base, size_t offset, int in_dim, int out_dim,
                    const float *x, float *y)
{
    const int nb = (in_dim + QK - 1) / QK;                         /* _blocksPerCol */
    for (int c = 0; c < out_dim; c++) {
        double dot = 0.0;
        const uint8_t *col = base + offset + (size_t)c * nb * BLK;
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = col + (size_t)b * BLK;
            const double d = qo_f16_to_f64(rd16(blk));
            const int8_t *qs = (const int8_t *)(blk + 2);
            const int eb = b * QK;
            for (int i = 0; i < QK && eb + i < in_dim; i++) {
                /* JS: dot += input[eb+i] * i8[..] * d  ->  ((x*q)*d) then add */
                double t = (double)x[eb + i] * (double)qs[i];
                t = t * d;
                dot = dot + t;
            }
        }
        y[c] = (float)dot;
    }
}

/* src/tensor.js:469-482 */
void qo_matmul_f32(const uint8_t *base, size_t offset, int in_dim, int out_dim,
                   const float *x, float *y)
{
    for (int c = 0; c < out_dim; c++) {
        double dot = 0.0;
        const uint8_t *col = base + offset + (size_t)c * in_dim * 4;
        for (int i = 0; i < in_dim; i++) {
            double t = (double)x[i] * (double)rdf32(col + (size_t)i * 4);
            dot = dot + t;
        }
        y[c] = (float)dot;
    }
}

/* src/tensor.js:485-496 */
int qo_matmul_generic(int type, const uint8_t *base, size_t offset, int in_dim,
                      int out_dim, const float *x, float *y)
{
    switch (type) {
    case QO_TYPE_F32:  qo_matmul_f32(base, offset, in_dim, out_dim, x, y);  return 0;
    case QO_TYPE_Q8_0: qo_matmul_q8_0(base, offset, in_dim, out_dim, x, y); return 0;
    default:           return -1;
    }
}

/* src/tensor.js:80-100 */
int qo_read_weight_f32(int type, const uint8_t *base, size_t offset, int n, float *out)
{
    if (type == QO_TYPE_F32) {
        for (int i = 0; i < n; i++) out[i] = rdf32(base + offset + (size_t)i * 4);
        return 0;
    }
    if (type == QO_TYPE_Q8_0) {
        const int nb = (n + QK - 1) / QK;
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = base + offset + (size_t)b * BLK;
            const double d = qo_f16_to_f64(rd16(blk));
            const int8_t *qs = (const int8_t *)(blk + 2);
            for (int i = 0; i < QK && b * QK + i < n; i++)
                out[b * QK + i] = (float)((double)qs[i] * d);
        }
        return 0;
    }
    return -1;
}

/* src/tensor.js:167-171: arr[i] *= 1.0 / (1.0 + Math.exp(-arr[i])) */
void qo_silu_inplace(float *a, int n)
{
    for (int i = 0; i < n; i++) {
        double v = (double)a[i];
        double s = 1.0 / (1.0 + exp(-v));
        a[i] = (float)(v * s);
    }
}

/* src/tensor.js:174-178 */
void qo_mul_inplace(float *a, const float *b, int n)
{
    for (int i = 0; i < n; i++) a[i] = (float)((double)a[i] * (double)b[i]);
}

/* src/tensor.js:181-185 */
void qo_add_vec(float *a, const float *b, int n)
{
    for (int i = 0; i < n; i++) a[i] = (float)((double)a[i] + (double)b[i]);
}

/* src/tensor.js:103-114 with wF32[i] == 1 */
void qo_rmsnorm_unit(const float *in, float *out, int n, double eps)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) {
        double t = (double)in[i] * (double)in[i];
        ss = ss + t;
    }
    const double inv = 1.0 / sqrt(ss / n + eps);
    for (int i = 0; i < n; i++) out[i] = (float)((1.0 * (double)in[i]) * inv);
}

/* src/lfm2-engine.js:489-505: expert e of a [inDim, hidDim, E] Q8_0 tensor */
static size_t expert_offset(int in_dim, int hid_dim, int e)
{
    const size_t bytes_per_col = (size_t)((in_dim + QK - 1) / QK) * BLK;
    return (size_t)e * hid_dim * bytes_per_col;
}

/* src/tensor.js:150-164 softmaxInPlace over a Float32Array: the max in fp32,
 * exp of the (exact) binary64 difference stored to fp32, a sequential binary64
 * sum of the stored values, then each value times 1/sum stored to fp32. */
static void softmax_f32(float *a, int n)
{
    float maxv = a[0];
    for (int i = 1; i < n; i++)
        if (a[i] > maxv) maxv = a[i];
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        a[i] = (float)exp((double)a[i] - (double)maxv);
        sum = sum + (double)a[i];
    }
    const double inv = 1.0 / sum;
    for (int i = 0; i < n; i++) a[i] = (float)((double)a[i] * inv);
}

/* src/qwen3-engine.js:305-330 for one token, logits already formed: softmax,
 * stable descending sort by probability, weights renormalised from 0. */
static int route_token_softmax(const qo_moe_layer *L, int32_t *idx_out, double *w_out,
                               float *probs_out, float *logits, int *order, float *rw,
                               double *inv_out)
{
    const int E = L->E, K = L->K;
    softmax_f32(logits, E);
    for (int e = 0; e < E; e++) rw[e] = logits[e];
    for (int e = 0; e < E; e++) order[e] = e;
    for (int i = 1; i < E; i++) {      /* stable insertion sort, as above */
        int v = order[i];
        int j = i - 1;
        while (j >= 0 && rw[order[j]] < rw[v]) {
            order[j + 1] = order[j];
            j--;
        }
        order[j + 1] = v;
    }
    double sumW = 0.0;
    for (int k = 0; k < K; k++) sumW = sumW + (double)rw[order[k]];
    const double invSum = sumW > 0 ? 1.0 / sumW : 0.0;
    for (int k = 0; k < K; k++) {
        if (idx_out) idx_out[k] = order[k];
        if (w_out) w_out[k] = (double)rw[order[k]] * invSum;
    }
    if (probs_out)
        for (int e = 0; e < E; e++) probs_out[e] = rw[e];
    *inv_out = invSum;
    return 0;
}

/* src/lfm2-engine.js:417-457 for one token: fills rw (probabilities),
 * order (rank order) and invSum; writes the telemetry outputs. */
static int route_token(const qo_moe_layer *L, const float *x, int32_t *idx_out,
                       double *w_out, float *probs_out, float *logits, float *rw,
                       float *sel, int *order, double *inv_out)
{
    const int H = L->H, E = L->E, K = L->K;

    /* 1. router logits (lfm2-engine.js:418) */
    if (qo_matmul_generic(L->router_type, L->router, L->router_off, H, E, x, logits))
        return -1;
    if (L->gating == QO_GATING_SOFTMAX) return route_token_softmax(L, idx_out, w_out, probs_out, logits, order, rw, inv_out);
    /* 2. sigmoid (lfm2-engine.js:420-424) */
    for (int e = 0; e < E; e++)
        rw[e] = (float)(1.0 / (1.0 + exp(-(double)logits[e])));
    /* 3. selection scores = probs + bias (lfm2-engine.js:426-431) */
    for (int e = 0; e < E; e++) sel[e] = rw[e];
    if (L->bias_type >= 0) {
        float *bias = (float *)malloc(sizeof(float) * E);
        if (!bias) return -1;
        if (qo_read_weight_f32(L->bias_type, L->bias, L->bias_off, E, bias)) {
            free(bias);
            return -1;
        }
        for (int e = 0; e < E; e++) sel[e] = (float)((double)sel[e] + (double)bias[e]);
        free(bias);
    }
    /* 4. stable descending sort (lfm2-engine.js:433-442); Array.prototype.sort
     *    is stable, so equal scores keep ascending expert order.  Insertion
     *    sort with a strict comparison is stable. */
    for (int e = 0; e < E; e++) order[e] = e;
    for (int i = 1; i < E; i++) {
        int v = order[i];
        int j = i - 1;
        while (j >= 0 && sel[order[j]] < sel[v]) {   /* comparator b-a > 0 */
            order[j + 1] = order[j];
            j--;
        }
        order[j + 1] = v;
    }
    /* 5. normalise (lfm2-engine.js:444-447) */
    double sumW = 1e-6;
    for (int k = 0; k < K; k++) sumW = sumW + (double)rw[order[k]];
    const double invSum = 1.0 / sumW;

    /* telemetry payload (lfm2-engine.js:449-457) */
    for (int k = 0; k < K; k++) {
        if (idx_out) idx_out[k] = order[k];
        if (w_out) w_out[k] = (double)rw[order[k]] * invSum;
    }
    if (probs_out)
        for (int e = 0; e < E; e++) probs_out[e] = rw[e];
    *inv_out = invSum;
    return 0;
}

/* src/lfm2-engine.js:413-487 for one token. */
static int moe_token(const qo_moe_layer *L, const float *x, float *hidden,
                     const uint8_t *mask, int32_t *idx_out, double *w_out,
                     float *probs_out, float *logits, float *rw, float *sel,
                     int *order, float *g, float *u, float *dn, float *acc)
{
    const int H = L->H, F = L->F, K = L->K;
    double invSum;
    if (route_token(L, x, idx_out, w_out, probs_out, logits, rw, sel, order, &invSum))
        return -1;

    /* 6. experts and weighted accumulate (lfm2-engine.js:459-483) */
    for (int i = 0; i < H; i++) acc[i] = 0.0f;
    for (int k = 0; k < K; k++) {
        const int e = order[k];
        if (mask && mask[e]) continue;
        const double weight = (double)rw[e] * invSum;
        qo_matmul_q8_0(L->gate, L->gate_off + expert_offset(H, F, e), H, F, x, g);
        qo_silu_inplace(g, F);
        qo_matmul_q8_0(L->up, L->up_off + expert_offset(H, F, e), H, F, x, u);
        qo_mul_inplace(g, u, F);
        qo_matmul_q8_0(L->down, L->down_off + expert_offset(F, H, e), F, H, g, dn);
        for (int i = 0; i < H; i++)
            acc[i] = (float)((double)acc[i] + weight * (double)dn[i]);
    }
    /* residual (lfm2-engine.js:486) */
    qo_add_vec(hidden, acc, H);
    return 0;
}

int qo_moe_ffn(const qo_moe_layer *L, const float *x, float *hidden, int T,
               const uint8_t *mask, int32_t *idx, double *w, float *probs)
{
    if (!L || L->H <= 0 || L->F <= 0 || L->E <= 0 || L->K <= 0 || L->K > L->E || T < 0)
        return -1;
    const int H = L->H, F = L->F, E = L->E, K = L->K;
    float *logits = (float *)malloc(sizeof(float) * E);
    float *rw = (float *)malloc(sizeof(float) * E);
    float *sel = (float *)malloc(sizeof(float) * E);
    int *order = (int *)malloc(sizeof(int) * E);
    float *g = (float *)malloc(sizeof(float) * F);
    float *u = (float *)malloc(sizeof(float) * F);
    float *dn = (float *)malloc(sizeof(float) * H);
    float *acc = (float *)malloc(sizeof(float) * H);
    int rc = 0;
    if (!logits || !rw || !sel || !order || !g || !u || !dn || !acc) rc = -1;
    for (int t = 0; t < T && rc == 0; t++)
        rc = moe_token(L, x + (size_t)t * H, hidden + (size_t)t * H, mask,
                       idx ? idx + (size_t)t * K : NULL, w ? w + (size_t)t * K : NULL,
                       probs ? probs + (size_t)t * E : NULL,
                       logits, rw, sel, order, g, u, dn, acc);
    free(logits); free(rw); free(sel); free(order);
    free(g); free(u); free(dn); free(acc);
    return rc;
}

int qo_moe_route(const qo_moe_layer *L, const float *x, int T, int32_t *idx, double *w,
                 float *probs)
{
    if (!L || L->H <= 0 || L->E <= 0 || L->K <= 0 || L->K > L->E || T < 0)
        return -1;
    const int H = L->H, E = L->E, K = L->K;
    float *logits = (float *)malloc(sizeof(float) * E);
    float *rw = (float *)malloc(sizeof(float) * E);
    float *sel = (float *)malloc(sizeof(float) * E);
    int *order = (int *)malloc(sizeof(int) * E);
    int rc = (logits && rw && sel && order) ? 0 : -1;
    double inv;
    for (int t = 0; t < T && rc == 0; t++)
        rc = route_token(L, x + (size_t)t * H, idx ? idx + (size_t)t * K : NULL,
                         w ? w + (size_t)t * K : NULL, probs ? probs + (size_t)t * E : NULL,
                         logits, rw, sel, order, &inv);
    free(logits); free(rw); free(sel); free(order);
    return rc;
}
