// router.hip -- LFM2-MoE router for token batches: binary64 logits, then
// sigmoid / expert-bias top-K / renormalisation (src/lfm2-engine.js:417-447).
#include "qq_device.h"

namespace qq {

// Router weight of expert e at input index k (F32: column e of [H, E]; Q8_0:
// block-major panel, exactly dequantised).  Products with a binary32
// activation are exact in binary64, so only the summation order differs from
// the reference's sequential loop.
struct RouterW {
    const float *f32;
    const int8_t *qs;
    const __half *d;
    int H, E, nb;
    __device__ __forceinline__ double at(int e, int k, bool q8) const
    {
        if (q8) {
            const size_t o = bm_index(0, nb, k >> 5, E, e);
            return (double)qs[o * QK + (k & 31)] * (double)__half2float(d[o]);
        }
        return (double)f32[(size_t)e * H + k];
    }
};

// Grid (ceil(T/TT), ceil(E/EB)); 256 threads split k; fixed-order reduction.
template <int TT, int EB, bool Q8>
__global__ __launch_bounds__(256) void router_logits_kernel(const float *__restrict__ x, int T,
                                                            RouterW W, float *__restrict__ logits)
{
    __shared__ double red[4][TT * EB];
    const int t0 = blockIdx.x * TT;
    const int e0 = blockIdx.y * EB;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int H = W.H, E = W.E;

    double acc[TT][EB];
#pragma unroll
    for (int a = 0; a < TT; a++)
#pragma unroll
        for (int b = 0; b < EB; b++) acc[a][b] = 0.0;

    for (int k = threadIdx.x; k < H; k += 256) {
        double xv[TT];
#pragma unroll
        for (int a = 0; a < TT; a++) xv[a] = (t0 + a < T) ? (double)x[(size_t)(t0 + a) * H + k] : 0.0;
#pragma unroll
        for (int b = 0; b < EB; b++) {
            const double wv = (e0 + b < E) ? W.at(e0 + b, k, Q8) : 0.0;
#pragma unroll
            for (int a = 0; a < TT; a++) acc[a][b] = fma(xv[a], wv, acc[a][b]);
        }
    }
#pragma unroll
    for (int a = 0; a < TT; a++)
#pragma unroll
        for (int b = 0; b < EB; b++) {
            const double v = wave_sum(acc[a][b]);
            if (lane == 0) red[wave][a * EB + b] = v;
        }
    __syncthreads();
    if (threadIdx.x < TT * EB) {
        const int a = threadIdx.x / EB, b = threadIdx.x % EB;
        const int i = threadIdx.x;
        const double s = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];
        if (t0 + a < T && e0 + b < E) logits[(size_t)(t0 + a) * E + e0 + b] = (float)s;
    }
}

// One wavefront per token.
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float *__restrict__ logits, int T, int E, int K, const float *__restrict__ bias,
    int32_t *__restrict__ idx, double *__restrict__ w, float *__restrict__ probs)
{
    constexpr int EPL = MAX_E / WAVE;
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (t >= T) return;
    float lg[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + WAVE * i;
        lg[i] = (e < E) ? logits[(size_t)t * E + e] : 0.0f;
    }
    WaveRoute<EPL> R;
    wave_route<EPL>(lg, E, K, bias, R);
    if (probs) {
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = lane + WAVE * i;
            if (e < E) probs[(size_t)t * E + e] = R.prob[i];
        }
    }
#pragma unroll
    for (int k = 0; k < MAX_K; k++) {
        if (k < K && lane == k) {
            idx[(size_t)t * K + k] = R.idx[k];
            w[(size_t)t * K + k] = (double)R.p[k] * R.inv;
        }
    }
}

int launch_router_topk(qq_ctx *ctx, const qq_moe *m, const float *x, int T, float *logits,
                       int32_t *idx, double *w, float *probs)
{
    if (T <= 0) return QQ_OK;
    const bool q8 = m->router_type == QQ_TYPE_Q8_0;
    RouterW W;
    W.f32 = m->router_f32;
    W.qs = q8 ? m->router_q8->qs : nullptr;
    W.d = q8 ? m->router_q8->d : nullptr;
    W.H = m->H;
    W.E = m->E;
    W.nb = (m->H + QK - 1) / QK;
#define QQ_RL(TT, EB)                                                                             \
    do {                                                                                          \
        dim3 g((T + TT - 1) / TT, (m->E + EB - 1) / EB);                                          \
        if (q8)                                                                                   \
            QQ_LAUNCH(ctx, (router_logits_kernel<TT, EB, true>), g, dim3(256), 0, \
                               x, T, W, logits);                                                  \
        else                                                                                      \
            QQ_LAUNCH(ctx, (router_logits_kernel<TT, EB, false>), g, dim3(256), 0, x, T, W, logits);                                     \
    } while (0)
    prof_begin(ctx, K_ROUTER_LOGITS);
    if (T <= 2)
        QQ_RL(1, 1);
    else if (T <= 32)
        QQ_RL(1, 8);
    else
        QQ_RL(4, 8);
    prof_end(ctx);
#undef QQ_RL
    QQ_HIP(ctx, hipGetLastError());
    prof_begin(ctx, K_ROUTER_TOPK);
    QQ_LAUNCH(ctx, router_topk_kernel, dim3((T + 3) / 4), dim3(256), 0, logits,
                       T, m->E, m->K, m->bias, idx, w, probs);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
