// moe.hip -- LFM2-MoE router, top-K and token-major expert kernels.
//
// Reference: Lfm2Engine._moEFFN, src/lfm2-engine.js:413-487.
//   1. logits = matmulGeneric(router, x)                      (fp64 sum, fp32 store)
//   2. p_e = fp32(1 / (1 + exp(-logit_e)))                    (binary64 math)
//   3. s_e = fp32(p_e + bias_e)                               (selection only)
//   4. stable descending sort of s, top K (ties -> lower expert index)
//   5. S = 1e-6 + sum_k p_k (rank order, binary64), w_k = p_k * (1/S)
//   6. per selected, unmasked expert: g = fp32(silu(gate.x)) * up.x, y = down.g,
//      acc = fp32(acc + w_k * y) in rank order; hidden += acc.
#include "qq_device.h"

#include <cfloat>
#include <climits>

namespace qq {

// ---------------------------------------------------------------------------
// Router logits in binary64.  Products of two binary32 values (or of a
// binary32 and an exactly dequantised Q8_0 weight) are exact in binary64, so
// the only departure from the reference's sequential sum is the summation
// order; the fp32-rounded logits agree except at rounding-boundary straddles.
// Grid (ceil(T/TT), ceil(E/EB)); 256 threads split k.
// ---------------------------------------------------------------------------
template <int TT, int EB, bool Q8>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const float *__restrict__ x, int T, int H, const float *__restrict__ wf,
    const int8_t *__restrict__ wq, const __half *__restrict__ wd, int kp, int nb, int E,
    float *__restrict__ logits)
{
    __shared__ double red[4][TT * EB];
    const int t0 = blockIdx.x * TT;
    const int e0 = blockIdx.y * EB;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;

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
            const int e = e0 + b;
            if (e >= E) break;
            double wv;
            if (Q8)
                wv = (double)wq[(size_t)e * kp + k] * (double)__half2float(wd[(size_t)e * nb + (k >> 5)]);
            else
                wv = (double)wf[(size_t)e * H + k];
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
        const double s = ((red[0][threadIdx.x] + red[1][threadIdx.x]) + red[2][threadIdx.x]) + red[3][threadIdx.x];
        if (t0 + a < T && e0 + b < E) logits[(size_t)(t0 + a) * E + e0 + b] = (float)s;
    }
}

// ---------------------------------------------------------------------------
// Sigmoid, bias, top-K, renormalisation: one wavefront per token, expert e in
// lane e % 64 (E <= 256).  Selection is K rounds of a 64-lane argmax with the
// order (score desc, index asc), which is exactly the order a stable
// descending sort produces.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool topk_better(float av, int ai, float bv, int bi)
{
    // is (av, ai) ranked before (bv, bi)?  index INT_MAX = empty
    if (ai == INT_MAX) return false;
    if (bi == INT_MAX) return true;
    return (av > bv) || (av == bv && ai < bi);
}

__global__ __launch_bounds__(256) void router_topk_kernel(
    const float *__restrict__ logits, int T, int E, int K, const float *__restrict__ bias,
    int32_t *__restrict__ idx, double *__restrict__ w, float *__restrict__ probs)
{
    constexpr int EPL = MAX_E / WAVE;
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (t >= T) return;

    float p[EPL], s[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + WAVE * i;
        p[i] = 0.0f;
        s[i] = 0.0f;
        if (e < E) {
            const double l = (double)logits[(size_t)t * E + e];
            p[i] = (float)(1.0 / (1.0 + exp(-l)));
            s[i] = p[i] + bias[e];
            if (probs) probs[(size_t)t * E + e] = p[i];
        }
    }
    uint32_t taken = 0;
    double sumW = 1e-6;
    int sel[MAX_K];
    float selp[MAX_K];
    for (int k = 0; k < K; k++) {
        float bv = 0.0f, bp = 0.0f;
        int bi = INT_MAX;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = lane + WAVE * i;
            if (e < E && !((taken >> i) & 1u) && (bi == INT_MAX || s[i] > bv)) {
                bv = s[i];
                bi = e;
                bp = p[i];
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(bv, o, WAVE);
            const int oi = __shfl_xor(bi, o, WAVE);
            const float op = __shfl_xor(bp, o, WAVE);
            if (topk_better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
                bp = op;
            }
        }
        if ((bi & (WAVE - 1)) == lane) taken |= 1u << (bi / WAVE);
        if (k < MAX_K) {
            sel[k] = bi;
            selp[k] = bp;
        }
        sumW = sumW + (double)bp;
    }
    const double inv = 1.0 / sumW;
    if (lane == 0) {
        for (int k = 0; k < K && k < MAX_K; k++) {
            idx[(size_t)t * K + k] = sel[k];
            w[(size_t)t * K + k] = (double)selp[k] * inv;
        }
    }
}

int launch_router_topk(qq_ctx *ctx, const qq_moe *m, const float *x, int T, float *logits,
                       int32_t *idx, double *w, float *probs)
{
    if (T <= 0) return QQ_OK;
    const bool q8 = m->router_type == QQ_TYPE_Q8_0;
    const int8_t *wq = q8 ? m->router_q8->qs : nullptr;
    const __half *wd = q8 ? m->router_q8->d : nullptr;
    const int kp = q8 ? m->router_q8->kp : 0, nb = q8 ? m->router_q8->nb : 0;
#define QQ_RL(TT, EB)                                                                           \
    do {                                                                                        \
        dim3 g((T + TT - 1) / TT, (m->E + EB - 1) / EB);                                        \
        if (q8)                                                                                 \
            hipLaunchKernelGGL((router_logits_kernel<TT, EB, true>), g, dim3(256), 0,         \
                               ctx->stream, x, T, m->H, m->router_f32, wq, wd, kp, nb, m->E,  \
                               logits);                                                         \
        else                                                                                    \
            hipLaunchKernelGGL((router_logits_kernel<TT, EB, false>), g, dim3(256), 0,        \
                               ctx->stream, x, T, m->H, m->router_f32, wq, wd, kp, nb, m->E,  \
                               logits);                                                         \
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
    hipLaunchKernelGGL(router_topk_kernel, dim3((T + 3) / 4), dim3(256), 0, ctx->stream, logits,
                       T, m->E, m->K, m->bias, idx, w, probs);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

// ---------------------------------------------------------------------------
// Token-major expert kernels (one (token, rank) pair per grid row).  Weights
// are read once per pair, which is optimal when the pairs select distinct
// experts (batch-1 decode).
// ---------------------------------------------------------------------------

// gate/up + SwiGLU.  Grid (ceil(F / (4*RPW)), T*K).
template <int NCH, int RPW>
__global__ __launch_bounds__(256) void gateup_tok_kernel(
    const float *__restrict__ x, int H, const int32_t *__restrict__ idx, int K, MaskBits mask,
    const int8_t *__restrict__ gq, const __half *__restrict__ gd, const int8_t *__restrict__ uq,
    const __half *__restrict__ ud, int F, int kp, int nb, float *__restrict__ g)
{
    const int pair = blockIdx.y;
    const int t = pair / K;
    const int e = idx[pair];
    if (mask_has(mask, e)) return;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;

    float xr[NCH][16], xs[NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int k0 = 1024 * j + 16 * lane;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float v = (k0 + i < H) ? x[(size_t)t * H + k0 + i] : 0.0f;
            xr[j][i] = v;
            s += v;
        }
        xs[j] = s;
    }

    const int f0 = (blockIdx.x * 4 + wave) * RPW;
    int4 qg[RPW][NCH], qu[RPW][NCH];
    float dg[RPW][NCH], du[RPW][NCH];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const size_t row = (size_t)e * F + min(f0 + r, F - 1);
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int k0 = 1024 * j + 16 * lane;
            if (k0 < kp) {
                qg[r][j] = *reinterpret_cast<const int4 *>(gq + row * kp + k0);
                qu[r][j] = *reinterpret_cast<const int4 *>(uq + row * kp + k0);
                dg[r][j] = __half2float(gd[row * nb + (k0 >> 5)]);
                du[r][j] = __half2float(ud[row * nb + (k0 >> 5)]);
            } else {
                qg[r][j] = qu[r][j] = make_int4(0, 0, 0, 0);
                dg[r][j] = du[r][j] = 0.0f;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float ga = 0.0f, ua = 0.0f;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            ga = fmaf(dot16_q8(qg[r][j], xr[j], xs[j]), dg[r][j], ga);
            ua = fmaf(dot16_q8(qu[r][j], xr[j], xs[j]), du[r][j], ua);
        }
        ga = wave_sum(ga);
        ua = wave_sum(ua);
        const int f = f0 + r;
        if (lane == 0 && f < F) {
            // siluInPlace then mulInPlace (src/tensor.js:167-178)
            const double gv = (double)ga;
            const float sg = (float)(gv * (1.0 / (1.0 + exp(-gv))));
            g[(size_t)pair * F + f] = sg * ua;
        }
    }
}

// down projection + weighted combine + residual.  Grid (ceil(H / (4*RPW)), T).
template <int NCH, int RPW>
__global__ __launch_bounds__(256) void down_combine_tok_kernel(
    const float *__restrict__ g, int F, const int32_t *__restrict__ idx,
    const double *__restrict__ w, int K, MaskBits mask, const int8_t *__restrict__ dq,
    const __half *__restrict__ dd, int H, int kp, int nb, float *__restrict__ hidden)
{
    const int t = blockIdx.y;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int j0 = (blockIdx.x * 4 + wave) * RPW;

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = 0.0f;

    for (int k = 0; k < K; k++) {
        const int pair = t * K + k;
        const int e = idx[pair];
        if (mask_has(mask, e)) continue;
        const double wk = w[pair];
        int4 q[RPW][NCH];
        float ds[RPW][NCH];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const size_t row = (size_t)e * H + min(j0 + r, H - 1);
#pragma unroll
            for (int j = 0; j < NCH; j++) {
                const int k0 = 1024 * j + 16 * lane;
                if (k0 < kp) {
                    q[r][j] = *reinterpret_cast<const int4 *>(dq + row * kp + k0);
                    ds[r][j] = __half2float(dd[row * nb + (k0 >> 5)]);
                } else {
                    q[r][j] = make_int4(0, 0, 0, 0);
                    ds[r][j] = 0.0f;
                }
            }
        }
        float gr[NCH][16], gs[NCH];
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int k0 = 1024 * j + 16 * lane;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float v = (k0 + i < F) ? g[(size_t)pair * F + k0 + i] : 0.0f;
                gr[j][i] = v;
                s += v;
            }
            gs[j] = s;
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float y = 0.0f;
#pragma unroll
            for (int j = 0; j < NCH; j++) y = fmaf(dot16_q8(q[r][j], gr[j], gs[j]), ds[r][j], y);
            y = wave_sum(y);
            acc[r] = (float)((double)acc[r] + wk * (double)y);
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int jj = j0 + r;
            if (jj < H) hidden[(size_t)t * H + jj] = hidden[(size_t)t * H + jj] + acc[r];
        }
    }
}

size_t moe_work_bytes(const qq_moe *m, int T)
{
    return (size_t)T * m->K * m->F * 4;   // g [T*K][F] f32
}

int launch_moe_experts(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                       const MaskBits &mask, const int32_t *idx, const double *w, void *work,
                       size_t work_bytes)
{
    if (T <= 0) return QQ_OK;
    const size_t need = (size_t)T * m->K * m->F * 4;
    if (work_bytes < need) return set_error(ctx, "internal: expert work area too small");
    float *g = static_cast<float *>(work);
    const qq_tensor *G = m->gate, *U = m->up, *D = m->down;
    constexpr int RPW = 2;
    {
        dim3 grid((m->F + 4 * RPW - 1) / (4 * RPW), T * m->K);
        const int nch = (G->kp + 1023) / 1024;
#define QQ_GU(NCH)                                                                              \
    hipLaunchKernelGGL((gateup_tok_kernel<NCH, RPW>), grid, dim3(256), 0, ctx->stream, x, m->H, \
                       idx, m->K, mask, G->qs, G->d, U->qs, U->d, m->F, G->kp, G->nb, g)
        prof_begin(ctx, K_GATEUP);
        switch (nch) {
        case 1: QQ_GU(1); break;
        case 2: QQ_GU(2); break;
        case 3: QQ_GU(3); break;
        case 4: QQ_GU(4); break;
        default: return set_error(ctx, "hidden size %d exceeds 4096", m->H);
        }
        prof_end(ctx);
#undef QQ_GU
        QQ_HIP(ctx, hipGetLastError());
    }
    {
        dim3 grid((m->H + 4 * RPW - 1) / (4 * RPW), T);
        const int nch = (D->kp + 1023) / 1024;
#define QQ_DC(NCH)                                                                               \
    hipLaunchKernelGGL((down_combine_tok_kernel<NCH, RPW>), grid, dim3(256), 0, ctx->stream, g, \
                       m->F, idx, w, m->K, mask, D->qs, D->d, m->H, D->kp, D->nb, hidden)
        prof_begin(ctx, K_DOWN_COMBINE);
        switch (nch) {
        case 1: QQ_DC(1); break;
        case 2: QQ_DC(2); break;
        case 3: QQ_DC(3); break;
        case 4: QQ_DC(4); break;
        default: return set_error(ctx, "expert size %d exceeds 4096", m->F);
        }
        prof_end(ctx);
#undef QQ_DC
        QQ_HIP(ctx, hipGetLastError());
    }
    return QQ_OK;
}

}  // namespace qq
