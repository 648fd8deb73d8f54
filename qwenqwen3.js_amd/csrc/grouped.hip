// grouped.hip -- token batches: dispatch by expert, grouped expert products,
// gather-based combine.
//
// The reference has no batching: a prompt is T sequential single-token calls
// (src/lfm2-engine.js:550-555), each row independent.  Here the T*K
// (token, rank) pairs are grouped by expert so that each expert's weights are
// read once per batch:
//   dispatch   counts[e], offsets[e] (exclusive scan), perm[slot] = pair and
//              inv[pair] = slot (order within an expert unspecified); pairs
//              whose expert is masked get inv = -1.
//   gate/up    grid (E, ceil(F/32)): the workgroup keeps its 32 gate and up
//              rows in registers and runs every slot of its expert against
//              them, MT tokens at a time from LDS -> g[slot][F].
//   down       grid (E, ceil(H/32)): same shape over down rows -> y[slot][H].
//   combine    hidden[t] += sum over ranks k in order of w[t,k] * y[inv[t,k]],
//              each step rounded to fp32 as in lfm2-engine.js:481-483; no
//              scatter, no atomics.
#include "qq_device.h"

namespace qq {

constexpr int GR_WAVES = 8;
constexpr int GR_THREADS = GR_WAVES * WAVE;
// tokens per LDS pass: 4, or 2 when a row spans more than 2048 values
template <int NBW>
struct GrMT {
    static constexpr int value = NBW >= 16 ? 2 : 4;
};

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of NT threads; pair p is handled by thread p % NT.
// Pass 1 counts pairs per expert with LDS atomics, one wave scans the counts
// into offsets (and cuts the row tiles), pass 2 hands out slots with LDS
// atomics.  The order of slots within an expert is therefore unspecified;
// nothing depends on it: every slot row is computed on its own and the
// combine reads slots through inv, so results are the same bit for bit.
// ---------------------------------------------------------------------------
constexpr int DISP_THREADS = 1024;
constexpr int DISP_ROUND = 16;   // pair loads in flight per thread

__global__ __launch_bounds__(DISP_THREADS) void moe_dispatch_kernel(
    const int32_t *__restrict__ idx, int P, int E, MaskBits mask, int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets, int32_t *__restrict__ perm, int32_t *__restrict__ inv,
    DispatchTiles tiles)
{
    __shared__ int cnt[MAX_E], cur[MAX_E], offs[MAX_E + 1];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    for (int e = tid; e < E; e += DISP_THREADS) {
        cnt[e] = 0;
        cur[e] = 0;
    }
    __syncthreads();
    constexpr int STEP = DISP_THREADS * DISP_ROUND;
    int ev[DISP_ROUND];
    for (int b0 = 0; b0 < P; b0 += STEP) {
#pragma unroll
        for (int i = 0; i < DISP_ROUND; i++) {
            const int p = b0 + tid + DISP_THREADS * i;
            ev[i] = p < P ? idx[p] : -1;
        }
#pragma unroll
        for (int i = 0; i < DISP_ROUND; i++) {
            const int e = ev[i];
            if ((unsigned)e < (unsigned)E && !mask_has(mask, e)) atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    if (wave == 0) {
        // exclusive scan of the expert counts, 64 experts at a time, then
        // row tiles of at most tiles.bm slots: lane e writes its expert's
        // tiles at the exclusive scan of the tile counts
        int run = 0, trun = 0;
        for (int e0 = 0; e0 < E; e0 += WAVE) {
            const int e = e0 + lane;
            const int c = e < E ? cnt[e] : 0;
            int tot;
            const int o = run + wave_excl_scan(c, &tot);
            if (e < E) {
                offs[e] = o;
                counts[e] = c;
                offsets[e] = o;
            }
            run += tot;
            if (tiles.bm > 0) {
                const int nte = (c + tiles.bm - 1) / tiles.bm;
                int ttot;
                int t = trun + wave_excl_scan(nte, &ttot);
                for (int m0 = 0; m0 < c && t < tiles.cap; m0 += tiles.bm, t++) {
                    tiles.e[t] = e;
                    tiles.m0[t] = m0;
                }
                trun += ttot;
            }
        }
        if (lane == 0) {
            offs[E] = run;
            offsets[E] = run;
            if (tiles.bm > 0) *tiles.n = min(trun, tiles.cap);
        }
    }
    __syncthreads();
    for (int b0 = 0; b0 < P; b0 += STEP) {
        // one chunk (P <= STEP): the expert ids of the counting pass are still held
        if (P > STEP) {
#pragma unroll
            for (int i = 0; i < DISP_ROUND; i++) {
                const int p = b0 + tid + DISP_THREADS * i;
                ev[i] = p < P ? idx[p] : -1;
            }
        }
#pragma unroll
        for (int i = 0; i < DISP_ROUND; i++) {
            const int p = b0 + tid + DISP_THREADS * i;
            if (p >= P) break;
            const int e = ev[i];
            const int pos = ((unsigned)e < (unsigned)E && !mask_has(mask, e)) ? offs[e] + atomicAdd(&cur[e], 1) : -1;
            if ((unsigned)pos < (unsigned)P) {   // (always, for a routed pair)
                perm[pos] = p;
                inv[p] = pos;
            } else {
                inv[p] = -1;
            }
        }
    }
}

struct GroupArgs {
    const float *x;          // [T][H]
    int H, F, K;
    int nbH, nbF;
    const int8_t *gq;
    const __half *gd;
    const int8_t *uq;
    const __half *ud;
    const int8_t *dq;
    const __half *dd;
    const int32_t *counts;
    const int32_t *offsets;
    const int32_t *perm;
    float *g;                // [slots][F]
    float *y;                // [slots][H]
};

// Activations of MT slots -> LDS (zero beyond `len` and beyond the group).
template <int XN, int MT>
__device__ __forceinline__ void stage_rows(float (*dst)[XN], float (*sums)[XN / 16],
                                           const float *__restrict__ src, int ld, int len,
                                           const int32_t *__restrict__ rowid, int mt)
{
    for (int i = threadIdx.x; i < MT * XN; i += GR_THREADS) {
        const int m = i / XN, kk = i - m * XN;
        dst[m][kk] = (m < mt && kk < len) ? src[(size_t)rowid[m] * ld + kk] : 0.0f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < MT * (XN / 16); i += GR_THREADS) {
        const int m = i / (XN / 16), hb = i - m * (XN / 16);
        float t = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) t += dst[m][hb * 16 + j];
        sums[m][hb] = t;
    }
    __syncthreads();
}

template <int NBW>
__global__ __launch_bounds__(GR_THREADS) void moe_grouped_gateup_kernel(GroupArgs a)
{
    constexpr int GR_MT = GrMT<NBW>::value;
    constexpr int XN = NBW * GR_WAVES * QK;
    __shared__ __align__(16) float xl[GR_MT][XN];
    __shared__ float xs[GR_MT][XN / 16];
    __shared__ float redg[GR_MT][GR_WAVES][QK];
    __shared__ float redu[GR_MT][GR_WAVES][QK];
    __shared__ int rowid[GR_MT];

    const int e = blockIdx.x, s = blockIdx.y;
    const int n = a.counts[e];
    if (n == 0) return;
    const int base = a.offsets[e];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int h = lane & 1;
    const int f = s * QK + lane / 2;
    const bool f_ok = f < a.F;

    // branch-free loads (clamped addresses, zero scale when out of range)
    int4 gq[NBW], uq[NBW];
    float gd[NBW], ud[NBW];
    const int fc = min(f, a.F - 1);
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const int b = wave + GR_WAVES * i;
        const size_t o = bm_index(e, a.nbH, min(b, a.nbH - 1), a.F, fc);
        gq[i] = *reinterpret_cast<const int4 *>(a.gq + o * QK + 16 * h);
        uq[i] = *reinterpret_cast<const int4 *>(a.uq + o * QK + 16 * h);
        gd[i] = __half2float(a.gd[o]);
        ud[i] = __half2float(a.ud[o]);
    }
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const bool bok = f_ok && (wave + GR_WAVES * i) < a.nbH;
        gd[i] = bok ? gd[i] : 0.0f;
        ud[i] = bok ? ud[i] : 0.0f;
    }
    // all loads above are issued before any of the arithmetic below
    __builtin_amdgcn_sched_barrier(0);

    for (int c0 = 0; c0 < n; c0 += GR_MT) {
        const int mt = min(GR_MT, n - c0);
        __syncthreads();
        if (threadIdx.x < GR_MT)
            rowid[threadIdx.x] = (threadIdx.x < mt) ? a.perm[base + c0 + threadIdx.x] / a.K : 0;
        __syncthreads();
        stage_rows<XN, GR_MT>(xl, xs, a.x, a.H, a.H, rowid, mt);
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            opaque(gq[i]);
            opaque(uq[i]);
        }
        float ga[GR_MT], ua[GR_MT];
#pragma unroll
        for (int m = 0; m < GR_MT; m++) ga[m] = ua[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            const int b = wave + GR_WAVES * i;   // < XN/32: reads stay inside xl
            float gw[16], uw[16];
            cvt16_off(gq[i], gw);
            cvt16_off(uq[i], uw);
#pragma unroll
            for (int m = 0; m < GR_MT; m++) {
                if (m < mt) {
                    const float *xp = &xl[m][b * QK + 16 * h];
                    const float xsm = xs[m][2 * b + h];
                    ga[m] = fmaf(dot16_off(gw, xp, xsm), gd[i], ga[m]);
                    ua[m] = fmaf(dot16_off(uw, xp, xsm), ud[i], ua[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < GR_MT; m++) {
            ga[m] += __shfl_xor(ga[m], 1, WAVE);
            ua[m] += __shfl_xor(ua[m], 1, WAVE);
            if (h == 0) {
                redg[m][wave][lane / 2] = ga[m];
                redu[m][wave][lane / 2] = ua[m];
            }
        }
        __syncthreads();
        if (threadIdx.x < GR_MT * QK) {
            const int m = threadIdx.x / QK, r = threadIdx.x % QK;
            const int fr = s * QK + r;
            if (m < mt && fr < a.F) {
                float G = redg[m][0][r], U = redu[m][0][r];
#pragma unroll
                for (int w = 1; w < GR_WAVES; w++) {
                    G += redg[m][w][r];
                    U += redu[m][w][r];
                }
                const double g64 = (double)G;
                const float sg = (float)(g64 * (1.0 / (1.0 + exp(-g64))));
                a.g[(size_t)(base + c0 + m) * a.F + fr] = sg * U;
            }
        }
    }
}

template <int NBW>
__global__ __launch_bounds__(GR_THREADS) void moe_grouped_down_kernel(GroupArgs a)
{
    constexpr int GR_MT = GrMT<NBW>::value;
    constexpr int XN = NBW * GR_WAVES * QK;
    __shared__ __align__(16) float gl[GR_MT][XN];
    __shared__ float gs[GR_MT][XN / 16];
    __shared__ float red[GR_MT][GR_WAVES][QK];
    __shared__ int rowid[GR_MT];

    const int e = blockIdx.x, jt = blockIdx.y;
    const int n = a.counts[e];
    if (n == 0) return;
    const int base = a.offsets[e];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int h = lane & 1;
    const int j = jt * QK + lane / 2;
    const bool j_ok = j < a.H;

    int4 dq[NBW];
    float dd[NBW];
    const int jc = min(j, a.H - 1);
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const int b = wave + GR_WAVES * i;
        const size_t o = bm_index(e, a.nbF, min(b, a.nbF - 1), a.H, jc);
        dq[i] = *reinterpret_cast<const int4 *>(a.dq + o * QK + 16 * h);
        dd[i] = __half2float(a.dd[o]);
    }
#pragma unroll
    for (int i = 0; i < NBW; i++) dd[i] = (j_ok && (wave + GR_WAVES * i) < a.nbF) ? dd[i] : 0.0f;
    // all loads above are issued before any of the arithmetic below
    __builtin_amdgcn_sched_barrier(0);

    for (int c0 = 0; c0 < n; c0 += GR_MT) {
        const int mt = min(GR_MT, n - c0);
        __syncthreads();
        if (threadIdx.x < GR_MT) rowid[threadIdx.x] = base + c0 + min((int)threadIdx.x, mt - 1);
        __syncthreads();
        stage_rows<XN, GR_MT>(gl, gs, a.g, a.F, a.F, rowid, mt);
#pragma unroll
        for (int i = 0; i < NBW; i++) opaque(dq[i]);
        float yv[GR_MT];
#pragma unroll
        for (int m = 0; m < GR_MT; m++) yv[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            const int b = wave + GR_WAVES * i;
            float dw[16];
            cvt16_off(dq[i], dw);
#pragma unroll
            for (int m = 0; m < GR_MT; m++)
                if (m < mt) yv[m] = fmaf(dot16_off(dw, &gl[m][b * QK + 16 * h], gs[m][2 * b + h]), dd[i], yv[m]);
        }
#pragma unroll
        for (int m = 0; m < GR_MT; m++) {
            yv[m] += __shfl_xor(yv[m], 1, WAVE);
            if (h == 0) red[m][wave][lane / 2] = yv[m];
        }
        __syncthreads();
        if (threadIdx.x < GR_MT * QK) {
            const int m = threadIdx.x / QK, r = threadIdx.x % QK;
            const int jr = jt * QK + r;
            if (m < mt && jr < a.H) {
                float v = red[m][0][r];
#pragma unroll
                for (int w = 1; w < GR_WAVES; w++) v += red[m][w][r];
                a.y[(size_t)(base + c0 + m) * a.H + jr] = v;
            }
        }
    }
}

// hidden[t][j] += sum_k fp32-rounded w[t,k] * y[inv[t,k]][j], ranks in order.
template <int KM>
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *__restrict__ y, int H, int K,
                                                          const int32_t *__restrict__ inv,
                                                          const double *__restrict__ w,
                                                          float *__restrict__ hidden)
{
    const int t = blockIdx.y;
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= H) return;
    int sv[KM];
    double wv[KM];
#pragma unroll
    for (int k = 0; k < KM; k++) {
        sv[k] = k < K ? inv[t * K + k] : -1;
        wv[k] = k < K ? w[t * K + k] : 0.0;
    }
    float v[KM];
#pragma unroll
    for (int k = 0; k < KM; k++) v[k] = sv[k] >= 0 ? y[(size_t)sv[k] * H + j] : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (sv[k] >= 0) acc = (float)((double)acc + wv[k] * (double)v[k]);
    hidden[(size_t)t * H + j] = hidden[(size_t)t * H + j] + acc;
}

int launch_dispatch(qq_ctx *ctx, const qq_moe *m, const int32_t *idx, int P, const MaskBits &mask,
                    int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                    const DispatchTiles &tiles)
{
    prof_begin(ctx, K_DISPATCH);
    QQ_LAUNCH(ctx, moe_dispatch_kernel, dim3(1), dim3(DISP_THREADS), 0, idx, P, m->E, mask, counts,
              offsets, perm, inv, tiles);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

// The same per element, four consecutive columns per thread (H % 4 == 0,
// 16-byte aligned rows); y rows in fp32 or, from the fp16 MFMA path, fp16.
template <typename YT, int KM>
__global__ __launch_bounds__(256) void moe_combine4_kernel(const YT *__restrict__ y, int H, int K,
                                                           const int32_t *__restrict__ inv,
                                                           const double *__restrict__ w,
                                                           float *__restrict__ hidden)
{
    const int t = blockIdx.y;
    const int j = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (j >= H) return;
    // slots and weights of every rank in one round trip, then every row
    int sv[KM];
    double wv[KM];
#pragma unroll
    for (int k = 0; k < KM; k++) {
        sv[k] = k < K ? inv[t * K + k] : -1;
        wv[k] = k < K ? w[t * K + k] : 0.0;
    }
    // the hidden values and every rank's row in flight at once: rows are
    // loaded at clamped slots (slot 0 for a masked rank) and pinned before
    // the sum, whose conditions would otherwise pull each load under a
    // branch, waited for where the branch joins -- one round trip per rank
    float4 *hp = reinterpret_cast<float4 *>(hidden + (size_t)t * H + j);
    float4 hv = *hp;
    float v[KM][4];
#pragma unroll
    for (int k = 0; k < KM; k++) {
        const int s = max(sv[k], 0);
        if constexpr (sizeof(YT) == 4) {
            const float4 q = *reinterpret_cast<const float4 *>(y + (size_t)s * H + j);
            v[k][0] = q.x; v[k][1] = q.y; v[k][2] = q.z; v[k][3] = q.w;
        } else {
            const uint2 q = *reinterpret_cast<const uint2 *>(y + (size_t)s * H + j);
            const _Float16 *h = reinterpret_cast<const _Float16 *>(&q);
#pragma unroll
            for (int i = 0; i < 4; i++) v[k][i] = (float)h[i];
        }
    }
#pragma unroll
    for (int k = 0; k < KM; k++)
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+v"(v[k][i]));
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < KM; k++) {
        if (sv[k] < 0) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = (float)((double)acc[i] + wv[k] * (double)v[k][i]);
    }
    hv.x = hv.x + acc[0];
    hv.y = hv.y + acc[1];
    hv.z = hv.z + acc[2];
    hv.w = hv.w + acc[3];
    *hp = hv;
}

int launch_combine(qq_ctx *ctx, const qq_moe *m, int T, const void *y, bool y_f16,
                   const int32_t *inv, const double *w, float *hidden)
{
    prof_begin(ctx, K_COMBINE);
    const bool vec = m->H % 4 == 0 && ((uintptr_t)hidden & 15) == 0 && ((uintptr_t)y & 15) == 0;
    if (y_f16 && !vec) return set_error(ctx, "combine: fp16 rows need H %% 4 == 0 and aligned buffers");
    const dim3 g4((m->H / 4 + 255) / 256, T), g1((m->H + 255) / 256, T);
    // every rank's slot, weight and row are loaded before the sum; KM ranks
    // at most, so the registers stay few
#define QQ_COMBINE(KM)                                                                            \
    if (y_f16)                                                                                    \
        QQ_LAUNCH(ctx, (moe_combine4_kernel<_Float16, KM>), g4, dim3(256), 0,                     \
                  static_cast<const _Float16 *>(y), m->H, m->K, inv, w, hidden);                  \
    else if (vec)                                                                                 \
        QQ_LAUNCH(ctx, (moe_combine4_kernel<float, KM>), g4, dim3(256), 0,                        \
                  static_cast<const float *>(y), m->H, m->K, inv, w, hidden);                     \
    else                                                                                          \
        QQ_LAUNCH(ctx, moe_combine_kernel<KM>, g1, dim3(256), 0, static_cast<const float *>(y),   \
                  m->H, m->K, inv, w, hidden);
    if (m->K <= 4) { QQ_COMBINE(4) }
    else if (m->K <= 8) { QQ_COMBINE(8) }
    else { QQ_COMBINE(MAX_K) }
#undef QQ_COMBINE
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

static int nbw_bucket(int nb)
{
    const int n = (nb + GR_WAVES - 1) / GR_WAVES;
    return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : 16;
}

size_t grouped_work_bytes(const qq_moe *m, int T)
{
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t P = (size_t)T * m->K;
    return al((size_t)m->E * 4) + al((size_t)(m->E + 1) * 4) + 2 * al(P * 4) + al(P * m->F * 4) +
           al(P * m->H * 4);
}

int launch_moe_grouped(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                       const MaskBits &mask, const int32_t *idx, const double *w, char *work)
{
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t P = (size_t)T * m->K;
    char *p = work;
    int32_t *counts = reinterpret_cast<int32_t *>(p);  p += al((size_t)m->E * 4);
    int32_t *offsets = reinterpret_cast<int32_t *>(p); p += al((size_t)(m->E + 1) * 4);
    int32_t *perm = reinterpret_cast<int32_t *>(p);    p += al(P * 4);
    int32_t *inv = reinterpret_cast<int32_t *>(p);     p += al(P * 4);
    float *g = reinterpret_cast<float *>(p);           p += al(P * m->F * 4);
    float *y = reinterpret_cast<float *>(p);

    int rc = launch_dispatch(ctx, m, idx, (int)P, mask, counts, offsets, perm, inv, DispatchTiles{});
    if (rc) return rc;

    GroupArgs a;
    a.x = x;
    a.H = m->H;
    a.F = m->F;
    a.K = m->K;
    a.nbH = (m->H + QK - 1) / QK;
    a.nbF = (m->F + QK - 1) / QK;
    a.gq = m->gate->qs;
    a.gd = m->gate->d;
    a.uq = m->up->qs;
    a.ud = m->up->d;
    a.dq = m->down->qs;
    a.dd = m->down->d;
    a.counts = counts;
    a.offsets = offsets;
    a.perm = perm;
    a.g = g;
    a.y = y;

    {
        const dim3 grid(m->E, a.nbF);
        prof_begin(ctx, K_GROUPED_GATEUP);
        switch (nbw_bucket(a.nbH)) {
        case 1: QQ_LAUNCH(ctx, moe_grouped_gateup_kernel<1>, grid, dim3(GR_THREADS), 0, a); break;
        case 2: QQ_LAUNCH(ctx, moe_grouped_gateup_kernel<2>, grid, dim3(GR_THREADS), 0, a); break;
        case 4: QQ_LAUNCH(ctx, moe_grouped_gateup_kernel<4>, grid, dim3(GR_THREADS), 0, a); break;
        case 8: QQ_LAUNCH(ctx, moe_grouped_gateup_kernel<8>, grid, dim3(GR_THREADS), 0, a); break;
        default: QQ_LAUNCH(ctx, moe_grouped_gateup_kernel<16>, grid, dim3(GR_THREADS), 0, a); break;
        }
        prof_end(ctx);
        QQ_HIP(ctx, hipGetLastError());
    }
    {
        const dim3 grid(m->E, (m->H + QK - 1) / QK);
        prof_begin(ctx, K_GROUPED_DOWN);
        switch (nbw_bucket(a.nbF)) {
        case 1: QQ_LAUNCH(ctx, moe_grouped_down_kernel<1>, grid, dim3(GR_THREADS), 0, a); break;
        case 2: QQ_LAUNCH(ctx, moe_grouped_down_kernel<2>, grid, dim3(GR_THREADS), 0, a); break;
        case 4: QQ_LAUNCH(ctx, moe_grouped_down_kernel<4>, grid, dim3(GR_THREADS), 0, a); break;
        case 8: QQ_LAUNCH(ctx, moe_grouped_down_kernel<8>, grid, dim3(GR_THREADS), 0, a); break;
        default: QQ_LAUNCH(ctx, moe_grouped_down_kernel<16>, grid, dim3(GR_THREADS), 0, a); break;
        }
        prof_end(ctx);
        QQ_HIP(ctx, hipGetLastError());
    }
    return launch_combine(ctx, m, T, y, false, inv, w, hidden);
}

}  // namespace qq
