// router.hip -- LFM2-MoE router for token batches: binary64 logits, then
// sigmoid / expert-bias top-K / renormalisation (src/lfm2-engine.js:417-447).
//
// logits[t][e] = fp32(sum_k x[t][k] * W[e][k]).  Every product of a binary32
// activation with a binary32 (or exactly dequantised Q8_0) weight is exact in
// binary64, so computing the sum in binary64 in any fixed order gives the
// reference's fp32 logit except when the two binary64 sums straddle an fp32
// rounding boundary (probability ~2^-29 per logit).
//
// The sum is a small [T x H] x [H x E] product on the binary64 matrix cores
// (v_mfma_f64_16x16x4f64): a workgroup takes 16 tokens x 32 experts x one
// slice of H; the slices' partial sums are stored in binary64 and added in
// slice order by the top-K kernel.
#include "qq_device.h"

namespace qq {

typedef double d4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// Router weight of expert e (F32: column e of [H, E] = E rows of H floats;
// Q8_0: block-major panel, exactly dequantised).
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
    // weights k .. k+3 of expert e (k % 4 == 0, k + 3 < H), zero when e >= E
    __device__ __forceinline__ void at4(int e, int k, bool q8, double (&w)[4]) const
    {
        const int ec = min(e, E - 1);
        const double z = e < E ? 1.0 : 0.0;
        if (q8) {
            const size_t o = bm_index(0, nb, k >> 5, E, ec);
            const int q = *reinterpret_cast<const int *>(qs + o * QK + (k & 31));
            const double sc = (double)__half2float(d[o]) * z;
#pragma unroll
            for (int j = 0; j < 4; j++) w[j] = (double)(int8_t)(q >> (8 * j)) * sc;
        } else {
            const float4 v = *reinterpret_cast<const float4 *>(f32 + (size_t)ec * H + k);
            w[0] = (double)v.x * z;
            w[1] = (double)v.y * z;
            w[2] = (double)v.z * z;
            w[3] = (double)v.w * z;
        }
    }
};

// ---------------------------------------------------------------------------
// Matrix-core logits.  Grid (ceil(T/16), KS, ceil(E/32)), 4 waves.  Lane l of
// a wave loads 4 consecutive k of token row l%16 and of expert rows l%16 and
// 16 + l%16 at k = k0 + 4*(l/16); the j-th of them feeds the j-th of four
// MFMAs, so the four instructions cover k0 .. k0+15 exactly once.  Waves take
// 16-wide k steps round robin inside the workgroup's slice; the four waves'
// accumulators are added in wave order.  part[ks][t][e] (binary64).
// f64 accumulator layout: lane l, element r -> row 4r + l/16, column l%16.
//
// NRM: x holds the residual rows, and the workgroup forms x = rmsnorm(row)
// (src/lfm2-engine.js:251-252) itself as it loads them: out of nw (or unit
// weights), eps and each token's 1 / sqrt(sum x^2 / H + eps), whose sum of
// squares is rmsnorm_kernel's own binary64 tree (wave w takes tokens 4w ..
// 4w + 3; lane l plays thread 64 v + l of the normalising block for v = 0 ..
// NORM_THREADS / 64 - 1), so logits and fp16 rows equal those of the two
// launches bit for bit.
// ---------------------------------------------------------------------------
template <bool Q8, bool NRM>
__global__ __launch_bounds__(256) void router_mfma_kernel(const float *__restrict__ x, int T,
                                                          RouterW W, int kchunk,
                                                          double *__restrict__ part,
                                                          _Float16 *__restrict__ xh,
                                                          const float *__restrict__ nw, double eps)
{
    static_assert(!(Q8 && NRM), "the norm is formed on the F32 router path only");
    __shared__ double red[4][16][33];
    __shared__ double sinv[16];
    const int t0 = blockIdx.x * 16, ks = blockIdx.y, e0 = blockIdx.z * 32;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int r16 = lane & 15, kq = lane >> 4;
    const int t = t0 + r16;
    const double tz = t < T ? 1.0 : 0.0;
    const float *xr = x + (size_t)min(t, T - 1) * W.H;
    const int ka = ks * kchunk, kb = min(W.H, ka + kchunk);
    double inv = 1.0;
    if constexpr (NRM) {
        constexpr int NV = NORM_THREADS / WAVE;
        constexpr int NJ = 4;   // values 4 x NORM_THREADS of a row per pass of loads
        for (int i0 = 0; i0 < 4; i0 += 2) {
            double s[2][NV];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int v = 0; v < NV; v++) s[i][v] = 0.0;
            // thread 64 v + l adds k = 64 v + l + 512 j for j = 0, 1, ... in
            // order; past H the term is an exact no-op (s + 0 with s >= +0).
            // Two tokens' loads of a pass go out together.
            for (int j0 = 0; j0 < W.H; j0 += NJ * NORM_THREADS) {
                float q[2][NJ][NV];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const float *hr = x + (size_t)min(t0 + 4 * wave + i0 + i, T - 1) * W.H;
#pragma unroll
                    for (int j = 0; j < NJ; j++)
#pragma unroll
                        for (int v = 0; v < NV; v++)
                            q[i][j][v] = hr[min(j0 + j * NORM_THREADS + WAVE * v + lane, W.H - 1)];
                }
                // every load above goes out before the first use (a load under
                // its own bounds branch is waited for inside that branch)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
#pragma unroll
                        for (int v = 0; v < NV; v++) asm volatile("" : "+v"(q[i][j][v]));
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
#pragma unroll
                        for (int v = 0; v < NV; v++) {
                            const int k = j0 + j * NORM_THREADS + WAVE * v + lane;
                            const double d = k < W.H ? (double)q[i][j][v] : 0.0;
                            s[i][v] = fma(d, d, s[i][v]);
                        }
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                double r = wave_sum_dpp(s[i][0]);
#pragma unroll
                for (int v = 1; v < NV; v++) r = r + wave_sum_dpp(s[i][v]);
                if (lane == 0) sinv[4 * wave + i0 + i] = rms_inv(r, W.H, eps);
            }
        }
        __syncthreads();
        inv = sinv[r16];
    }

    d4_t acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
    auto step = [&](const float4 xv, const double (&wa)[4], const double (&wb)[4]) {
        const double xd[4] = {(double)xv.x * tz, (double)xv.y * tz, (double)xv.z * tz,
                              (double)xv.w * tz};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(xd[j], wa[j], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(xd[j], wb[j], acc1, 0, 0, 0);
        }
    };
    int k = ka + 16 * wave;
    if constexpr (!Q8) {
        // F32 router: the raw rows of RB steps are loaded before any of them
        // is used (one round trip per RB steps, not per step); steps past
        // the slice load clamped addresses and are skipped
        constexpr int RB = 4;
        const int ea = min(e0 + r16, W.E - 1), eb = min(e0 + 16 + r16, W.E - 1);
        const double za = e0 + r16 < W.E ? 1.0 : 0.0, zb = e0 + 16 + r16 < W.E ? 1.0 : 0.0;
        for (; k < kb; k += 64 * RB) {
            float4 xv[RB], va[RB], vb[RB], nv[RB];
#pragma unroll
            for (int u = 0; u < RB; u++) {
                const int kk = min(k + 64 * u, kb - 16) + 4 * kq;
                xv[u] = *reinterpret_cast<const float4 *>(xr + kk);
                va[u] = *reinterpret_cast<const float4 *>(W.f32 + (size_t)ea * W.H + kk);
                vb[u] = *reinterpret_cast<const float4 *>(W.f32 + (size_t)eb * W.H + kk);
                nv[u] = (NRM && nw) ? *reinterpret_cast<const float4 *>(nw + kk) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            }
            // keeps the loads above the skip test below (otherwise each is
            // sunk into its step's branch and waited for there)
#pragma unroll
            for (int u = 0; u < RB; u++)
                asm volatile("" : "+v"(xv[u].x), "+v"(xv[u].y), "+v"(xv[u].z), "+v"(xv[u].w),
                                  "+v"(va[u].x), "+v"(va[u].y), "+v"(va[u].z), "+v"(va[u].w),
                                  "+v"(vb[u].x), "+v"(vb[u].y), "+v"(vb[u].z), "+v"(vb[u].w));
            if constexpr (NRM) {
                // rmsnorm_kernel's out[k] = fp32(w[k] * x[k] * inv)
#pragma unroll
                for (int u = 0; u < RB; u++) {
                    const float4 wv = nv[u];
                    xv[u].x = (float)((double)wv.x * (double)xv[u].x * inv);
                    xv[u].y = (float)((double)wv.y * (double)xv[u].y * inv);
                    xv[u].z = (float)((double)wv.z * (double)xv[u].z * inv);
                    xv[u].w = (float)((double)wv.w * (double)xv[u].w * inv);
                }
            }
#pragma unroll
            for (int u = 0; u < RB; u++) {
                if (k + 64 * u >= kb) break;
                const double wa[4] = {(double)va[u].x * za, (double)va[u].y * za, (double)va[u].z * za,
                                      (double)va[u].w * za};
                const double wb[4] = {(double)vb[u].x * zb, (double)vb[u].y * zb, (double)vb[u].z * zb,
                                      (double)vb[u].w * zb};
                step(xv[u], wa, wb);
                // the fp16 copy of x for the prefill GEMMs (xh != nullptr):
                // every (token, k) of the slice once, rounded to nearest even
                if (xh && t < T && blockIdx.z == 0) {
                    const h2_t lo = {(_Float16)xv[u].x, (_Float16)xv[u].y};
                    const h2_t hi = {(_Float16)xv[u].z, (_Float16)xv[u].w};
                    *reinterpret_cast<uint2 *>(xh + (size_t)t * W.H + k + 64 * u + 4 * kq) =
                        make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
                }
            }
        }
    } else {
        for (; k < kb; k += 64) {
            const int kk = k + 4 * kq;
            const float4 xv = *reinterpret_cast<const float4 *>(xr + kk);
            double wa[4], wb[4];
            W.at4(e0 + r16, kk, Q8, wa);
            W.at4(e0 + 16 + r16, kk, Q8, wb);
            step(xv, wa, wb);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        red[wave][4 * r + kq][r16] = acc0[r];
        red[wave][4 * r + kq][16 + r16] = acc1[r];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 16 * 32; i += 256) {
        const int tt = i >> 5, ee = i & 31;
        const double s = ((red[0][tt][ee] + red[1][tt][ee]) + red[2][tt][ee]) + red[3][tt][ee];
        if (t0 + tt < T && e0 + ee < W.E) part[((size_t)ks * T + t0 + tt) * W.E + e0 + ee] = s;
    }
}

// ---------------------------------------------------------------------------
// Vector-unit logits for shapes the matrix-core kernel does not take (H not a
// multiple of 16).  Grid (ceil(T/TT), ceil(E/EB)); 256 threads split k; fixed-
// order reduction.  Writes part[0][t][e].
// ---------------------------------------------------------------------------
template <int TT, int EB, bool Q8>
__global__ __launch_bounds__(256) void router_logits_kernel(const float *__restrict__ x, int T,
                                                            RouterW W, double *__restrict__ part)
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
        if (t0 + a < T && e0 + b < E) part[(size_t)(t0 + a) * E + e0 + b] = s;
    }
}

// One wavefront per token: logit = fp32(sum of the KS partial sums in order),
// then the layer's gating (sigmoid + bias, or softmax), stable top-K and
// renormalisation.  EPL = experts per lane (E <= 64 EPL).
template <int EPL>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const double *__restrict__ part, int KS, int T, int E, int K, const float *__restrict__ bias,
    int softmax, int32_t *__restrict__ idx, double *__restrict__ w, float *__restrict__ probs)
{
    __shared__ RouteLds<EPL> rl[4];
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (t >= T) return;
    // every partial sum of this lane in flight at once (loaded at clamped
    // slices, unconditionally), then added in slice order
    double pv[EPL][ROUTER_MAX_SPLIT];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = min(lane + WAVE * i, E - 1);
#pragma unroll
        for (int ks = 0; ks < ROUTER_MAX_SPLIT; ks++)
            pv[i][ks] = part[((size_t)min(ks, KS - 1) * T + t) * E + e];
    }
    float lg[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        double s = pv[i][0];
#pragma unroll
        for (int ks = 1; ks < ROUTER_MAX_SPLIT; ks++)
            if (ks < KS) s += pv[i][ks];
        lg[i] = (lane + WAVE * i < E) ? (float)s : 0.0f;
    }
    float bl[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) bl[i] = bias[min(lane + WAVE * i, E - 1)];
    WaveRoute<EPL> R;
    wave_route<EPL>(lg, bl, E, K, softmax != 0, R, rl[threadIdx.x / WAVE]);
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

// ---------------------------------------------------------------------------
// Small token batches: router logits, top-K and the dispatch in one launch.
// A 1-D grid of 256-thread workgroups, every one resident.  The dispatcher
// deals workgroups to the 8 XCDs round robin (XCD = blockIdx % 8), and all
// KS x ceil(E/32) workgroups of a token tile are placed on one XCD
// (rf_place), so the exchange of the partial logits stays in that XCD's L2.
//  1. Each workgroup forms the binary64 partial logits of its 16 tokens x 32
//     experts x H slice on the matrix cores (as router_mfma_kernel) and
//     publishes each as two tagged words (low and high half) into its XCD's
//     table (L2) and, for a tile whose workgroups did not land on one XCD,
//     into a device-coherent copy, which the waits fall back to after
//     RF_LOCAL_TICKS.  The publishing waves are not the routing waves: a wave
//     that has just stored device-scope words waits for their acknowledgement
//     at its next load.
//  2. The workgroups of expert tile 0 then take 16 / KS tokens each, one wave
//     per token: the KS partials of every expert, added in slice order, the
//     gating and stable top-K of router_topk_kernel (wave_route); the token's
//     routing is stored and its expert ids published as tagged words.
//  3. Workgroup 0 gathers the T K expert ids and does the dispatch of
//     moe_dispatch_kernel: counts, exclusive offsets, row tiles, and slots
//     handed out with LDS atomics (order within an expert unspecified).
// Tags are the decode kernel's: the device epoch + 1, advanced by workgroup 0
// at the end, after every workgroup has published (and so read the epoch).
// Every wait is bounded; on expiry the error word is set and the workgroup
// skips what is left.
// ---------------------------------------------------------------------------
struct FusedRouteArgs {
    const float *x;
    int T;
    RouterW W;
    int kchunk, KS;
    const float *bias;
    int softmax, K;
    MaskBits mask;
    int32_t *idx;          // [T][K]
    double *w;             // [T][K]
    float *probs;          // [T][E] or NULL
    int32_t *counts, *offsets, *perm, *inv;
    DispatchTiles tiles;
    uint32_t *epoch_word;
    uint64_t *pw;          // [KS][T][E][2] tagged halves of the partial logits, XCD-local copy
    uint64_t *pwd;         // the same, device-coherent copy
    uint64_t *iw;          // [T][K] tagged expert ids
    uint32_t *err;
    uint64_t wait_ticks;
};

// blockIdx.x -> (token tile, slice, expert tile): the NXY = KS ceil(E/32)
// workgroups of token tile x take blocks x % 8 + 8 (NXY (x / 8) + j),
// j < NXY, all on XCD x % 8.  False for the blocks past the tiles.
__device__ __forceinline__ bool rf_place(int nx, int KS, int nxy, int &x, int &ks, int &z)
{
    const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3;
    x = xcd + 8 * (loc / nxy);
    const int j = loc - nxy * (loc / nxy);
    ks = j % KS;
    z = j / KS;
    return x < nx;
}

constexpr int FR_MAX_KS = 8;
constexpr int FR_MAX_P = 1024;      // T K pairs dispatched by one workgroup
constexpr int FR_MAX_TILES = FR_MAX_P / 16 + MAX_E;   // row tiles of at least 16 slots

template <int EPL>
__global__ __launch_bounds__(256) void route_dispatch_kernel(FusedRouteArgs a)
{
    __shared__ double red[4][16][33];
    __shared__ int cnt[MAX_E], cur[MAX_E], offs[MAX_E + 1];
    __shared__ int pe[FR_MAX_P];
    __shared__ int tle[FR_MAX_TILES], tlm[FR_MAX_TILES];
    __shared__ int sh_ntiles;
    __shared__ RouteLds<EPL> rl[4];
    __shared__ uint32_t sh_tag;
    __shared__ int sh_fail;
    int T = a.T, E = a.W.E, K = a.K, KS = a.KS, softmax = a.softmax;
    // held in registers: otherwise reloaded from the argument segment (and
    // waited for) at every use in the routing and dispatch below
    asm volatile("" : "+s"(T), "+s"(E), "+s"(K), "+s"(KS), "+s"(softmax));
    int bx, ks, bz;
    if (!rf_place((T + 15) / 16, KS, KS * ((E + 31) / 32), bx, ks, bz)) return;
    const int t0 = bx * 16, e0 = bz * 32;
    const bool wg0 = bx == 0 && ks == 0 && bz == 0;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int TPW = 16 / KS;   // routing waves (tokens) per workgroup of expert tile 0
    const uint32_t epoch = __hip_atomic_load(a.epoch_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        sh_tag = epoch + 1u;
        sh_fail = 0;
    }
    // the expert biases of the routing waves, loaded now rather than after
    // their wait
    float bl[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) bl[i] = a.bias[min(lane + WAVE * i, E - 1)];

    // ---- 1. partial logits of 16 tokens x 32 experts over slice ks ----
    {
        const int r16 = lane & 15, kq = lane >> 4;
        const int t = t0 + r16;
        const double tz = t < T ? 1.0 : 0.0;
        const float *xr = a.x + (size_t)min(t, T - 1) * a.W.H;
        const int ka = ks * a.kchunk, kb = min(a.W.H, ka + a.kchunk);
        d4_t acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
        constexpr int RB = 4;
        const int ea = min(e0 + r16, E - 1), eb = min(e0 + 16 + r16, E - 1);
        const double za = e0 + r16 < E ? 1.0 : 0.0, zb = e0 + 16 + r16 < E ? 1.0 : 0.0;
        for (int k = ka + 16 * wave; k < kb; k += 64 * RB) {
            float4 xv[RB], va[RB], vb[RB];
#pragma unroll
            for (int u = 0; u < RB; u++) {
                const int kk = min(k + 64 * u, kb - 16) + 4 * kq;
                xv[u] = *reinterpret_cast<const float4 *>(xr + kk);
                va[u] = *reinterpret_cast<const float4 *>(a.W.f32 + (size_t)ea * a.W.H + kk);
                vb[u] = *reinterpret_cast<const float4 *>(a.W.f32 + (size_t)eb * a.W.H + kk);
            }
#pragma unroll
            for (int u = 0; u < RB; u++)
                asm volatile("" : "+v"(xv[u].x), "+v"(xv[u].y), "+v"(xv[u].z), "+v"(xv[u].w),
                                  "+v"(va[u].x), "+v"(va[u].y), "+v"(va[u].z), "+v"(va[u].w),
                                  "+v"(vb[u].x), "+v"(vb[u].y), "+v"(vb[u].z), "+v"(vb[u].w));
#pragma unroll
            for (int u = 0; u < RB; u++) {
                if (k + 64 * u >= kb) break;
                const double xd[4] = {(double)xv[u].x * tz, (double)xv[u].y * tz, (double)xv[u].z * tz,
                                      (double)xv[u].w * tz};
                const double wa[4] = {(double)va[u].x * za, (double)va[u].y * za, (double)va[u].z * za,
                                      (double)va[u].w * za};
                const double wb[4] = {(double)vb[u].x * zb, (double)vb[u].y * zb, (double)vb[u].z * zb,
                                      (double)vb[u].w * zb};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(xd[j], wa[j], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(xd[j], wb[j], acc1, 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            red[wave][4 * r + kq][r16] = acc0[r];
            red[wave][4 * r + kq][16 + r16] = acc1[r];
        }
    }
    // (kept here: not sunk to its use behind the wait)
#pragma unroll
    for (int i = 0; i < EPL; i++) asm volatile("" : "+v"(bl[i]));
    __syncthreads();
    const uint32_t tag = sh_tag;
    // publishers: the waves that do not route (all four when every wave routes)
    const int pw0 = (bz == 0 && TPW < 4) ? TPW : 0;
    if (wave >= pw0) {
        for (int i = tid - WAVE * pw0; i < 16 * 32; i += WAVE * (4 - pw0)) {
            const int tt = i >> 5, ee = i & 31;
            const double s = ((red[0][tt][ee] + red[1][tt][ee]) + red[2][tt][ee]) + red[3][tt][ee];
            if (t0 + tt < T && e0 + ee < E) {
                const uint64_t b = __double_as_longlong(s);
                const size_t o = (((size_t)ks * T + t0 + tt) * E + e0 + ee) * 2;
                store_tagged_local(a.pw + o, tag, (uint32_t)b);
                store_tagged_local(a.pw + o + 1, tag, (uint32_t)(b >> 32));
                store_tagged(a.pwd + o, tag, (uint32_t)b);
                store_tagged(a.pwd + o + 1, tag, (uint32_t)(b >> 32));
            }
        }
    }

    // ---- 2. routing of 16 / KS tokens (one wave each), expert tile 0 only ----
    bool ok = true;
    const int t = t0 + ks * TPW + wave;
    if (bz == 0 && wave < TPW && t < T) {
        constexpr int NW = EPL * FR_MAX_KS * 2;
        const uint64_t *p[NW];
        bool want[NW];
        uint32_t v[NW];
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = min(lane + WAVE * i, E - 1);
#pragma unroll
            for (int k2 = 0; k2 < FR_MAX_KS; k2++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int n = (i * FR_MAX_KS + k2) * 2 + h;
                    p[n] = a.pw + (((size_t)min(k2, KS - 1) * T + t) * E + e) * 2 + h;
                    want[n] = k2 < KS && lane + WAVE * i < E;
                    v[n] = 0;
                }
        }
        ok = wave_wait<NW>(p, want, tag, v, a.wait_ticks, a.err, a.pwd - a.pw);
        if (ok) {
            float lg[EPL];
#pragma unroll
            for (int i = 0; i < EPL; i++) {
                double s = 0.0;
#pragma unroll
                for (int k2 = 0; k2 < FR_MAX_KS; k2++) {
                    const int n = (i * FR_MAX_KS + k2) * 2;
                    const double d = __longlong_as_double((long long)(((uint64_t)v[n + 1] << 32) | v[n]));
                    if (k2 == 0) s = d;
                    else if (k2 < KS) s += d;
                }
                lg[i] = (lane + WAVE * i < E) ? (float)s : 0.0f;
            }
            WaveRoute<EPL> R;
            wave_route<EPL>(lg, bl, E, K, softmax != 0, R, rl[wave]);
            if (a.probs) {
#pragma unroll
                for (int i = 0; i < EPL; i++) {
                    const int e = lane + WAVE * i;
                    if (e < E) a.probs[(size_t)t * E + e] = R.prob[i];
                }
            }
#pragma unroll
            for (int k = 0; k < MAX_K; k++) {
                if (k < K && lane == k) {
                    a.idx[(size_t)t * K + k] = R.idx[k];
                    a.w[(size_t)t * K + k] = (double)R.p[k] * R.inv;
                    store_tagged(&a.iw[(size_t)t * K + k], tag, (uint32_t)R.idx[k]);
                }
            }
        }
        if (!ok && lane == 0) sh_fail = 1;
    }

    // ---- 3. the dispatch, by workgroup 0 ----
    // After a failed wait it still writes a consistent, empty dispatch (no
    // slots, every pair unrouted), so the expert kernels behind it do nothing.
    if (wg0) {
        __syncthreads();
        const int P = T * K;
        constexpr int PPT = FR_MAX_P / 256;
        if (sh_fail == 0) {
            const uint64_t *p[PPT];
            bool want[PPT];
            uint32_t v[PPT];
#pragma unroll
            for (int i = 0; i < PPT; i++) {
                const int q = tid + 256 * i;
                p[i] = &a.iw[min(q, P - 1)];
                want[i] = q < P;
                v[i] = 0;
            }
            if (!wave_wait<PPT>(p, want, tag, v, a.wait_ticks, a.err)) sh_fail = 1;
#pragma unroll
            for (int i = 0; i < PPT; i++)
                if (tid + 256 * i < P) pe[tid + 256 * i] = (int)v[i];
        }
        for (int e = tid; e < E; e += 256) {
            cnt[e] = 0;
            cur[e] = 0;
        }
        __syncthreads();
        const bool good = sh_fail == 0;
        if (good) {
            for (int q = tid; q < P; q += 256) {
                const int e = pe[q];
                if ((unsigned)e < (unsigned)E && !mask_has(a.mask, e)) atomicAdd(&cnt[e], 1);
            }
        }
        __syncthreads();
        // exclusive scans of the expert counts and of their row tiles, into
        // LDS only: the global copies go out after the last barrier (a
        // barrier waits for the stores before it)
        if (wave == 0) {
            int run = 0, trun = 0;
            for (int eb = 0; eb < E; eb += WAVE) {
                const int e = eb + lane;
                const int c = e < E ? cnt[e] : 0;
                int tot;
                const int o = run + wave_excl_scan(c, &tot);
                if (e < E) offs[e] = o;
                run += tot;
                if (a.tiles.bm > 0) {
                    const int nte = (c + a.tiles.bm - 1) / a.tiles.bm;
                    int ttot;
                    int tt = trun + wave_excl_scan(nte, &ttot);
                    for (int m0 = 0; m0 < c && tt < a.tiles.cap; m0 += a.tiles.bm, tt++) {
                        tle[tt] = e;
                        tlm[tt] = m0;
                    }
                    trun += ttot;
                }
            }
            if (lane == 0) {
                offs[E] = run;
                sh_ntiles = min(trun, a.tiles.cap);
            }
        }
        __syncthreads();
        for (int e = tid; e <= E; e += 256) {
            a.offsets[e] = offs[e];
            if (e < E) a.counts[e] = cnt[e];
        }
        if (a.tiles.bm > 0) {
            const int nt = sh_ntiles;
            for (int i = tid; i < nt; i += 256) {
                a.tiles.e[i] = tle[i];
                a.tiles.m0[i] = tlm[i];
            }
            if (tid == 0) *a.tiles.n = nt;
        }
        for (int q = tid; q < P; q += 256) {
            const int e = good ? pe[q] : -1;
            const int pos = ((unsigned)e < (unsigned)E && !mask_has(a.mask, e)) ? offs[e] + atomicAdd(&cur[e], 1) : -1;
            if ((unsigned)pos < (unsigned)P) {   // (always, for a routed pair)
                a.perm[pos] = q;
                a.inv[q] = pos;
            } else {
                a.inv[q] = -1;
            }
        }
        if (tid == 0) {
            if (!good) atomicOr(a.err, 1u);
            // every workgroup has published its partials, so has read the epoch
            __hip_atomic_store(a.epoch_word, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (!ok && lane == 0) {
        atomicOr(a.err, 1u);
    }
}

// Number of H slices for T tokens: enough workgroups to spread over the chip,
// at most ROUTER_MAX_SPLIT, and slices of at least 64 k.
static int router_split(const qq_moe *m, int T)
{
    if (m->H % 16 != 0) return 1;
    const int tiles = ((T + 15) / 16) * ((m->E + 31) / 32);
    int ks = 1;
    while (ks < ROUTER_MAX_SPLIT && tiles * ks < 512 && m->H / (2 * ks) >= 64) ks *= 2;
    return ks;
}

size_t router_work_bytes(const qq_moe *m, int T)
{
    return (size_t)router_split(m, T) * T * m->E * sizeof(double);
}

bool router_norm_supported(const qq_moe *m, const float *hidden, const float *norm_w)
{
    return m->router_type == QQ_TYPE_F32 && m->H % 16 == 0 && ((uintptr_t)hidden & 15) == 0 &&
           ((uintptr_t)norm_w & 15) == 0;
}

int launch_router_topk(qq_ctx *ctx, const qq_moe *m, const float *x, int T, double *part,
                       int32_t *idx, double *w, float *probs, void *xh, bool *xh_done,
                       const NormArgs *norm)
{
    if (xh_done) *xh_done = false;
    if (T <= 0) return QQ_OK;
    if (norm && !(router_norm_supported(m, x, norm->w) && xh && xh_done))
        return set_error(ctx, "router: the norm is formed only by the F32 matrix-core router with fp16 rows");
    const bool q8 = m->router_type == QQ_TYPE_Q8_0;
    RouterW W;
    W.f32 = m->router_f32;
    W.qs = q8 ? m->router_q8->qs : nullptr;
    W.d = q8 ? m->router_q8->d : nullptr;
    W.H = m->H;
    W.E = m->E;
    W.nb = (m->H + QK - 1) / QK;
    const int KS = ((uintptr_t)x & 15) == 0 ? router_split(m, T) : 1;

    prof_begin(ctx, K_ROUTER_LOGITS);
    if (m->H % 16 == 0 && ((uintptr_t)x & 15) == 0) {
        const int kchunk = ((m->H + KS * 64 - 1) / (KS * 64)) * 64;
        const dim3 g((T + 15) / 16, KS, (m->E + 31) / 32);
        if (q8) {
            QQ_LAUNCH(ctx, (router_mfma_kernel<true, false>), g, dim3(256), 0, x, T, W, kchunk, part, nullptr,
                      nullptr, 0.0);
        } else if (norm) {
            QQ_LAUNCH(ctx, (router_mfma_kernel<false, true>), g, dim3(256), 0, x, T, W, kchunk, part,
                      static_cast<_Float16 *>(xh), norm->w, norm->eps);
            *xh_done = true;
        } else {
            QQ_LAUNCH(ctx, (router_mfma_kernel<false, false>), g, dim3(256), 0, x, T, W, kchunk, part,
                      static_cast<_Float16 *>(xh), nullptr, 0.0);
            if (xh && xh_done) *xh_done = true;
        }
    } else {
        const dim3 g((T + 3) / 4, (m->E + 7) / 8);
        if (q8)
            QQ_LAUNCH(ctx, (router_logits_kernel<4, 8, true>), g, dim3(256), 0, x, T, W, part);
        else
            QQ_LAUNCH(ctx, (router_logits_kernel<4, 8, false>), g, dim3(256), 0, x, T, W, part);
    }
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    prof_begin(ctx, K_ROUTER_TOPK);
    const int sm = m->gating == QQ_GATING_SOFTMAX ? 1 : 0;
    if (m->E <= WAVE)
        QQ_LAUNCH(ctx, router_topk_kernel<1>, dim3((T + 3) / 4), dim3(256), 0, part, KS, T, m->E, m->K,
                  m->bias, sm, idx, w, probs);
    else if (m->E <= 2 * WAVE)
        QQ_LAUNCH(ctx, router_topk_kernel<2>, dim3((T + 3) / 4), dim3(256), 0, part, KS, T, m->E, m->K,
                  m->bias, sm, idx, w, probs);
    else
        QQ_LAUNCH(ctx, (router_topk_kernel<MAX_E / WAVE>), dim3((T + 3) / 4), dim3(256), 0, part, KS, T,
                  m->E, m->K, m->bias, sm, idx, w, probs);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

bool route_dispatch_supported(const qq_ctx *ctx, const qq_moe *m, int T, const float *x)
{
    if (m->router_type != QQ_TYPE_F32 || m->H % 16 != 0 || ((uintptr_t)x & 15) != 0 || m->E > 2 * WAVE)
        return false;
    const int KS = router_split(m, T);
    const size_t wgs = (size_t)((T + 15) / 16) * KS * ((m->E + 31) / 32);
    // 16 / KS routing waves per workgroup of 4 waves
    return KS >= 4 && KS <= FR_MAX_KS && 16 % KS == 0 && T * m->K <= FR_MAX_P &&
           (size_t)KS * T * m->E * 2 <= SYNC_RP_WORDS && (size_t)T * m->K <= SYNC_RI_WORDS &&
           wgs <= (size_t)ctx->num_cus;
}

int launch_route_dispatch(qq_ctx *ctx, const qq_moe *m, const float *x, int T, const MaskBits &mask,
                          int32_t *idx, double *w, float *probs, int32_t *counts, int32_t *offsets,
                          int32_t *perm, int32_t *inv, const DispatchTiles &tiles)
{
    FusedRouteArgs a;
    a.x = x;
    a.T = T;
    a.W.f32 = m->router_f32;
    a.W.qs = nullptr;
    a.W.d = nullptr;
    a.W.H = m->H;
    a.W.E = m->E;
    a.W.nb = (m->H + QK - 1) / QK;
    a.KS = router_split(m, T);
    a.kchunk = ((m->H + a.KS * 64 - 1) / (a.KS * 64)) * 64;
    a.bias = m->bias;
    a.softmax = m->gating == QQ_GATING_SOFTMAX ? 1 : 0;
    a.K = m->K;
    a.mask = mask;
    a.idx = idx;
    a.w = w;
    a.probs = probs;
    a.counts = counts;
    a.offsets = offsets;
    a.perm = perm;
    a.inv = inv;
    a.tiles = tiles;
    if (tiles.cap > FR_MAX_TILES) return set_error(ctx, "route_dispatch: %d row tiles, at most %d", tiles.cap, FR_MAX_TILES);
    a.epoch_word = ctx->sync_epoch;
    a.pw = ctx->sync_rp;
    a.pwd = ctx->sync_rp + SYNC_RP_WORDS;
    a.iw = ctx->sync_ri;
    a.err = ctx->sync_err;
    a.wait_ticks = ctx->dec_wait_ticks;
    const int nxy = a.KS * ((m->E + 31) / 32);
    const dim3 g(8u * (unsigned)(((T + 15) / 16 + 7) / 8) * (unsigned)nxy);
    prof_begin(ctx, K_ROUTE_DISPATCH);
    if (m->E <= WAVE) QQ_LAUNCH(ctx, route_dispatch_kernel<1>, g, dim3(256), 0, a);
    else QQ_LAUNCH(ctx, route_dispatch_kernel<2>, g, dim3(256), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

// The routing record of the WebGPU engines' top-K shaders
// (src/webgpu.js:1236-1240): per row, K selected experts as floats, their K
// weights rounded to fp32, the E probabilities.  One thread per record word.
__global__ __launch_bounds__(256) void route_record_kernel(const int32_t *__restrict__ idx,
                                                           const double *__restrict__ w,
                                                           const float *__restrict__ probs, int T, int K,
                                                           int E, float *__restrict__ rec)
{
    const int L = 2 * K + E;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * L) return;
    const int t = (int)(i / L), j = (int)(i - (size_t)t * L);
    float v;
    if (j < K)
        v = (float)idx[(size_t)t * K + j];
    else if (j < 2 * K)
        v = (float)w[(size_t)t * K + j - K];
    else
        v = probs[(size_t)t * E + j - 2 * K];
    rec[i] = v;
}

int launch_route_record(qq_ctx *ctx, const int32_t *idx, const double *w, const float *probs, int T,
                        int K, int E, float *rec)
{
    const size_t n = (size_t)T * (2 * K + E);
    prof_begin(ctx, K_ROUTER_TOPK);
    QQ_LAUNCH(ctx, route_record_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, idx, w, probs, T, K, E,
              rec);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
