// lfm2.hip -- kernels of the LFM2 single-token device forward.
//
// Reference: Lfm2Engine.forward, src/lfm2-engine.js:228-280, and the blocks
// it calls (_shortConv :282-327, _selfAttention :329-392, _denseFfn
// :394-403); the MoE block runs through decode.hip.
//
// One token per call.  The matrix products are Q8_0 x fp32 matvecs
// (matmulQ80xF32, src/tensor.js:26-53) over the repacked block-major panels
// of q8_0.hip, and every elementwise step of the reference is folded into
// the matvec that produces or consumes its operands:
//   * the RMSNorm in front of a block (attn_norm, ffn_norm, the output norm:
//     src/tensor.js:103-114) is formed by every workgroup of the matvec that
//     reads it, from the residual row (binary64 sum of squares);
//   * residual adds (addVec, src/tensor.js:181-185) are the epilogue of the
//     matvec whose output is added (hidden = fp32(hidden + fp32(W x)));
//   * short-conv: a workgroup owns 8 channels d and computes rows d, H + d
//     and 2H + d of in_proj (B, C, x), then bx = B * x, the depthwise causal
//     conv over its channels' state, the state shift and y = C * conv;
//   * attention: q, k and v are one matvec over their concatenated rows (v
//     goes straight into the KV cache); each attention workgroup forms the
//     per-head RMSNorm and split-half RoPE of its q head and of the new k row
//     itself, and one workgroup per KV head stores that k row;
//   * dense FFN: rows f of gate and up in one workgroup, silu(g) * u.
// Where the reference stores into a Float32Array the kernels round to fp32 at
// the same step, and its binary64 expressions are kept in binary64 without
// contraction into fused multiply-adds.
#include "qq_device.h"

// binary64 expressions of the reference stay separate multiplies and adds
#pragma clang fp contract(off)

namespace qq {

constexpr int LM_MAX_IN = 8192;  // longest input row staged in LDS
constexpr int LM_MAX_L = 4;      // short-conv kernel length (l_cache) supported
constexpr int LM_HEAD = 64;      // head_dim supported by the QKV epilogue and attention
constexpr int LM_MAX_CTX = 4096; // the reference caps the context at 4096 (lfm2-engine.js:33)
constexpr int LM_ATTN_THREADS = 256;
constexpr int LM_CHUNK = 256;    // positions of the one-workgroup attention, and of a long-context chunk

struct LmMat {
    const int8_t *qs;
    const __half *dcm;   // scales row by row: dcm[r * nbp + b]
    int rows, nbp;
};

struct LmArgs {
    const float *x;      // input row (in_dim floats)
    int in_dim, nb;      // nb = ceil(in_dim / 32)
    int norm;            // x = rmsnorm(x) * norm_w first
    const float *norm_w;
    double eps;
    LmMat m[3];          // PLAIN/RESID/CONV: m[0]; SWIGLU: gate, up; QKV: q, k, v
    float *y;            // output (RESID: added into)
    // short-conv: state [L-1][H] (oldest first), kernel [H][L]
    float *state;
    const float *kern;
    int L, H;
    // attention: raw q and k rows out, V into the KV cache of this layer
    // [n_kv_heads][max_ctx][64]
    float *q, *kraw;
    float *kc, *vc;
    const float *qn, *kn;   // per-head norm weights [64]
    int n_heads, n_kv_heads, pos, max_ctx;
    const double *freq;     // RoPE frequencies 1 / base^(i / 32), i < 32
};

// Sum of one value per thread over a block of NW waves: waves by DPP, then
// the wave sums in wave order (the order of block_sum_f64).  Its barrier
// orders LDS only, so global loads issued before it stay in flight.
template <int NW>
__device__ __forceinline__ double lm_block_sum(double v, double *red)
{
    v = wave_sum_dpp(v);
    if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = v;
    lds_barrier();
    double s = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) s = s + red[w];
    return s;
}

template <int NW>
__device__ __forceinline__ float lm_block_max(float v, float *red)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = fmaxf(m, red[w]);
    return m;
}

// First row of matrix `mat` owned by row group g (RPW rows) of this workgroup.
// 16 weight bytes read once per token: a non-temporal load, so the weight
// stream does not evict the activations, caches and state other launches
// read again
__device__ __forceinline__ uint4 load_nt16(const int8_t *p)
{
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int MODE, int G, int RPW>
__device__ __forceinline__ int lm_row(const LmArgs &a, int g, int &mat)
{
    const int j = blockIdx.x;
    if (MODE == LM_PLAIN || MODE == LM_RESID) {
        mat = 0;
        return G * RPW * j + RPW * g;
    }
    if (MODE == LM_SWIGLU) {   // group 0: gate rows, group 1: the same up rows
        mat = g;
        return RPW * j;
    }
    if (MODE == LM_CONV) {     // group g: rows g*H + channels of the workgroup
        mat = 0;
        return g * a.H + RPW * j;
    }
    // QKV: the rows of q, then k, then v, G * RPW of them per workgroup
    // (head sizes are multiples of it, so a workgroup stays in one matrix)
    const int r = G * RPW * j + RPW * g;
    const int nq = a.n_heads * LM_HEAD, nkv = a.n_kv_heads * LM_HEAD;
    mat = r < nq ? 0 : (r < nq + nkv ? 1 : 2);
    return r - (mat >= 1 ? nq : 0) - (mat == 2 ? nkv : 0);
}

// BPL int8 weights (offset binary after the XOR) against BPL activations:
// sum q_i x_i = sum (q_i + 128) x_i - 128 sum x_i, each byte converted by one
// v_cvt_f32_ubyte.
template <int BPL>
__device__ __forceinline__ float lm_dot(const uint32_t (&w)[BPL / 4], const float *x, float xsum)
{
    float xr[BPL];
#pragma unroll
    for (int i = 0; i < BPL / 4; i++) {
        const float4 v = reinterpret_cast<const float4 *>(x)[i];
        xr[4 * i] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < BPL / 4; i++) {
        const uint32_t u = w[i] ^ 0x80808080u;
#pragma unroll
        for (int b = 0; b < 4; b++) acc = fmaf((float)((u >> (8 * b)) & 0xffu), xr[4 * i + b], acc);
    }
    return fmaf(-128.0f, xsum, acc);
}

// G row groups of RPW rows, WPG waves each.  A wave's lanes take a row,
// a 16-byte half of a block and a block slot: lane l holds half l & 1, row
// (l >> 1) % RPW and slot l / (2 RPW), so one 16-byte load per lane covers
// the group's RPW rows x SPW = 64 / (2 RPW) block columns (each a contiguous
// run of 32 RPW bytes).  A wave keeps NBW such loads in flight per lane
// (blocks of a chunk of WPG * SPW * NBW); the row sums are added over the
// lanes of a wave by shuffles, then over the group's waves in wave order.
// Fewer rows per group spread a matrix over more workgroups (CUs): one CU
// pulls only a few tens of GB/s.  Each thread loads XR values of the input
// row (XR * threads >= nb * 32) before the weights.
template <int MODE, int G, int WPG, int NBW, int RPW, int XR>
__global__ __launch_bounds__(G * WPG * WAVE) void lfm2_mv_kernel(LmArgs a)
{
    constexpr int NT = G * WPG * WAVE;
    constexpr int NW = G * WPG;
    constexpr int SPW = WAVE / (2 * RPW);   // block slots per wave
    constexpr int BPR = WPG * SPW;          // block columns per round of a row group
    static_assert(SPW * 2 * RPW == WAVE, "lane layout");
    static_assert(MODE != LM_QKV || LM_HEAD % (G * RPW) == 0, "a workgroup within one head");
    extern __shared__ __align__(16) float lm_lds[];
    float *xl = lm_lds;                  // nb * 32 activations (zero padded)
    float *xs = lm_lds + a.nb * QK;      // sums of every 16-value half block
    __shared__ float red[G][WPG][RPW];
    __shared__ double redd[NW];
    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = tid / WAVE;
    const int kp = a.nb * QK;

    // ---- row groups: lane l takes row (l >> 1) % RPW, half l & 1 of slot l / (2 RPW) ----
    const int g = wave / WPG, wg = wave % WPG;
    int mat;
    const int row0 = lm_row<MODE, G, RPW>(a, g, mat);
    const LmMat M = a.m[mat];
    const int h = lane & 1, rr = (lane >> 1) & (RPW - 1), sl = lane / (2 * RPW);
    const int row = row0 + rr;
    const int rc = min(row, M.rows - 1);
    const int first = wg * SPW + sl;     // this lane's first block of a chunk
    uint4 q[NBW];
    float dd[NBW];
    // NBW blocks from chunk c0 on (stride BPR), at clamped addresses and
    // without a condition on the loaded values (a value selected against a
    // condition lets the compiler move its load under a branch, whose join
    // then waits for every load in flight).  Blocks past nb are skipped in
    // the products; a row past the matrix reads row rows - 1 and is never
    // stored.  Scales come from the row-major copy (a group's rows' scales
    // are lines no other workgroup reads).
    auto load = [&](int c0) {
#pragma unroll
        for (int u = 0; u < NBW; u++) {
            const int b = min(c0 + first + BPR * u, a.nb - 1);
            const size_t o = bm_index(0, a.nb, b, M.rows, rc);
            q[u] = load_nt16(M.qs + o * QK + 16 * h);
            dd[u] = __half2float(M.dcm[(size_t)rc * M.nbp + b]);
        }
    };
    // ---- loads first: this thread's share of the input row (and norm
    // weights), then the first chunk of weight blocks, then the operands of
    // the epilogue.  Loads complete in issue order and the barriers below
    // order LDS only, so the row is normalised and staged while the weight
    // bytes are still in flight. ----
    // (unconditional loads at clamped indices, values selected once they
    // arrive: a load under a branch is waited for where the branch joins)
    float xr[XR], wr[XR];
    const float *nw = a.norm_w ? a.norm_w : a.x;
#pragma unroll
    for (int i = 0; i < XR; i++) {
        const int k = min(tid + NT * i, a.in_dim - 1);
        xr[i] = a.x[k];
        wr[i] = nw[k];
    }
    __builtin_amdgcn_sched_barrier(0);
    load(0);
    // epilogue operands: the residual value (RESID), the conv state and
    // kernel taps of this thread's channel (CONV)
    float yold = 0.0f;
    float st[LM_MAX_L], kw[LM_MAX_L];
    if (MODE == LM_RESID && tid < G * RPW) {
        const int orow = G * RPW * blockIdx.x + tid;
        if (orow < a.m[0].rows) yold = a.y[orow];
    }
    if (MODE == LM_CONV) {   // clamped, unconditional (used only where in range)
        const int d = min(RPW * (int)blockIdx.x + tid, a.H - 1);
#pragma unroll
        for (int k = 0; k < LM_MAX_L; k++) {
            st[k] = a.state[(size_t)min(k, a.L - 2) * a.H + d];
            kw[k] = a.kern[(size_t)d * a.L + min(k, a.L - 1)];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- input row -> LDS, normalised when asked (src/tensor.js:103-114) ----
    double inv = 1.0;
    if (a.norm) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < XR; i++)
            if (tid + NT * i < a.in_dim) {
                const double v = (double)xr[i];
                ss = fma(v, v, ss);
            }
        inv = rms_inv(lm_block_sum<NW>(ss, redd), a.in_dim, a.eps);
    }
#pragma unroll
    for (int i = 0; i < XR; i++) {
        const int k = tid + NT * i;
        if (k < kp) {
            float v = k < a.in_dim ? xr[i] : 0.0f;
            if (a.norm && k < a.in_dim)
                v = (float)((double)(a.norm_w ? wr[i] : 1.0f) * (double)v * inv);
            xl[k] = v;
        }
    }
    lds_barrier();
    for (int i = tid; i < kp / 16; i += NT) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) s += xl[16 * i + j];
        xs[i] = s;
    }
    lds_barrier();

    float acc = 0.0f;
    for (int c0 = 0;;) {
#pragma unroll
        for (int u = 0; u < NBW; u++) {
            const int b = c0 + first + BPR * u;
            if (b < a.nb) {
                const uint32_t w4[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
                acc = fmaf(lm_dot<16>(w4, &xl[b * QK + 16 * h], xs[2 * b + h]), dd[u], acc);
            }
        }
        c0 += NBW * BPR;
        if (c0 >= a.nb) break;
        load(c0);
        __builtin_amdgcn_sched_barrier(0);   // every load of the chunk before its arithmetic
    }
    acc += __shfl_xor(acc, 1, WAVE);
#pragma unroll
    for (int o = 2 * RPW; o < WAVE; o <<= 1) acc += __shfl_xor(acc, o, WAVE);
    if (lane < 2 * RPW && h == 0) red[g][wg][rr] = acc;
    __syncthreads();

    // ---- epilogues ----
    auto rowsum = [&](int gg, int r) {
        float v = red[gg][0][r];
#pragma unroll
        for (int w = 1; w < WPG; w++) v += red[gg][w][r];
        return v;
    };
    if (MODE == LM_PLAIN || MODE == LM_RESID) {
        if (tid < G * RPW) {
            const int gg = tid / RPW, r = tid % RPW;
            const int orow = G * RPW * blockIdx.x + RPW * gg + r;
            if (orow < a.m[0].rows) {
                const float v = rowsum(gg, r);
                a.y[orow] = MODE == LM_RESID ? yold + v : v;
            }
        }
    } else if (MODE == LM_SWIGLU) {
        // siluInPlace, mulInPlace (src/tensor.js:167-179)
        const int f = RPW * blockIdx.x + tid;
        if (tid < RPW && f < a.m[0].rows) {
            const float gv = rowsum(0, tid), uv = rowsum(1, tid);
            const double g64 = (double)gv;
            const float s = (float)(g64 * (1.0 / (1.0 + exp(-g64))));
            a.y[f] = s * uv;
        }
    } else if (MODE == LM_CONV) {
        // _shortConv steps 3-6 (src/lfm2-engine.js:297-322) for channel d
        const int d = RPW * blockIdx.x + tid;
        if (tid < RPW && d < a.H) {
            const float B = rowsum(0, tid), C = rowsum(1, tid), X = rowsum(2, tid);
            const float bx = B * X;
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < LM_MAX_L; k++) {
                if (k >= a.L) break;
                const double w = (double)kw[k];
                const double t = w * (double)(k < a.L - 1 ? st[k] : bx);
                s = k == 0 ? t : s + t;
            }
            const float co = (float)s;
#pragma unroll
            for (int k = 0; k + 1 < LM_MAX_L - 1; k++)
                if (k + 1 < a.L - 1) a.state[(size_t)k * a.H + d] = st[k + 1];
            a.state[(size_t)(a.L - 2) * a.H + d] = bx;
            a.y[d] = C * co;
        }
    } else {
        // QKV: raw q and k rows; v rows straight into the cache (KVCache.store,
        // src/kv-cache.js:16-32)
        if (tid < G * RPW) {
            const int r = G * RPW * blockIdx.x + tid;
            const int nq = a.n_heads * LM_HEAD, nkv = a.n_kv_heads * LM_HEAD;
            const float v = rowsum(tid / RPW, tid % RPW);
            if (r < nq) a.q[r] = v;
            else if (r < nq + nkv) a.kraw[r - nq] = v;
            else if (r < nq + 2 * nkv) {
                const int rv = r - nq - nkv;
                a.vc[((size_t)(rv / LM_HEAD) * a.max_ctx + a.pos) * LM_HEAD + rv % LM_HEAD] = v;
            }
        }
    }
}

// perHeadRMSNorm (src/tensor.js:117-129) then applyRoPE (:132-147) of one
// 64-value head `raw` into LDS `out`, by one wave (lane l holds value l):
// the sum of squares in order in binary64 (every lane runs the same
// sequence), (w * x) * inv, and x0' = fp32(x0 cos - x1 sin),
// x1' = fp32(x0 sin + x1 cos) in binary64.
__device__ __forceinline__ void lm_head_prep(const float *__restrict__ raw, const float *__restrict__ nw,
                                             double eps, int pos, const double *__restrict__ freq,
                                             float *out)
{
    static_assert(LM_HEAD == WAVE, "one value per lane");
    const int l = threadIdx.x & (WAVE - 1);
    const float x = raw[l];
    const float w = nw[l];
    const double fr = freq[l & (LM_HEAD / 2 - 1)];
    const int xb = __float_as_int(x);
    double ss = 0.0;
    for (int i = 0; i < LM_HEAD; i++) {
        const double v = (double)__int_as_float(__builtin_amdgcn_readlane(xb, i));
        ss = ss + v * v;
    }
    const double inv = 1.0 / sqrt(ss / (double)LM_HEAD + eps);
    const float t = (float)((double)w * (double)x * inv);
    const float other = __shfl(t, (l + LM_HEAD / 2) & (WAVE - 1), WAVE);   // lane i < 32: value i + 32
    if (l < LM_HEAD / 2) {
        const double th = (double)pos * fr;
        const double c = cos(th), s = sin(th);
        const double x0 = (double)t, x1 = (double)other;
        out[l] = (float)(x0 * c - x1 * s);
        out[l + LM_HEAD / 2] = (float)(x0 * s + x1 * c);
    }
}

// The query head hq and the new k row of its kv head g, normed and rotated,
// into LDS; the first query head of each kv head (in the last chunk) stores
// the k row into the cache, which nobody reads in this launch (position
// n - 1 takes kpos).
struct LmAttnIn {
    const float *q, *kraw;
    const float *qn, *kn;
    const double *freq;
    double eps;
};

__device__ __forceinline__ bool lm_first_of_group(int hq, int g, int n_heads, int n_kv_heads)
{
    return hq == 0 || (int)(((long long)(hq - 1) * n_kv_heads) / n_heads) != g;
}

// blockIdx.x -> (query head hq, chunk c) of the attention kernels.  The
// dispatcher deals workgroups to the 8 XCDs round robin, so the GQ =
// n_heads / n_kv_heads query heads of one (chunk, KV head) unit get block
// indices 8 apart: they run on one XCD and read that KV head's rows into one
// L2 (head hq of KV head hq / GQ, as (h * n_kv_heads / n_heads) | 0 with
// n_heads a multiple of n_kv_heads).  False for the padding blocks.
__device__ __forceinline__ bool lm_attn_unit(int n_heads, int n_kv_heads, int nch, int &hq, int &c)
{
    const int GQ = n_heads / n_kv_heads;
    const int x = blockIdx.x & 7, r = blockIdx.x >> 3;
    const int u = (r / GQ) * 8 + x;   // unit c * n_kv_heads + KV head
    if (u >= n_kv_heads * nch) return false;
    c = u / n_kv_heads;
    hq = (u - c * n_kv_heads) * GQ + r % GQ;
    return true;
}

static unsigned lm_attn_grid(int n_heads, int n_kv_heads, int nch)
{
    return 8u * (unsigned)((n_kv_heads * nch + 7) / 8) * (unsigned)(n_heads / n_kv_heads);
}

// GQA attention of one token (src/lfm2-engine.js:354-388), one workgroup
// per query head h over kv head (h * n_kv_heads / n_heads) | 0 and positions
// 0..n-1:
//   score_p = fp32(dot(q, k_p) * scale)   dot in binary64, in dimension order
//   softmaxInPlace (src/tensor.js:150-164): max, e_p = fp32(exp(s_p - max)),
//     w_p = fp32(e_p * (1 / sum e))
//   out[d] = fp32 sum of v_p[d] * w_p
// The sum of the exponentials is a tree (not the reference's one-by-one
// order) and out[d] is accumulated in four position classes joined at the
// end, so those two steps agree with the reference to rounding, not bit for bit.
__global__ __launch_bounds__(LM_ATTN_THREADS) void lfm2_attn_kernel(LmAttnIn in, float *__restrict__ kc,
                                                                   const float *__restrict__ vc,
                                                                   int n_heads, int n_kv_heads,
                                                                   int max_ctx, int n, double scale,
                                                                   float *__restrict__ out)
{
    constexpr int NW = LM_ATTN_THREADS / WAVE;
    __shared__ __align__(16) float qh[LM_HEAD];
    __shared__ __align__(16) float kpos[LM_HEAD];
    __shared__ float sc[LM_MAX_CTX];
    __shared__ float redf[NW];
    __shared__ double redd[NW];
    __shared__ float part[NW][LM_HEAD];
    const int tid = threadIdx.x;
    int hq, c;
    if (!lm_attn_unit(n_heads, n_kv_heads, 1, hq, c)) return;
    const int g = (int)(((long long)hq * n_kv_heads) / n_heads);
    const float *K = kc + (size_t)g * max_ctx * LM_HEAD;
    const float *V = vc + (size_t)g * max_ctx * LM_HEAD;
    const int d = tid % LM_HEAD, cls = tid / LM_HEAD;
    // loads that depend on nothing are issued first: this thread's first K
    // row (cached positions only: position n - 1 is this call's) and every
    // value of its V column it sums (positions cls, cls + NW, ...)
    constexpr int VPT = LM_CHUNK / NW;   // V values per thread
    static_assert(LM_ATTN_THREADS == LM_CHUNK, "up to LM_CHUNK positions");
    float4 kr[LM_HEAD / 4];
    auto load_k = [&](int p) {
        if (p >= n - 1) return;
        const float4 *src = reinterpret_cast<const float4 *>(K + (size_t)p * LM_HEAD);
#pragma unroll
        for (int i = 0; i < LM_HEAD / 4; i++) kr[i] = src[i];
    };
#pragma unroll
    for (int i = 0; i < LM_HEAD / 4; i++) kr[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    load_k(tid);
    float vv[VPT];
#pragma unroll
    for (int u = 0; u < VPT; u++) vv[u] = V[(size_t)min(cls + NW * u, n - 1) * LM_HEAD + d];
    // this query head (wave 0) and the new k row (wave 1), normed and rotated
    if (tid / WAVE == 0) lm_head_prep(in.q + (size_t)hq * LM_HEAD, in.qn, in.eps, n - 1, in.freq, qh);
    else if (tid / WAVE == 1) lm_head_prep(in.kraw + (size_t)g * LM_HEAD, in.kn, in.eps, n - 1, in.freq, kpos);
    __syncthreads();
    if (lm_first_of_group(hq, g, n_heads, n_kv_heads) && tid < LM_HEAD)
        kc[((size_t)g * max_ctx + n - 1) * LM_HEAD + tid] = kpos[tid];
    float mx = -INFINITY;
    for (int p = tid; p < n; p += LM_ATTN_THREADS) {
        double dot = 0.0;
        const bool self = p == n - 1;
#pragma unroll
        for (int i = 0; i < LM_HEAD / 4; i++) {
            const float4 kv = self ? reinterpret_cast<const float4 *>(kpos)[i] : kr[i];
            dot = fma((double)qh[4 * i], (double)kv.x, dot);
            dot = fma((double)qh[4 * i + 1], (double)kv.y, dot);
            dot = fma((double)qh[4 * i + 2], (double)kv.z, dot);
            dot = fma((double)qh[4 * i + 3], (double)kv.w, dot);
        }
        const float s = (float)(dot * scale);
        sc[p] = s;
        mx = fmaxf(mx, s);
        if (p + LM_ATTN_THREADS < n) load_k(p + LM_ATTN_THREADS);
    }
    const float M = lm_block_max<NW>(mx, redf);
    double ls = 0.0;
    for (int p = tid; p < n; p += LM_ATTN_THREADS) {
        const float e = (float)exp((double)sc[p] - (double)M);
        sc[p] = e;
        ls += (double)e;
    }
    const double inv = 1.0 / block_sum_f64<NW>(ls, redd);
    for (int p = tid; p < n; p += LM_ATTN_THREADS) sc[p] = (float)((double)sc[p] * inv);
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const int p = cls + NW * u;
        if (p >= n) break;
        const float w = sc[p];
        if (w != 0.0f) acc = (float)fma((double)vv[u], (double)w, (double)acc);
    }
    part[cls][d] = acc;
    __syncthreads();
    if (tid < LM_HEAD) {
        float o = part[0][tid];
#pragma unroll
        for (int c = 1; c < NW; c++) o = o + part[c][tid];
        out[(size_t)hq * LM_HEAD + tid] = o;
    }
}

// Long contexts: the same attention split over chunks of LM_CHUNK positions
// (one workgroup per head and chunk, so the K and V rows of a head are read
// by many CUs at once).  Chunk c writes its score max m_c, the binary64 sum
// l_c of fp32(exp(s - m_c)) and o_c[d] = sum fp32(exp(s - m_c)) * v[d]
// (binary64); lfm2_attn_join_kernel then forms
// out[d] = fp32(sum_c o_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M)), M = max m_c,
// over the chunks in order.  Equal to the one-workgroup form to rounding.
constexpr int LM_MAX_CHUNKS = LM_MAX_CTX / LM_CHUNK;
constexpr int LM_PART = LM_HEAD + 2;   // doubles per (head, chunk): o[64], m, l

__global__ __launch_bounds__(LM_ATTN_THREADS) void lfm2_attn_chunk_kernel(
    LmAttnIn in, float *__restrict__ kc, const float *__restrict__ vc, int n_heads,
    int n_kv_heads, int max_ctx, int n, int nch, double scale, double *__restrict__ part)
{
    constexpr int NW = LM_ATTN_THREADS / WAVE;
    constexpr int VPT = LM_CHUNK / NW;   // V values per thread
    static_assert(LM_ATTN_THREADS == LM_CHUNK, "one position per thread");
    __shared__ __align__(16) float qh[LM_HEAD];
    __shared__ __align__(16) float kpos[LM_HEAD];
    __shared__ float ex[LM_CHUNK];
    __shared__ float redf[NW];
    __shared__ double redd[NW];
    __shared__ double po[NW][LM_HEAD];
    const int tid = threadIdx.x;
    int hq, c;
    if (!lm_attn_unit(n_heads, n_kv_heads, nch, hq, c)) return;
    const int g = (int)(((long long)hq * n_kv_heads) / n_heads);
    const float *K = kc + (size_t)g * max_ctx * LM_HEAD;
    const float *V = vc + (size_t)g * max_ctx * LM_HEAD;
    const int p0 = c * LM_CHUNK;
    const int d = tid % LM_HEAD, cls = tid / LM_HEAD;
    // independent loads first: this thread's K row (cached positions only:
    // position n - 1 is this call's) and its V column values
    float4 kr[LM_HEAD / 4];
#pragma unroll
    for (int i = 0; i < LM_HEAD / 4; i++) kr[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (p0 + tid < n - 1) {
        const float4 *src = reinterpret_cast<const float4 *>(K + (size_t)(p0 + tid) * LM_HEAD);
#pragma unroll
        for (int i = 0; i < LM_HEAD / 4; i++) kr[i] = src[i];
    }
    float vv[VPT];
#pragma unroll
    for (int u = 0; u < VPT; u++) vv[u] = V[(size_t)min(p0 + cls + NW * u, n - 1) * LM_HEAD + d];
    // this query head (wave 0) and the new k row (wave 1), normed and rotated
    if (tid / WAVE == 0) lm_head_prep(in.q + (size_t)hq * LM_HEAD, in.qn, in.eps, n - 1, in.freq, qh);
    else if (tid / WAVE == 1) lm_head_prep(in.kraw + (size_t)g * LM_HEAD, in.kn, in.eps, n - 1, in.freq, kpos);
    __syncthreads();
    if (c == (n - 1) / LM_CHUNK && lm_first_of_group(hq, g, n_heads, n_kv_heads) && tid < LM_HEAD)
        kc[((size_t)g * max_ctx + n - 1) * LM_HEAD + tid] = kpos[tid];
    const bool valid = p0 + tid < n;
    const bool self = p0 + tid == n - 1;
    double dot = 0.0;
#pragma unroll
    for (int i = 0; i < LM_HEAD / 4; i++) {
        const float4 kv = self ? reinterpret_cast<const float4 *>(kpos)[i] : kr[i];
        dot = fma((double)qh[4 * i], (double)kv.x, dot);
        dot = fma((double)qh[4 * i + 1], (double)kv.y, dot);
        dot = fma((double)qh[4 * i + 2], (double)kv.z, dot);
        dot = fma((double)qh[4 * i + 3], (double)kv.w, dot);
    }
    const float sc = valid ? (float)(dot * scale) : -INFINITY;
    const float m = lm_block_max<NW>(sc, redf);
    const float e = valid ? (float)exp((double)sc - (double)m) : 0.0f;
    ex[tid] = e;
    const double l = block_sum_f64<NW>((double)e, redd);   // contains the barrier ex[] needs
    double o = 0.0;
#pragma unroll
    for (int u = 0; u < VPT; u++) o = fma((double)vv[u], (double)ex[cls + NW * u], o);
    po[cls][d] = o;
    __syncthreads();
    if (tid < LM_HEAD) {
        double t = po[0][tid];
#pragma unroll
        for (int w = 1; w < NW; w++) t = t + po[w][tid];
        double *pp = part + ((size_t)hq * LM_MAX_CHUNKS + c) * LM_PART;
        pp[tid] = t;
        if (tid == 0) {
            pp[LM_HEAD] = (double)m;
            pp[LM_HEAD + 1] = l;
        }
    }
}

__global__ __launch_bounds__(LM_HEAD) void lfm2_attn_join_kernel(const double *__restrict__ part, int nchunks,
                                                                 float *__restrict__ out)
{
    const int hq = blockIdx.x, d = threadIdx.x;
    const double *pp = part + (size_t)hq * LM_MAX_CHUNKS * LM_PART;
    // every chunk's values in flight at once, then the join in chunk order
    double mv[LM_MAX_CHUNKS], lv[LM_MAX_CHUNKS], ov[LM_MAX_CHUNKS];
#pragma unroll
    for (int c = 0; c < LM_MAX_CHUNKS; c++) {
        const int cc = min(c, nchunks - 1);
        mv[c] = pp[cc * LM_PART + LM_HEAD];
        lv[c] = pp[cc * LM_PART + LM_HEAD + 1];
        ov[c] = pp[cc * LM_PART + d];
    }
    double M = -INFINITY;
#pragma unroll
    for (int c = 0; c < LM_MAX_CHUNKS; c++)
        if (c < nchunks) M = fmax(M, mv[c]);
    double L = 0.0, O = 0.0;
#pragma unroll
    for (int c = 0; c < LM_MAX_CHUNKS; c++) {
        if (c >= nchunks) break;
        const double f = exp(mv[c] - M);
        L = L + lv[c] * f;
        O = O + ov[c] * f;
    }
    out[(size_t)hq * LM_HEAD + d] = (float)(O / L);
}

// embeddingLookupQ80 (src/tensor.js:56-77) of column `token` of the repacked
// [H, vocab] table: hidden[i] = q * d (exact in fp32).  One value per thread,
// so the row costs one round trip to memory.
__global__ __launch_bounds__(256) void lfm2_embed_kernel(const int8_t *__restrict__ qs,
                                                        const __half *__restrict__ d, int nb,
                                                        int vocab, int token, int H,
                                                        float *__restrict__ out)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H) return;
    const size_t o = bm_index(0, nb, i / QK, vocab, token);
    out[i] = (float)qs[o * QK + i % QK] * __half2float(d[o]);
}

__global__ __launch_bounds__(256) void lfm2_zero_kernel(float *__restrict__ p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0.0f;
}

// ---------------------------------------------------------------------------

static LmMat lm_mat(const qq_tensor *t) { return LmMat{t->qs, t->dcm, t->out_dim, t->nbp}; }

// One launch of lfm2_mv_kernel; XR, the input values each thread holds, is
// the smaller of two instances (rows of up to 2048 values, or up to
// LM_MAX_IN) whose threads cover the row's nb * 32 values.
template <int MODE, int G, int WPG, int NBW, int RPW>
static void mv_launch(qq_ctx *ctx, int grid, size_t shm, const LmArgs &a)
{
    constexpr int NT = G * WPG * WAVE;
    constexpr int XS = (2048 + NT - 1) / NT, XL = (LM_MAX_IN + NT - 1) / NT;
    if (a.nb * QK <= XS * NT)
        QQ_LAUNCH(ctx, (lfm2_mv_kernel<MODE, G, WPG, NBW, RPW, XS>), dim3(grid), dim3(NT), shm, a);
    else
        QQ_LAUNCH(ctx, (lfm2_mv_kernel<MODE, G, WPG, NBW, RPW, XL>), dim3(grid), dim3(NT), shm, a);
}

int launch_lfm2_mv(qq_ctx *ctx, int mode, const LmLaunch &l)
{
    LmArgs a{};
    a.x = l.x;
    a.in_dim = l.mats[0]->in_dim;
    a.nb = l.mats[0]->nb;
    a.norm = l.norm;
    a.norm_w = l.norm_w;
    a.eps = l.eps;
    for (int i = 0; i < 3; i++)
        if (l.mats[i]) a.m[i] = lm_mat(l.mats[i]);
    a.y = l.y;
    a.state = l.state;
    a.kern = l.kern;
    a.L = l.L;
    a.H = l.H;
    a.q = l.q;
    a.kraw = l.kraw;
    a.kc = l.kc;
    a.vc = l.vc;
    a.qn = l.qn;
    a.kn = l.kn;
    a.n_heads = l.n_heads;
    a.n_kv_heads = l.n_kv_heads;
    a.pos = l.pos;
    a.max_ctx = l.max_ctx;
    a.freq = l.freq;
    if (a.in_dim > LM_MAX_IN) return set_error(ctx, "lfm2: input row of %d > %d", a.in_dim, LM_MAX_IN);
    if (mode == LM_CONV && (a.L < 2 || a.L > LM_MAX_L)) return set_error(ctx, "lfm2: short-conv length %d", a.L);
    // LDS: the activations and the sums of their 16-value halves
    const size_t shm = (size_t)a.nb * QK * 4 + (size_t)a.nb * 2 * 4;
    prof_begin(ctx, K_LFM2_MV);
    // rows per group and waves per row group chosen so that a 2048-row matrix
    // spreads over 256 to 512 workgroups with every block of a row in flight
    // (a 2048-value input row is 64 blocks: one chunk of WPG * SPW * NBW);
    // measured on the LFM2-8B-A1B token against 2 to 32 rows per group and 1
    // to 16 waves
    switch (mode) {
    case LM_PLAIN:   // the output head: 65536 rows
        mv_launch<LM_PLAIN, 1, 16, 4, 32>(ctx, (a.m[0].rows + 31) / 32, shm, a);
        break;
    case LM_RESID:   // 2048 inputs (64 blocks), or the dense FFN's 7168 (224)
        if (a.nb <= 64)
            mv_launch<LM_RESID, 1, 8, 1, 4>(ctx, (a.m[0].rows + 3) / 4, shm, a);
        else
            mv_launch<LM_RESID, 1, 16, 4, 8>(ctx, (a.m[0].rows + 7) / 8, shm, a);
        break;
    case LM_SWIGLU:
        mv_launch<LM_SWIGLU, 2, 8, 4, 16>(ctx, (a.m[0].rows + 15) / 16, shm, a);
        break;
    case LM_CONV:
        mv_launch<LM_CONV, 3, 5, 4, 8>(ctx, (a.H + 7) / 8, shm, a);
        break;
    default:
        mv_launch<LM_QKV, 1, 8, 1, 4>(ctx, (a.n_heads + 2 * a.n_kv_heads) * LM_HEAD / 4, shm, a);
        break;
    }
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

size_t lfm2_attn_work_bytes(int n_heads) { return (size_t)n_heads * LM_MAX_CHUNKS * LM_PART * 8; }

int launch_lfm2_attn(qq_ctx *ctx, const float *q, const float *kraw, const float *qn, const float *kn,
                     const double *freq, double eps, float *kc, const float *vc, int n_heads,
                     int n_kv_heads, int max_ctx, int n, double scale, float *out, double *work)
{
    if (n < 1 || n > LM_MAX_CTX || n > max_ctx) return set_error(ctx, "lfm2: %d positions", n);
    const LmAttnIn in{q, kraw, qn, kn, freq, eps};
    prof_begin(ctx, K_LFM2_ATTN);
    if (n <= LM_CHUNK) {
        QQ_LAUNCH(ctx, lfm2_attn_kernel, dim3(lm_attn_grid(n_heads, n_kv_heads, 1)), dim3(LM_ATTN_THREADS), 0,
                  in, kc, vc, n_heads, n_kv_heads, max_ctx, n, scale, out);
    } else {
        const int nch = (n + LM_CHUNK - 1) / LM_CHUNK;
        QQ_LAUNCH(ctx, lfm2_attn_chunk_kernel, dim3(lm_attn_grid(n_heads, n_kv_heads, nch)),
                  dim3(LM_ATTN_THREADS), 0, in, kc, vc, n_heads, n_kv_heads, max_ctx, n, nch, scale, work);
        QQ_LAUNCH(ctx, lfm2_attn_join_kernel, dim3(n_heads), dim3(LM_HEAD), 0, work, nch, out);
    }
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

int launch_lfm2_embed(qq_ctx *ctx, const qq_tensor *t, int token, float *out)
{
    prof_begin(ctx, K_LFM2_EMBED);
    QQ_LAUNCH(ctx, lfm2_embed_kernel, dim3((t->in_dim + 255) / 256), dim3(256), 0, t->qs, t->d, t->nb,
              t->out_dim, token, t->in_dim, out);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

int launch_lfm2_zero(qq_ctx *ctx, float *p, size_t n)
{
    if (!n) return QQ_OK;
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    QQ_LAUNCH(ctx, lfm2_zero_kernel, dim3(grid), dim3(256), 0, p, n);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
