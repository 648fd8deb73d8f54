// decode.hip -- batch-1 decode of one MoE layer in two launches.
//
// Reference: Lfm2Engine._moEFFN, src/lfm2-engine.js:413-487 (sigmoid + bias
// gating), and Qwen3Engine._moEFFN, src/qwen3-engine.js:304-363 (softmax
// gating), for one token.
//
// Launch 1 (moe_decode_experts): 8 * ceil(E/8) router workgroups + K*NS
// expert-unit workgroups (NS = ceil(F/32)).
//   * router workgroup i (group g = i / 8): binary64 dots of x with router
//     columns 8g .. 8g+7 (one per wave), fp32 logits, published
//     as 64-bit words slot[e] = (epoch << 32) | value.  Sigmoid gating
//     publishes the selection score s_e = fp32(p_e + bias_e) at slot[e] and
//     p_e = fp32 sigmoid (binary64 math) at slot[SYNC_PROB + e]; softmax
//     gating publishes the logit at slot[e] (the softmax needs all of them,
//     so every waiter takes it itself).
//     Workgroups are dealt to the 8 XCDs round robin, so the 8 copies of a
//     group land on the 8 XCDs: each writes the table of its own XCD, which
//     stays in that XCD's L2, and copy 0 also writes SYNC_REPLICAS
//     device-coherent copies of the table.
//   * expert-unit workgroup (k, s): stages x in LDS (and its 3-level int8
//     decomposition), waits in wave 0 (bounded) until all E slots carry this
//     call's epoch -- polling its XCD's table through L2 first, and the
//     device-coherent copy u % SYNC_REPLICAS if that has not filled within
//     DEC_LOCAL_TICKS (so progress never depends on where the dispatcher
//     placed the router workgroups) -- takes the softmax if asked, ranks the
//     experts itself (rank of e = number of experts ordered before it by
//     (score desc, index asc): the order of a stable descending sort;
//     identical in every workgroup), then streams one F-slice of the rank-k
//     expert: gate and up rows f in [32s, 32s+32) (2 x 32 rows x H), SwiGLU,
//     and the matching down block column s (H rows x 32), writing the partial
//     down product partial[k][s][0..H).  Every weight load is issued before
//     any arithmetic; dot products use v_dot4_i32_i8.
//   Value and epoch travel together in one word, so no fence (and no cache
//   write-back or invalidate) is needed on either side, and every expert has
//   its own words, so nothing is contended.  The epoch is a device word that
//   the combine launch of each call advances, so replaying a recorded graph
//   of decode calls draws a fresh epoch every time.
//   Workgroup (0, 0) also writes the routing outputs.
// Launch 2 (moe_decode_combine): y_k = sum_s partial[k][s] in a fixed order,
//   acc = fp32(acc + w_k * y_k) in rank order, hidden += acc.
//
// Nothing waits on another workgroup except on the router slots, and the
// router workgroups have the lowest ids, so they are dispatched first and never
// wait themselves.  The wait is bounded by the wall clock; on expiry the
// workgroup sets the context's error word and returns.
#include "qq_device.h"

namespace qq {

constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * WAVE;
constexpr uint64_t DEC_WAIT_TICKS = 5000000;   // 50 ms at the 100 MHz wall clock
constexpr uint64_t DEC_LOCAL_TICKS = 1000;     // 10 us on the XCD's own table, then the copies
constexpr int RT_EPW = 8;                      // experts per router workgroup (one per wave)
constexpr int RT_COPIES = 8;                   // router workgroups per expert group
static_assert(RT_EPW == DEC_WAVES && RT_EPW * 8 == WAVE, "router lane layout");
static_assert(MAX_E <= 4 * WAVE, "at most four experts per lane");

// XCD (accelerator complex die) this wave runs on.
__device__ __forceinline__ uint32_t xcc_id()
{
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
    return x;
}


struct DecodeArgs {
    const float *x;       // the MoE input, or the residual row when norm
    int norm;             // x = rmsnorm(x) * norm_w is formed in every workgroup
    const float *norm_w;  // NULL: unit weight
    double eps;
    int H, F, E, K;
    int nbH, nbF, NS;
    const float *rf32;
    const int8_t *rq;
    const __half *rd;
    int router_q8;
    int router_vec4;      // F32 router, H % 4 == 0
    int n_router;         // router workgroups: RT_COPIES * ceil(E / RT_EPW)
    int softmax;          // Qwen3-MoE gating: routers publish logits, waiters take the softmax
    const float *bias;
    const int8_t *gq;
    const __half *gd;
    const int8_t *uq;
    const __half *ud;
    const int8_t *dq;
    const __half *dd;
    MaskBits mask;
    const uint32_t *epoch_word;   // this call's epoch is *epoch_word + 1
    // Slot tables, persistent across calls, each [0, E) epoch << 32 | selection
    // score bits (softmax gating: logit bits), [SYNC_PROB, SYNC_PROB + E)
    // epoch << 32 | probability bits (sigmoid gating only):
    //   slots: SYNC_REPLICAS device-coherent copies, SYNC_REPLICA_WORDS apart;
    //   local: one table per XCD (SYNC_LOCAL_WORDS apart), kept in that XCD's L2
    uint64_t *slots;
    uint64_t *local;
    float *partial;       // [K][NS][H]
    int32_t *route_idx;   // [K]
    double *route_w;      // [K]
    int32_t *out_idx;     // optional outputs
    double *out_w;
    float *out_probs;
    uint32_t *err;
};

// Bounded wait until words [0, E) of a slot table carry `epoch` (lane l
// holds words l, l + 64, ...: EPL of them); returns them in v.  Polls the
// XCD's own table (`loc`) while `use_loc` and for DEC_LOCAL_TICKS, then the
// device-coherent copy `glob`; use_loc tells on return which table answered.
// Both are device-scope loads: for a line written from the same XCD one is
// answered by that XCD's L2 in about 0.2 us, against about 1-2 us for a line
// written from another XCD.
template <int EPL>
__device__ __forceinline__ void wait_slots(const uint64_t *loc, const uint64_t *glob, int E,
                                           uint32_t epoch, int lane, int &ok, bool &use_loc,
                                           uint64_t (&v)[EPL])
{
    const uint64_t t0 = wall_clock64();
    while (true) {
        bool all = true;
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const int e = lane + WAVE * j;
            if (e < E)
                v[j] = __hip_atomic_load(use_loc ? &loc[e] : &glob[e], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            else
                v[j] = (uint64_t)epoch << 32;
            all = all && (uint32_t)(v[j] >> 32) == epoch;
        }
        if (__all(all)) break;
        const uint64_t dt = wall_clock64() - t0;
        if (dt > DEC_LOCAL_TICKS) use_loc = false;
        if (dt > DEC_WAIT_TICKS) {
            ok = 0;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// NBW = blocks of H per wave (and 32-row chunks of H per wave) = ceil(ceil(H/32)/8);
// EPL = experts per lane of the waiting waves (1: E <= 64, 2: E <= 128, 4: E <= 256).
template <int NBW, int EPL>
__global__ __launch_bounds__(DEC_THREADS) void moe_decode_experts_kernel(DecodeArgs a)
{
    constexpr int XN = NBW * DEC_WAVES * QK;    // activations, zero padded
    constexpr int NHB = XN / 16;                // 16-value chunks
    __shared__ __align__(16) float xl[XN];
    __shared__ __align__(16) int4 xq1[NHB], xq2[NHB], xq3[NHB];
    __shared__ float xsig[NHB];
    __shared__ __align__(16) float gl[QK];
    __shared__ __align__(16) int4 gq1[2], gq2[2], gq3[2];
    __shared__ float gsig[2];
    __shared__ float redg[DEC_WAVES][QK];
    __shared__ float redu[DEC_WAVES][QK];
    __shared__ double rsum[DEC_WAVES];
    __shared__ int sh_ok;
    __shared__ int rank_part[DEC_WAVES][EPL * WAVE];
    __shared__ int sh_rank_e[MAX_K];
    __shared__ float sh_rank_p[MAX_K];
    __shared__ __align__(16) float sh_score[EPL * WAVE];
    __shared__ float sh_prob[EPL * WAVE];

    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    // advanced by the previous call's combine kernel, so identical in every workgroup
    const uint32_t epoch = a.epoch_word[0] + 1u;

    const bool router = (int)blockIdx.x < a.n_router;
    // router workgroup i: experts 8g .. 8g + 7 of group g = i / RT_COPIES, one a wave
    const int e_r = min((int)(blockIdx.x / RT_COPIES) * RT_EPW + wave, a.E - 1);
    const int H4 = a.H >> 2;
    float4 rw[NBW];
    if (router && a.router_vec4) {
        // issued before x is staged; columns past H meet the zero padding of xl
        const float4 *w4 = reinterpret_cast<const float4 *>(a.rf32) + (size_t)e_r * H4;
#pragma unroll
        for (int i = 0; i < NBW; i++) rw[i] = w4[min(lane + WAVE * i, H4 - 1)];
    }

    // ---- x -> LDS (ffn_norm first when asked: lfm2-engine.js:251-252) ----
    {
        static_assert(DEC_THREADS == NORM_THREADS, "the decode kernel normalises like rmsnorm_kernel");
        constexpr int XPT = (XN + DEC_THREADS - 1) / DEC_THREADS;
        float xv[XPT];
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int k = threadIdx.x + DEC_THREADS * i;
            xv[i] = (k < a.H) ? a.x[k] : 0.0f;
        }
        if (a.norm) {
            float wv[XPT];
#pragma unroll
            for (int i = 0; i < XPT; i++) {
                const int k = threadIdx.x + DEC_THREADS * i;
                wv[i] = (a.norm_w && k < a.H) ? a.norm_w[k] : 1.0f;
            }
            double ss = 0.0;   // padding adds exact zeros
#pragma unroll
            for (int i = 0; i < XPT; i++) ss = fma((double)xv[i], (double)xv[i], ss);
            const double inv = rms_inv(block_sum_f64<DEC_WAVES>(ss, rsum), a.H, a.eps);
#pragma unroll
            for (int i = 0; i < XPT; i++) xv[i] = (float)((double)wv[i] * (double)xv[i] * inv);
        }
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int k = threadIdx.x + DEC_THREADS * i;
            if (k < XN) xl[k] = xv[i];
        }
    }
    __syncthreads();

    if (router) {
        // ---- router workgroup: logits, then sigmoid and scores or softmax
        // logits (lfm2-engine.js:418-431; qwen3-engine.js:306-307) ----
        // Workgroup i runs on XCD i % 8 (the dispatcher deals workgroups to the
        // XCDs round robin), so each XCD gets a full set of router workgroups
        // and its table fills from its own L2.  Nothing depends on that for
        // correctness: copy 0 of each group also fills the device-coherent
        // tables, which waiters fall back to.
        double acc = 0.0;
        if (a.router_vec4) {
            // four independent chains (one per float4 component), then joined
            const float4 *x4 = reinterpret_cast<const float4 *>(xl);
            double ax = 0.0, ay = 0.0, az = 0.0, aw = 0.0;
#pragma unroll
            for (int i = 0; i < NBW; i++) {
                const float4 xv = x4[lane + WAVE * i];
                ax = fma((double)xv.x, (double)rw[i].x, ax);
                ay = fma((double)xv.y, (double)rw[i].y, ay);
                az = fma((double)xv.z, (double)rw[i].z, az);
                aw = fma((double)xv.w, (double)rw[i].w, aw);
            }
            acc = (ax + ay) + (az + aw);
        } else {
            for (int k = lane; k < a.H; k += WAVE) {
                double wv;
                if (a.router_q8) {
                    const size_t o = bm_index(0, a.nbH, k >> 5, a.E, e_r);
                    wv = (double)a.rq[o * QK + (k & 31)] * (double)__half2float(a.rd[o]);
                } else {
                    wv = (double)a.rf32[(size_t)e_r * a.H + k];
                }
                acc = fma((double)xl[k], wv, acc);
            }
        }
        acc = wave_sum_dpp(acc);
        if (lane == 0) rsum[wave] = acc;
        __syncthreads();
        if (wave == 0) {
            // lane = 8 q + r: expert 8g + q; copies r and r + 8 of the device table
            const int q = lane >> 3, r = lane & 7;
            const int e = (blockIdx.x / RT_COPIES) * RT_EPW + q;
            if (e < a.E) {
                const float logit = (float)rsum[q];
                // sigmoid gating: probability and selection score; softmax
                // gating: the logit (the softmax needs all of them and is taken
                // by every waiter)
                float p = 0.0f, sc = logit;
                if (!a.softmax) {
                    p = (float)(1.0 / (1.0 + exp(-(double)logit)));
                    sc = p + a.bias[e];
                }
                const uint64_t ep = (uint64_t)epoch << 32;
                uint64_t *ltab = a.local + (size_t)xcc_id() * SYNC_LOCAL_WORDS;
                if (r == 0) {
                    if (!a.softmax)
                        __hip_atomic_store(&ltab[SYNC_PROB + e], ep | __float_as_uint(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    __hip_atomic_store(&ltab[e], ep | __float_as_uint(sc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
                if (blockIdx.x % RT_COPIES == 0) {
#pragma unroll
                    for (int c = r; c < SYNC_REPLICAS; c += 8) {
                        uint64_t *tab = a.slots + (size_t)c * SYNC_REPLICA_WORDS;
                        if (!a.softmax)
                            __hip_atomic_store(&tab[SYNC_PROB + e], ep | __float_as_uint(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(&tab[e], ep | __float_as_uint(sc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
        return;
    }

    const int unit = blockIdx.x - a.n_router;
    const uint64_t *tab = a.slots + (size_t)(unit % SYNC_REPLICAS) * SYNC_REPLICA_WORDS;
    const uint64_t *loc = a.local + (size_t)xcc_id() * SYNC_LOCAL_WORDS;
    const int kslot = unit / a.NS;
    const int s = unit - kslot * a.NS;

    // ---- x -> three int8 levels, four lanes per 16-value chunk ----
    // (whole waves take part: 4 * NHB is a multiple of 64)
    for (int t = threadIdx.x; t < 4 * NHB; t += DEC_THREADS) {
        const float4 v = reinterpret_cast<const float4 *>(xl)[t];   // x[4t .. 4t+3]
        float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        m = fmaxf(m, __shfl_xor(m, 1, WAVE));
        m = fmaxf(m, __shfl_xor(m, 2, WAVE));
        const float inv = (m > 0.0f) ? 127.0f / m : 0.0f;
        uint32_t p1, p2, p3;
        decompose4(v, inv, p1, p2, p3);
        reinterpret_cast<uint32_t *>(xq1)[t] = p1;
        reinterpret_cast<uint32_t *>(xq2)[t] = p2;
        reinterpret_cast<uint32_t *>(xq3)[t] = p3;
        if ((t & 3) == 0) xsig[t >> 2] = m * (1.0f / 127.0f);
    }

    // ---- routing (lfm2-engine.js:433-447; qwen3-engine.js:306-321) ----
    bool use_loc = true;
    if (wave == 0) {
        int ok = 1;
        uint64_t v[EPL];
        wait_slots<EPL>(loc, tab, a.E, epoch, lane, ok, use_loc, v);
        if (a.softmax) {
            // every workgroup takes the same softmax of the same logits
            float lg[EPL], pr[EPL];
#pragma unroll
            for (int j = 0; j < EPL; j++) lg[j] = __uint_as_float((uint32_t)v[j]);
            softmax_probs<EPL>(lg, a.E, pr);
#pragma unroll
            for (int j = 0; j < EPL; j++) {
                const int e = lane + WAVE * j;
                sh_score[e] = (e < a.E) ? pr[j] : -INFINITY;
                sh_prob[e] = pr[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < EPL; j++) {
                const int e = lane + WAVE * j;
                sh_score[e] = (e < a.E) ? __uint_as_float((uint32_t)v[j]) : -INFINITY;
            }
        }
        if (lane == 0) {
            sh_ok = ok;
            if (!ok) atomicOr(a.err, 1u);
        }
    }
    __syncthreads();
    if (!sh_ok) return;
    // rank of expert e = lane + 64j: experts ordered before it by (score
    // desc, index asc), so the rank-k expert is the k-th element of a stable
    // descending sort.  Wave w counts over slots 8*EPL*w .. 8*EPL*(w+1) - 1
    // (slots >= E hold -inf and never rank before a real expert); every wave
    // then sums the counts.
    {
        constexpr int NQ = 2 * EPL;   // float4 reads of the wave's 8*EPL slots
        float qq[4 * NQ];
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const float4 q4 = reinterpret_cast<const float4 *>(sh_score)[NQ * wave + u];
            qq[4 * u] = q4.x;
            qq[4 * u + 1] = q4.y;
            qq[4 * u + 2] = q4.z;
            qq[4 * u + 3] = q4.w;
        }
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const int e = lane + WAVE * j;
            const float sc = sh_score[e];
            int part = 0;
#pragma unroll
            for (int u = 0; u < 4 * NQ; u++) {
                const int i = 4 * NQ * wave + u;
                part += (int)(qq[u] > sc) | ((int)(qq[u] == sc) & (int)(i < e));
            }
            rank_part[wave][e] = part;
        }
    }
    __syncthreads();
    int rank[EPL];
    int e = -1;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        rank[j] = 0;
#pragma unroll
        for (int w = 0; w < DEC_WAVES; w++) rank[j] += rank_part[w][lane + WAVE * j];
        if (lane + WAVE * j >= a.E) rank[j] = INT_MAX;
        const uint64_t hit = __ballot(rank[j] == kslot);   // the same in every wave
        if (hit) e = WAVE * j + (int)__builtin_ctzll(hit);
    }
    if (e < 0) return;
    if (unit == 0 && wave == 0) {
        // probabilities (telemetry) and normalised weights (lfm2-engine.js:444-457;
        // qwen3-engine.js:317-329: the sum starts at 0 and a zero sum gives zero weights)
        float p[EPL];
        if (a.softmax) {
#pragma unroll
            for (int j = 0; j < EPL; j++) p[j] = sh_prob[lane + WAVE * j];
        } else {
            int okp = 1;
            uint64_t pv[EPL];
            wait_slots<EPL>(loc + SYNC_PROB, tab + SYNC_PROB, a.E, epoch, lane, okp, use_loc, pv);
            if (!okp && lane == 0) atomicOr(a.err, 2u);
#pragma unroll
            for (int j = 0; j < EPL; j++) p[j] = __uint_as_float((uint32_t)pv[j]);
        }
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const int ee = lane + WAVE * j;
            if (a.out_probs && ee < a.E) a.out_probs[ee] = p[j];
            if (rank[j] < a.K) {
                sh_rank_e[rank[j]] = ee;
                sh_rank_p[rank[j]] = p[j];
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) {
            double sumW = a.softmax ? 0.0 : 1e-6;
            for (int k = 0; k < a.K; k++) sumW = sumW + (double)sh_rank_p[k];
            const double inv = a.softmax ? (sumW > 0.0 ? 1.0 / sumW : 0.0) : 1.0 / sumW;
            for (int k = 0; k < a.K; k++) {
                const double wk = (double)sh_rank_p[k] * inv;
                a.route_idx[k] = sh_rank_e[k];
                a.route_w[k] = wk;
                if (a.out_idx) a.out_idx[k] = sh_rank_e[k];
                if (a.out_w) a.out_w[k] = wk;
            }
        }
    }
    if (mask_has(a.mask, e)) return;   // the combine skips masked ranks

    const int h = lane & 1;
    const int f = s * QK + lane / 2;
    const bool f_ok = f < a.F;

    // ---- issue every weight load of this workgroup ----
    // All addresses are clamped in bounds so every load is unconditional and
    // the compiler issues them back to back; out-of-range rows / blocks get a
    // zero scale afterwards.  One 64-bit base per tensor, uniform strides.
    int4 gq[NBW], uq[NBW], dq[NBW];
    __half gdh[NBW], udh[NBW], ddh[NBW];
    {
        const int fc = min(f, a.F - 1);
        const int ilast = (a.nbH - 1 - wave) >= 0 ? (a.nbH - 1 - wave) / DEC_WAVES : 0;
        const size_t row0 = ((size_t)e * a.nbH + min(wave, a.nbH - 1)) * a.F + fc;
        const size_t rstride = (size_t)DEC_WAVES * a.F;
        const int8_t *gp = a.gq + row0 * QK + 16 * h;
        const int8_t *up = a.uq + row0 * QK + 16 * h;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            const size_t o = (size_t)min(i, ilast) * rstride;
            gq[i] = *reinterpret_cast<const int4 *>(gp + o * QK);
            uq[i] = *reinterpret_cast<const int4 *>(up + o * QK);
            gdh[i] = a.gd[row0 + o];
            udh[i] = a.ud[row0 + o];
        }
        // down rows j = (wave + 8i)*32 + lane/2 of block column s
        const size_t dsbase = ((size_t)e * a.nbF + s) * a.H;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            const int j = min((wave + DEC_WAVES * i) * QK + lane / 2, a.H - 1);
            dq[i] = *reinterpret_cast<const int4 *>(a.dq + (dsbase + j) * QK + 16 * h);
            ddh[i] = a.dd[dsbase + j];
        }
    }
    // every load above is issued before any of the work below
    __builtin_amdgcn_sched_barrier(0);

    // ---- gate / up rows, SwiGLU (tensor.js:167-178) ----
    float ga = 0.0f, ua = 0.0f;
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        // blocks past nbH: zero scale and zero activations (x is padded)
        const int b = wave + DEC_WAVES * i;
        const int c = 2 * b + h;
        const bool bok = f_ok && b < a.nbH;
        const float sg = bok ? __half2float(gdh[i]) : 0.0f;
        const float su = bok ? __half2float(udh[i]) : 0.0f;
        const int4 l1 = xq1[c], l2 = xq2[c], l3 = xq3[c];
        const float sig = xsig[c];
        ga = fmaf(dot16_lev3(gq[i], l1, l2, l3, sig), sg, ga);
        ua = fmaf(dot16_lev3(uq[i], l1, l2, l3, sig), su, ua);
    }
    ga += __shfl_xor(ga, 1, WAVE);
    ua += __shfl_xor(ua, 1, WAVE);
    if (h == 0) {
        redg[wave][lane / 2] = ga;
        redu[wave][lane / 2] = ua;
    }
    __syncthreads();
    if (threadIdx.x < QK) {
        const int r = threadIdx.x;
        float G = redg[0][r], U = redu[0][r];
#pragma unroll
        for (int w = 1; w < DEC_WAVES; w++) {
            G += redg[w][r];
            U += redu[w][r];
        }
        float gv = 0.0f;
        if (s * QK + r < a.F) {
            const double g64 = (double)G;
            const float sg = (float)(g64 * (1.0 / (1.0 + exp(-g64))));
            gv = sg * U;
        }
        gl[r] = gv;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        Lev3 L;
        decompose16(&gl[16 * threadIdx.x], L);
        gq1[threadIdx.x] = L.l1;
        gq2[threadIdx.x] = L.l2;
        gq3[threadIdx.x] = L.l3;
        gsig[threadIdx.x] = L.sig;
    }
    __syncthreads();

    // ---- partial down product over this slice ----
    float *part = a.partial + ((size_t)kslot * a.NS + s) * a.H;
    const int4 m1 = gq1[h], m2 = gq2[h], m3 = gq3[h];
    const float msig = gsig[h];
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const int j = (wave + DEC_WAVES * i) * QK + lane / 2;
        const float sdd = (j < a.H) ? __half2float(ddh[i]) : 0.0f;
        float y = dot16_lev3(dq[i], m1, m2, m3, msig) * sdd;
        y += __shfl_xor(y, 1, WAVE);
        if (h == 0 && j < a.H) part[j] = y;
    }
}

// 256 threads per CW outputs: thread (group q, output jl) sums the slices
// s = q, q + NG, ... (NSP of them, NG = 256 / CW groups) of up to 4 ranks,
// with all its loads in flight at once; the NG groups are then summed in a
// fixed order.
template <int CW, int NSP>
__global__ __launch_bounds__(256) void moe_decode_combine_kernel(
    const float *__restrict__ partial, int H, int NS, int K, const int32_t *__restrict__ route_idx,
    const double *__restrict__ route_w, MaskBits mask, float *__restrict__ hidden,
    uint32_t *__restrict__ epoch_word)
{
    constexpr int NG = 256 / CW;
    // the experts kernel of this call has finished: the next call takes a new epoch
    if (blockIdx.x == 0 && threadIdx.x == 0) epoch_word[0] = epoch_word[0] + 1u;
    __shared__ float red[MAX_K][NG][CW];
    __shared__ int sh_e[MAX_K];
    __shared__ double sh_w[MAX_K];
    const int jl = threadIdx.x % CW;
    const int q = threadIdx.x / CW;
    const int j = blockIdx.x * CW + jl;
    const int jc = min(j, H - 1);
    // the routing and the residual row are loaded with the partial sums, in
    // the same round trip
    const int tid = threadIdx.x;
    if (tid >= CW && tid < CW + K) {
        sh_e[tid - CW] = route_idx[tid - CW];
        sh_w[tid - CW] = route_w[tid - CW];
    }
    const float h_in = hidden[jc];
    for (int k0 = 0; k0 < K; k0 += 4) {
        float v[4][NSP];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int k = min(k0 + kk, K - 1);
#pragma unroll
            for (int i = 0; i < NSP; i++) {
                const int s = min(q + NG * i, NS - 1);
                v[kk][i] = partial[((size_t)k * NS + s) * H + jc];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            float y = 0.0f;
#pragma unroll
            for (int i = 0; i < NSP; i++)
                if (q + NG * i < NS) y += v[kk][i];
            if (k0 + kk < K) red[k0 + kk][q][jl] = y;
        }
    }
    __syncthreads();
    if (threadIdx.x < CW && j < H) {
        float acc = 0.0f;
        for (int k = 0; k < K; k++) {
            const int e = sh_e[k];
            if ((unsigned)e >= (unsigned)MAX_E || mask_has(mask, e)) continue;
            float y = red[k][0][jl];
#pragma unroll
            for (int p = 1; p < NG; p++) y += red[k][p][jl];
            acc = (float)((double)acc + sh_w[k] * (double)y);
        }
        hidden[j] = h_in + acc;
    }
}

bool decode_supported(const qq_moe *m, int T)
{
    return T == 1 && m->E <= MAX_E && m->K <= m->E && m->H <= 8 * DEC_WAVES * QK;
}

size_t decode_work_bytes(const qq_moe *m)
{
    const int NS = (m->F + QK - 1) / QK;
    return (size_t)m->K * NS * m->H * 4 + 256 + 256 + (size_t)m->K * 4 + 256;
}

template <int NBW, int EPL>
static void launch_experts(qq_ctx *ctx, const DecodeArgs &a, dim3 grid)
{
    QQ_LAUNCH(ctx, (moe_decode_experts_kernel<NBW, EPL>), grid, dim3(DEC_THREADS), 0, a);
}

template <int EPL>
static void launch_experts_nbw(qq_ctx *ctx, const DecodeArgs &a, dim3 grid, int nbw)
{
    if (nbw <= 1) launch_experts<1, EPL>(ctx, a, grid);
    else if (nbw <= 2) launch_experts<2, EPL>(ctx, a, grid);
    else if (nbw <= 4) launch_experts<4, EPL>(ctx, a, grid);
    else launch_experts<8, EPL>(ctx, a, grid);
}

int launch_moe_decode(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden,
                      const MaskBits &mask, int32_t *out_idx, double *out_w, float *out_probs,
                      char *work, const NormArgs *norm)
{
    DecodeArgs a;
    a.x = x;
    a.norm = norm != nullptr;
    a.norm_w = norm ? norm->w : nullptr;
    a.eps = norm ? norm->eps : 0.0;
    a.H = m->H;
    a.F = m->F;
    a.E = m->E;
    a.K = m->K;
    a.nbH = (m->H + QK - 1) / QK;
    a.nbF = (m->F + QK - 1) / QK;
    a.NS = a.nbF;
    a.router_q8 = m->router_type == QQ_TYPE_Q8_0;
    a.rf32 = m->router_f32;
    a.rq = a.router_q8 ? m->router_q8->qs : nullptr;
    a.rd = a.router_q8 ? m->router_q8->d : nullptr;
    a.bias = m->bias;
    a.gq = m->gate->qs;
    a.gd = m->gate->d;
    a.uq = m->up->qs;
    a.ud = m->up->d;
    a.dq = m->down->qs;
    a.dd = m->down->d;
    a.mask = mask;
    a.slots = ctx->sync_slots;
    a.local = ctx->sync_local;
    a.router_vec4 = !a.router_q8 && (m->H & 3) == 0;
    a.softmax = m->gating == QQ_GATING_SOFTMAX;
    const int epl = m->E <= WAVE ? 1 : m->E <= 2 * WAVE ? 2 : 4;
    a.n_router = RT_COPIES * ((m->E + RT_EPW - 1) / RT_EPW);
    a.epoch_word = ctx->sync_epoch;
    a.err = ctx->sync_err;
    const size_t part_b = ((size_t)m->K * a.NS * m->H * 4 + 255) & ~(size_t)255;
    a.partial = reinterpret_cast<float *>(work);
    a.route_w = reinterpret_cast<double *>(work + part_b);
    a.route_idx = reinterpret_cast<int32_t *>(reinterpret_cast<char *>(a.route_w) + 256);
    a.out_idx = out_idx;
    a.out_w = out_w;
    a.out_probs = out_probs;

    const int nbw = (a.nbH + DEC_WAVES - 1) / DEC_WAVES;
    const dim3 grid(a.n_router + m->K * a.NS);
    prof_begin(ctx, K_DECODE_EXPERTS);
    if (epl == 1) launch_experts_nbw<1>(ctx, a, grid, nbw);
    else if (epl == 2) launch_experts_nbw<2>(ctx, a, grid, nbw);
    else launch_experts_nbw<4>(ctx, a, grid, nbw);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());

    // 32 outputs per workgroup (16 or 8, with more workgroups, measured slower)
    constexpr int CW = 32, NG = 256 / CW;
    const int nsp = (a.NS + NG - 1) / NG;
    const dim3 cgrid((m->H + CW - 1) / CW);
#define QQ_CB(N)                                                                                 \
    QQ_LAUNCH(ctx, (moe_decode_combine_kernel<CW, N>), cgrid, dim3(256), 0, a.partial, \
                       m->H, a.NS, m->K, a.route_idx, a.route_w, mask, hidden, ctx->sync_epoch)
    prof_begin(ctx, K_DECODE_COMBINE);
    if (nsp <= 1) QQ_CB(1);
    else if (nsp <= 2) QQ_CB(2);
    else if (nsp <= 4) QQ_CB(4);
    else if (nsp <= 8) QQ_CB(8);
    else if (nsp <= 16) QQ_CB(16);
    else QQ_CB(32);
    prof_end(ctx);
#undef QQ_CB
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
