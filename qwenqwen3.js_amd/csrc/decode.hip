// decode.hip -- batch-1 decode of one MoE layer in one launch.
//
// Reference: Lfm2Engine._moEFFN, src/lfm2-engine.js:413-487 (sigmoid + bias
// gating), and Qwen3Engine._moEFFN, src/qwen3-engine.js:304-363 (softmax
// gating), for one token.
//
// The grid is G workgroups of 512 threads, one per CU (G = 256 on MI355X),
// dealt by the dispatcher to the 8 XCDs round robin: workgroup j belongs to
// group x = j % 8 (its XCD) as member i = j / 8 of M = G / 8.  Each group
// runs the whole layer for its own eighth of the F features:
//
//  1. Routing.  Member i forms the binary64 router dots of experts i, i + M,
//     ... with x (forming x = rmsnorm(hidden) first when asked) and publishes
//     the fp32 logits in its group's table (with more experts than members,
//     E > M: workgroup j forms expert j's logit alone and publishes it to the
//     device-coherent tables, so the router is read once, not once per
//     group); every workgroup waits for the E logits of its own table (or of
//     the device-coherent one), takes the sigmoid + bias (or softmax) scores
//     and ranks the experts itself (stable descending order, ties to the
//     lower index), so every workgroup holds the same idx[K], p[K], w[K].
//  2. Gate/up.  Group x owns F blocks [x nbF / 8, (x + 1) nbF / 8) of all K
//     selected experts; its (rank, feature) columns are split evenly over the
//     members (28 each at H=2048, F=1792, K=4).  A member issues every weight
//     load of its share at once -- its gate and up columns and the down rows
//     it needs in step 3 -- takes v_dot4 products of the int8 weights against
//     a 3-level int8 split of x, SwiGLU, and publishes its h values.
//  3. Down.  Every member waits for its group's h values (K x F/8), then
//     forms the partial down products of its M-th of the H rows over the
//     group's F blocks from the down weights already in its registers, and
//     publishes them.
//  4. Combine.  Workgroup j finishes rows [j H/G, (j+1) H/G): y_k = sum of the
//     8 groups' partials in group order, acc = fp32(acc + w_k y_k) in rank
//     order, hidden += acc.
//
// Every exchange is a table of 64-bit words (tag << 32) | value bits, written
// once per call, so a reader knows a word is this call's from the word
// itself: no fences, no cache write-back or invalidation.  The routing and h
// tables of a group are written with workgroup-scope stores, which stay in
// that XCD's L2, and read with device-scope loads that the L2 answers in about
// 0.2 us; every word also goes to a device-coherent copy, which a reader falls
// back to after DEC_LOCAL_TICKS (so progress never depends on where the
// dispatcher put a workgroup).  Partials go to device-coherent words only.
//
// The tag of a call is the device epoch word + 1.  Every workgroup reads the
// epoch first thing and publishes an arrival word once it has read the epoch,
// x and hidden.  Workgroup 0 advances the epoch after its final wait, which
// covers all G arrival words, so every workgroup has read the old epoch by
// then.  A replayed graph of decode launches so draws a fresh tag every time.
//
// A workgroup writes its hidden rows only after all G arrival words carry the
// tag, so hidden may be the input row itself (the fused ffn_norm).
//
// All G workgroups must be resident at once (one per CU; nothing else on the
// device keeps a CU busy for long).  Every wait is bounded by the wall clock;
// on expiry the workgroup sets the context's error word and skips the rest.
#include "qq_device.h"

namespace qq {

constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * WAVE;
constexpr int DEC_GROUPS = 8;                  // one per XCD
static_assert(DEC_GROUPS == 8, "group blocks are found with shifts by 3");
constexpr uint64_t DEC_LOCAL_TICKS = 1000;     // 10 us on the group's own table, then the copy
constexpr int DEC_CCH = 32;                    // gate/up columns per chunk (two lanes each)
constexpr int DEC_DCH = 8;                     // down loads per lane
static_assert(DEC_THREADS == NORM_THREADS, "the decode kernel normalises like rmsnorm_kernel");

struct DecodeArgs {
    const float *x;       // the MoE input, or the residual row when norm
    int norm;             // x = rmsnorm(x) * norm_w is formed in every workgroup
    double eps;
    float *hidden;
    int H, F, E, K;
    int nbH, nbF;
    int router_q8;
    int xr;               // router logits across the grid: workgroup j forms expert j's
                          // (E > 32, one layer); else member i of each group forms
                          // experts i, i + M, ... for its group
    int softmax;          // Qwen3-MoE gating
    int nbpH;
    int L;                // layers of a stack launch (1 otherwise)
    DecodeLayer one;      // the layer of a single-layer launch
    const DecodeLayer *layers;   // [L]: the layers of a stack launch
    MaskBits mask;
    uint32_t *epoch_word;
    // exchange tables (tag << 32 | bits):
    uint64_t *rloc;       // per group: router logits [SYNC_LOCAL_WORDS apart]
    uint64_t *rdev;       // SYNC_REPLICAS device-coherent copies of group 0's
    uint64_t *hloc;       // h values [K][F] (each group writes its own features)
    uint64_t *hdev;       // device-coherent copy
    uint64_t *part;       // partial down sums [8][K][H], device-coherent
    uint64_t *arrive;     // [G]
    uint64_t *hxl;        // stack: each group's residual row after layer l, table l % 2
    uint64_t *hxd;        //   [2][8][SYNC_X_WORDS]: group-local and device-coherent copies
    int32_t *out_idx;     // optional outputs (a stack's: layer l at l K, l K, l E)
    double *out_w;
    float *out_probs;
    float *out_rec;       // [K idx as float | K w rounded to fp32 | E probs]
    uint32_t *err;
    uint64_t wait_ticks;  // bound on every device-side wait (100 MHz wall clock)
};

// A pointer read from memory (a stack's layer table) has no known address
// space: loads through it compile to flat loads, which also count in lgkmcnt,
// so every LDS barrier would wait for the whole weight stream.  Typed as a
// global-memory pointer at the table, loads through it are global loads.
#if defined(__HIP_DEVICE_COMPILE__)
template <typename T>
using gptr = T __attribute__((address_space(1))) *;
#else
template <typename T>
using gptr = T *;
#endif
template <typename T>
__device__ __forceinline__ gptr<T> as_global(T *p)
{
    return (gptr<T>)p;
}

__device__ __forceinline__ uint64_t tag_word(uint32_t tag, float v)
{
    return ((uint64_t)tag << 32) | __float_as_uint(v);
}

__device__ __forceinline__ void store_local(uint64_t *p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void store_dev(uint64_t *p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait of the first NT threads for their words: thread t polls the
// words of its items s < IPT with want[s] for tag[s] (loads issued together, each wave
// on its own with wave votes), at pl[s] -- its group's table -- and after
// DEC_LOCAL_TICKS at pd[s], the device-coherent copy (pd[s] = pl[s] when
// there is none).  Once a word carries `tag` its low half goes to *dst[s]
// (LDS; NULL: not kept).  The item addresses are worked out by the caller
// once, so a poll round is only loads and compares.  The other waves go
// straight to the closing barrier.  (Stores count in the same in-order
// counter as loads here, so a wave that has just written device-scope words
// would wait for their acknowledgement before every poll: the waves that
// publish are kept out of the waits that follow.)  Returns false (in every
// thread) when some wave's wait expired, or -- once a wait has run past
// DEC_LOCAL_TICKS -- when the error word says another workgroup gave up (its
// words will not come, so the failure spreads in ~10 us instead of a bound).
template <int NT, int IPT>
__device__ __forceinline__ bool block_wait(const uint32_t (&tag)[IPT], int *sh_fail, const uint64_t *(&pl)[IPT],
                                           const uint64_t *(&pd)[IPT], bool (&want)[IPT],
                                           float *(&dst)[IPT], uint64_t wait_ticks, const uint32_t *err)
{
    bool fail = false;
    if ((int)threadIdx.x < NT) {
        const uint64_t t0 = wall_clock64();
        bool loc = true;
        while (true) {
            uint64_t v[IPT];
#pragma unroll
            for (int s = 0; s < IPT; s++)
                v[s] = want[s] ? __hip_atomic_load(loc ? pl[s] : pd[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : 0;
            bool mine = true;
#pragma unroll
            for (int s = 0; s < IPT; s++) {
                if (!want[s]) continue;
                if ((uint32_t)(v[s] >> 32) == tag[s]) {
                    want[s] = false;
                    if (dst[s]) *dst[s] = __uint_as_float((uint32_t)v[s]);
                } else {
                    mine = false;
                }
            }
            if (__all(mine)) break;
            const uint64_t dt = wall_clock64() - t0;
            if (dt >= wait_ticks ||
                (dt > DEC_LOCAL_TICKS && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
                fail = true;
                break;
            }
            if (dt > DEC_LOCAL_TICKS) loc = false;
            __builtin_amdgcn_s_sleep(1);
        }
    }
    if (fail) *sh_fail = 1;
    lds_barrier();
    return *sh_fail == 0;
}

// 32-value blocks of the LDS row v[0, 32 nblk) -> three int8 levels (row l of
// lev, LS bytes apart, holds level l at the values' positions) and the block
// scale, eight lanes a block (lane 8b + q takes values 32b + 4q .. 32b + 4q + 3).
template <int LS>
__device__ __forceinline__ void decompose32(const float *v, int nblk, int8_t *lev, float *sig)
{
    for (int t = threadIdx.x; t < 8 * nblk; t += DEC_THREADS) {
        const float4 f = reinterpret_cast<const float4 *>(v)[t];
        float m = fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w)));
        m = fmaxf(m, xor1_dpp(m));
        m = fmaxf(m, xor2_dpp(m));
        m = fmaxf(m, __shfl_xor(m, 4));
        const float inv = (m > 0.0f) ? 127.0f / m : 0.0f;
        uint32_t p1, p2, p3;
        decompose4(f, inv, p1, p2, p3);
        reinterpret_cast<uint32_t *>(lev)[t] = p1;
        reinterpret_cast<uint32_t *>(lev + LS)[t] = p2;
        reinterpret_cast<uint32_t *>(lev + 2 * LS)[t] = p3;
        if ((t & 7) == 0) sig[t >> 3] = m * (1.0f / 127.0f);
    }
}

typedef int mf_v4i __attribute__((ext_vector_type(4)));
typedef int mf_v16i __attribute__((ext_vector_type(16)));

// One 32 x 32 x 32 int8 product on the matrix cores, C[m][n] = sum_k A[m][k]
// B[k][n]: lane l holds 16 bytes of row l % 32 of A and the same 16 k of
// column l % 32 of B (any split of k that A and B share gives the same sum);
// C[m][n] comes back in lane n + 32 ((m / 4) % 2), element 4 (m / 8) + m % 4.
__device__ __forceinline__ mf_v16i mfma_i8(const int4 a, const int4 b)
{
    const mf_v4i av = {a.x, a.y, a.z, a.w};
    const mf_v4i bv = {b.x, b.y, b.z, b.w};
    const mf_v16i z = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, z, 0, 0, 0);
}

// The three levels' sums in rows 0..2 of C (lanes 0..31): c0 + c1/254 + c2/254^2.
__device__ __forceinline__ float lev3_sum(const mf_v16i c)
{
    return fmaf(fmaf((float)c[2], 1.0f / 254.0f, (float)c[1]), 1.0f / 254.0f, (float)c[0]);
}

// 16 weight bytes read once per call: a non-temporal load, so the stream of
// expert weights does not push the exchange tables and activations out of L2.
__device__ __forceinline__ int4 load_stream16(gptr<const int8_t> p)
{
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i v = __builtin_nontemporal_load((gptr<const v4i>)p);
    return make_int4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float f16_bits(uint32_t b) { return __half2float(__ushort_as_half((uint16_t)b)); }

// q / d for 0 <= q < 2^20 and 1 <= d < 2^12 without an integer division:
// the float product is within 2^-9 of the quotient, which is never that close
// to the next integer.
__device__ __forceinline__ int div_small(int q, float inv_d) { return (int)(((float)q + 0.5f) * inv_d); }

// The NBW consecutive fp16 scales at p (2 NBW bytes, aligned to that size)
// in one load: element i is (s[i / 2] >> 16 (i % 2)) & 0xffff.
template <int NBW>
struct ScaleRun {
    uint32_t s[(NBW + 1) / 2];
    __device__ __forceinline__ void load(gptr<const __half> p)
    {
        if constexpr (NBW == 8) {
            const uint4 v = *(gptr<const uint4>)p;
            s[0] = v.x; s[1] = v.y; s[2] = v.z; s[3] = v.w;
        } else if constexpr (NBW == 4) {
            const uint2 v = *(gptr<const uint2>)p;
            s[0] = v.x; s[1] = v.y;
        } else if constexpr (NBW == 2) {
            s[0] = *(gptr<const uint32_t>)p;
        } else {
            s[0] = *(gptr<const uint16_t>)p;
        }
    }
    __device__ __forceinline__ float get(int i) const { return f16_bits(s[i / 2] >> (16 * (i % 2))); }
};

// Limits of one launch (checked by decode_supported on the host).
constexpr int DEC_MAX_HW = 2048;               // h values of one group (K x F-range)
constexpr int DEC_MAX_FIN = 3 * DEC_THREADS;   // partial + arrival words read by one workgroup
constexpr int DEC_MAX_FIN_STACK = 5 * DEC_THREADS;   // ... by one member of a stack launch

// NBW = blocks of H per wave = ceil(ceil(H/32)/8) in {1, 2, 4, 8}; RE = router
// experts per member (>= ceil(E/M); 1 with xr, one expert per workgroup);
// EPL = experts per lane (>= ceil(E/64));
// PP2: a wave takes two (rank, row half) pairs of down rows (K x halves > 8);
// STACK: the launch runs a.L layers (ffn_norm folded in) on one residual row.
//
// Stack launches.  Layer l uses tag epoch + 1 + l.  The combine is done by
// every group for all H rows: member i of each group waits for the 8 groups'
// partials of its rows [i RM, (i + 1) RM), adds them up and publishes its rows
// of the new residual in its group's table (group-local, with a device-
// coherent copy); layer l + 1 starts with every member gathering its group's
// H rows.  So the only device-wide exchange of a layer is the partials; the
// residual row passes between layers inside each XCD.  Only group 0 writes
// hidden, at the last layer, once the arrival words of the first layer (every
// workgroup has read the input row) are in.
// Groups are coupled only through the partials, so one group can run up to a
// layer ahead of another: the partials and the device copies of the routing
// logits (the tables other groups read) alternate between two halves by layer
// parity.  A member publishes layer l + 2 words there only after its group
// has gathered the layer l + 1 residual, which every member of every group
// publishes only after it has read all of its layer-l words.  Group-local
// tables are reused each layer (a member writes layer l + 1 words only after
// every member of its group has published its layer-l residual rows, and so
// has finished layer l); the residual tables alternate by parity as well.
// The next layer's router rows, bias and norm weights are loaded while the
// current layer's partials are exchanged.
template <int NBW, int RE, int EPL, bool PP2, bool STACK>
__global__ __launch_bounds__(DEC_THREADS) void moe_decode_kernel(DecodeArgs a)
{
    constexpr int XN = NBW * DEC_WAVES * QK;    // activations, zero padded
    constexpr int XPT = (XN + DEC_THREADS - 1) / DEC_THREADS;
    __shared__ __align__(16) float xl[XN];
    // x and h in three int8 levels (rows 0..2) and a row of zeros (row 3):
    // lane l of an MFMA reads row min(l % 32, 3)
    __shared__ __align__(16) int8_t xlev[4][XN];
    __shared__ float xsig[XN / QK];
    __shared__ double rsum[RE][DEC_WAVES];
    __shared__ double nsum[DEC_WAVES];
    __shared__ float sh_lg[EPL * WAVE];
    __shared__ int sh_idx[MAX_K];                // the routing, formed by wave 0
    __shared__ __align__(16) float sh_pr[MAX_K];
    __shared__ double sh_w[MAX_K];
    __shared__ uint32_t sh_mrank;
    // ranking slots (>= E): 32 RE, or 64 EPL for the xr instantiations (RE = 1)
    constexpr int SLOTS = (EPL > RE) ? WAVE * EPL : 32 * RE;
    __shared__ __align__(16) uint64_t sh_key[SLOTS];
    __shared__ float redg[DEC_WAVES][DEC_CCH];
    __shared__ float redu[DEC_WAVES][DEC_CCH];
    __shared__ __align__(16) float hl[DEC_MAX_HW];
    // (8 blocks of padding: the down units past a pair's blocks read there)
    __shared__ __align__(16) int8_t hlev[4][DEC_MAX_HW + 8 * QK];
    __shared__ float hsig[DEC_MAX_HW / QK + 8];
    __shared__ float sh_pd[2 * DEC_WAVES][32];   // sums of the (rank, row half) pairs
    __shared__ float pf[STACK ? DEC_MAX_FIN_STACK : DEC_MAX_FIN];
    __shared__ float hraw[STACK ? XN : 1];       // the layer's input residual row
    __shared__ uint32_t sh_tag;
    __shared__ int sh_fail;

    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int G = gridDim.x;
    const int j = blockIdx.x;
    const int mi = j / DEC_GROUPS;   // member
    const int M = G / DEC_GROUPS;
    const int NL = STACK ? a.L : 1;

    // a field of layer i (each read where it is used, so no layer's pointers
    // are held in scalar registers across the layer)
#define LAYER(i, f) as_global(STACK ? as_global(A.layers)[i].f : A.one.f)
#define LAYER0(f) as_global(STACK ? as_global(a.layers)[0].f : a.one.f)

    // ---- every load of the routing phase, unconditional (clamped addresses) ----
    const uint32_t epoch = __hip_atomic_load(a.epoch_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // rows this workgroup finishes, and their residual values
    const int RF = (a.H + G - 1) / G;
    const int q0 = j * RF;
    const int RFm = max(min(RF, a.H - q0), 0);
    float hin = STACK ? 0.0f : a.hidden[min(q0 + tid, a.H - 1)];   // (stack: hraw)
    float xv[XPT], wv[XPT];
    {
        const gptr<const float> nw = LAYER0(norm_w) ? LAYER0(norm_w) : as_global(a.x);
#pragma unroll
        for (int s = 0; s < XPT; s++) {
            const int k = min(tid + DEC_THREADS * s, a.H - 1);
            xv[s] = a.x[k];
            wv[s] = nw[k];
        }
    }
    // router rows of this member's experts e = mi + M t (F32 router; with
    // xr, expert j)
    float rw[RE][XPT];
    if (!a.router_q8) {
#pragma unroll
        for (int t = 0; t < RE; t++) {
            const int e = min(a.xr ? j : mi + M * t, a.E - 1);
#pragma unroll
            for (int s = 0; s < XPT; s++)
                rw[t][s] = LAYER0(rf32)[(size_t)e * a.H + min(tid + DEC_THREADS * s, a.H - 1)];
        }
    }
    // selection bias of experts lane, lane + 64, ...
    float bias_l[EPL];
#pragma unroll
    for (int t = 0; t < EPL; t++) bias_l[t] = LAYER0(bias)[min(lane + WAVE * t, a.E - 1)];
#pragma unroll
    for (int s = 0; s < XPT; s++) {
        const bool in = tid + DEC_THREADS * s < a.H;
        xv[s] = in ? xv[s] : 0.0f;
        wv[s] = (in && LAYER0(norm_w)) ? wv[s] : 1.0f;
    }
    if (tid == 0) {
        sh_tag = epoch + 1u;
        sh_fail = 0;
    }
    lds_barrier();
    const uint32_t tag0 = sh_tag;
    bool ok = true;
    constexpr int PUB = (DEC_WAVES - 1) * WAVE;

#define A a
    for (int l = 0; l < NL; l++) {
    // The index work of a layer is the same for every layer; computed from
    // opaque copies of the ids it stays inside the loop instead of being
    // hoisted out of it and held, spilled, across all the layers.
    int tid = threadIdx.x, j = blockIdx.x;
    asm volatile("" : "+v"(tid), "+s"(j));
    const int lane = tid & (WAVE - 1);
    const int wave = tid / WAVE;
    const int gx = j % DEC_GROUPS;
    const int mi = j / DEC_GROUPS;
    const uint32_t tag = tag0 + (uint32_t)l;
    const bool last = l == NL - 1;
    if (STACK && l > 0) {
        // ---- the residual row after layer l - 1, from the members of the group ----
        const uint64_t *pl[XPT], *pd[XPT];
        bool want[XPT];
        float *dst[XPT];
        const size_t xo = ((size_t)((l - 1) & 1) * DEC_GROUPS + gx) * SYNC_X_WORDS;
#pragma unroll
        for (int s = 0; s < XPT; s++) {
            const int k = tid + DEC_THREADS * s;
            pl[s] = A.hxl + xo + min(k, A.H - 1);
            pd[s] = A.hxd + xo + min(k, A.H - 1);
            want[s] = k < A.H;
            dst[s] = &xl[min(k, XN - 1)];
        }
        uint32_t tg[XPT];
#pragma unroll
        for (int s = 0; s < XPT; s++) tg[s] = tag - 1u;
        ok = block_wait<DEC_THREADS, XPT>(tg, &sh_fail, pl, pd, want, dst, A.wait_ticks, A.err);
        if (!ok) break;
#pragma unroll
        for (int s = 0; s < XPT; s++) {
            const int k = tid + DEC_THREADS * s;
            xv[s] = (k < A.H) ? xl[k] : 0.0f;
        }
    }

    if constexpr (STACK) {
#pragma unroll
        for (int s = 0; s < XPT; s++) {
            const int k = tid + DEC_THREADS * s;
            if (k < XN) hraw[k] = xv[s];
        }
    }
    // ---- x -> LDS (ffn_norm first when asked: lfm2-engine.js:251-252) ----
    if (A.norm) {
        double ss = 0.0;   // padding adds exact zeros
#pragma unroll
        for (int s = 0; s < XPT; s++) ss = fma((double)xv[s], (double)xv[s], ss);
        const double inv = rms_inv(block_sum_f64<DEC_WAVES>(ss, nsum), A.H, A.eps);
#pragma unroll
        for (int s = 0; s < XPT; s++) xv[s] = (float)((double)wv[s] * (double)xv[s] * inv);
    }
#pragma unroll
    for (int s = 0; s < XPT; s++) {
        const int k = tid + DEC_THREADS * s;
        if (k < XN) xl[k] = xv[s];
    }
    // ---- router dots (lfm2-engine.js:418, tensor.js:469-482): exact products, binary64 sums ----
    const int re = A.xr ? (j < A.E ? 1 : 0) : (A.E > mi) ? (A.E - mi + M - 1) / M : 0;
#pragma unroll
    for (int t = 0; t < RE; t++) {
        double acc = 0.0;
        if (A.router_q8) {
            const int e = min(A.xr ? j : mi + M * t, A.E - 1);
#pragma unroll
            for (int s = 0; s < XPT; s++) {
                const int k = min(tid + DEC_THREADS * s, A.H - 1);
                const size_t o = bm_index(0, A.nbH, k >> 5, A.E, e);
                acc = fma((double)xv[s], (double)LAYER(l, rq)[o * QK + (k & 31)] * (double)__half2float(LAYER(l, rd)[o]), acc);
            }
        } else {
#pragma unroll
            for (int s = 0; s < XPT; s++) acc = fma((double)xv[s], (double)rw[t][s], acc);
        }
        acc = wave_sum_dpp(acc);
        if (lane == 0) rsum[t][wave] = acc;
    }
    // (the residual rows have arrived before the arrival word goes out)
    if constexpr (!STACK) asm volatile("" : "+v"(hin));
    lds_barrier();
    // the last wave publishes (arrival, at the first layer: x and hidden
    // have been read; the router logits); waves 0..3 poll
    if (l == 0 && tid == PUB) store_dev(&A.arrive[j], (uint64_t)tag << 32);
    if (tid >= PUB && tid - PUB < re) {
        const int t = tid - PUB;
        const int e = A.xr ? j : mi + M * t;
        double s = rsum[t][0];
#pragma unroll
        for (int w = 1; w < DEC_WAVES; w++) s = s + rsum[t][w];
        const uint64_t word = tag_word(tag, (float)s);
        if (!A.xr) store_local(&A.rloc[(size_t)gx * SYNC_LOCAL_WORDS + e], word);
        if (gx == 0 || A.xr) {
            // (stack launches: replicas [0, 8) for even layers, [8, 16) for odd)
            constexpr int NREP = STACK ? SYNC_REPLICAS / 2 : SYNC_REPLICAS;
            const int c0 = STACK ? (l & 1) * NREP : 0;
#pragma unroll
            for (int c = 0; c < NREP; c++) store_dev(&A.rdev[(size_t)(c0 + c) * SYNC_REPLICA_WORDS + e], word);
        }
    }
    // x -> three int8 levels for the MFMA products; the rows of zeros
    decompose32<XN>(xl, XN / QK, &xlev[0][0], xsig);
    if (l == 0) {
        for (int i = tid; i < XN / 16; i += DEC_THREADS) reinterpret_cast<int4 *>(xlev[3])[i] = make_int4(0, 0, 0, 0);
        for (int i = tid; i < (DEC_MAX_HW + 8 * QK) / 16; i += DEC_THREADS)
            reinterpret_cast<int4 *>(hlev[3])[i] = make_int4(0, 0, 0, 0);
    }

    {
        const int rc = STACK ? (l & 1) * (SYNC_REPLICAS / 2) + j % (SYNC_REPLICAS / 2) : j % SYNC_REPLICAS;
        const uint64_t *pd[1] = {&A.rdev[(size_t)rc * SYNC_REPLICA_WORDS + min(tid, A.E - 1)]};
        // with xr every logit comes from the device-coherent tables
        const uint64_t *pl[1] = {A.xr ? pd[0] : &A.rloc[(size_t)gx * SYNC_LOCAL_WORDS + min(tid, A.E - 1)]};
        bool want[1] = {tid < A.E};
        float *dst[1] = {&sh_lg[min(tid, EPL * WAVE - 1)]};
        const uint32_t tg[1] = {tag};
        ok = block_wait<4 * WAVE, 1>(tg, &sh_fail, pl, pd, want, dst, A.wait_ticks, A.err);
    }

    // ---- this workgroup's share (independent of the routing) ----
    const int fb0 = gx * A.nbF / DEC_GROUPS, fb1 = (gx + 1) * A.nbF / DEC_GROUPS;
    const int FRb = fb1 - fb0;                        // F blocks of the group (<= 8)
    const int f0 = fb0 * QK;
    const int FR = max(min(fb1 * QK, A.F) - f0, 0);   // features of the group
    const float inv_fr = 1.0f / (float)max(FR, 1);
    const float inv_frb = 1.0f / (float)max(FRb, 1);
    const int NC = A.K * FR;                          // its (rank, feature) columns
    const int CPM = (NC + M - 1) / M;
    const int c0 = mi * CPM;
    const int nc = max(min(CPM, NC - c0), 0);         // this member's columns (<= 32)
    const int RM = (A.H + M - 1) / M;                 // down rows per member (<= 64)
    const int r0 = mi * RM;
    const int RMm = max(min(RM, A.H - r0), 0);
    const int NRH = RM > 32 ? 2 : 1;                  // 32-row halves of the member's rows
    const int NP2 = (FRb > 0 && RMm > 0) ? A.K * NRH : 0;   // (rank, row half) pairs
    const int PPW = (NP2 + DEC_WAVES - 1) / DEC_WAVES;      // pairs per wave
    const int NUW = PPW * FRb;                               // down units per lane (<= 8)
    const int hh = lane >> 5;
    const int cs = lane & 31;
    // gate/up: lane c + 32h takes column c0 + c (lanes past the member's
    // columns repeat its last one: no extra lines), bytes 16h .. 16h + 15 of
    // blocks NBW w .. NBW w + NBW - 1; row offsets within an expert
    const int cl = c0 + max(min(cs, nc - 1), 0);
    const int ck = (nc > 0) ? div_small(cl, inv_fr) : 0;   // rank of the column
    const int cf = (nc > 0) ? f0 + cl - ck * FR : 0;        // feature
    uint32_t goff[NBW];
#pragma unroll
    for (int i = 0; i < NBW; i++) goff[i] = (uint32_t)(min(NBW * wave + i, A.nbH - 1) * A.F + cf);
    // down: wave w takes the (rank, row half) pairs w, w + 8 over the group's
    // blocks, lane r + 32h row r of the half; row offsets within an expert
    int pk2[2];   // ranks of this wave's two pairs
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int p = min(wave + DEC_WAVES * t, max(NP2 - 1, 0));
        pk2[t] = min((NRH == 2) ? (p >> 1) : p, A.K - 1);
    }
    uint32_t doff[DEC_DCH];
    bool dsec[DEC_DCH];   // unit of the second pair
    bool don[DEC_DCH];    // unit in use (pair, block and row exist)
    int dhb[DEC_DCH];     // its 32-value block of the group's h values
#pragma unroll
    for (int i = 0; i < DEC_DCH; i++) {
        const int t = PP2 ? min(div_small(i, inv_frb), 1) : 0;
        const int bl = min(i - t * FRb, max(FRb - 1, 0));
        const int p = min(wave + DEC_WAVES * t, max(NP2 - 1, 0));
        const int rh = (NRH == 2) ? (p & 1) : 0;
        const int rl = min(rh * 32 + cs, max(RMm - 1, 0));
        doff[i] = (uint32_t)(min(fb0 + bl, A.nbF - 1) * A.H + min(r0 + rl, A.H - 1));
        dsec[i] = t != 0;
        don[i] = i < NUW && wave + DEC_WAVES * t < NP2 && rh * 32 + cs < RMm;
        // one pair: the units' blocks are consecutive (immediate LDS offsets)
        dhb[i] = PP2 ? pk2[t] * FRb + bl : pk2[0] * FRb + i;
    }

    // ---- routing (lfm2-engine.js:420-447; qwen3-engine.js:305-321), formed by
    // wave 0 alone (one wave per SIMD runs faster than eight sharing four):
    // scores, then the rank of each expert among them -- a stable descending
    // sort, ties to the lower index -- from 64-bit keys (order-preserving
    // score bits, complemented index), and the top K.  The weights w_k =
    // p_k / S (lfm2-engine.js:444-447; qwen3-engine.js:317-321) follow once
    // the weight loads are out ----
    float pr[EPL];
    if (ok && wave == 0) {
        float lg[EPL];
#pragma unroll
        for (int t = 0; t < EPL; t++) lg[t] = sh_lg[min(lane + WAVE * t, A.E - 1)];
        if (A.softmax) {
            softmax_probs<EPL>(lg, A.E, pr);
        } else {
#pragma unroll
            for (int t = 0; t < EPL; t++) pr[t] = (float)(1.0 / (1.0 + exp(-(double)lg[t])));
        }
        uint64_t key[EPL];
#pragma unroll
        for (int t = 0; t < EPL; t++) {
            const int e = lane + WAVE * t;
            const float sc = (A.softmax ? pr[t] : pr[t] + bias_l[t]) + 0.0f;   // -0 -> +0
            const uint32_t u = __float_as_uint(sc);
            const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            key[t] = (e < A.E) ? (((uint64_t)ord << 32) | (uint32_t)~e) : 0;
            if (e < SLOTS) sh_key[e] = key[t];
        }
        // (a wave's LDS accesses are done in order, so its lanes read what
        // its other lanes wrote above without a barrier)
        int rank[EPL];
#pragma unroll
        for (int t = 0; t < EPL; t++) rank[t] = 0;
#pragma unroll 16
        for (int u = 0; u < SLOTS / 2; u++) {
            const ulonglong2 q = reinterpret_cast<const ulonglong2 *>(sh_key)[u];
#pragma unroll
            for (int t = 0; t < EPL; t++) rank[t] += (int)(q.x > key[t]) + (int)(q.y > key[t]);
        }
#pragma unroll
        for (int t = 0; t < EPL; t++) {
            const int e = lane + WAVE * t;
            if (e < A.E && rank[t] < A.K) {
                sh_idx[rank[t]] = e;
                sh_pr[rank[t]] = pr[t];
            }
        }
        // bit k: the rank-k expert is masked (lfm2-engine.js:464)
        const uint64_t mb = __ballot(lane < A.K && mask_has(A.mask, sh_idx[min(lane, MAX_K - 1)]));
        if (lane == 0) sh_mrank = (uint32_t)mb;
    }
    lds_barrier();
    const uint32_t mrank = ok ? sh_mrank : 0u;

    // The loads are issued unconditionally (expert 0 stands in when the
    // routing failed), so no control-flow join sits between them and their
    // uses for the compiler to place conversions -- and waits -- at.
    int4 gq[NBW], uq[NBW], dq[DEC_DCH];
    ScaleRun<NBW> gs, us;
    uint32_t ddb[DEC_DCH];
    bool cok = false;
    const int eg = ok ? sh_idx[ck] : 0;
    const int ed0 = ok ? sh_idx[pk2[0]] : 0, ed1 = ok ? sh_idx[pk2[1]] : 0;
    const size_t dst0 = (size_t)ed0 * A.nbF * A.H, dst1 = (size_t)ed1 * A.nbF * A.H;
    const gptr<const uint16_t> dd16 = (gptr<const uint16_t>)LAYER(l, dd);
    {
        // The scales go out first: small requests to pages the weight rows do
        // not touch are otherwise served after the whole stream.
        const size_t grow = (size_t)eg * A.F + cf;
        gs.load(LAYER(l, gdcm) + grow * A.nbpH + NBW * wave);
        us.load(LAYER(l, udcm) + grow * A.nbpH + NBW * wave);
#pragma unroll
        for (int i = 0; i < DEC_DCH; i++) ddb[i] = dd16[(dsec[i] ? dst1 : dst0) + doff[i]];
        cok = ok && cs < nc && !((mrank >> ck) & 1u);
        const gptr<const int8_t> gbase = LAYER(l, gq) + (size_t)eg * A.nbH * A.F * QK + 16 * hh;
        const gptr<const int8_t> ubase = LAYER(l, uq) + (size_t)eg * A.nbH * A.F * QK + 16 * hh;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            gq[i] = load_stream16(gbase + (size_t)goff[i] * QK);
            uq[i] = load_stream16(ubase + (size_t)goff[i] * QK);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();
    // ---- the weights, by wave 0 while the weight bytes stream in ----
    if (ok && wave == 0) {
        float pk[MAX_K];
#pragma unroll
        for (int u = 0; u < MAX_K / 4; u++) {
            const float4 v = reinterpret_cast<const float4 *>(sh_pr)[u];
            pk[4 * u] = v.x;
            pk[4 * u + 1] = v.y;
            pk[4 * u + 2] = v.z;
            pk[4 * u + 3] = v.w;
        }
        double sumW = A.softmax ? 0.0 : 1e-6;
#pragma unroll
        for (int k = 0; k < MAX_K; k++)
            if (k < A.K) sumW = sumW + (double)pk[k];
        const double inv = A.softmax ? (sumW > 0.0 ? 1.0 / sumW : 0.0) : 1.0 / sumW;
        const double wl = (double)sh_pr[min(lane, MAX_K - 1)] * inv;   // w of rank `lane`
        if (lane < A.K) sh_w[lane] = wl;
        if (j == 0) {
            if (lane < A.K) {
                if (A.out_idx) A.out_idx[l * A.K + lane] = sh_idx[lane];
                if (A.out_w) A.out_w[l * A.K + lane] = wl;
            }
            if (A.out_probs) {
#pragma unroll
                for (int t = 0; t < EPL; t++)
                    if (lane + WAVE * t < A.E) A.out_probs[l * A.E + lane + WAVE * t] = pr[t];
            }
            if (A.out_rec) {
                if (lane < A.K) {
                    A.out_rec[lane] = (float)sh_idx[lane];
                    A.out_rec[A.K + lane] = (float)wl;
                }
#pragma unroll
                for (int t = 0; t < EPL; t++)
                    if (lane + WAVE * t < A.E) A.out_rec[2 * A.K + lane + WAVE * t] = pr[t];
            }
        }
    }

    // The group's h values (zero for masked ranks and padding) and the
    // partials (zero for groups without blocks and masked ranks) start
    // cleared; the barrier after the gate/up products orders this before
    // the waits that fill them.
    {
        const int HW = A.K * FRb * QK;
        for (int i = tid; i < HW; i += DEC_THREADS) hl[i] = 0.0f;
        for (int i = tid; i < (STACK ? DEC_MAX_FIN_STACK : DEC_MAX_FIN); i += DEC_THREADS) pf[i] = 0.0f;
    }

    // the next layer's router rows, bias and norm weights (stack launches)
    float rwn[RE][XPT] = {}, wvn[XPT] = {}, bsn[EPL] = {};

    // ---- gate / up columns, SwiGLU (tensor.js:167-178), h out ----
    if (ok) {
        // block b of the wave: C = (x levels of b) x (b's bytes of the 32
        // columns) on the matrix cores, column c's three level sums in lane c
        const int8_t *xa = &xlev[min(cs, 3)][16 * hh];
        float ga = 0.0f, ua = 0.0f;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            const int b = NBW * wave + i;
            const int4 av = *reinterpret_cast<const int4 *>(xa + QK * b);
            const float fg = lev3_sum(mfma_i8(av, gq[i]));
            const float fu = lev3_sum(mfma_i8(av, uq[i]));
            const bool bok = cok && b < A.nbH;
            const float sx = xsig[b];
            ga = fmaf(fg, bok ? sx * gs.get(i) : 0.0f, ga);
            ua = fmaf(fu, bok ? sx * us.get(i) : 0.0f, ua);
        }
        // The down rows are requested only once this wave's gate/up bytes
        // have arrived: every workgroup's gate/up requests then reach HBM
        // ahead of any down request, so the h values are ready early, and
        // the down bytes stream in while the h values are exchanged.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < DEC_DCH; i++)
            dq[i] = load_stream16(LAYER(l, dq) + ((dsec[i] ? dst1 : dst0) + doff[i]) * QK + 16 * hh);
        __builtin_amdgcn_sched_barrier(0);
        if (hh == 0) {
            redg[wave][cs] = ga;
            redu[wave][cs] = ua;
        }
        lds_barrier();
        if (tid >= PUB && tid - PUB < nc) {
            const int cc = tid - PUB;
            const int c = c0 + cc;
            const int k = div_small(c, inv_fr);
            const int f = f0 + c - k * FR;
            if (!((mrank >> k) & 1u)) {
                float G = redg[0][cc], U = redu[0][cc];
#pragma unroll
                for (int w = 1; w < DEC_WAVES; w++) {
                    G += redg[w][cc];
                    U += redu[w][cc];
                }
                const double g64 = (double)G;
                const float sg = (float)(g64 * (1.0 / (1.0 + exp(-g64))));
                const uint64_t word = tag_word(tag, sg * U);
                store_local(&A.hloc[(size_t)k * A.F + f], word);
                store_dev(&A.hdev[(size_t)k * A.F + f], word);
            }
        }
    }

    // ---- the group's h values -> LDS (zero for masked ranks and padding,
    // cleared above); waves 0..6 poll while wave 7 forms and publishes its h ----
    if (ok && NP2 > 0) {
        constexpr int IPT = (DEC_MAX_HW + PUB - 1) / PUB;
        const uint64_t *pl[IPT], *pd[IPT];
        bool want[IPT];
        float *dst[IPT];
        uint32_t tg[IPT];
#pragma unroll
        for (int s2 = 0; s2 < IPT; s2++) {
            tg[s2] = tag;
            const int i = min(tid + PUB * s2, NC - 1);
            const int k = div_small(i, inv_fr);
            const int f = f0 + i - k * FR;
            pl[s2] = &A.hloc[(size_t)k * A.F + f];
            pd[s2] = &A.hdev[(size_t)k * A.F + f];
            want[s2] = tid + PUB * s2 < NC && !((mrank >> k) & 1u);
            dst[s2] = &hl[k * FRb * QK + (i - k * FR)];
        }
        ok = block_wait<PUB, IPT>(tg, &sh_fail, pl, pd, want, dst, A.wait_ticks, A.err);
    }
    if (ok && NP2 > 0) {
        decompose32<DEC_MAX_HW + 8 * QK>(hl, A.K * FRb, &hlev[0][0], hsig);
        lds_barrier();
        // ---- partial down products: lane r of wave w adds up the products
        // of its row r of pairs w and w + 8 over the group's blocks (in block
        // order), one MFMA a block: C = (h levels of the block) x (the block's
        // bytes of the 32 rows) ----
        const int8_t *ha = &hlev[min(cs, 3)][16 * hh];
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int i = 0; i < DEC_DCH; i++) {
            const int hb = dhb[i];
            // the scale bits pass an empty asm here (ordered after the
            // barriers above), so the compiler cannot convert them -- and wait
            // for the down loads -- before the gate/up products
            uint32_t db = ddb[i];
            asm volatile("" : "+v"(db));
            const int4 av = *reinterpret_cast<const int4 *>(ha + QK * hb);
            const float y = lev3_sum(mfma_i8(av, dq[i])) * hsig[hb] * f16_bits(db);
            if (PP2) {
                acc0 += (don[i] && !dsec[i]) ? y : 0.0f;
                acc1 += (don[i] && dsec[i]) ? y : 0.0f;
            } else {
                acc0 += don[i] ? y : 0.0f;
            }
        }
        if (hh == 0) {
            sh_pd[wave][cs] = acc0;
            sh_pd[DEC_WAVES + wave][cs] = acc1;
        }
    }
    // the next layer's router rows, bias and norm weights: requested once the
    // down products are done (the weight registers are free), they arrive
    // while the partials and the residual row are exchanged
    if (STACK && ok && !last) {
        if (!A.router_q8) {
#pragma unroll
            for (int t = 0; t < RE; t++) {
                const int e = min(mi + M * t, A.E - 1);
#pragma unroll
                for (int s = 0; s < XPT; s++)
                    rwn[t][s] = LAYER(l + 1, rf32)[(size_t)e * A.H + min(tid + DEC_THREADS * s, A.H - 1)];
            }
        }
#pragma unroll
        for (int t = 0; t < EPL; t++) bsn[t] = LAYER(l + 1, bias)[min(lane + WAVE * t, A.E - 1)];
#pragma unroll
        for (int s = 0; s < XPT; s++) {
            const int k = tid + DEC_THREADS * s;
            wvn[s] = (LAYER(l + 1, norm_w) && k < A.H) ? LAYER(l + 1, norm_w)[k] : 1.0f;
        }
    }
    lds_barrier();
    // waves 4..7 publish the pairs' sums (the polling waves 0..3 then hold no
    // device stores to wait for); stack launches alternate two halves
    const size_t ppar = STACK ? (size_t)(l & 1) * DEC_GROUPS * A.K * A.H : 0;
    if (ok && NP2 > 0) {
        for (int t = tid - DEC_THREADS / 2; t >= 0 && t < NP2 * 32; t += DEC_THREADS / 2) {
            const int p = t >> 5;
            const int r = t & 31;
            const int k = (NRH == 2) ? (p >> 1) : p;
            const int rl = ((NRH == 2) ? (p & 1) : 0) * 32 + r;
            if (rl < RMm && !((mrank >> k) & 1u))
                store_dev(&A.part[ppar + ((size_t)gx * A.K + k) * A.H + r0 + rl], tag_word(tag, sh_pd[p][r]));
        }
    }

    // ---- combine (lfm2-engine.js:459-486): y_k = sum of the groups' partials,
    // acc = fp32(acc + w_k y_k) in rank order, hidden += acc.  The arrival
    // words (of the first layer) are waited for before hidden is written ----
    if constexpr (STACK) {
        // member mi of every group: the 8 groups' partials of rows
        // [r0, r0 + RM) (and, at the last layer, the arrival words)
        const int NPm = DEC_GROUPS * A.K * RM;
        if (ok) {
            constexpr int IPT = DEC_MAX_FIN_STACK / DEC_THREADS;
            const uint64_t *pl[IPT];
            bool want[IPT];
            float *dst[IPT];
            uint32_t tg[IPT];
            const float inv_krm = 1.0f / (float)(A.K * RM), inv_rm = 1.0f / (float)RM;
#pragma unroll
            for (int s2 = 0; s2 < IPT; s2++) {
                const int i = tid + DEC_THREADS * s2;
                const int ip = min(i, NPm - 1);
                const int x = div_small(ip, inv_krm);
                const int r = ip - x * A.K * RM;
                const int k = div_small(r, inv_rm);
                const int q = r - k * RM;
                const int xb0 = (x * A.nbF) >> 3, xb1 = ((x + 1) * A.nbF) >> 3;   // DEC_GROUPS = 8
                const uint64_t *pp = &A.part[ppar + ((size_t)x * A.K + k) * A.H + min(r0 + q, A.H - 1)];
                const uint64_t *pa = &A.arrive[min(max(i - NPm, 0), G - 1)];
                const bool isp = i < NPm;
                pl[s2] = isp ? pp : pa;
                want[s2] = isp ? (q < RMm && xb1 > xb0 && !((mrank >> k) & 1u)) : (last && i < NPm + G);
                dst[s2] = isp ? &pf[min(i, DEC_MAX_FIN_STACK - 1)] : nullptr;
                tg[s2] = isp ? tag : tag0;
            }
            ok = block_wait<DEC_THREADS, IPT>(tg, &sh_fail, pl, pl, want, dst, A.wait_ticks, A.err);
        }
        if (ok && tid < RMm) {
            float acc = 0.0f;
            for (int k0 = 0; k0 < A.K; k0 += 4) {   // four ranks' reads issued together
                float v[4][DEC_GROUPS];
                double w4[4];
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const int k = min(k0 + kk, A.K - 1);
#pragma unroll
                    for (int x = 0; x < DEC_GROUPS; x++) v[kk][x] = pf[(x * A.K + k) * RM + tid];
                    w4[kk] = sh_w[k];
                }
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    float y = 0.0f;
#pragma unroll
                    for (int x = 0; x < DEC_GROUPS; x++) y += v[kk][x];
                    const int k = k0 + kk;
                    if (k < A.K && !((mrank >> k) & 1u)) acc = (float)((double)acc + w4[kk] * (double)y);
                }
            }
            const float hn = hraw[r0 + tid] + acc;
            if (last) {
                if (gx == 0) A.hidden[r0 + tid] = hn;
            } else {
                const size_t xo = ((size_t)(l & 1) * DEC_GROUPS + gx) * SYNC_X_WORDS + r0 + tid;
                const uint64_t word = tag_word(tag, hn);
                store_local(&A.hxl[xo], word);
                store_dev(&A.hxd[xo], word);
            }
        }
    } else {
    const int NP = DEC_GROUPS * A.K * RF;
    if (ok) {
        constexpr int NT = DEC_THREADS / 2;
        constexpr int IPT = DEC_MAX_FIN / NT;
        const uint64_t *pl[IPT];
        bool want[IPT];
        float *dst[IPT];
        uint32_t tg[IPT];   // arrival words carry the first layer's tag
        const float inv_krf = 1.0f / (float)(A.K * RF), inv_rf = 1.0f / (float)RF;
#pragma unroll
        for (int s2 = 0; s2 < IPT; s2++) {
            // item i: partial (x, k, q) of the group sums, or arrival word i - NP;
            // both worked out and selected (no branch, no integer division:
            // this runs right after the partials go out)
            const int i = tid + NT * s2;
            const int ip = min(i, NP - 1);
            const int x = div_small(ip, inv_krf);
            const int r = ip - x * A.K * RF;
            const int k = div_small(r, inv_rf);
            const int q = r - k * RF;
            const int xb0 = (x * A.nbF) >> 3, xb1 = ((x + 1) * A.nbF) >> 3;   // DEC_GROUPS = 8
            const uint64_t *pp = &A.part[((size_t)x * A.K + k) * A.H + min(q0 + q, A.H - 1)];
            const uint64_t *pa = &A.arrive[min(max(i - NP, 0), G - 1)];
            const bool isp = i < NP;
            pl[s2] = isp ? pp : pa;
            want[s2] = isp ? (q < RFm && xb1 > xb0 && !((mrank >> k) & 1u)) : (last && i < NP + G);
            dst[s2] = isp ? &pf[min(i, DEC_MAX_FIN - 1)] : nullptr;
            tg[s2] = isp ? tag : tag0;
        }
        ok = block_wait<NT, IPT>(tg, &sh_fail, pl, pl, want, dst, A.wait_ticks, A.err);
    }
    if (ok && tid < RFm) {
        float acc = 0.0f;
        for (int k0 = 0; k0 < A.K; k0 += 4) {   // four ranks' reads issued together
            float v[4][DEC_GROUPS];
            double w4[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int k = min(k0 + kk, A.K - 1);
#pragma unroll
                for (int x = 0; x < DEC_GROUPS; x++) v[kk][x] = pf[(x * A.K + k) * RF + tid];
                w4[kk] = sh_w[k];
            }
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                float y = 0.0f;
#pragma unroll
                for (int x = 0; x < DEC_GROUPS; x++) y += v[kk][x];
                const int k = k0 + kk;
                if (k < A.K && !((mrank >> k) & 1u)) acc = (float)((double)acc + w4[kk] * (double)y);
            }
        }
        A.hidden[q0 + tid] = hin + acc;
    }
    }
    if constexpr (STACK) {
        if (!ok) break;
#pragma unroll
        for (int t = 0; t < RE; t++)
#pragma unroll
            for (int s = 0; s < XPT; s++) rw[t][s] = rwn[t][s];
#pragma unroll
        for (int s = 0; s < XPT; s++) wv[s] = wvn[s];
#pragma unroll
        for (int t = 0; t < EPL; t++) bias_l[t] = bsn[t];
    }
    }   // layers

    if (tid == 0) {
        if (!ok) atomicOr(a.err, 1u);
        // workgroup 0 has seen every arrival word carry the first tag (or gave
        // up waiting), so every workgroup has read the epoch: the next call
        // draws the tags after this call's
        if (j == 0) __hip_atomic_store(a.epoch_word, tag0 + (uint32_t)NL - 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#undef LAYER
#undef LAYER0
#undef A
}

static int decode_grid(const qq_ctx *ctx)
{
    return (std::min(ctx->num_cus, SYNC_ARRIVE_WORDS) / DEC_GROUPS) * DEC_GROUPS;
}

bool decode_supported(const qq_ctx *ctx, const qq_moe *m, int T)
{
    if (T != 1 || m->E > MAX_E || m->K > m->E || m->H > 8 * DEC_WAVES * QK) return false;
    const int G = decode_grid(ctx);
    if (G < DEC_GROUPS) return false;
    const int M = G / DEC_GROUPS;
    const int nbF = (m->F + QK - 1) / QK;
    const int frb = (nbF + DEC_GROUPS - 1) / DEC_GROUPS;   // blocks of the largest group
    const int cpm = (m->K * frb * QK + M - 1) / M;
    const int RM = (m->H + M - 1) / M;
    const int nrh = RM > 32 ? 2 : 1;
    const int RF = (m->H + G - 1) / G;
    const int ppw = (m->K * nrh + DEC_WAVES - 1) / DEC_WAVES;
    return (m->E + M - 1) / M <= 8 && RM <= 64 && cpm <= DEC_CCH && ppw <= 2 && ppw * frb <= DEC_DCH &&
           m->K * frb * QK <= DEC_MAX_HW &&
           DEC_GROUPS * m->K * RF + G <= DEC_MAX_FIN &&
           (size_t)m->K * m->F <= SYNC_H_WORDS && (size_t)m->K * m->H * DEC_GROUPS <= SYNC_P_WORDS;
}

template <int NBW, int RE, int EPL, bool STACK>
static void launch_t(qq_ctx *ctx, const DecodeArgs &a, dim3 grid, bool pp2)
{
    if (pp2) QQ_LAUNCH(ctx, (moe_decode_kernel<NBW, RE, EPL, true, STACK>), grid, dim3(DEC_THREADS), 0, a);
    else QQ_LAUNCH(ctx, (moe_decode_kernel<NBW, RE, EPL, false, STACK>), grid, dim3(DEC_THREADS), 0, a);
}

// (RE, EPL) pairs: with M <= 32 members per group, ceil(E / M) <= RE implies
// ceil(E / 64) <= EPL for these four
bool stack_decode_supported(const qq_ctx *ctx, const qq_moe *m)
{
    if (!decode_supported(ctx, m, 1) || m->H > SYNC_X_WORDS) return false;
    const int M = decode_grid(ctx) / DEC_GROUPS;
    const int RM = (m->H + M - 1) / M;
    return DEC_GROUPS * m->K * RM + decode_grid(ctx) <= DEC_MAX_FIN_STACK &&
           2 * (size_t)DEC_GROUPS * m->K * m->H <= SYNC_P_WORDS;
}

template <int NBW, bool STACK>
static void launch_re(qq_ctx *ctx, const DecodeArgs &a, dim3 grid, int re, bool pp2)
{
    if constexpr (!STACK) {
        if (a.xr) {   // one expert per workgroup
            if (a.E <= 2 * WAVE) launch_t<NBW, 1, 2, STACK>(ctx, a, grid, pp2);
            else launch_t<NBW, 1, 4, STACK>(ctx, a, grid, pp2);
            return;
        }
    }
    if (re <= 1) launch_t<NBW, 1, 1, STACK>(ctx, a, grid, pp2);
    else if (re <= 2) launch_t<NBW, 2, 1, STACK>(ctx, a, grid, pp2);
    else if (re <= 4) launch_t<NBW, 4, 2, STACK>(ctx, a, grid, pp2);
    else launch_t<NBW, 8, 4, STACK>(ctx, a, grid, pp2);
}

DecodeLayer decode_layer_of(const qq_moe *m, const float *norm_w)
{
    DecodeLayer d;
    const bool q8 = m->router_type == QQ_TYPE_Q8_0;
    d.rf32 = m->router_f32;
    d.rq = q8 ? m->router_q8->qs : nullptr;
    d.rd = q8 ? m->router_q8->d : nullptr;
    d.bias = m->bias;
    d.gq = m->gate->qs;
    d.gdcm = m->gate->dcm;
    d.uq = m->up->qs;
    d.udcm = m->up->dcm;
    d.dq = m->down->qs;
    d.dd = m->down->d;
    d.norm_w = norm_w;
    return d;
}

static void decode_common(qq_ctx *ctx, const qq_moe *m, DecodeArgs &a)
{
    a.H = m->H;
    a.F = m->F;
    a.E = m->E;
    a.K = m->K;
    a.nbH = (m->H + QK - 1) / QK;
    a.nbF = (m->F + QK - 1) / QK;
    a.router_q8 = m->router_type == QQ_TYPE_Q8_0;
    a.xr = 0;
    a.softmax = m->gating == QQ_GATING_SOFTMAX;
    a.nbpH = m->gate->nbp;
    a.epoch_word = ctx->sync_epoch;
    a.rloc = ctx->sync_local;
    a.rdev = ctx->sync_slots;
    a.hloc = ctx->sync_hloc;
    a.hdev = ctx->sync_hdev;
    a.part = ctx->sync_part;
    a.arrive = ctx->sync_arrive;
    a.hxl = ctx->sync_hx;
    a.hxd = ctx->sync_hx + 2 * DEC_GROUPS * SYNC_X_WORDS;
    a.err = ctx->sync_err;
    a.wait_ticks = ctx->dec_wait_ticks;
}

template <bool STACK>
static int decode_launch(qq_ctx *ctx, const qq_moe *m, const DecodeArgs &a)
{
    const int G = decode_grid(ctx);
    const int re = (m->E + G / DEC_GROUPS - 1) / (G / DEC_GROUPS);
    const int nbw = (a.nbH + DEC_WAVES - 1) / DEC_WAVES;
    const int RM = (m->H + G / DEC_GROUPS - 1) / (G / DEC_GROUPS);
    const bool pp2 = m->K * (RM > 32 ? 2 : 1) > DEC_WAVES;
    const dim3 grid(G);
    prof_begin(ctx, K_DECODE);
    if (nbw <= 1) launch_re<1, STACK>(ctx, a, grid, re, pp2);
    else if (nbw <= 2) launch_re<2, STACK>(ctx, a, grid, re, pp2);
    else if (nbw <= 4) launch_re<4, STACK>(ctx, a, grid, re, pp2);
    else launch_re<8, STACK>(ctx, a, grid, re, pp2);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

int launch_moe_decode(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden,
                      const MaskBits &mask, int32_t *out_idx, double *out_w, float *out_probs,
                      const NormArgs *norm, float *out_rec)
{
    DecodeArgs a;
    decode_common(ctx, m, a);
    a.x = x;
    a.norm = norm != nullptr;
    a.eps = norm ? norm->eps : 0.0;
    a.hidden = hidden;
    a.L = 1;
    a.one = decode_layer_of(m, norm ? norm->w : nullptr);
    a.layers = nullptr;
    a.mask = mask;
    a.out_idx = out_idx;
    a.out_w = out_w;
    a.out_probs = out_probs;
    a.out_rec = out_rec;
    // more experts than a group has members: each workgroup forms one logit
    // (the router is read once, not once per group), exchanged device-wide
    a.xr = m->E > decode_grid(ctx) / DEC_GROUPS && m->E <= decode_grid(ctx);
    return decode_launch<false>(ctx, m, a);
}

int launch_moe_stack_decode(qq_ctx *ctx, const qq_moe *m0, const DecodeLayer *layers_dev, int L, float *hidden,
                            double eps, const MaskBits &mask, int32_t *out_idx, double *out_w, float *out_probs)
{
    DecodeArgs a;
    decode_common(ctx, m0, a);
    a.x = hidden;
    a.norm = 1;
    a.eps = eps;
    a.hidden = hidden;
    a.L = L;
    a.one = decode_layer_of(m0, nullptr);
    a.layers = layers_dev;
    a.mask = mask;
    a.out_idx = out_idx;
    a.out_w = out_w;
    a.out_probs = out_probs;
    a.out_rec = nullptr;
    return decode_launch<true>(ctx, m0, a);
}

}  // namespace qq
