// stream.hip -- decode batches (a few to a few dozen tokens per expert) on
// the matrix cores at fp32 accuracy.
//
// With ~8 rows per expert (64 tokens, 32 experts, top-4) every weight is used
// by very few rows, so the layer is bound by streaming the experts' Q8_0
// weights from HBM once.  A workgroup owns one expert, one tile of 16*MF
// slots and a group of weight columns (two halves of 16 NFH: 64 or 112 gate
// and the same up features, 128 down columns); its 4 waves split the reduction
// dimension block by block (each streaming its blocks straight into
// registers, a few blocks ahead, below) and their partial sums are added in
// wave order through LDS.
//
// Accuracy (the fp32 path's 1e-4 relative L2): activations are split into
// two fp16 halves, a = a_hi + a_lo (22 significant bits); the int8 weights
// are exact in fp16.  Per 32-value block two MFMAs give the block's partial
// sum a_hi*q + a_lo*q with exact products and fp32 accumulation, and the
// block's fp16 scale is applied to that fp32 partial (one FMA per output),
// as the reference applies d per block.  Error ~1e-7 relative, like the fp32
// kernels.
//   gate/up  A = x rows of the tile's tokens (gathered by perm), B = 64 gate +
//            64 up columns; epilogue silu(g) * u -> act[slot][F] (fp32)
//   down     A = act rows, B = 128 down columns -> y[slot][H] (fp32)
// followed by the gather combine.
#include "qq_device.h"

namespace qq {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int ST_THREADS = 256;   // 4 waves split the reduction dimension

struct StreamArgs {
    const float *x;          // [T][H] activations
    float *act;              // [slots][F] SwiGLU products
    float *y;                // [slots][H] expert outputs
    const int32_t *perm, *counts, *offsets;
    const int32_t *tile_e, *tile_m0, *n_tiles;
    const int8_t *gq, *uq, *dq;
    const uint16_t *gd, *ud, *dd;   // fp16 scale bits
    uint64_t *part;          // partial sums of split items (st_work), tagged words
    uint32_t *seg_ctr;       // per split item: segments done (zero between launches)
    uint32_t *seg_gen;       // [0] generation: a launch's partials carry gen + 1;
                             // [1] split items done in the launch (zero between launches)
    uint32_t *err;           // device error word (a bounded wait expired)
    uint64_t wait_ticks;
    int H, F, K, nbH, nbF;
    int G;                   // resident workgroups (2 per CU)
    int tile_cap;            // row tiles the grid is sized for
};

// 8 consecutive fp32 values -> high and low fp16 halves.  hi is rounded
// toward zero (v_cvt_pkrtz_f16_f32); v - hi is exact in fp32 and its fp16
// rounding is the split's only loss.
__device__ __forceinline__ void split8(const float4 a, const float4 b, h8_t &hi, h8_t &lo)
{
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2_t h = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(v[2 * i], v[2 * i + 1]));
        hw[i] = __builtin_bit_cast(uint32_t, h);
        lw[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(v[2 * i] - (float)h[0],
                                                                          v[2 * i + 1] - (float)h[1]));
    }
    hi = __builtin_bit_cast(h8_t, make_uint4(hw[0], hw[1], hw[2], hw[3]));
    lo = __builtin_bit_cast(h8_t, make_uint4(lw[0], lw[1], lw[2], lw[3]));
}

// 8 int8 weights (one lane's share of a 16x32 fragment) -> 8 fp16 holding
// the same integers exactly (four conversions per four weights; the
// offset-binary form, bytes paired with the exponent byte 0x64 and 1152
// subtracted, took five).
__device__ __forceinline__ h8_t int8_to_f16x8(const uint2 q)
{
    return __builtin_bit_cast(h8_t, make_uint4(i8pair_f16<0>(q.x), i8pair_f16<2>(q.x), i8pair_f16<0>(q.y),
                                               i8pair_f16<2>(q.y)));
}

// ---------------------------------------------------------------------------
// Operand stream.  Wave w reduces blocks w, w+4, w+8, ... of the reduction
// dimension.  Every operand of a block goes straight to registers: the
// lane's 8 activations of each of its MF rows (two float4), its 8 weight
// bytes of each of the 2 NFH fragment columns (uint2) and one fp16 scale per
// 64 columns of a half: load u of lane l reads column c0[h] + 64u + l's, and
// a fragment's scale is taken from the lane that loaded it (fragment f of a
// half: load f/4, lanes 16(f%4) .. 16(f%4)+15).  Each wave keeps st_pf
// blocks in flight: block i + st_pf is requested as soon as block i's
// products are done.  (Staged through LDS the stream is held to ~100 KB in
// flight per CU by the LDS size.)
// Fragment j: column 16*(j%NFH) + lane%16 of half j/NFH; lane l holds row
// l%16 of A and column l%16 of B at k = 8*(l/16) .. 8*(l/16) + 7 of the block.
// ---------------------------------------------------------------------------
template <int MF, int NFH>
struct StBlock {
    static constexpr int NF = 2 * NFH;      // fragments
    static constexpr int NS = (NFH + 3) / 4;   // scale loads per column half
    float4 a[MF][2];     // rows 16m + lane%16, k = 8*(lane/16) .. +7
    uint2 q[NF];         // fragment j's 8 weight bytes
    uint32_t ds[2][NS];  // scale bits of column c0[h] + 64 s + lane of half h
};

// blocks in flight per wave: ~12-14 KB of weights either way
template <int MF, int NFH>
constexpr int st_pf() { return MF == 1 && NFH == 4 ? 3 : 2; }

template <int MF, int NFH>
struct StSrc {
    static constexpr int NS = (NFH + 3) / 4;
    const char *abase;          // activation rows (bytes)
    uint32_t arow[MF];          // lane's row 16m + lane%16: byte offset + its k chunk
    const int8_t *qb[2];        // weights of column halves 0 / 1 at the expert's block 0
    const uint16_t *db[2];      // their scales
    int cb[2];                  // column half h: the lane's column c0[h] + lane%16 (fragment f of the half adds 16 f)
    int cmax;                   // last column (loads clamp to it)
    uint32_t sc[2][NS];         // column of this lane's scale load s in half h (clamped)
    uint32_t qk;                // the lane's byte offset within a column's 32 bytes
    uint32_t qstep, dstep;      // one block: rows * 32 bytes, rows scales
    uint32_t okm;               // bit j: fragment j's column in range (else its scale is zero)
};

// 32-bit offsets from workgroup-uniform bases (one VGPR per address).
template <int MF, int NFH>
__device__ __forceinline__ void st_load(StBlock<MF, NFH> &b, const StSrc<MF, NFH> &s, int kb)
{
    const uint32_t ak = (uint32_t)kb * (QK * 4), qk = (uint32_t)kb * s.qstep, dk = (uint32_t)kb * s.dstep;
#pragma unroll
    for (int m = 0; m < MF; m++) {
        b.a[m][0] = *reinterpret_cast<const float4 *>(s.abase + (size_t)(s.arow[m] + ak));
        b.a[m][1] = *reinterpret_cast<const float4 *>(s.abase + (size_t)(s.arow[m] + ak + 16));
    }
    // one row tile per expert (MF == 1: at most 16 rows on average) reads
    // every weight byte once, so those loads are non-temporal; with more
    // rows the expert's other row tiles read the same bytes through the L2
#pragma unroll
    for (int j = 0; j < 2 * NFH; j++) {
        const uint32_t c = (uint32_t)min(s.cb[j / NFH] + 16 * (j % NFH), s.cmax);
        const uint2 *src = reinterpret_cast<const uint2 *>(s.qb[j / NFH] + (size_t)(qk + c * QK + s.qk));
        if constexpr (MF == 1) {
            typedef unsigned int v2u __attribute__((ext_vector_type(2)));
            const v2u v = __builtin_nontemporal_load(reinterpret_cast<const v2u *>(src));
            b.q[j] = make_uint2(v.x, v.y);
        } else {
            b.q[j] = *src;
        }
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int u = 0; u < StSrc<MF, NFH>::NS; u++)
            b.ds[h][u] = *reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(s.db[h]) +
                                                             (size_t)(2u * (dk + s.sc[h][u])));
}

// The block's int8 weights enter the MFMA exactly (as fp16 integers); the
// block's scale is applied to the block's fp32 partial sum:
//   acc += d * (a_hi * q + a_lo * q).
// A lane's four outputs of a fragment share one column, hence one scale.
template <int MF, int NFH>
__device__ __forceinline__ void st_block(const StBlock<MF, NFH> &b, const StSrc<MF, NFH> &s,
                                         f4_t (&acc)[MF][2 * NFH])
{
    h8_t ah[MF], al[MF];
#pragma unroll
    for (int m = 0; m < MF; m++) split8(b.a[m][0], b.a[m][1], ah[m], al[m]);
    const int l16 = threadIdx.x & 15;
#pragma unroll
    for (int j = 0; j < 2 * NFH; j++) {
        const int f = j % NFH;
        const uint32_t bits = (uint32_t)__shfl((int)b.ds[j / NFH][f / 4], 16 * (f & 3) + l16, WAVE);
        const float d = ((s.okm >> j) & 1u) ? (float)__builtin_bit_cast(_Float16, (uint16_t)bits) : 0.0f;
        const h8_t qh = int8_to_f16x8(b.q[j]);
#pragma unroll
        for (int m = 0; m < MF; m++) {
            f4_t p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[m], qh, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            p = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[m], qh, p, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[m][j][r] = fmaf(p[r], d, acc[m][j][r]);
        }
    }
}

// Wave w reduces blocks kb0 + w, kb0 + w + 4, ... of the nb blocks from kb0
// on, with st_pf blocks in flight.
template <int MF, int NFH>
__device__ __forceinline__ void st_mainloop(const StSrc<MF, NFH> &s, int kb0, int nb, int wave,
                                            f4_t (&acc)[MF][2 * NFH])
{
    constexpr int PF = st_pf<MF, NFH>();
    const int nblk = (nb - wave + 3) / 4;
    const int kw = kb0 + wave;
    StBlock<MF, NFH> r[PF];
#pragma unroll
    for (int u = 0; u < PF; u++)
        if (u < nblk) st_load<MF, NFH>(r[u], s, kw + 4 * u);
    for (int i = 0; i < nblk; i += PF) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            if (i + u < nblk) {
                st_block<MF, NFH>(r[u], s, acc);
                // the refill goes out only after the products, so the
                // compiler waits for this block alone, not the ones behind it
                __builtin_amdgcn_sched_barrier(0);
                if (i + u + PF < nblk) st_load<MF, NFH>(r[u], s, kw + 4 * (i + u + PF));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

// Load offsets: activation row r of the tile has byte offset rowoff(r);
// weight halves start at columns c0[0], c0[1] of a matrix with `rows`
// columns per block (clamped into range).
template <int MF, int NFH, typename RowOff>
__device__ __forceinline__ void st_offsets(StSrc<MF, NFH> &s, RowOff rowoff, const int (&c0)[2],
                                           int rows, int lane)
{
#pragma unroll
    for (int m = 0; m < MF; m++) s.arow[m] = rowoff(16 * m + (lane & 15)) + 32 * (lane >> 4);
    s.qk = 8 * (lane >> 4);
    s.cb[0] = c0[0] + (lane & 15);
    s.cb[1] = c0[1] + (lane & 15);
    s.cmax = rows - 1;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int u = 0; u < StSrc<MF, NFH>::NS; u++) s.sc[h][u] = (uint32_t)min(c0[h] + 64 * u + lane, rows - 1);
    s.okm = 0;
#pragma unroll
    for (int j = 0; j < 2 * NFH; j++)
        s.okm |= (c0[j / NFH] + 16 * (j % NFH) + (lane & 15) < rows ? 1u : 0u) << j;
}

// Cross-wave sums of fragment row block m: each wave writes its fragments of
// half 0 to red0 and of half 1 to red1 ([wave][16 rows][16 NFH + 1 columns]).
template <int MF, int NFH>
__device__ __forceinline__ void st_spill(float (*red0)[16][16 * NFH + 1], float (*red1)[16][16 * NFH + 1],
                                         const f4_t (&acc)[MF][2 * NFH], int m, int wave, int lane)
{
    const int cl = lane & 15, rq = 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 2 * NFH; j++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            (j < NFH ? red0 : red1)[wave][rq + r][16 * (j % NFH) + cl] = acc[m][j][r];
}

template <int NFH>
__device__ __forceinline__ float wave_order_sum(const float (*red)[16][16 * NFH + 1], int row, int c)
{
    return ((red[0][row][c] + red[1][row][c]) + red[2][row][c]) + red[3][row][c];
}

// LDS: the cross-wave reduction tiles only
template <int NFH>
constexpr int st_lds() { return 2 * 4 * 16 * (16 * NFH + 1) * 4; }

// The work of one workgroup among R items (row tile x column group, row-tile
// major).  Items that fill whole rounds of the G resident workgroups run
// whole.  A remainder of L < G items would run as a round of its own on L
// workgroups, each streaming only as fast as its own blocks in flight allow:
// a tail as long as a full round for a few percent of the work.  Instead each
// remainder item is split into S segments of the reduction dimension (S L <=
// G / 2, at least 8 blocks each, and S L within the grid's room past the
// whole items, which is sized for the most row tiles there can be; the
// remainder is widened back to the first tile of its first expert, so all
// rows of an expert are summed the same way whatever their order within the
// expert) run by S L more workgroups, which store
// their fp32 partial sums as tagged words (tag = the kernel's generation + 1,
// new in every launch); the last segment to finish adds them in segment order
// and applies the epilogue (st_last, st_seg_sum).  The tags stand in for a
// release / acquire pair, whose device-scope fences would write back the
// whole L2.
constexpr int ST_SEG_MAX = 8;   // segments of a split item

struct StWork {
    int item;         // tile * ncg + column group
    int seg, nseg;    // segment of the reduction dimension; nseg == 1: whole
    int li;           // remainder item: counter li, partial slot li * nseg + seg
    int L;            // remainder items (split when nseg > 1)
};

__device__ __forceinline__ bool st_work(int R, int G, int nb, int ncg, int bm, const int32_t *tile_m0,
                                        StWork &w)
{
    int W = R;                               // items run whole
    int L = 0, S = 1;
    // R mod G by subtraction (R / G is a few rounds at most): the divisions
    // below sit on every workgroup's way to its first load, so they are
    // taken only where a split can follow (S >= 2: G >= 4 L, blocks >= 16;
    // widening the remainder only narrows S)
    int rem = R;
    while (rem >= G) rem -= G;
    if (rem && 4 * rem <= G && nb >= 16) {
        const int t = (R - rem) / ncg;      // tile of the first remainder item
        W = (t - tile_m0[t] / bm) * ncg;
        L = R - W;
        const int room = (int)gridDim.x - 8 * ((W + 7) >> 3);
        S = max(1, min(min(min(G / (2 * L), nb / 8), ST_SEG_MAX), room / L));
        if (S == 1) {
            W = R;
            L = 0;
        }
    }
    const int per = (W + 7) >> 3;
    const int b = blockIdx.x;
    w.L = L;
    if (b < 8 * per) {
        // the dispatcher deals workgroups to the 8 XCDs round robin (one XCD
        // runs blocks x, x+8, ...); each XCD takes a contiguous run of the
        // items, so the column groups of a row tile read its activation rows
        // through one L2
        const int x = b & 7, i = b >> 3, it = x * per + i;
        if (it >= W) return false;
        w.item = it;
        w.seg = 0;
        w.nseg = 1;
        w.li = 0;
        return true;
    }
    const int q = b - 8 * per;
    if (S == 1 || q >= L * S) return false;
    w.li = q / S;
    w.seg = q - w.li * S;
    w.nseg = S;
    w.item = W + w.li;
    return true;
}

// Counts this workgroup's segment of a split item in once its partial sums
// are stored; true in the workgroup of the last segment to arrive.  That
// workgroup returns the counter to zero for the next launch.  sh: one int of
// LDS.
__device__ __forceinline__ bool st_last(uint32_t *ctr, int nseg, int *sh)
{
    wait_vm<0>();   // this wave's tagged stores are out
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == (uint32_t)nseg - 1u;
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *sh = last;
    }
    __syncthreads();
    return *sh != 0;
}

// The last segment's workgroup, after its reduction: counts the item done;
// the last of the launch's L split items moves the generation on (every
// segment of the launch read it before its item's counter reached the end).
__device__ __forceinline__ void st_item_done(uint32_t *gen, int L, uint32_t tag)
{
    if (threadIdx.x == 0) {
        const uint32_t d = __hip_atomic_fetch_add(gen + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == (uint32_t)L - 1u) {
            __hip_atomic_store(gen + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Sums of a split item's partial sums: the 4 words from offset o[i] of each
// segment (segments PSZ words apart) into r[i], added in segment order.  All
// loads go out before the first add; words not yet carrying `tag` are read
// again (bounded by wait_ticks: false when the wait expired).
template <int PSZ, int NO>
__device__ __forceinline__ bool st_seg_sum(const uint64_t *p0, const int (&o)[NO], int nseg, uint32_t tag,
                                           uint64_t wait_ticks, float (&r)[NO][4])
{
    uint64_t v[ST_SEG_MAX][NO][4];
    uint64_t t0 = 0;
    for (bool first = true;; first = false) {
        bool ok = true;
#pragma unroll
        for (int sg = 0; sg < ST_SEG_MAX; sg++)
#pragma unroll
            for (int i = 0; i < NO; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (sg < nseg)
                        v[sg][i][j] = __hip_atomic_load(p0 + (size_t)sg * PSZ + o[i] + j, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int sg = 0; sg < ST_SEG_MAX; sg++)
#pragma unroll
            for (int i = 0; i < NO; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (sg < nseg) ok = ok && (uint32_t)(v[sg][i][j] >> 32) == tag;
        if (ok) break;
        if (first) {
            t0 = wall_clock64();
        } else if (wall_clock64() - t0 >= wait_ticks) {
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float x = __uint_as_float((uint32_t)v[0][i][j]);
#pragma unroll
            for (int sg = 1; sg < ST_SEG_MAX; sg++)
                if (sg < nseg) x += __uint_as_float((uint32_t)v[sg][i][j]);
            r[i][j] = x;
        }
    return true;
}

__device__ __forceinline__ float silu_mul(float g, float u)
{
    const double g64 = (double)g;
    return (float)(g64 * (1.0 / (1.0 + exp(-g64)))) * u;
}

// ---------------------------------------------------------------------------
// gate/up: column half 0 = gate features f0 .. f0 + 16 NFH - 1, half 1 = the
// same up features.
// ---------------------------------------------------------------------------
template <int MF, int NFH>
__global__ __launch_bounds__(ST_THREADS, 2) void moe_stream_gateup_kernel(StreamArgs a)
{
    constexpr int NC = 16 * NFH;   // features per workgroup
    __shared__ __align__(16) char lds[st_lds<NFH>()];
    __shared__ int sh_last;
    const int ncg = (a.F + NC - 1) / NC;
    StWork wk;
    if (!st_work(min(*a.n_tiles, a.tile_cap) * ncg, a.G, a.nbH, ncg, 16 * MF, a.tile_m0, wk)) return;
    const int tile = wk.item / ncg, cg = wk.item - tile * ncg;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(16 * MF, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int f0 = cg * NC;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;

    StSrc<MF, NFH> src;
    src.abase = reinterpret_cast<const char *>(a.x);
    const size_t eb = (size_t)e * a.nbH * a.F;     // expert's first block-row
    src.qb[0] = a.gq + eb * QK;
    src.qb[1] = a.uq + eb * QK;
    src.db[0] = a.gd + eb;
    src.db[1] = a.ud + eb;
    src.qstep = (uint32_t)a.F * QK;
    src.dstep = (uint32_t)a.F;
    const int c0[2] = {f0, f0};
    st_offsets<MF, NFH>(src, [&](int r) {
        return (uint32_t)(a.perm[slot0 + min(r, n - 1)] / a.K) * a.H * 4;
    }, c0, a.F, lane);

    f4_t acc[MF][2 * NFH];
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
        for (int j = 0; j < 2 * NFH; j++) acc[m][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int kb0 = wk.nseg > 1 ? wk.seg * a.nbH / wk.nseg : 0;
    const int kb1 = wk.nseg > 1 ? (wk.seg + 1) * a.nbH / wk.nseg : a.nbH;
    const uint32_t tag =
        wk.nseg > 1 ? __hip_atomic_load(a.seg_gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u : 0u;
    st_mainloop<MF, NFH>(src, kb0, kb1 - kb0, wave, acc);
    float (*red0)[16][NC + 1] = reinterpret_cast<float (*)[16][NC + 1]>(lds);
    float (*red1)[16][NC + 1] = red0 + 4;
    // split item: partial [16 MF rows][NC gate | NC up] of each segment
    constexpr int PSZ = 16 * MF * 2 * NC;
    uint64_t *pp = a.part + (size_t)(wk.li * wk.nseg + wk.seg) * PSZ;
#pragma unroll
    for (int m = 0; m < MF; m++) {
        __syncthreads();
        st_spill<MF, NFH>(red0, red1, acc, m, wave, lane);
        __syncthreads();
        // the tile's rows only (a split item's last segment reads those alone)
        const int nr = min(16, n - 16 * m);
        for (int i = threadIdx.x; i < nr * NC; i += ST_THREADS) {
            const int row = i / NC, c = i % NC;
            const int f = f0 + c;
            const float g = wave_order_sum<NFH>(red0, row, c), u = wave_order_sum<NFH>(red1, row, c);
            if (wk.nseg > 1) {
                store_tagged(pp + (16 * m + row) * 2 * NC + c, tag, __float_as_uint(g));
                store_tagged(pp + (16 * m + row) * 2 * NC + NC + c, tag, __float_as_uint(u));
            } else if (f < a.F) {
                a.act[(size_t)(slot0 + 16 * m + row) * a.F + f] = silu_mul(g, u);
            }
        }
    }
    if (wk.nseg == 1 || !st_last(a.seg_ctr + wk.li, wk.nseg, &sh_last)) return;
    const uint64_t *p0 = a.part + (size_t)wk.li * wk.nseg * PSZ;
    constexpr int NC4 = NC / 4;
    for (int i = threadIdx.x; i < 16 * MF * NC4; i += ST_THREADS) {
        const int row = i / NC4, c = 4 * (i - row * NC4);
        if (row >= n) continue;
        const int o[2] = {row * 2 * NC + c, row * 2 * NC + NC + c};
        float gu[2][4];
        if (!st_seg_sum<PSZ, 2>(p0, o, wk.nseg, tag, a.wait_ticks, gu)) atomicOr(a.err, 8u);
        float *dst = a.act + (size_t)(slot0 + row) * a.F + f0 + c;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (f0 + c + j < a.F) dst[j] = silu_mul(gu[0][j], gu[1][j]);
    }
    st_item_done(a.seg_gen, wk.L, tag);
}

// ---------------------------------------------------------------------------
// down: 128 output columns h0 .. h0+127 (halves h0 and h0 + 64).
// ---------------------------------------------------------------------------
template <int MF>
__global__ __launch_bounds__(ST_THREADS, 2) void moe_stream_down_kernel(StreamArgs a)
{
    constexpr int NFH = 4;
    __shared__ __align__(16) char lds[st_lds<NFH>()];
    __shared__ int sh_last;
    const int ncg = (a.H + 127) / 128;
    StWork wk;
    if (!st_work(min(*a.n_tiles, a.tile_cap) * ncg, a.G, a.nbF, ncg, 16 * MF, a.tile_m0, wk)) return;
    const int tile = wk.item / ncg, cg = wk.item - tile * ncg;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(16 * MF, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int h0 = cg * 128;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;

    StSrc<MF, NFH> src;
    src.abase = reinterpret_cast<const char *>(a.act);
    const size_t eb = (size_t)e * a.nbF * a.H;
    src.qb[0] = src.qb[1] = a.dq + eb * QK;
    src.db[0] = src.db[1] = a.dd + eb;
    src.qstep = (uint32_t)a.H * QK;
    src.dstep = (uint32_t)a.H;
    const int c0[2] = {h0, h0 + 64};
    st_offsets<MF, NFH>(src, [&](int r) { return (uint32_t)(slot0 + min(r, n - 1)) * a.F * 4; }, c0,
                        a.H, lane);

    f4_t acc[MF][2 * NFH];
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
        for (int j = 0; j < 2 * NFH; j++) acc[m][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int kb0 = wk.nseg > 1 ? wk.seg * a.nbF / wk.nseg : 0;
    const int kb1 = wk.nseg > 1 ? (wk.seg + 1) * a.nbF / wk.nseg : a.nbF;
    const uint32_t tag =
        wk.nseg > 1 ? __hip_atomic_load(a.seg_gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u : 0u;
    st_mainloop<MF, NFH>(src, kb0, kb1 - kb0, wave, acc);
    float (*red0)[16][65] = reinterpret_cast<float (*)[16][65]>(lds);
    float (*red1)[16][65] = red0 + 4;
    // split item: partial [16 MF rows][128 columns] of each segment
    constexpr int PSZ = 16 * MF * 128;
    uint64_t *pp = a.part + (size_t)(wk.li * wk.nseg + wk.seg) * PSZ;
#pragma unroll
    for (int m = 0; m < MF; m++) {
        __syncthreads();
        st_spill<MF, NFH>(red0, red1, acc, m, wave, lane);
        __syncthreads();
        // the tile's rows only (a split item's last segment reads those alone)
        const int nr = min(16, n - 16 * m);
        for (int i = threadIdx.x; i < nr * 128; i += ST_THREADS) {
            const int row = i >> 7, c = i & 127;
            const int h = h0 + c;
            const float v = wave_order_sum<NFH>(c < 64 ? red0 : red1, row, c & 63);
            if (wk.nseg > 1)
                store_tagged(pp + (16 * m + row) * 128 + c, tag, __float_as_uint(v));
            else if (h < a.H)
                a.y[(size_t)(slot0 + 16 * m + row) * a.H + h] = v;
        }
    }
    if (wk.nseg == 1 || !st_last(a.seg_ctr + wk.li, wk.nseg, &sh_last)) return;
    const uint64_t *p0 = a.part + (size_t)wk.li * wk.nseg * PSZ;
    for (int i = threadIdx.x; i < 16 * MF * 32; i += ST_THREADS) {
        const int row = i >> 5, c = 4 * (i & 31);
        if (row >= n) continue;
        const int o[1] = {row * 128 + c};
        float v[1][4];
        if (!st_seg_sum<PSZ, 1>(p0, o, wk.nseg, tag, a.wait_ticks, v)) atomicOr(a.err, 8u);
        float *dst = a.y + (size_t)(slot0 + row) * a.H + h0 + c;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (h0 + c + j < a.H) dst[j] = v[0][j];
    }
    st_item_done(a.seg_gen, wk.L, tag);
}

// ---------------------------------------------------------------------------

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

// slots per tile: 16 for groups of up to ~16 rows on average, else 32
static int stream_mf(const qq_moe *m, int T) { return (size_t)T * m->K <= (size_t)16 * m->E ? 1 : 2; }

static int stream_cap(const qq_moe *m, int T, int bm) { return T * m->K / bm + m->E; }

size_t stream_work_bytes(const qq_moe *m, int T)
{
    const size_t P = (size_t)T * m->K;
    const size_t cap = (size_t)stream_cap(m, T, 16);
    return al256((size_t)m->E * 4) + al256((size_t)(m->E + 1) * 4) + 2 * al256(P * 4) +
           2 * al256(cap * 4) + 256 + al256(P * m->F * 4) + al256(P * m->H * 4);
}

// work: counts | offsets | perm | inv | tile e | tile m0 | tile count | act | y
StreamDispatch stream_dispatch(const qq_moe *m, int T, char *work)
{
    const size_t P = (size_t)T * m->K;
    StreamDispatch d;
    char *p = work;
    d.counts = reinterpret_cast<int32_t *>(p);  p += al256((size_t)m->E * 4);
    d.offsets = reinterpret_cast<int32_t *>(p); p += al256((size_t)(m->E + 1) * 4);
    d.perm = reinterpret_cast<int32_t *>(p);    p += al256(P * 4);
    d.inv = reinterpret_cast<int32_t *>(p);     p += al256(P * 4);
    d.tiles.bm = 16 * stream_mf(m, T);
    d.tiles.cap = stream_cap(m, T, d.tiles.bm);
    d.tiles.e = reinterpret_cast<int32_t *>(p); p += al256((size_t)stream_cap(m, T, 16) * 4);
    d.tiles.m0 = reinterpret_cast<int32_t *>(p);
    p += al256((size_t)stream_cap(m, T, 16) * 4);
    d.tiles.n = reinterpret_cast<int32_t *>(p);
    return d;
}

// Gate/up features per column half of a workgroup, 16 NFH.  Each workgroup
// keeps a fixed number of blocks in flight, so a kernel whose items fill the
// resident slots (2 per CU) only partly in its last round streams that round
// at a fraction of the rate.  The wider items are taken where they need
// fewer item-rounds x width, counting the row tiles of even routing
// (ceil(T K / 16 / E) per expert, clipped to T K / 16 + E).
static int stream_gateup_nfh(const qq_ctx *ctx, const qq_moe *m, int T)
{
    if (stream_mf(m, T) != 1) return 4;
    const long slots = 2L * ctx->num_cus;
    const long per_e = ((long)T * m->K + 16L * m->E - 1) / (16L * m->E);
    const long tiles = std::min((long)stream_cap(m, T, 16), per_e * m->E);
    long best = 0, best_cost = 0;
    for (const int nfh : {4, 7}) {
        const long items = tiles * ((m->F + 16 * nfh - 1) / (16 * nfh));
        const long cost = ((items + slots - 1) / slots) * nfh;
        if (!best || cost < best_cost) {
            best = nfh;
            best_cost = cost;
        }
    }
    return (int)best;
}

int launch_moe_stream(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                      const MaskBits &mask, const int32_t *idx, const double *w, char *work,
                      bool dispatched)
{
    const size_t P = (size_t)T * m->K;
    const int MF = stream_mf(m, T);
    const StreamDispatch d = stream_dispatch(m, T, work);
    const int cap = d.tiles.cap;
    int32_t *counts = d.counts, *offsets = d.offsets, *perm = d.perm, *inv = d.inv;
    const DispatchTiles &tiles = d.tiles;
    char *p = work + al256((size_t)m->E * 4) + al256((size_t)(m->E + 1) * 4) + 2 * al256(P * 4) +
              2 * al256((size_t)stream_cap(m, T, 16) * 4) + 256;
    float *act = reinterpret_cast<float *>(p);         p += al256(P * m->F * 4);
    float *y = reinterpret_cast<float *>(p);

    if (!dispatched) {
        const int rc = launch_dispatch(ctx, m, idx, (int)P, mask, counts, offsets, perm, inv, tiles);
        if (rc) return rc;
    }

    StreamArgs a;
    a.x = x;
    a.act = act;
    a.y = y;
    a.perm = perm;
    a.counts = counts;
    a.offsets = offsets;
    a.tile_e = tiles.e;
    a.tile_m0 = tiles.m0;
    a.n_tiles = tiles.n;
    a.gq = m->gate->qs;
    a.uq = m->up->qs;
    a.dq = m->down->qs;
    a.gd = reinterpret_cast<const uint16_t *>(m->gate->d);
    a.ud = reinterpret_cast<const uint16_t *>(m->up->d);
    a.dd = reinterpret_cast<const uint16_t *>(m->down->d);
    a.H = m->H;
    a.F = m->F;
    a.K = m->K;
    a.nbH = m->H / QK;
    a.nbF = m->F / QK;
    a.part = ctx->seg_part;
    a.seg_ctr = ctx->sync_seg;
    a.seg_gen = ctx->sync_seg + SEG_CTR_WORDS / 4;
    a.err = ctx->sync_err;
    a.wait_ticks = ctx->dec_wait_ticks;
    a.G = 2 * ctx->num_cus;
    a.tile_cap = cap;

    // a split item's partial sums: [16 MF rows][2 x 16 NFH or 128 columns]
    if (16 * MF * std::max(2 * 16 * stream_gateup_nfh(ctx, m, T), 128) > SEG_PART_WORDS)
        return set_error(ctx, "stream path: partial sums exceed %d words", SEG_PART_WORDS);

    // grids (st_work): 8 * ceil(items / 8) workgroups for the items of cap
    // row tiles; split items' segments take the room past the items there are
    const int nfh = stream_gateup_nfh(ctx, m, T);
    const unsigned g1 = 8u * (unsigned)(((size_t)cap * ((m->F + 16 * nfh - 1) / (16 * nfh)) + 7) / 8);
    const unsigned g2 = 8u * (unsigned)(((size_t)cap * ((m->H + 127) / 128) + 7) / 8);
    prof_begin(ctx, K_STREAM_GATEUP);
    if (MF == 1 && nfh == 7)
        QQ_LAUNCH(ctx, (moe_stream_gateup_kernel<1, 7>), dim3(g1), dim3(ST_THREADS), 0, a);
    else if (MF == 1)
        QQ_LAUNCH(ctx, (moe_stream_gateup_kernel<1, 4>), dim3(g1), dim3(ST_THREADS), 0, a);
    else
        QQ_LAUNCH(ctx, (moe_stream_gateup_kernel<2, 4>), dim3(g1), dim3(ST_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    prof_begin(ctx, K_STREAM_DOWN);
    a.seg_ctr = ctx->sync_seg + SEG_CTR_WORDS / 2;
    a.seg_gen = ctx->sync_seg + 3 * SEG_CTR_WORDS / 4;
    if (MF == 1)
        QQ_LAUNCH(ctx, moe_stream_down_kernel<1>, dim3(g2), dim3(ST_THREADS), 0, a);
    else
        QQ_LAUNCH(ctx, moe_stream_down_kernel<2>, dim3(g2), dim3(ST_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return launch_combine(ctx, m, T, y, false, inv, w, hidden);
}

}  // namespace qq
