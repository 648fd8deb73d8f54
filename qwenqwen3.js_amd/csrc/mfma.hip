// mfma.hip -- prefill chunks on the matrix cores: grouped fp16 MFMA GEMMs.
//
// For a chunk of prompt tokens the (token, rank) pairs routed to one expert
// form a dense [n_e x H] x [H x F] contraction (the reference runs them as
// n_e separate matvecs, src/lfm2-engine.js:471-478 per token).  After the
// dispatch (grouped.hip) every expert's slots are cut into row tiles of
// MF_BM slots, and per (row tile, column tile):
//   gate/up  A = fp16 activations of the tile's tokens (gathered by perm),
//            B = 64 gate + 64 up columns dequantised from Q8_0 into LDS as
//            fp16 w = fp16(q * d); v_mfma_f32_16x16x32_f16 with fp32
//            accumulators; epilogue silu(g) * u -> fp16 act[slot][F]
//   down     A = act rows of the tile, B = 128 down columns dequantised
//            likewise -> y[slot][H] fp16
// followed by the gather combine of the fp32 path (rank order, fp32 steps).
// One Q8_0 block (32 values of the reduction dimension) is one MFMA K step;
// the next block's global loads are in flight while the current block's
// MFMAs run, and LDS is double buffered with one barrier per step.
//
// Accuracy: fp16 activations, weights and expert outputs (relative rounding
// 2^-11 each), fp32 accumulation: ~1e-3 relative L2 on the layer output,
// inside the 1e-2 bound of the MFMA path.  SwiGLU products, weights and
// expert outputs must stay inside the fp16 range (|v| < 65504); beyond it
// they become inf and show in the output.
#include "qq_device.h"

namespace qq {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int MF_BM = 128;       // slots per row tile
constexpr int MF_BN = 128;       // weight columns per workgroup
constexpr int MF_THREADS = 256;  // 4 waves, 2 x 2 over the 128 x 128 tile

struct MfmaArgs {
    const _Float16 *xh;      // [T][H] activations in fp16
    _Float16 *act;           // [slots][F] SwiGLU products (down input)
    _Float16 *y;             // [slots][H] expert outputs (fp16)
    const int32_t *perm, *counts, *offsets;
    const int32_t *tile_e, *tile_m0, *n_tiles;
    const int8_t *gq, *uq, *dq;
    const uint16_t *gd, *ud, *dd;   // fp16 scale bits
    int H, F, K, nbH, nbF;
};

// x fp32 -> fp16 (round to nearest even), 4 values per thread.
__global__ __launch_bounds__(256) void cast_f16_kernel(const float4 *__restrict__ x,
                                                       uint2 *__restrict__ y, size_t n4)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 v = x[i];
    const h2_t a = {(_Float16)v.x, (_Float16)v.y};
    const h2_t b = {(_Float16)v.z, (_Float16)v.w};
    y[i] = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

// 16 int8 weights of one column (half a Q8_0 block) and the block's fp16
// scale -> 16 fp16 values w = fp16(q * d), in k order.  Each byte is made
// offset binary (u = q + 128) and paired with the exponent byte 0x64, so the
// half 0x64uu is exactly 1024 + u; subtracting 1152 gives q exactly, and the
// multiply by d is the one rounding.
__device__ __forceinline__ void dequant16(const uint4 q, const _Float16 d, uint4 &lo, uint4 &hi)
{
    const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u,
                           q.w ^ 0x80808080u};
    const h2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2_t dd = {d, d};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // bytes {b0, 0x64, b1, 0x64} and {b2, 0x64, b3, 0x64}
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u);
        const h2_t a = (__builtin_bit_cast(h2_t, p0) + off) * dd;
        const h2_t b = (__builtin_bit_cast(h2_t, p1) + off) * dd;
        o[2 * i] = __builtin_bit_cast(uint32_t, a);
        o[2 * i + 1] = __builtin_bit_cast(uint32_t, b);
    }
    lo = make_uint4(o[0], o[1], o[2], o[3]);
    hi = make_uint4(o[4], o[5], o[6], o[7]);
}

__device__ __forceinline__ _Float16 half_bits(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// LDS tile of one operand and stage: 128 rows x KB Q8_0 blocks (32*KB halves,
// 4*KB chunks of 16 bytes).  Chunk c of row r sits at r*64*KB + 16*(c ^ s(r)).
// For KB = 1, s(r) = ((r >> 1) ^ (r >> 2)) & 3: any 8 consecutive rows of a
// fragment read (same chunk) fall in 8 different 16-byte groups of a 128-byte
// bank row and any 16 in 16 different groups of a 256-byte one; so do the
// staging writes.  For KB = 2, s(r) = (r >> 1) & 7.
template <int KB>
struct MfTile {
    static constexpr int BYTES = MF_BM * 64 * KB;
    static __device__ __forceinline__ int off(int r, int c)
    {
        return r * 64 * KB + 16 * (c ^ (KB == 1 ? (((r >> 1) ^ (r >> 2)) & 3) : ((r >> 1) & 7)));
    }
};

// Per-thread staging sources: 32 bytes (16 halves) of one A row and 16 int8 of
// one B column per Q8_0 block, advanced by a fixed stride per block.
struct MfSrc {
    const char *a;           // A row, this thread's half of block 0
    const int8_t *q;         // B column, this thread's half of block 0
    const uint16_t *d;       // the column's scale at block 0
    size_t qstep, dstep;     // one block of the B matrix (rows * 32 bytes, rows halves)
    bool ok;                 // B column in range (else zero scale)
};

// Shared main loop of the two GEMMs over nb blocks (nb % KB == 0).  Stage = A
// tile + B tile (fp16) of KB blocks; two stages double buffered; the next
// stage's global loads are in flight while this stage's MFMAs run; one
// barrier per stage.  Wave fragments: A rows arow[i], B columns bcol[j] (row
// bases of 16-row fragments within the tile).
template <int KB>
__device__ __forceinline__ void mf_mainloop(const MfSrc &src, int nb, char *lds, int sr, int sh,
                                            const int (&arow)[4], const int (&bcol)[4],
                                            f4_t (&acc)[4][4])
{
    using T = MfTile<KB>;
    const int lane = threadIdx.x & (WAVE - 1);
    // staging offsets: block b of this thread's row sr, chunks 4b + 2sh, +1
    int w0[KB], w1[KB];
#pragma unroll
    for (int b = 0; b < KB; b++) {
        w0[b] = T::off(sr, 4 * b + 2 * sh);
        w1[b] = T::off(sr, 4 * b + 2 * sh + 1);
    }
    // fragment offsets: row base + lane%16, chunk 4b + lane/16
    int ao[KB][4], bo[KB][4];
#pragma unroll
    for (int b = 0; b < KB; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            ao[b][i] = T::off(arow[i] + (lane & 15), 4 * b + (lane >> 4));
            bo[b][i] = T::BYTES + T::off(bcol[i] + (lane & 15), 4 * b + (lane >> 4));
        }

    const char *ap = src.a;
    const int8_t *qp = src.q;
    const uint16_t *dp = src.d;
    uint4 xa[KB], xb[KB], wv[KB];
    uint16_t ws[KB];
    auto load = [&]() {
#pragma unroll
        for (int b = 0; b < KB; b++) {
            xa[b] = *reinterpret_cast<const uint4 *>(ap + b * QK * 2);
            xb[b] = *reinterpret_cast<const uint4 *>(ap + b * QK * 2 + 16);
            wv[b] = *reinterpret_cast<const uint4 *>(qp + b * src.qstep);
            ws[b] = dp[b * src.dstep];
        }
        ap += KB * QK * 2;
        qp += KB * src.qstep;
        dp += KB * src.dstep;
    };
    auto store = [&](char *st) {
#pragma unroll
        for (int b = 0; b < KB; b++) {
            *reinterpret_cast<uint4 *>(st + w0[b]) = xa[b];
            *reinterpret_cast<uint4 *>(st + w1[b]) = xb[b];
            uint4 lo, hi;
            dequant16(wv[b], src.ok ? half_bits(ws[b]) : (_Float16)0.0f, lo, hi);
            *reinterpret_cast<uint4 *>(st + T::BYTES + w0[b]) = lo;
            *reinterpret_cast<uint4 *>(st + T::BYTES + w1[b]) = hi;
        }
    };
    auto compute = [&](const char *st) {
#pragma unroll
        for (int b = 0; b < KB; b++) {
            h8_t af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = *reinterpret_cast<const h8_t *>(st + ao[b][i]);
#pragma unroll
            for (int j = 0; j < 4; j++) bf[j] = *reinterpret_cast<const h8_t *>(st + bo[b][j]);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    const int nst = nb / KB;
    load();
    store(lds);
    __syncthreads();
    for (int k = 0; k < nst; k++) {
        char *cur = lds + (k & 1) * 2 * T::BYTES;
        char *nxt = lds + ((k + 1) & 1) * 2 * T::BYTES;
        const bool more = k + 1 < nst;
        if (more) load();
        compute(cur);
        if (more) store(nxt);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// gate/up: tile = MF_BM slots x 64 features (64 gate + 64 up columns).
// Wave (wm, wn): slots wm*64 .. +64, features wn*32 .. +32 -> 4 x (2 gate +
// 2 up) fragments of 16 x 16.
// ---------------------------------------------------------------------------
template <int KB>
__global__ __launch_bounds__(MF_THREADS, 4) void moe_mfma_gateup_kernel(MfmaArgs a)
{
    __shared__ __align__(16) char lds[4 * MfTile<KB>::BYTES];
    __shared__ int rowtok[MF_BM];

    const int nft = (a.F + 63) / 64;
    const int tile = blockIdx.x / nft, ft = blockIdx.x - tile * nft;
    if (tile >= *a.n_tiles) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(MF_BM, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int f0 = ft * 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    if (tid < MF_BM) rowtok[tid] = a.perm[slot0 + min(tid, n - 1)] / a.K;
    __syncthreads();

    // staging: thread -> row / column tid/2, 16-value half tid&1
    const int sr = tid >> 1, sh = tid & 1;
    const int f = f0 + (sr & 63);
    const int fc = min(f, a.F - 1);
    MfSrc src;
    src.a = reinterpret_cast<const char *>(a.xh + (size_t)rowtok[sr] * a.H) + sh * 32;
    const size_t o = bm_index(e, a.nbH, 0, a.F, fc);
    src.q = (sr < 64 ? a.gq : a.uq) + o * QK + sh * 16;
    src.d = (sr < 64 ? a.gd : a.ud) + o;
    src.qstep = (size_t)a.F * QK;
    src.dstep = (size_t)a.F;
    src.ok = f < a.F;

    const int arow[4] = {wm * 64, wm * 64 + 16, wm * 64 + 32, wm * 64 + 48};
    const int bcol[4] = {wn * 32, wn * 32 + 16, 64 + wn * 32, 64 + wn * 32 + 16};
    f4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    mf_mainloop<KB>(src, a.nbH, lds, sr, sh, arow, bcol, acc);

    // lane holds rows 4*(lane/16) + r, column lane % 16 of each fragment
    const int cl = lane & 15, rq = 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int ff = f0 + wn * 32 + j * 16 + cl;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = wm * 64 + i * 16 + rq + r;
                if (row < n && ff < a.F) {
                    const float g = acc[i][j][r], u = acc[i][j + 2][r];
                    // hardware exp and reciprocal (~1 ulp each), far inside the fp16 rounding
                    const float v = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                    a.act[(size_t)(slot0 + row) * a.F + ff] = (_Float16)v;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// down: tile = MF_BM slots x 128 output columns; wave (wm, wn): slots
// wm*64 .. +64, columns wn*64 .. +64 -> 4 x 4 fragments.
// ---------------------------------------------------------------------------
template <int KB>
__global__ __launch_bounds__(MF_THREADS, 4) void moe_mfma_down_kernel(MfmaArgs a)
{
    __shared__ __align__(16) char lds[4 * MfTile<KB>::BYTES];

    const int nht = (a.H + MF_BN - 1) / MF_BN;
    const int tile = blockIdx.x / nht, ht = blockIdx.x - tile * nht;
    if (tile >= *a.n_tiles) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(MF_BM, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int h0 = ht * MF_BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    const int sr = tid >> 1, sh = tid & 1;
    const int h = h0 + sr;
    const int hc = min(h, a.H - 1);
    MfSrc src;
    src.a = reinterpret_cast<const char *>(a.act + (size_t)(slot0 + min(sr, n - 1)) * a.F) + sh * 32;
    const size_t o = bm_index(e, a.nbF, 0, a.H, hc);
    src.q = a.dq + o * QK + sh * 16;
    src.d = a.dd + o;
    src.qstep = (size_t)a.H * QK;
    src.dstep = (size_t)a.H;
    src.ok = h < a.H;

    const int arow[4] = {wm * 64, wm * 64 + 16, wm * 64 + 32, wm * 64 + 48};
    const int bcol[4] = {wn * 64, wn * 64 + 16, wn * 64 + 32, wn * 64 + 48};
    f4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    mf_mainloop<KB>(src, a.nbF, lds, sr, sh, arow, bcol, acc);

    const int cl = lane & 15, rq = 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int hh = h0 + wn * 64 + j * 16 + cl;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = wm * 64 + i * 16 + rq + r;
                if (row < n && hh < a.H) a.y[(size_t)(slot0 + row) * a.H + hh] = (_Float16)acc[i][j][r];
            }
        }
}

// ---------------------------------------------------------------------------

bool mfma_supported(const qq_moe *m) { return m->H % QK == 0 && m->F % QK == 0; }

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

static int tile_cap(const qq_moe *m, int T) { return T * m->K / MF_BM + m->E; }

size_t mfma_work_bytes(const qq_moe *m, int T)
{
    const size_t P = (size_t)T * m->K;
    const size_t cap = (size_t)tile_cap(m, T);
    return al256((size_t)m->E * 4) + al256((size_t)(m->E + 1) * 4) + 2 * al256(P * 4) +
           2 * al256(cap * 4) + 256 + al256((size_t)T * m->H * 2) + al256(P * m->F * 2) +
           al256(P * m->H * 2);
}

int launch_moe_mfma(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                    const MaskBits &mask, const int32_t *idx, const double *w, char *work)
{
    const size_t P = (size_t)T * m->K;
    const int cap = tile_cap(m, T);
    char *p = work;
    int32_t *counts = reinterpret_cast<int32_t *>(p);  p += al256((size_t)m->E * 4);
    int32_t *offsets = reinterpret_cast<int32_t *>(p); p += al256((size_t)(m->E + 1) * 4);
    int32_t *perm = reinterpret_cast<int32_t *>(p);    p += al256(P * 4);
    int32_t *inv = reinterpret_cast<int32_t *>(p);     p += al256(P * 4);
    DispatchTiles tiles;
    tiles.bm = MF_BM;
    tiles.cap = cap;
    tiles.e = reinterpret_cast<int32_t *>(p);          p += al256((size_t)cap * 4);
    tiles.m0 = reinterpret_cast<int32_t *>(p);         p += al256((size_t)cap * 4);
    tiles.n = reinterpret_cast<int32_t *>(p);          p += 256;
    _Float16 *xh = reinterpret_cast<_Float16 *>(p);    p += al256((size_t)T * m->H * 2);
    _Float16 *act = reinterpret_cast<_Float16 *>(p);   p += al256(P * m->F * 2);
    _Float16 *y = reinterpret_cast<_Float16 *>(p);

    int rc = launch_dispatch(ctx, m, idx, (int)P, mask, counts, offsets, perm, inv, tiles);
    if (rc) return rc;

    const size_t n4 = (size_t)T * m->H / 4;
    prof_begin(ctx, K_CAST_F16);
    QQ_LAUNCH(ctx, cast_f16_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
              reinterpret_cast<const float4 *>(x), reinterpret_cast<uint2 *>(xh), n4);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());

    MfmaArgs a;
    a.xh = xh;
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

    // one Q8_0 block per pipeline stage: two per stage halve the barriers but
    // double the LDS per workgroup, and the lost occupancy costs more
    const dim3 g1((unsigned)cap * ((m->F + 63) / 64)), g2((unsigned)cap * ((m->H + MF_BN - 1) / MF_BN));
    prof_begin(ctx, K_MFMA_GATEUP);
    QQ_LAUNCH(ctx, moe_mfma_gateup_kernel<1>, g1, dim3(MF_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    prof_begin(ctx, K_MFMA_DOWN);
    QQ_LAUNCH(ctx, moe_mfma_down_kernel<1>, g2, dim3(MF_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return launch_combine(ctx, m, T, y, true, inv, w, hidden);
}

}  // namespace qq
