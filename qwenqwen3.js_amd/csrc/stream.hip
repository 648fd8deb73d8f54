// stream.hip -- decode batches (a few to a few dozen tokens per expert) on
// the matrix cores at fp32 accuracy.
//
// With ~8 rows per expert (64 tokens, 32 experts, top-4) every weight is used
// by very few rows, so the layer is bound by streaming the experts' Q8_0
// weights from HBM once.  Weights go straight from HBM into registers (no
// LDS): a workgroup owns one expert, one tile of 16*MF slots and a group of
// 128 weight columns; its 4 waves split the reduction dimension block by
// block and their partial sums are added in wave order through LDS.
//
// Accuracy (the fp32 path's 1e-4 relative L2): every operand is split into
// two fp16 halves, a = a_hi + a_lo, w = w_hi + w_lo, and each 16x16x32 tile
// takes three MFMAs, a_hi*w_hi + a_hi*w_lo + a_lo*w_hi, with fp32
// accumulation.  w = q * d needs 19 significant bits; w_hi = fp16(q*d) and
// w_lo = fp16(q*d - w_hi) (one fused multiply-add) hold it exactly unless
// w_lo falls below the fp16 normal range.  The dropped a_lo*w_lo term and the
// fp16 rounding of the low halves are ~2^-22 relative, so the products are
// accurate to ~1e-7 like the fp32 kernels.
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
constexpr int ST_NF = 8;          // 16-column fragments per workgroup (128 columns)

struct StreamArgs {
    const float *x;          // [T][H] activations
    float *act;              // [slots][F] SwiGLU products
    float *y;                // [slots][H] expert outputs
    const int32_t *perm, *counts, *offsets;
    const int32_t *tile_e, *tile_m0, *n_tiles;
    const int8_t *gq, *uq, *dq;
    const uint16_t *gd, *ud, *dd;   // fp16 scale bits
    int H, F, K, nbH, nbF;
};

// 8 consecutive fp32 values -> high and low fp16 halves (v - hi is exact in
// fp32; its fp16 rounding is the split's only loss).
__device__ __forceinline__ void split8(const float4 a, const float4 b, h8_t &hi, h8_t &lo)
{
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const _Float16 h = (_Float16)v[i];
        hi[i] = h;
        lo[i] = (_Float16)(v[i] - (float)h);
    }
}

// 8 int8 weights (one lane's share of a 16x32 fragment) and their fp16 scale
// -> w_hi = fp16(q*d), w_lo = fp16(q*d - w_hi).  Bytes are made offset binary
// and paired with the exponent byte 0x64 (half 0x64uu = 1024 + u), so
// subtracting 1152 gives q exactly in fp16.
__device__ __forceinline__ void dequant8_split(const uint2 q, const _Float16 d, h8_t &hi, h8_t &lo)
{
    const uint32_t w[2] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u};
    const h2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2_t dd = {d, d};
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u);
        const h2_t q0 = __builtin_bit_cast(h2_t, p0) + off;
        const h2_t q1 = __builtin_bit_cast(h2_t, p1) + off;
        const h2_t h0 = q0 * dd, h1 = q1 * dd;
        const h2_t l0 = __builtin_elementwise_fma(q0, dd, -h0);
        const h2_t l1 = __builtin_elementwise_fma(q1, dd, -h1);
        hi[4 * i] = h0[0];
        hi[4 * i + 1] = h0[1];
        hi[4 * i + 2] = h1[0];
        hi[4 * i + 3] = h1[1];
        lo[4 * i] = l0[0];
        lo[4 * i + 1] = l0[1];
        lo[4 * i + 2] = l1[0];
        lo[4 * i + 3] = l1[1];
    }
}

// One reduction block (32 values) of a wave's operands.
template <int MF>
struct StBlk {
    float4 a[MF][2];         // A: row lane%16 (+16 m), k = 8*(lane/16) .. +7
    uint2 q[ST_NF];          // B: column lane%16 of fragment j, same k
    uint16_t s[ST_NF];       // B scales
};

// Where fragment j's 16 columns come from: matrix pointer and column index.
struct ColSrc {
    const int8_t *q;
    const uint16_t *d;
    int col;                 // clamped into range
    bool ok;
};

template <int MF>
__device__ __forceinline__ void st_load(StBlk<MF> &b, const float *const (&arow)[MF], int kb, int e,
                                        int nb, int rows, const ColSrc (&src)[ST_NF], int lane)
{
    const int ko = kb * QK + 8 * (lane >> 4);
#pragma unroll
    for (int m = 0; m < MF; m++) {
        b.a[m][0] = *reinterpret_cast<const float4 *>(arow[m] + ko);
        b.a[m][1] = *reinterpret_cast<const float4 *>(arow[m] + ko + 4);
    }
#pragma unroll
    for (int j = 0; j < ST_NF; j++) {
        const size_t o = bm_index(e, nb, kb, rows, src[j].col);
        b.q[j] = *reinterpret_cast<const uint2 *>(src[j].q + o * QK + 8 * (lane >> 4));
        b.s[j] = src[j].d[o];
    }
}

template <int MF>
__device__ __forceinline__ void st_compute(const StBlk<MF> &b, const ColSrc (&src)[ST_NF],
                                           f4_t (&acc)[MF][ST_NF])
{
    h8_t ah[MF], al[MF];
#pragma unroll
    for (int m = 0; m < MF; m++) split8(b.a[m][0], b.a[m][1], ah[m], al[m]);
#pragma unroll
    for (int j = 0; j < ST_NF; j++) {
        h8_t wh, wl;
        const _Float16 d = src[j].ok ? __builtin_bit_cast(_Float16, b.s[j]) : (_Float16)0.0f;
        dequant8_split(b.q[j], d, wh, wl);
#pragma unroll
        for (int m = 0; m < MF; m++) {
            acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[m], wh, acc[m][j], 0, 0, 0);
            acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[m], wl, acc[m][j], 0, 0, 0);
            acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[m], wh, acc[m][j], 0, 0, 0);
        }
    }
}

// Wave w reduces blocks w, w+4, w+8, ... of nb; two blocks are in flight
// while one is multiplied.  Loads are branch-free (clamped block index).
template <int MF>
__device__ __forceinline__ void st_mainloop(const float *const (&arow)[MF], int e, int nb, int rows,
                                            const ColSrc (&src)[ST_NF], int wave, int lane,
                                            f4_t (&acc)[MF][ST_NF])
{
    const int last = nb - 1;
    StBlk<MF> b0, b1;
    st_load<MF>(b0, arow, min(wave, last), e, nb, rows, src, lane);
    st_load<MF>(b1, arow, min(wave + 4, last), e, nb, rows, src, lane);
    for (int kb = wave; kb < nb; kb += 8) {
        StBlk<MF> n0, n1;
        st_load<MF>(n0, arow, min(kb + 8, last), e, nb, rows, src, lane);
        st_compute<MF>(b0, src, acc);
        st_load<MF>(n1, arow, min(kb + 12, last), e, nb, rows, src, lane);
        if (kb + 4 < nb) st_compute<MF>(b1, src, acc);
        b0 = n0;
        b1 = n1;
    }
}

// Partial sums of the 4 waves -> red[wave][row][col] (fp32).
template <int MF>
__device__ __forceinline__ void st_spill(float (*red)[16 * MF][16 * ST_NF + 1],
                                         const f4_t (&acc)[MF][ST_NF], int wave, int lane)
{
    const int cl = lane & 15, rq = 4 * (lane >> 4);
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
        for (int j = 0; j < ST_NF; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[wave][16 * m + rq + r][16 * j + cl] = acc[m][j][r];
}

// ---------------------------------------------------------------------------
// gate/up: columns 0..63 of the workgroup are gate features f0 .. f0+63,
// 64..127 the same up features.
// ---------------------------------------------------------------------------
template <int MF>
__global__ __launch_bounds__(ST_THREADS) void moe_stream_gateup_kernel(StreamArgs a)
{
    __shared__ float red[4][16 * MF][16 * ST_NF + 1];
    const int ncg = (a.F + 63) / 64;
    const int tile = blockIdx.x / ncg, cg = blockIdx.x - tile * ncg;
    if (tile >= *a.n_tiles) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(16 * MF, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int f0 = cg * 64;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;

    const float *arow[MF];
#pragma unroll
    for (int m = 0; m < MF; m++) {
        const int r = min(16 * m + (lane & 15), n - 1);
        arow[m] = a.x + (size_t)(a.perm[slot0 + r] / a.K) * a.H;
    }
    ColSrc src[ST_NF];
#pragma unroll
    for (int j = 0; j < ST_NF; j++) {
        const int f = f0 + 16 * (j & 3) + (lane & 15);
        src[j].q = j < 4 ? a.gq : a.uq;
        src[j].d = j < 4 ? a.gd : a.ud;
        src[j].col = min(f, a.F - 1);
        src[j].ok = f < a.F;
    }
    f4_t acc[MF][ST_NF];
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
        for (int j = 0; j < ST_NF; j++) acc[m][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    st_mainloop<MF>(arow, e, a.nbH, a.F, src, wave, lane, acc);
    st_spill<MF>(red, acc, wave, lane);
    __syncthreads();
    for (int i = threadIdx.x; i < 16 * MF * 64; i += ST_THREADS) {
        const int row = i >> 6, c = i & 63;
        const int f = f0 + c;
        if (row < n && f < a.F) {
            const float g = ((red[0][row][c] + red[1][row][c]) + red[2][row][c]) + red[3][row][c];
            const float u = ((red[0][row][64 + c] + red[1][row][64 + c]) + red[2][row][64 + c]) +
                            red[3][row][64 + c];
            const double g64 = (double)g;
            const float sg = (float)(g64 * (1.0 / (1.0 + exp(-g64))));
            a.act[(size_t)(slot0 + row) * a.F + f] = sg * u;
        }
    }
}

// ---------------------------------------------------------------------------
// down: 128 output columns h0 .. h0+127.
// ---------------------------------------------------------------------------
template <int MF>
__global__ __launch_bounds__(ST_THREADS) void moe_stream_down_kernel(StreamArgs a)
{
    __shared__ float red[4][16 * MF][16 * ST_NF + 1];
    const int ncg = (a.H + 127) / 128;
    const int tile = blockIdx.x / ncg, cg = blockIdx.x - tile * ncg;
    if (tile >= *a.n_tiles) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(16 * MF, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int h0 = cg * 128;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;

    const float *arow[MF];
#pragma unroll
    for (int m = 0; m < MF; m++)
        arow[m] = a.act + (size_t)(slot0 + min(16 * m + (lane & 15), n - 1)) * a.F;
    ColSrc src[ST_NF];
#pragma unroll
    for (int j = 0; j < ST_NF; j++) {
        const int h = h0 + 16 * j + (lane & 15);
        src[j].q = a.dq;
        src[j].d = a.dd;
        src[j].col = min(h, a.H - 1);
        src[j].ok = h < a.H;
    }
    f4_t acc[MF][ST_NF];
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
        for (int j = 0; j < ST_NF; j++) acc[m][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    st_mainloop<MF>(arow, e, a.nbF, a.H, src, wave, lane, acc);
    st_spill<MF>(red, acc, wave, lane);
    __syncthreads();
    for (int i = threadIdx.x; i < 16 * MF * 128; i += ST_THREADS) {
        const int row = i >> 7, c = i & 127;
        const int h = h0 + c;
        if (row < n && h < a.H)
            a.y[(size_t)(slot0 + row) * a.H + h] =
                ((red[0][row][c] + red[1][row][c]) + red[2][row][c]) + red[3][row][c];
    }
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

int launch_moe_stream(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                      const MaskBits &mask, const int32_t *idx, const double *w, char *work)
{
    const size_t P = (size_t)T * m->K;
    const int MF = stream_mf(m, T);
    const int cap = stream_cap(m, T, 16 * MF);
    char *p = work;
    int32_t *counts = reinterpret_cast<int32_t *>(p);  p += al256((size_t)m->E * 4);
    int32_t *offsets = reinterpret_cast<int32_t *>(p); p += al256((size_t)(m->E + 1) * 4);
    int32_t *perm = reinterpret_cast<int32_t *>(p);    p += al256(P * 4);
    int32_t *inv = reinterpret_cast<int32_t *>(p);     p += al256(P * 4);
    DispatchTiles tiles;
    tiles.bm = 16 * MF;
    tiles.cap = cap;
    tiles.e = reinterpret_cast<int32_t *>(p);          p += al256((size_t)stream_cap(m, T, 16) * 4);
    tiles.m0 = reinterpret_cast<int32_t *>(p);         p += al256((size_t)stream_cap(m, T, 16) * 4);
    tiles.n = reinterpret_cast<int32_t *>(p);          p += 256;
    float *act = reinterpret_cast<float *>(p);         p += al256(P * m->F * 4);
    float *y = reinterpret_cast<float *>(p);

    int rc = launch_dispatch(ctx, m, idx, (int)P, mask, counts, offsets, perm, inv, tiles);
    if (rc) return rc;

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

    const unsigned g1 = (unsigned)cap * ((m->F + 63) / 64);
    const unsigned g2 = (unsigned)cap * ((m->H + 127) / 128);
    prof_begin(ctx, K_STREAM_GATEUP);
    if (MF == 1)
        QQ_LAUNCH(ctx, moe_stream_gateup_kernel<1>, dim3(g1), dim3(ST_THREADS), 0, a);
    else
        QQ_LAUNCH(ctx, moe_stream_gateup_kernel<2>, dim3(g1), dim3(ST_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    prof_begin(ctx, K_STREAM_DOWN);
    if (MF == 1)
        QQ_LAUNCH(ctx, moe_stream_down_kernel<1>, dim3(g2), dim3(ST_THREADS), 0, a);
    else
        QQ_LAUNCH(ctx, moe_stream_down_kernel<2>, dim3(g2), dim3(ST_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return launch_combine(ctx, m, T, y, inv, w, hidden);
}

}  // namespace qq
