// q8_0.hip -- one-time Q8_0 repack and the Q8_0 x fp32 matvec (matmulQ80xF32).
//
// Reference: matmulQ80xF32, src/tensor.js:26-53.  Block = {fp16 d, int8 qs[32]}
// (src/tensor.js:1-2); a GGUF [in_dim, out_dim] tensor stores column c as
// ceil(in_dim/32) consecutive blocks (src/tensor.js:4-5, 36).
//
// Device layout (block-major panels): for matrix m and block column b, the 32
// quants of every row r are contiguous, rows in order:
//   qs[((m*nb + b)*rows + r)*32 + i],   d[(m*nb + b)*rows + r]
// A wavefront load of 64 lanes x 16 bytes is then 32 rows x one block: 1 KiB
// contiguous, whichever rows a kernel owns.  The scales are also kept row by
// row, dcm[(m*rows + r)*nbp + b] (nbp = nb rounded up to 8, zero padded).
#include "qq_device.h"

namespace qq {

// ---------------------------------------------------------------------------
// Repack.  One thread per GGUF block; reads are consecutive 34-byte blocks.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void repack_q8_0_kernel(const uint8_t *__restrict__ src,
                                                          int8_t *__restrict__ qs,
                                                          __half *__restrict__ d,
                                                          __half *__restrict__ dcm, size_t nblocks,
                                                          int rows, int nb, int nbp)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(src + i * QBLK);  // 2-byte aligned
    const size_t col = i / nb;                  // m*rows + r (GGUF column)
    const int b = (int)(i - col * nb);
    const int m = (int)(col / rows);
    const int r = (int)(col - (size_t)m * rows);
    const size_t o = bm_index(m, nb, b, rows, r);
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = (uint32_t)s16[1 + 2 * j] | ((uint32_t)s16[2 + 2 * j] << 16);
    int4 *dst = reinterpret_cast<int4 *>(qs + o * QK);
    dst[0] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    dst[1] = make_int4((int)w[4], (int)w[5], (int)w[6], (int)w[7]);
    d[o] = __ushort_as_half(s16[0]);
    dcm[col * nbp + b] = __ushort_as_half(s16[0]);
}

int launch_repack_q8_0(qq_ctx *ctx, const uint8_t *gguf_dev, qq_tensor *t)
{
    const size_t nblocks = (size_t)t->n_mats * t->out_dim * t->nb;
    const unsigned grid = (unsigned)((nblocks + 255) / 256);
    prof_begin(ctx, K_REPACK);
    QQ_LAUNCH(ctx, repack_q8_0_kernel, dim3(grid), dim3(256), 0, gguf_dev,
                       t->qs, t->d, t->dcm, nblocks, t->out_dim, t->nb, t->nbp);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

// ---------------------------------------------------------------------------
// Matvec over R input vectors.  A workgroup (4 waves) owns 32 output rows; lane l of every wave
// takes row l/2 and half l%2 of a block, wave w takes block columns
// w, w+4, ...  The R input vectors sit in LDS (a window of up to MV_WIN
// blocks at a time) together with the sum of every 16-value half block.
// Per lane: 16 weights x R vectors per block; lanes pair up at the end and
// the 4 waves are summed through LDS in a fixed order.
// ---------------------------------------------------------------------------
// MV_WIN = blocks of activations staged per pass: 32 KiB of LDS for R vectors.
template <int R, int MV_WIN = 256 / R>
__global__ __launch_bounds__(256) void q8_0_matvec_kernel(
    const int8_t *__restrict__ qs, const __half *__restrict__ dsc, int mat, int rows, int nb,
    int in_dim, const float *__restrict__ x, int ldx, float *__restrict__ y, int ldy, int nvec)
{
    __shared__ __align__(16) float xl[R][MV_WIN * QK];
    __shared__ float xs[R][2 * MV_WIN];
    __shared__ float red[4][R][32];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int v0 = blockIdx.y * R;
    const int row = blockIdx.x * 32 + lane / 2;
    const int h = lane & 1;
    const bool row_ok = row < rows;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int b0 = 0; b0 < nb; b0 += MV_WIN) {
        const int nbw = min(MV_WIN, nb - b0);
        __syncthreads();
        for (int i = threadIdx.x; i < R * nbw * QK; i += 256) {
            const int r = i / (nbw * QK), kk = i - r * nbw * QK;
            const int k = b0 * QK + kk;
            xl[r][kk] = (v0 + r < nvec && k < in_dim) ? x[(size_t)(v0 + r) * ldx + k] : 0.0f;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < R * 2 * nbw; i += 256) {
            const int r = i / (2 * nbw), hb = i - r * 2 * nbw;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) s += xl[r][hb * 16 + j];
            xs[r][hb] = s;
        }
        __syncthreads();
        // four blocks per wave in flight
        for (int bb = wave; bb < nbw; bb += 16) {
            int4 q[4];
            float dd[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {   // branch-free: clamped address, zero scale
                const int b = bb + 4 * u;
                const size_t o = bm_index(mat, nb, b0 + min(b, nbw - 1), rows, min(row, rows - 1));
                q[u] = *reinterpret_cast<const int4 *>(qs + o * QK + 16 * h);
                dd[u] = __half2float(dsc[o]);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) dd[u] = (row_ok && bb + 4 * u < nbw) ? dd[u] : 0.0f;
            // all loads above are issued before any of the arithmetic below
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int b = bb + 4 * u;
                if (b < nbw) {
#pragma unroll
                    for (int r = 0; r < R; r++)
                        acc[r] = fmaf(dot16_q8_lds(q[u], &xl[r][b * QK + 16 * h], xs[r][2 * b + h]),
                                      dd[u], acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        acc[r] += __shfl_xor(acc[r], 1, WAVE);
        if (h == 0) red[wave][r][lane / 2] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < R * 32) {
        const int r = threadIdx.x / 32, rr = threadIdx.x % 32;
        const int orow = blockIdx.x * 32 + rr;
        if (orow < rows && v0 + r < nvec)
            y[(size_t)(v0 + r) * ldy + orow] = ((red[0][r][rr] + red[1][r][rr]) + red[2][r][rr]) + red[3][r][rr];
    }
}

// Single input vector.  A workgroup owns RPW output rows and all of their
// block columns; lane l of a wave takes half h = l & 1 of a block, row
// (l >> 1) % RPW and block slot l / (2 RPW), so one 16-byte load per lane
// covers RPW rows x 64 / (2 RPW) block columns (each a contiguous run of
// 32 RPW bytes); scales come from the row-major copy, so the RPW rows' scales
// are whole lines no other workgroup reads.  Every lane issues the weight and scale loads of its first
// NBW blocks before the input row is staged in LDS, so at 1024 -> 3072 the
// whole matrix is requested at once by 384 workgroups; a kernel that only
// loads the same weights takes as long.  Each lane forms its own half-block
// sums; rows are summed over the lanes of a wave and then over the waves in
// wave order.  RAG: in_dim is not a multiple of 32 (the missing activations
// of the last block read as zero).
constexpr int MV1_MAX_NB = 384;   // 48 KiB of activations in LDS

template <int RPW, int NWV, int NBW, bool RAG>
__global__ __launch_bounds__(NWV * WAVE) void q8_0_matvec1_kernel(const int8_t *__restrict__ qs,
                                                                  const __half *__restrict__ dcm, int mat,
                                                                  int rows, int nb, int nbp, int in_dim,
                                                                  const float *__restrict__ x,
                                                                  float *__restrict__ y)
{
    constexpr int SPW = WAVE / (2 * RPW);   // block slots per wave
    constexpr int BPR = NWV * SPW;          // block columns per round of the workgroup
    constexpr int NT = NWV * WAVE;
    extern __shared__ __align__(16) float mv_x[];   // nb * 32 activations
    __shared__ float red[NWV][RPW];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int h = lane & 1, r = (lane >> 1) & (RPW - 1), s = lane / (2 * RPW);
    const int row = blockIdx.x * RPW + r;
    const bool row_ok = row < rows;
    const int rc = min(row, rows - 1);
    const int first = wave * SPW + s;
    int4 q[NBW];
    float dd[NBW];
    // branch-free: clamped block, zero scale past the last one
    auto load = [&](int c0) {
#pragma unroll
        for (int u = 0; u < NBW; u++) {
            const int bc = min(c0 + first + BPR * u, nb - 1);
            const size_t o = bm_index(mat, nb, bc, rows, rc);
            q[u] = *reinterpret_cast<const int4 *>(qs + o * QK + 16 * h);
            dd[u] = __half2float(dcm[((size_t)mat * rows + rc) * nbp + bc]);
        }
#pragma unroll
        for (int u = 0; u < NBW; u++) dd[u] = (row_ok && c0 + first + BPR * u < nb) ? dd[u] : 0.0f;
    };
    load(0);
    const int kp = nb * QK;
    for (int k = 4 * threadIdx.x; k < kp; k += 4 * NT) {
        float4 v;
        if (!RAG || k + 4 <= in_dim) {
            v = *reinterpret_cast<const float4 *>(x + k);
        } else {
            v.x = k < in_dim ? x[k] : 0.0f;
            v.y = k + 1 < in_dim ? x[k + 1] : 0.0f;
            v.z = k + 2 < in_dim ? x[k + 2] : 0.0f;
            v.w = k + 3 < in_dim ? x[k + 3] : 0.0f;
        }
        *reinterpret_cast<float4 *>(&mv_x[k]) = v;
    }
    __syncthreads();
    float acc = 0.0f;
    for (int c0 = 0;;) {
#pragma unroll
        for (int u = 0; u < NBW; u++) {
            const int bc = min(c0 + first + BPR * u, nb - 1);
            float xr[16];
            const float4 *p = reinterpret_cast<const float4 *>(&mv_x[bc * QK + 16 * h]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = p[i];
                xr[4 * i] = v.x;
                xr[4 * i + 1] = v.y;
                xr[4 * i + 2] = v.z;
                xr[4 * i + 3] = v.w;
            }
            float xs = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) xs += xr[j];
            acc = fmaf(dot16_q8(q[u], xr, xs), dd[u], acc);
        }
        c0 += NBW * BPR;
        if (c0 >= nb) break;
        load(c0);
    }
    acc += __shfl_xor(acc, 1, WAVE);
#pragma unroll
    for (int o = 2 * RPW; o < WAVE; o <<= 1) acc += __shfl_xor(acc, o, WAVE);
    if (lane < 2 * RPW && h == 0) red[wave][r] = acc;
    __syncthreads();
    if (threadIdx.x < RPW) {
        const int orow = blockIdx.x * RPW + threadIdx.x;
        if (orow < rows) {
            float v = red[0][threadIdx.x];
#pragma unroll
            for (int w = 1; w < NWV; w++) v += red[w][threadIdx.x];
            y[orow] = v;
        }
    }
}

template <bool RAG>
static void launch_matvec1(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, float *y)
{
    // launch shapes measured at 1024 -> 3072, 2048 -> 2048, 7168 -> 2048 and
    // 2048 -> 7168: 8 rows per workgroup, 4 waves up to 32 block columns,
    // else 8; up to 2 blocks in flight per lane for 64 block columns, else 4
    constexpr int RPW = 8;
    const dim3 grid((t->out_dim + RPW - 1) / RPW);
    const size_t shm = (size_t)t->nb * QK * sizeof(float);
    if (t->nb <= 16)
        QQ_LAUNCH(ctx, (q8_0_matvec1_kernel<RPW, 4, 1, RAG>), grid, dim3(4 * WAVE), shm, t->qs, t->dcm, mat,
                  t->out_dim, t->nb, t->nbp, t->in_dim, x, y);
    else if (t->nb <= 32)
        QQ_LAUNCH(ctx, (q8_0_matvec1_kernel<RPW, 4, 2, RAG>), grid, dim3(4 * WAVE), shm, t->qs, t->dcm, mat,
                  t->out_dim, t->nb, t->nbp, t->in_dim, x, y);
    else if (t->nb <= 64)
        QQ_LAUNCH(ctx, (q8_0_matvec1_kernel<RPW, 8, 2, RAG>), grid, dim3(8 * WAVE), shm, t->qs, t->dcm, mat,
                  t->out_dim, t->nb, t->nbp, t->in_dim, x, y);
    else
        QQ_LAUNCH(ctx, (q8_0_matvec1_kernel<RPW, 8, 4, RAG>), grid, dim3(8 * WAVE), shm, t->qs, t->dcm, mat,
                  t->out_dim, t->nb, t->nbp, t->in_dim, x, y);
}

int launch_q8_0_matvec(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, int ldx,
                       float *y, int ldy, int rows)
{
    if (rows <= 0) return QQ_OK;
    const unsigned gx = (unsigned)((t->out_dim + 31) / 32);
    prof_begin(ctx, K_MATVEC);
    // one vector whose activations fit in LDS (in_dim <= 12288)
    if (rows == 1 && ((uintptr_t)x & 15) == 0 && t->nb <= MV1_MAX_NB) {
        if (t->in_dim % QK)
            launch_matvec1<true>(ctx, t, mat, x, y);
        else
            launch_matvec1<false>(ctx, t, mat, x, y);
    } else if (rows >= 4)
        QQ_LAUNCH(ctx, (q8_0_matvec_kernel<4>), dim3(gx, (rows + 3) / 4), dim3(256), 0, t->qs, t->d, mat, t->out_dim, t->nb, t->in_dim, x, ldx, y,
                           ldy, rows);
    else if (rows >= 2)
        QQ_LAUNCH(ctx, (q8_0_matvec_kernel<2>), dim3(gx, (rows + 1) / 2), dim3(256), 0, t->qs, t->d, mat, t->out_dim, t->nb, t->in_dim, x, ldx, y,
                           ldy, rows);
    else
        QQ_LAUNCH(ctx, (q8_0_matvec_kernel<1>), dim3(gx, rows), dim3(256), 0,
                           t->qs, t->d, mat, t->out_dim, t->nb, t->in_dim, x, ldx, y, ldy, rows);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
