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
// Matvec.  A workgroup (4 waves) owns 32 output rows; lane l of every wave
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

int launch_q8_0_matvec(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, int ldx,
                       float *y, int ldy, int rows)
{
    if (rows <= 0) return QQ_OK;
    const unsigned gx = (unsigned)((t->out_dim + 31) / 32);
    prof_begin(ctx, K_MATVEC);
    if (rows >= 4)
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
