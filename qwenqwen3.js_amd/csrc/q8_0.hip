// q8_0.hip -- one-time Q8_0 repack and the Q8_0 x fp32 matvec (matmulQ80xF32).
//
// Reference: matmulQ80xF32, src/tensor.js:26-53.  Block = {fp16 d, int8 qs[32]}
// (src/tensor.js:1-2); a GGUF [in_dim, out_dim] tensor stores column c as
// ceil(in_dim/32) consecutive blocks (src/tensor.js:4-5, 36).
#include "qq_device.h"

namespace qq {

// ---------------------------------------------------------------------------
// Repack: GGUF AoS blocks -> qs[row][kp] (int8, k contiguous) + d[row][nb].
// One thread per block; consecutive threads read consecutive 34-byte blocks.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void repack_q8_0_kernel(const uint8_t *__restrict__ src,
                                                          int8_t *__restrict__ qs,
                                                          __half *__restrict__ d, size_t nblocks,
                                                          int nb)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(src + i * QBLK);  // 2-byte aligned
    const size_t row = i / nb;
    const int b = (int)(i - row * nb);
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = (uint32_t)s16[1 + 2 * j] | ((uint32_t)s16[2 + 2 * j] << 16);
    int4 *dst = reinterpret_cast<int4 *>(qs + row * (size_t)nb * QK + (size_t)b * QK);
    dst[0] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    dst[1] = make_int4((int)w[4], (int)w[5], (int)w[6], (int)w[7]);
    d[i] = __ushort_as_half(s16[0]);
}

int launch_repack_q8_0(qq_ctx *ctx, const uint8_t *gguf_dev, qq_tensor *t)
{
    const size_t nblocks = (size_t)t->n_mats * t->out_dim * t->nb;
    const unsigned grid = (unsigned)((nblocks + 255) / 256);
    prof_begin(ctx, K_REPACK);
    hipLaunchKernelGGL(repack_q8_0_kernel, dim3(grid), dim3(256), 0, ctx->stream, gguf_dev,
                       t->qs, t->d, nblocks, t->nb);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

// ---------------------------------------------------------------------------
// Matvec.  A wavefront owns one output column (one repacked row) at a time:
// lane l reads the 16 contiguous weight bytes at k = 1024*j + 16*l, so each
// wave-wide load is one 1 KiB coalesced segment.  The R input vectors'
// activations for those k live in registers for the whole block; the scale of
// the lane's block is one fp16.  Lanes reduce with a 64-wide butterfly.
// NCH = ceil(kp/1024) chunks per row, RPW rows per wave issued together.
// ---------------------------------------------------------------------------
template <int NCH, int R, int RPW>
__global__ __launch_bounds__(256) void q8_0_matvec_kernel(
    const int8_t *__restrict__ qs, const __half *__restrict__ dsc, int out_dim, int kp, int nb,
    int in_dim, const float *__restrict__ x, int ldx, float *__restrict__ y, int ldy, int nvec)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int v0 = blockIdx.y * R;

    float xr[R][NCH][16];
    float xs[R][NCH];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int k0 = 1024 * j + 16 * lane;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int k = k0 + i;
                const float v = (v0 + r < nvec && k < in_dim) ? x[(size_t)(v0 + r) * ldx + k] : 0.0f;
                xr[r][j][i] = v;
                s += v;
            }
            xs[r][j] = s;
        }
    }

    const int row0 = (blockIdx.x * 4 + wave) * RPW;
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
        const int c = row0 + rr;
        if (c >= out_dim) break;
        int4 q[NCH];
        float dd[NCH];
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int k0 = 1024 * j + 16 * lane;
            if (k0 < kp) {
                q[j] = *reinterpret_cast<const int4 *>(qs + (size_t)c * kp + k0);
                dd[j] = __half2float(dsc[(size_t)c * nb + (k0 >> 5)]);
            } else {
                q[j] = make_int4(0, 0, 0, 0);
                dd[j] = 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < NCH; j++) acc = fmaf(dot16_q8(q[j], xr[r][j], xs[r][j]), dd[j], acc);
            acc = wave_sum(acc);
            if (lane == 0 && v0 + r < nvec) y[(size_t)(v0 + r) * ldy + c] = acc;
        }
    }
}

// Fallback for rows longer than 4096 weights: activations re-read per row.
__global__ __launch_bounds__(256) void q8_0_matvec_long_kernel(
    const int8_t *__restrict__ qs, const __half *__restrict__ dsc, int out_dim, int kp, int nb,
    int in_dim, const float *__restrict__ x, int ldx, float *__restrict__ y, int ldy)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x / WAVE;
    const int c = blockIdx.x * 4 + wave;
    const int v = blockIdx.y;
    if (c >= out_dim) return;
    const float *xv = x + (size_t)v * ldx;
    float acc = 0.0f;
    for (int k0 = 16 * lane; k0 < kp; k0 += 1024) {
        const int4 q = *reinterpret_cast<const int4 *>(qs + (size_t)c * kp + k0);
        float xr[16];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            xr[i] = (k0 + i < in_dim) ? xv[k0 + i] : 0.0f;
            s += xr[i];
        }
        acc = fmaf(dot16_q8(q, xr, s), __half2float(dsc[(size_t)c * nb + (k0 >> 5)]), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[(size_t)v * ldy + c] = acc;
}

int launch_q8_0_matvec(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, int ldx,
                       float *y, int ldy, int rows)
{
    if (rows <= 0) return QQ_OK;
    const size_t moff = (size_t)mat * t->out_dim;
    const int8_t *qs = t->qs + moff * t->kp;
    const __half *d = t->d + moff * t->nb;
    const int nch = (t->kp + 1023) / 1024;
    constexpr int RPW = 2;
    const unsigned gx = (unsigned)((t->out_dim + 4 * RPW - 1) / (4 * RPW));
#define QQ_MV(NCH, R)                                                                          \
    hipLaunchKernelGGL((q8_0_matvec_kernel<NCH, R, RPW>), dim3(gx, (rows + R - 1) / R),      \
                       dim3(256), 0, ctx->stream, qs, d, t->out_dim, t->kp, t->nb, t->in_dim, \
                       x, ldx, y, ldy, rows)
    prof_begin(ctx, K_MATVEC);
    switch (nch) {
    case 1: if (rows >= 2) QQ_MV(1, 2); else QQ_MV(1, 1); break;
    case 2: if (rows >= 2) QQ_MV(2, 2); else QQ_MV(2, 1); break;
    case 3: QQ_MV(3, 1); break;
    case 4: QQ_MV(4, 1); break;
    default:
        hipLaunchKernelGGL(q8_0_matvec_long_kernel, dim3((t->out_dim + 3) / 4, rows), dim3(256),
                           0, ctx->stream, qs, d, t->out_dim, t->kp, t->nb, t->in_dim, x, ldx,
                           y, ldy);
    }
    prof_end(ctx);
#undef QQ_MV
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
