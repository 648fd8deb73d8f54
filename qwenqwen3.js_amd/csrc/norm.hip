// norm.hip -- RMSNorm of the residual stream, the step that feeds the MoE
// block (src/lfm2-engine.js:251-252):
//   out[i] = fp32(w[i] * x[i] * (1 / sqrt(sum_j x[j]^2 / n + eps)))
// with the reference's binary64 arithmetic (src/tensor.js:103-114); the sum
// of squares is a fixed-order binary64 tree instead of a sequential loop (the
// same tree as the normalisation inside the decode kernel).
#include "qq_device.h"

namespace qq {

__global__ __launch_bounds__(NORM_THREADS) void rmsnorm_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               float *__restrict__ out, int H,
                                                               double eps)
{
    __shared__ double red[NORM_THREADS / WAVE];
    const float *xr = x + (size_t)blockIdx.x * H;
    float *orow = out + (size_t)blockIdx.x * H;
    double s = 0.0;
    for (int i = threadIdx.x; i < H; i += NORM_THREADS) {
        const double v = (double)xr[i];
        s = fma(v, v, s);
    }
    const double inv = rms_inv(block_sum_f64<NORM_THREADS / WAVE>(s, red), H, eps);
    for (int i = threadIdx.x; i < H; i += NORM_THREADS) {
        const double wv = w ? (double)w[i] : 1.0;
        orow[i] = (float)(wv * (double)xr[i] * inv);
    }
}

int launch_rmsnorm(qq_ctx *ctx, const float *x, const float *w, float *out, int T, int H,
                   double eps)
{
    prof_begin(ctx, K_RMSNORM);
    QQ_LAUNCH(ctx, rmsnorm_kernel, dim3(T), dim3(NORM_THREADS), 0, x, w, out, H, eps);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

}  // namespace qq
