// qq_device.h -- device helpers shared by the kernels (wave reductions, Q8_0 dot).
#pragma once

#include "qq_internal.h"

namespace qq {

// Butterfly sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// 16 int8 weights (one int4 = 4 dwords) against 16 fp32 activations.
// Each dword is flipped to offset binary (q + 128) so that every byte
// converts with a single v_cvt_f32_ubyteN; the constant 128 * sum(x) is
// removed afterwards with the chunk's precomputed activation sum.
__device__ __forceinline__ float dot16_q8(const int4 q, const float *x, float xsum)
{
    const uint32_t w[4] = {(uint32_t)q.x ^ 0x80808080u, (uint32_t)q.y ^ 0x80808080u,
                           (uint32_t)q.z ^ 0x80808080u, (uint32_t)q.w ^ 0x80808080u};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float u = (float)((w[i] >> (8 * b)) & 0xffu);
            acc = fmaf(u, x[4 * i + b], acc);
        }
    }
    return fmaf(-128.0f, xsum, acc);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h)
{
    return __half2float(__ushort_as_half(h));
}

}  // namespace qq
