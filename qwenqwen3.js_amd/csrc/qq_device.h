// qq_device.h -- device helpers shared by the kernels.
#pragma once

#include "qq_internal.h"

#include <climits>

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

// v from the lane picked by the DPP control CTRL (a permutation within each
// row of 16 lanes), both halves moved by the data-parallel-primitive path
// rather than through LDS.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v)
{
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

__device__ __forceinline__ double readlane_f64(double v, int l)
{
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sum over the 64 lanes of a wavefront (all lanes active), the same value in
// every lane: quads by quad permutations, rows of 16 by row rotations, then
// the four row sums in row order.
__device__ __forceinline__ double wave_sum_dpp(double v)
{
    v += dpp_f64<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f64<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f64<0x124>(v);   // row_ror:4
    v += dpp_f64<0x128>(v);   // row_ror:8
    return ((readlane_f64(v, 0) + readlane_f64(v, 16)) + readlane_f64(v, 32)) + readlane_f64(v, 48);
}

// Sum over a block of NW wavefronts: waves by wave_sum_dpp, then the NW wave
// sums in wave order (red: NW doubles of LDS).  Contains a __syncthreads.
template <int NW>
__device__ __forceinline__ double block_sum_f64(double v, double *red)
{
    v = wave_sum_dpp(v);
    if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    double s = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) s = s + red[w];
    return s;
}

// RMSNorm of one row (src/tensor.js:103-114) by a block of NORM_THREADS:
// thread t sums x[k]^2 for k = t, t + NORM_THREADS, ... in order (exact
// squares, binary64), block_sum_f64 joins the threads; every kernel that
// normalises a row goes through this, so they agree bit for bit.
constexpr int NORM_THREADS = 512;
__device__ __forceinline__ double rms_inv(double sumsq, int H, double eps)
{
    return 1.0 / sqrt(sumsq / (double)H + eps);
}

// Two int8 values of w (bytes LO, LO + 1) -> two fp16 halves holding the
// same integers exactly: v_cvt_f16_i16 on a sign-extended byte (SDWA byte
// select), the second written into the high half with the low half kept.
template <int LO>
__device__ __forceinline__ uint32_t i8pair_f16(uint32_t w)
{
    static_assert(LO == 0 || LO == 2, "byte pair 0-1 or 2-3");
    uint32_t o;
    if constexpr (LO == 0) {
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(o) : "v"(w));
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1"
            : "+v"(o) : "v"(w));
    } else {
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(o) : "v"(w));
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
            : "+v"(o) : "v"(w));
    }
    return o;
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_u32(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

// global_load_lds: each lane copies `size` bytes from its own address to
// LDS (M0 + lane * size).  Issued from inline assembly: the compiler then
// adds no waits of its own for these copies (with the builtin it cannot
// tell the ring stages of one LDS array apart and drains every copy in flight
// before each LDS read), so callers wait for them explicitly (s_waitcnt
// vmcnt) before reading what they fill.  M0 is read when the copy issues; it
// is saved and restored around the copy (one wait state after an SALU write
// to M0), so any value the compiler keeps in M0 survives.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds)
{
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save) : "v"(g), "s"(lds) : "memory");
}

__device__ __forceinline__ void dma4(const void *g, uint32_t lds)
{
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save) : "v"(g), "s"(lds) : "memory");
}
// The same with a wave-uniform base address (SGPR pair) and a 32-bit
// per-lane byte offset: one VGPR per lane instead of two.
__device__ __forceinline__ void dma16s(uint32_t off, const void *base, uint32_t lds)
{
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save) : "v"(off), "s"(base), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4s(uint32_t off, const void *base, uint32_t lds)
{
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save) : "v"(off), "s"(base), "s"(lds) : "memory");
}

// Four dwordx4 copies and one dword copy (each lane its own 32-bit offset
// from a wave-uniform base, to LDS M0 + lane * size) in one statement: M0 is
// saved once and restored once for the five.  A copy reads M0 one wait
// state after the SALU write that set it.
__device__ __forceinline__ void dma5s(uint32_t o0, const void *b0, uint32_t l0, uint32_t o1, const void *b1,
                                      uint32_t l1, uint32_t o2, const void *b2, uint32_t l2, uint32_t o3,
                                      const void *b3, uint32_t l3, uint32_t o4, const void *b4, uint32_t l4)
{
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %4, %5\n\t"
                 "s_mov_b32 m0, %9\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %7, %8\n\t"
                 "s_mov_b32 m0, %12\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %10, %11\n\t"
                 "s_mov_b32 m0, %15\n\ts_nop 0\n\tglobal_load_lds_dword %13, %14\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "v"(o0), "s"(b0), "s"(l0), "v"(o1), "s"(b1), "s"(l1), "v"(o2), "s"(b2), "s"(l2),
                   "v"(o3), "s"(b3), "s"(l3), "v"(o4), "s"(b4), "s"(l4)
                 : "memory");
}

// Value of lane ^ 1 (resp. lane ^ 2) by a DPP quad permutation: a VALU
// operation, where __shfl_xor goes through the LDS permute unit.
__device__ __forceinline__ float xor1_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));
}
__device__ __forceinline__ float xor2_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false));
}

// Maximum over each row of 16 lanes (all 16 active), the same value in every
// lane of the row: rotations by 8, 4, 2 and 1 within the row.
__device__ __forceinline__ float row_max16(float v)
{
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xf, 0xf, false)));
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xf, 0xf, false)));
}

// Maximum over the 64 lanes of a wavefront (all lanes active), the same value
// in every lane: quads and rows of 16 by DPP, then the four row maxima.
__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Stable top-K of E scores held by one wavefront (score of expert lane + 64 t
// in sc[t]; slots past E must hold -inf): K rounds of a DPP maximum and a
// ballot for the lowest expert holding it, so ties go to the lower index --
// the order of a stable descending sort.  idx[k] / p[k] get the rank-k expert
// and pr[] of it, the same in every lane.  Scores must not be NaN.
template <int EPL>
__device__ __forceinline__ void wave_topk(const float (&sc)[EPL], const float (&pr)[EPL], int K,
                                          int (&idx)[MAX_K], float (&p)[MAX_K])
{
    const int lane = threadIdx.x & (WAVE - 1);
    float v[EPL];
#pragma unroll
    for (int t = 0; t < EPL; t++) v[t] = sc[t];
#pragma unroll
    for (int k = 0; k < MAX_K; k++) {
        idx[k] = 0;
        p[k] = 0.0f;
        if (k >= K) continue;
        float m = v[0];
#pragma unroll
        for (int t = 1; t < EPL; t++) m = fmaxf(m, v[t]);
        m = wave_max_dpp(m);
        int win = -1;
        float pw = 0.0f;
#pragma unroll
        for (int t = EPL - 1; t >= 0; t--) {
            const uint64_t hit = __ballot(v[t] == m);
            if (hit) {
                const int l = (int)__builtin_ctzll(hit);
                win = WAVE * t + l;
                pw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[t]), l));
            }
        }
        idx[k] = win;
        p[k] = pw;
#pragma unroll
        for (int t = 0; t < EPL; t++)
            if (WAVE * t + lane == win) v[t] = -INFINITY;
    }
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// operations, not for its global loads and stores (words exchanged with other
// workgroups carry their own tags and need no fence).
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
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

// Same, activations read from LDS as four float4.
__device__ __forceinline__ float dot16_q8_lds(const int4 q, const float *xl, float xsum)
{
    float xr[16];
    const float4 *p = reinterpret_cast<const float4 *>(xl);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = p[i];
        xr[4 * i] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
    return dot16_q8(q, xr, xsum);
}

// Hide a register value from loop-invariant code motion: without it the
// compiler hoists the int8->float conversion of every weight out of a token
// loop and runs out of registers.
__device__ __forceinline__ void opaque(int4 &q)
{
    asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
}

// 16 int8 weights -> 16 floats in offset binary (q + 128), one
// v_cvt_f32_ubyteN each; pair with dot16_off.
__device__ __forceinline__ void cvt16_off(const int4 q, float *w)
{
    const uint32_t d[4] = {(uint32_t)q.x ^ 0x80808080u, (uint32_t)q.y ^ 0x80808080u,
                           (uint32_t)q.z ^ 0x80808080u, (uint32_t)q.w ^ 0x80808080u};
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int b = 0; b < 4; b++) w[4 * i + b] = (float)((d[i] >> (8 * b)) & 0xffu);
}

// sum_i (q_i + 128) * x_i - 128 * sum_i x_i, x from LDS.
__device__ __forceinline__ float dot16_off(const float *w, const float *xl, float xsum)
{
    const float4 *p = reinterpret_cast<const float4 *>(xl);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = p[i];
        acc = fmaf(w[4 * i], v.x, acc);
        acc = fmaf(w[4 * i + 1], v.y, acc);
        acc = fmaf(w[4 * i + 2], v.z, acc);
        acc = fmaf(w[4 * i + 3], v.w, acc);
    }
    return fmaf(-128.0f, xsum, acc);
}

// ---- int8 dot products on a 3-level decomposition of fp32 activations ----
// A chunk of 16 activations with sigma = max|x|/127 is written as
//   x ~= sigma * (a1 + a2/254 + a3/254^2),  a1, a2, a3 in [-127, 127],
// each level a rounded residual of the previous one.  The representation
// error is below sigma * 2^-15 + |x| * 2^-23 per value, about 1e-7 of the
// chunk's largest value, so a dot product against int8 weights keeps fp32
// accuracy while each group of 4 weights costs one v_dot4 per level.
struct Lev3 {
    int4 l1, l2, l3;
    float sig;
};

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d)
{
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// t (|t| <= 127) -> three int8 levels, t ~ a1 + a2 / 254 + a3 / 254^2.
__device__ __forceinline__ void decompose1(float t, int &q1, int &q2, int &q3)
{
    const float a1 = fminf(fmaxf(rintf(t), -127.0f), 127.0f);
    const float t2 = (t - a1) * 254.0f;
    const float a2 = fminf(fmaxf(rintf(t2), -127.0f), 127.0f);
    const float t3 = (t2 - a2) * 254.0f;
    const float a3 = fminf(fmaxf(rintf(t3), -127.0f), 127.0f);
    q1 = (int)a1;
    q2 = (int)a2;
    q3 = (int)a3;
}

// Three levels of four values, packed as they are formed (few live registers).
__device__ __forceinline__ void decompose4(const float4 v, float inv, uint32_t &p1, uint32_t &p2,
                                           uint32_t &p3)
{
    const float vv[4] = {v.x, v.y, v.z, v.w};
    int q1[4], q2[4], q3[4];
#pragma unroll
    for (int i = 0; i < 4; i++) decompose1(vv[i] * inv, q1[i], q2[i], q3[i]);
    p1 = pack4_i8(q1[0], q1[1], q1[2], q1[3]);
    p2 = pack4_i8(q2[0], q2[1], q2[2], q2[3]);
    p3 = pack4_i8(q3[0], q3[1], q3[2], q3[3]);
}

// v: 16 values, 16-byte aligned.
__device__ __forceinline__ void decompose16(const float *v, Lev3 &o)
{
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    float m = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 q = v4[g];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(q.x), fabsf(q.y)), fmaxf(fabsf(q.z), fabsf(q.w))));
    }
    const float inv = (m > 0.0f) ? 127.0f / m : 0.0f;
    o.sig = m * (1.0f / 127.0f);
    uint32_t a[4], b[4], c[4];
#pragma unroll
    for (int g = 0; g < 4; g++) decompose4(v4[g], inv, a[g], b[g], c[g]);
    o.l1 = make_int4((int)a[0], (int)a[1], (int)a[2], (int)a[3]);
    o.l2 = make_int4((int)b[0], (int)b[1], (int)b[2], (int)b[3]);
    o.l3 = make_int4((int)c[0], (int)c[1], (int)c[2], (int)c[3]);
}

// q . a over four int8 pairs, the accumulator starting at zero: the
// three-operand form with an inline-constant zero (the compiler's choice, the
// accumulating form, first needs a v_mov of zero into the destination).
__device__ __forceinline__ int sdot4_first(int q, int a)
{
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(q), "v"(a));
    return r;
}

__device__ __forceinline__ int sdot16(const int4 q, const int4 a)
{
    int s = sdot4_first(q.x, a.x);
    s = __builtin_amdgcn_sdot4(q.y, a.y, s, false);
    s = __builtin_amdgcn_sdot4(q.z, a.z, s, false);
    return __builtin_amdgcn_sdot4(q.w, a.w, s, false);
}

// sum_i q_i * x_i for 16 int8 weights against a decomposed chunk.
__device__ __forceinline__ float dot16_lev3(const int4 q, const int4 l1, const int4 l2, const int4 l3,
                                            float sig)
{
    const float s1 = (float)sdot16(q, l1);
    const float s2 = (float)sdot16(q, l2);
    const float s3 = (float)sdot16(q, l3);
    return fmaf(fmaf(s3, 1.0f / 254.0f, s2), 1.0f / 254.0f, s1) * sig;
}

// Offsets in the block-major device layout of a qq_tensor:
//   qs[(mat*nb + b)*rows + r][32],  d[(mat*nb + b)*rows + r]
__device__ __forceinline__ size_t bm_index(int mat, int nb, int b, int rows, int r)
{
    return ((size_t)mat * nb + b) * rows + r;
}

// ---- tagged 64-bit exchange words: (tag << 32) | 32 data bits ----
constexpr uint64_t RF_LOCAL_TICKS = 1000;   // 10 us on an XCD-local table, then the copy

// Bounded wait of one wave for its N words per lane at p[i] (want[i]) to
// carry `tag`; the low halves go to v[i].  With dev != 0, after
// RF_LOCAL_TICKS the words are read at p[i] + dev instead (the device-
// coherent copy).  Returns false when it gave up.
template <int N>
__device__ __forceinline__ bool wave_wait(const uint64_t *(&p)[N], const bool (&want)[N], uint32_t tag,
                                          uint32_t (&v)[N], uint64_t wait_ticks, const uint32_t *err,
                                          ptrdiff_t dev = 0)
{
    bool need[N];
#pragma unroll
    for (int i = 0; i < N; i++) need[i] = want[i];
    const uint64_t t0 = wall_clock64();
    ptrdiff_t off = 0;
    while (true) {
        uint64_t u[N];
#pragma unroll
        for (int i = 0; i < N; i++)
            u[i] = need[i] ? __hip_atomic_load(p[i] + off, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
        bool mine = true;
#pragma unroll
        for (int i = 0; i < N; i++) {
            if (!need[i]) continue;
            if ((uint32_t)(u[i] >> 32) == tag) {
                need[i] = false;
                v[i] = (uint32_t)u[i];
            } else {
                mine = false;
            }
        }
        if (__all(mine)) return true;
        const uint64_t dt = wall_clock64() - t0;
        if (dt >= wait_ticks ||
            (dt > RF_LOCAL_TICKS && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)))
            return false;
        if (dt > RF_LOCAL_TICKS) off = dev;
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void store_tagged(uint64_t *p, uint32_t tag, uint32_t bits)
{
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The same into the L2 of this XCD only (read there by agent-scope loads of
// workgroups on the same XCD).
__device__ __forceinline__ void store_tagged_local(uint64_t *p, uint32_t tag, uint32_t bits)
{
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Exclusive scan over the 64 lanes; *total = sum of all lanes.  The
// inclusive scan runs on DPP lane moves (no LDS round trips): within each row
// of 16 lanes by shifts of 1, 2, 4 and 8 (lanes shifted in from outside the
// row add 0), then across rows: lane 15 of rows 0 and 2 into rows 1 and 3,
// and lane 31 into rows 2 and 3.  The whole wave must be active.
__device__ __forceinline__ int wave_excl_scan(int v, int *total)
{
    int x = v;
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31
    *total = __builtin_amdgcn_readlane(x, WAVE - 1);
    return x - v;
}

// Sigmoid routing for one token in one wavefront (lfm2-engine.js:420-447).
// Lane e (+64*i) holds the fp32 logit of expert e.  Every lane returns the
// same ranked selection: idx[k], unbiased probability p[k] and 1/S with
// S = 1e-6 + sum_k p[k] accumulated in rank order in binary64.  The ranking
// is a stable descending sort by selection score (ties to the lower index).
template <int EPL>
struct WaveRoute {
    int idx[MAX_K];
    float p[MAX_K];
    double inv;
    float prob[EPL];   // this lane's sigmoid probabilities (expert lane + 64*i)
};

// LDS of one wave for wave_route: the sort keys and the selection.
template <int EPL>
struct __align__(16) RouteLds {
    uint64_t key[EPL * WAVE];
    int idx[MAX_K];
    float p[MAX_K];
};

// Softmax gating (Qwen3-MoE, src/qwen3-engine.js:305-321 with softmaxInPlace,
// src/tensor.js:150-164): probabilities p_e = fp32(fp32(exp(l_e - max)) * (1/S))
// with S the binary64 sum of the fp32 exponentials in expert order (as the
// reference adds them; a tree sum where that is provably the same value),
// selection by p_e itself,
// and the weights renormalised from 0 (1/sum, or 0 when the sum is 0).
template <int EPL>
__device__ __forceinline__ void softmax_probs(const float (&logit)[EPL], int E, float (&prob)[EPL])
{
    const int lane = threadIdx.x & (WAVE - 1);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; i++)
        if (lane + WAVE * i < E) mx = fmaxf(mx, logit[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, WAVE));
    float ex[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++)
        ex[i] = (lane + WAVE * i < E) ? (float)exp((double)logit[i] - (double)mx) : 0.0f;
    // When every term is 0 or in [2^-22, 1], all terms are multiples of 2^-45
    // and every partial sum is at most E <= 2^8: each is exact in binary64
    // (53 bits), so the sequential sum equals the exact sum and any order of
    // addition gives it.  Otherwise one lane adds the terms in expert order.
    static_assert(EPL * WAVE <= 256, "exact-sum bound");
    bool exact = true;
#pragma unroll
    for (int i = 0; i < EPL; i++) exact = exact && (ex[i] == 0.0f || (ex[i] >= 0x1p-22f && ex[i] <= 1.0f));
    double sum = 0.0;
    if (__all(exact)) {
        double part = 0.0;
#pragma unroll
        for (int i = 0; i < EPL; i++) part += (double)ex[i];   // zero past E
        sum = wave_sum_dpp(part);
    } else {
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int n = min(WAVE, E - WAVE * i);
            const int bits = __float_as_int(ex[i]);
            for (int l = 0; l < n; l++)
                sum = sum + (double)__int_as_float(__builtin_amdgcn_readlane(bits, l));
        }
    }
    const double inv = 1.0 / sum;
#pragma unroll
    for (int i = 0; i < EPL; i++) prob[i] = (float)((double)ex[i] * inv);
}

// softmax: Qwen3 gating (bias unused); otherwise LFM2's sigmoid + bias.
// bias[i] is the selection bias of expert lane + 64 i (any value past E).
// The rank of each expert is the number of experts whose 64-bit key --
// order-preserving score bits, then the complemented index -- is larger: a
// stable descending sort, ties to the lower index (-0 counts as +0).  Every
// lane counts against all keys at once (LDS broadcast reads), so no chain of
// cross-lane steps sits on the path.  A wave's LDS accesses complete in
// order, so its lanes read what its other lanes wrote without a barrier.
template <int EPL>
__device__ __forceinline__ void wave_route(const float (&logit)[EPL], const float (&bias)[EPL], int E,
                                           int K, bool softmax, WaveRoute<EPL> &out, RouteLds<EPL> &lds)
{
    const int lane = threadIdx.x & (WAVE - 1);
    float s[EPL];
    if (softmax) {
        softmax_probs<EPL>(logit, E, out.prob);
#pragma unroll
        for (int i = 0; i < EPL; i++) s[i] = out.prob[i];
    } else {
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = lane + WAVE * i;
            out.prob[i] = 0.0f;
            s[i] = 0.0f;
            if (e < E) {
                out.prob[i] = (float)(1.0 / (1.0 + exp(-(double)logit[i])));
                s[i] = out.prob[i] + bias[i];
            }
        }
    }
    uint64_t key[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + WAVE * i;
        const uint32_t u = __float_as_uint(s[i] + 0.0f);
        const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        key[i] = e < E ? (((uint64_t)ord << 32) | (uint32_t)~e) : 0;
        lds.key[e] = key[i];
    }
    int rank[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) rank[i] = 0;
    const int n2 = (E + 1) / 2;
    for (int u = 0; u < n2; u++) {
        const ulonglong2 q = reinterpret_cast<const ulonglong2 *>(lds.key)[u];
#pragma unroll
        for (int i = 0; i < EPL; i++) rank[i] += (int)(q.x > key[i]) + (int)(q.y > key[i]);
    }
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + WAVE * i;
        if (e < E && rank[i] < K) {
            lds.idx[rank[i]] = e;
            lds.p[rank[i]] = out.prob[i];
        }
    }
    double sumW = softmax ? 0.0 : 1e-6;
#pragma unroll
    for (int k = 0; k < MAX_K; k++) {   // fully unrolled: idx/p stay in registers
        out.idx[k] = INT_MAX;
        out.p[k] = 0.0f;
        if (k >= K) continue;
        out.idx[k] = lds.idx[k];
        out.p[k] = lds.p[k];
        sumW = sumW + (double)out.p[k];
    }
    out.inv = softmax ? (sumW > 0.0 ? 1.0 / sumW : 0.0) : 1.0 / sumW;
}

}  // namespace qq
