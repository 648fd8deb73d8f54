// mfma.hip -- prefill chunks on the matrix cores: grouped fp16 MFMA GEMMs.
//
// For a chunk of prompt tokens the (token, rank) pairs routed to one expert
// form a dense [n_e x H] x [H x F] contraction (the reference runs them as
// n_e separate matvecs, src/lfm2-engine.js:471-478 per token).  After the
// dispatch (grouped.hip) every expert's slots are cut into row tiles of
// MG_BM slots, and per (row tile, column tile):
//   gate/up  A = fp16 activations of the tile's tokens (gathered by perm),
//            B = gate and up columns dequantised from Q8_0 to fp16
//            w = fp16(q * d); fp32 accumulators; epilogue silu(g) * u ->
//            fp16 act[slot][F]
//   down     A = act rows of the tile, B = down columns likewise ->
//            y[slot][H] fp16
// followed by the gather combine of the fp32 path (rank order, fp32 steps).
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
// scale -> 16 fp16 values w = fp16(q * d), in k order: q converts exactly
// (|q| <= 128), and the multiply by d is the one rounding.  Six instructions
// per four weights (an offset-binary form, bytes paired with the exponent
// byte 0x64 by v_perm and 1152 subtracted, took seven: 1.5-2 % slower GEMMs).
__device__ __forceinline__ void dequant16(const uint4 q, const _Float16 d, uint4 &lo, uint4 &hi)
{
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const h2_t dd = {d, d};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2_t a = __builtin_bit_cast(h2_t, i8pair_f16<0>(w[i])) * dd;
        const h2_t b = __builtin_bit_cast(h2_t, i8pair_f16<2>(w[i])) * dd;
        o[2 * i] = __builtin_bit_cast(uint32_t, a);
        o[2 * i + 1] = __builtin_bit_cast(uint32_t, b);
    }
    lo = make_uint4(o[0], o[1], o[2], o[3]);
    hi = make_uint4(o[4], o[5], o[6], o[7]);
}

__device__ __forceinline__ _Float16 half_bits(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// ---------------------------------------------------------------------------
// Grouped GEMM on v_mfma_f32_32x32x16_f16.
//
// Workgroup = one row tile (MG_BM slots of one expert) x a column tile; its
// 4 waves split the columns, and every wave computes all MG_BM rows of its
// columns for two 32-column B matrices (gate/up: the same 32 features of the
// gate and of the up tensor; down: two adjacent 32-column groups).  Wave tile
// 128 x 64, accumulators 4 row fragments x 2 x 16 floats.
//
// Per Q8_0 block (32 values of the reduction dimension) and stage:
//   A  the tile's 128 rows x 32 halves (8 KB), copied by the 4 waves with
//      global_load_lds_dwordx4 in an XOR-swizzled row order, shared by all;
//   B  each wave's raw int8 columns (2 x 32 columns x 32 B), copied as is;
//      each wave reads back only its own columns and dequantises them in
//      registers to fp16 w = fp16(q * d);
//   d  the fp16 scales of the tile's columns (waves 0 and 1, 256 B each; waves
//      2 and 3 copy them again, unread, so all waves issue 5 copies).
// The copies run MG_AHEAD blocks ahead through a ring of MG_STAGES stages;
// one barrier per block.  The reduction index is permuted identically in A
// and B: lane half h = lane / 32 carries k = 16h + 8s + j in MFMA step s,
// so a lane's B operand is the 16 contiguous bytes 16h .. 16h+15 of its
// column's block and its A operand is chunk 2h + s of its row.
// ---------------------------------------------------------------------------
typedef float f16v_t __attribute__((ext_vector_type(16)));

constexpr int MG_BM = 128;
constexpr int MG_THREADS = 256;
#ifndef MG_STAGES_CFG
#define MG_STAGES_CFG 4
#define MG_AHEAD_CFG 2
#define MG_OCC_CFG 2
#endif
constexpr int MG_STAGES = MG_STAGES_CFG;
constexpr int MG_AHEAD = MG_AHEAD_CFG;       // blocks copied ahead of the one being read
constexpr int MG_A = MG_BM * 64;             // A: 128 rows x 64 B
constexpr int MG_B = 4 * 2 * 1024;           // B: 4 waves x 2 matrices x 32 columns x 32 B
// scales: 2 x 128 columns x 2 B, copied by waves 0 and 1; waves 2 and 3
// copy the same bytes into the other half, so that every wave issues the
// same copies per block and waits for the same counts
constexpr int MG_S = 4 * 256;
constexpr int MG_STAGE = MG_A + MG_B + MG_S;
// The copy of block h + MG_AHEAD is issued after the barrier of block h.  A
// wave may then still be reading stage h (B operands of block h) and stage
// h - 1 (A fragments of block h - 1), and the stage rewritten held block
// h + MG_AHEAD - MG_STAGES, whose last read precedes barrier h when
// MG_AHEAD <= MG_STAGES - 2.
static_assert(MG_STAGES >= MG_AHEAD + 2 && MG_AHEAD >= 1, "ring stage written while still read");

// A slot of (row r, 16-byte chunk c): rows of 4 chunks, chunk order XORed
// with s(r) = ((r >> 1) ^ (r >> 2)) & 3, so that the 16 rows a 16-lane group
// of a fragment read touches 16 different 16-byte bank groups.
__device__ __forceinline__ int mg_aslot(int r, int c) { return 4 * r + (c ^ (((r >> 1) ^ (r >> 2)) & 3)); }

// B slot of (column f in 0..31, half h): lanes 0-15, 16-31, 32-47, 48-63 of a
// fragment read land in 16 consecutive slots each.
__device__ __forceinline__ int mg_bslot(int f, int h) { return (f & 15) + 16 * h + 32 * (f >> 4); }

// Copy sources of block 0: wave-uniform bases plus 32-bit per-lane offsets.
struct MgSrc {
    const char *abase, *bbase0, *bbase1, *sbase;
    uint32_t a0, a1;           // this lane's A chunks for its two copies
    uint32_t b0, b1;           // this lane's 16 B of the two B matrices
    uint32_t sc;               // waves 0, 1: this lane's 4 bytes of scales
    size_t bstep, sstep;       // one block of B (columns * 32 B) and of the scales (columns * 2 B)
};

// s_waitcnt vmcnt(PER * later), later = 0 .. 6 blocks still in flight behind this one
template <int PER>
__device__ __forceinline__ void mg_wait(int later)
{
    switch (later) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<PER>(); break;
    case 2: wait_vm<2 * PER>(); break;
    case 3: wait_vm<3 * PER>(); break;
    case 4: wait_vm<4 * PER>(); break;
    case 5: wait_vm<5 * PER>(); break;
    default: wait_vm<6 * PER>(); break;
    }
}
static_assert(MG_AHEAD <= 6, "mg_wait covers up to 6 blocks in flight");

template <int NFR>
__device__ __forceinline__ void mg_mainloop(const MgSrc &src, int nb, char *lds, int sc_off0, int sc_off1,
                                            f16v_t (&acc)[4][2])
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: SGPR operands
    const uint32_t base = lds_u32(lds);
    // copy destinations within a stage (wave-uniform)
    const uint32_t da0 = base + (128 * wave) * 16, da1 = da0 + 64 * 16;
    const uint32_t db0 = base + MG_A + (wave * 2) * 1024, db1 = db0 + 1024;
    const uint32_t ds = base + MG_A + MG_B + wave * 256;
    // fragment reads within a stage: row 32i + x has the swizzle of row x
    // (s(r) depends on r mod 8 only), so fragment i is fragment 0 + 2048 i
    int ao[2];
#pragma unroll
    for (int st = 0; st < 2; st++) ao[st] = 16 * mg_aslot(lane & 31, 2 * (lane >> 5) + st);
    const int bo = MG_A + (wave * 2) * 1024 + 16 * mg_bslot(lane & 31, lane >> 5);

    // (stage st of the ring: block b % MG_STAGES; a literal in the unrolled loop)
    auto issue_s = [&](int b, int st) {
        const uint32_t so = (uint32_t)st * MG_STAGE;
        const char *ab = src.abase + (size_t)b * 64;
        dma5s(src.a0, ab, da0 + so, src.a1, ab, da1 + so, src.b0, src.bbase0 + (size_t)b * src.bstep, db0 + so,
              src.b1, src.bbase1 + (size_t)b * src.bstep, db1 + so, src.sc, src.sbase + (size_t)b * src.sstep,
              ds + so);
    };
    auto issue = [&](int b) { issue_s(b, b % MG_STAGES); };
    // the wait for the block after the one just issued while MG_AHEAD - 1
    // more are in flight behind it (5 copies a block per wave)
    auto wait_steady = [&]() { wait_vm<5 * (MG_AHEAD - 1)>(); };
    // Wait until block x's copies landed when blocks up to `upto` have been
    // issued.
    auto wait_block = [&](int x, int upto) { mg_wait<5>(min(nb - 1, upto) - x); };
    // Operands fetched one block ahead: B dequantised (both matrices, both
    // MFMA steps) and the A fragments of MFMA step 0.
    struct Frag {
        h8_t b[2][2];
        h8_t a0[NFR];
    };
    auto fetch_s = [&](int sg, Frag &f) {
        const char *st = lds + sg * MG_STAGE;
        const uint4 q0 = *reinterpret_cast<const uint4 *>(st + bo);
        const uint4 q1 = *reinterpret_cast<const uint4 *>(st + bo + 1024);
        const _Float16 d0 = *reinterpret_cast<const _Float16 *>(st + sc_off0);
        const _Float16 d1 = *reinterpret_cast<const _Float16 *>(st + sc_off1);
#pragma unroll
        for (int i = 0; i < NFR; i++) f.a0[i] = *reinterpret_cast<const h8_t *>(st + ao[0] + 2048 * i);
        uint4 lo0, hi0, lo1, hi1;
        dequant16(q0, d0, lo0, hi0);
        dequant16(q1, d1, lo1, hi1);
        f.b[0][0] = __builtin_bit_cast(h8_t, lo0);
        f.b[0][1] = __builtin_bit_cast(h8_t, hi0);
        f.b[1][0] = __builtin_bit_cast(h8_t, lo1);
        f.b[1][1] = __builtin_bit_cast(h8_t, hi1);
    };
    auto fetch = [&](int b, Frag &f) { fetch_s(b % MG_STAGES, f); };
    // block b's MFMAs; the step-1 A fragments are read here, under step 0's MFMAs
    auto mma_s = [&](int sg, const Frag &f) {
        const char *st = lds + sg * MG_STAGE;
        h8_t a1[NFR];
#pragma unroll
        for (int i = 0; i < NFR; i++) a1[i] = *reinterpret_cast<const h8_t *>(st + ao[1] + 2048 * i);
#pragma unroll
        for (int i = 0; i < NFR; i++) {
            acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a0[i], f.b[0][0], acc[i][0], 0, 0, 0);
            acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a0[i], f.b[1][0], acc[i][1], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NFR; i++) {
            acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[i], f.b[0][1], acc[i][0], 0, 0, 0);
            acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[i], f.b[1][1], acc[i][1], 0, 0, 0);
        }
    };
    auto mma = [&](int b, const Frag &f) { mma_s(b % MG_STAGES, f); };

    // Software pipeline: block b+1's B operands and step-0 A fragments are
    // read (and B dequantised) while block b's MFMAs run (two register sets,
    // loop unrolled by two).
#pragma unroll
    for (int b = 0; b < MG_AHEAD; b++)
        if (b < nb) issue(b);
    Frag f0, f1;
    wait_block(0, MG_AHEAD - 1);
    __syncthreads();
    fetch(0, f0);
    int b = 0;
    // steady state: every copy of an iteration goes out and every wait leaves
    // MG_AHEAD - 1 blocks in flight.  Four blocks an iteration from b = 0, so
    // the ring stage of each is a literal (no stage arithmetic per block).
    static_assert(MG_STAGES == 4, "four blocks per steady iteration, one per stage");
    for (; b + 3 + MG_AHEAD < nb; b += 4) {
        issue_s(b + MG_AHEAD, MG_AHEAD % 4);
        wait_steady();
        __syncthreads();
        fetch_s(1, f1);
        mma_s(0, f0);
        issue_s(b + 1 + MG_AHEAD, (1 + MG_AHEAD) % 4);
        wait_steady();
        __syncthreads();
        fetch_s(2, f0);
        mma_s(1, f1);
        issue_s(b + 2 + MG_AHEAD, (2 + MG_AHEAD) % 4);
        wait_steady();
        __syncthreads();
        fetch_s(3, f1);
        mma_s(2, f0);
        issue_s(b + 3 + MG_AHEAD, (3 + MG_AHEAD) % 4);
        wait_steady();
        __syncthreads();
        fetch_s(0, f0);
        mma_s(3, f1);
    }
    for (; b + 1 + MG_AHEAD < nb; b += 2) {
        issue(b + MG_AHEAD);
        wait_steady();
        __syncthreads();
        fetch(b + 1, f1);
        mma(b, f0);
        issue(b + 1 + MG_AHEAD);
        wait_steady();
        __syncthreads();
        fetch(b + 2, f0);
        mma(b + 1, f1);
    }
    // the last blocks, with waits that count down to zero
    for (; b + 1 < nb; b += 2) {
        // f0 holds block b
        if (b + MG_AHEAD < nb) issue(b + MG_AHEAD);
        wait_block(b + 1, b + MG_AHEAD);
        __syncthreads();
        fetch(b + 1, f1);
        mma(b, f0);
        // f1 holds block b + 1
        if (b + 1 + MG_AHEAD < nb) issue(b + 1 + MG_AHEAD);
        if (b + 2 < nb) {
            wait_block(b + 2, b + 1 + MG_AHEAD);
            __syncthreads();
            fetch(b + 2, f0);
        }
        mma(b + 1, f1);
    }
    if (b < nb) mma(b, f0);   // odd block count: the last block, fetched above
}

// blockIdx -> (row tile, column tile): the dispatcher deals workgroups to the
// 8 XCDs round robin, so XCD x runs blocks x, x+8, ...; each XCD takes a
// contiguous run of the real work items (row-tile major), so the column
// tiles of a row tile share its A rows, and the row tiles of an expert its
// weights, in one L2.  False once past the real items.
__device__ __forceinline__ bool mg_item(int n_tiles, int nct, int &tile, int &ct)
{
    const int R = n_tiles * nct;
    const int per = (R + 7) >> 3;
    const int x = blockIdx.x & 7, i = blockIdx.x >> 3;
    const int w = x * per + i;
    if (i >= per || w >= R) return false;
    tile = w / nct;
    ct = w - tile * nct;
    return true;
}

// MODE 0: gate/up -> SwiGLU -> act (column tile = 128 features: wave w takes
//         features 32w..32w+31 of the gate and of the up tensor);
// MODE 1: down -> y (column tile = 256 outputs: wave w takes 64w..64w+63).
template <int MODE>
__global__ __launch_bounds__(MG_THREADS, MG_OCC_CFG) void moe_mg_kernel(MfmaArgs a)
{
    __shared__ __align__(16) char lds[MG_STAGES * MG_STAGE];
    __shared__ uint32_t rowoff[MG_BM];

    const int ncols = MODE == 0 ? a.F : a.H;          // columns of a B matrix
    const int tw = MODE == 0 ? 128 : 256;             // columns per column tile
    const int nct = (ncols + tw - 1) / tw;
    int tile, ct;
    if (!mg_item(*a.n_tiles, nct, tile, ct)) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int n = min(MG_BM, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = MODE == 0 ? a.nbH : a.nbF;
    const int kdim = MODE == 0 ? a.H : a.F;

    // A row offsets (bytes): gate/up gathers token rows of xh, down reads act rows
    if (tid < MG_BM) {
        const int r = min(tid, n - 1);
        rowoff[tid] = (uint32_t)((MODE == 0 ? (size_t)(a.perm[slot0 + r] / a.K) : (size_t)(slot0 + r)) * kdim * 2);
    }
    __syncthreads();

    MgSrc src;
    src.abase = MODE == 0 ? reinterpret_cast<const char *>(a.xh) : reinterpret_cast<const char *>(a.act);
    {
        const int s0 = 128 * wave + lane, s1 = s0 + 64;
        const int r0 = s0 >> 2, r1 = s1 >> 2;
        src.a0 = rowoff[r0] + 16 * ((s0 & 3) ^ (((r0 >> 1) ^ (r0 >> 2)) & 3));
        src.a1 = rowoff[r1] + 16 * ((s1 & 3) ^ (((r1 >> 1) ^ (r1 >> 2)) & 3));
    }
    // this wave's two 32-column groups (clamped into range; stores are masked)
    const int c0 = MODE == 0 ? ct * 128 + 32 * wave : ct * 256 + 64 * wave;
    const int c1 = MODE == 0 ? c0 : c0 + 32;
    const int8_t *q0 = MODE == 0 ? a.gq : a.dq;
    const int8_t *q1 = MODE == 0 ? a.uq : a.dq;
    const uint16_t *dd0 = MODE == 0 ? a.gd : a.dd;
    const uint16_t *dd1 = MODE == 0 ? a.ud : a.dd;
    {
        const int f = (lane & 15) + 16 * (lane >> 5), h = (lane >> 4) & 1;   // inverse of mg_bslot
        const int g0 = min(c0, ncols - 32) + f, g1 = min(c1, ncols - 32) + f;
        src.bbase0 = reinterpret_cast<const char *>(q0 + bm_index(e, nb, 0, ncols, 0) * QK);
        src.bbase1 = reinterpret_cast<const char *>(q1 + bm_index(e, nb, 0, ncols, 0) * QK);
        src.b0 = (uint32_t)(g0 * QK + 16 * h);
        src.b1 = (uint32_t)(g1 * QK + 16 * h);
        // scales: wave 0 -> columns [cs, cs+128) of matrix 0, wave 1 -> of matrix 1
        // (gate/up) or the next 128 (down); 2 per lane
        const int cs = MODE == 0 ? ct * 128 : ct * 256 + 128 * (wave & 1);
        const uint16_t *dsrc = (MODE == 0 && wave == 1) ? dd1 : dd0;
        src.sbase = reinterpret_cast<const char *>(dsrc + bm_index(e, nb, 0, ncols, 0));
        src.sc = (uint32_t)(2 * min(cs + 2 * lane, ncols - 2));
        src.bstep = (size_t)ncols * QK;
        src.sstep = (size_t)ncols * 2;
    }
    // scale offsets within a stage for this lane's columns of the two matrices
    int so0, so1;
    if (MODE == 0) {
        so0 = MG_A + MG_B + (32 * wave + (lane & 31)) * 2;
        so1 = so0 + 256;
    } else {
        const int l0 = 64 * wave + (lane & 31), l1 = l0 + 32;
        so0 = MG_A + MG_B + (l0 >> 7) * 256 + (l0 & 127) * 2;
        so1 = MG_A + MG_B + (l1 >> 7) * 256 + (l1 & 127) * 2;
    }

    f16v_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    const int nfr = (n + 31) >> 5;
    switch (nfr) {
    case 1: mg_mainloop<1>(src, nb, lds, so0, so1, acc); break;
    case 2: mg_mainloop<2>(src, nb, lds, so0, so1, acc); break;
    case 3: mg_mainloop<3>(src, nb, lds, so0, so1, acc); break;
    default: mg_mainloop<4>(src, nb, lds, so0, so1, acc); break;
    }

    // lane holds column lane % 32 and rows 8*(r/4) + 4*(lane/32) + r%4 of each fragment
    const int cl = lane & 31, rh = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (32 * i >= n) break;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = 32 * i + 8 * (r >> 2) + rh + (r & 3);
            if (row >= n) continue;
            if (MODE == 0) {
                const int ff = c0 + cl;
                if (ff < a.F) {
                    const float g = acc[i][0][r], u = acc[i][1][r];
                    // hardware exp and reciprocal (~1 ulp each), far inside the fp16 rounding
                    const float v = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                    a.act[(size_t)(slot0 + row) * a.F + ff] = (_Float16)v;
                }
            } else {
                _Float16 *yr = a.y + (size_t)(slot0 + row) * a.H;
                if (c0 + cl < a.H) yr[c0 + cl] = (_Float16)acc[i][0][r];
                if (c1 + cl < a.H) yr[c1 + cl] = (_Float16)acc[i][1][r];
            }
        }
    }
}

// ---------------------------------------------------------------------------

bool mfma_supported(const qq_moe *m) { return m->H % QK == 0 && m->F % QK == 0; }

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

static int tile_cap(const qq_moe *m, int T) { return T * m->K / MG_BM + m->E; }

size_t mfma_work_bytes(const qq_moe *m, int T)
{
    const size_t P = (size_t)T * m->K;
    const size_t cap = (size_t)tile_cap(m, T);
    return al256((size_t)m->E * 4) + al256((size_t)(m->E + 1) * 4) + 2 * al256(P * 4) +
           2 * al256(cap * 4) + 256 + al256((size_t)T * m->H * 2) + al256(P * m->F * 2) +
           al256(P * m->H * 2);
}

void *mfma_xh(const qq_moe *m, int T, char *work)
{
    const size_t P = (size_t)T * m->K;
    const size_t cap = (size_t)tile_cap(m, T);
    return work + al256((size_t)m->E * 4) + al256((size_t)(m->E + 1) * 4) + 2 * al256(P * 4) +
           2 * al256(cap * 4) + 256;
}

int launch_moe_mfma(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                    const MaskBits &mask, const int32_t *idx, const double *w, char *work,
                    bool x_cast)
{
    const size_t P = (size_t)T * m->K;
    const int cap = tile_cap(m, T);
    char *p = work;
    int32_t *counts = reinterpret_cast<int32_t *>(p);  p += al256((size_t)m->E * 4);
    int32_t *offsets = reinterpret_cast<int32_t *>(p); p += al256((size_t)(m->E + 1) * 4);
    int32_t *perm = reinterpret_cast<int32_t *>(p);    p += al256(P * 4);
    int32_t *inv = reinterpret_cast<int32_t *>(p);     p += al256(P * 4);
    DispatchTiles tiles;
    tiles.bm = MG_BM;
    tiles.cap = cap;
    tiles.e = reinterpret_cast<int32_t *>(p);          p += al256((size_t)cap * 4);
    tiles.m0 = reinterpret_cast<int32_t *>(p);         p += al256((size_t)cap * 4);
    tiles.n = reinterpret_cast<int32_t *>(p);          p += 256;
    _Float16 *xh = reinterpret_cast<_Float16 *>(p);    p += al256((size_t)T * m->H * 2);
    _Float16 *act = reinterpret_cast<_Float16 *>(p);   p += al256(P * m->F * 2);
    _Float16 *y = reinterpret_cast<_Float16 *>(p);

    int rc = launch_dispatch(ctx, m, idx, (int)P, mask, counts, offsets, perm, inv, tiles);
    if (rc) return rc;

    if (static_cast<void *>(xh) != mfma_xh(m, T, work)) return set_error(ctx, "mfma: scratch layout");
    if (!x_cast) {   // else the router launch stored the fp16 rows
        const size_t n4 = (size_t)T * m->H / 4;
        prof_begin(ctx, K_CAST_F16);
        QQ_LAUNCH(ctx, cast_f16_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                  reinterpret_cast<const float4 *>(x), reinterpret_cast<uint2 *>(xh), n4);
        prof_end(ctx);
        QQ_HIP(ctx, hipGetLastError());
    }

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

    // XCD-aware grids (mg_item): 8 * ceil(items / 8) workgroups at most
    const unsigned g1 = 8u * (unsigned)(((size_t)cap * ((m->F + 127) / 128) + 7) / 8);
    const unsigned g2 = 8u * (unsigned)(((size_t)cap * ((m->H + 255) / 256) + 7) / 8);
    prof_begin(ctx, K_MFMA_GATEUP);
    QQ_LAUNCH(ctx, moe_mg_kernel<0>, dim3(g1), dim3(MG_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    prof_begin(ctx, K_MFMA_DOWN);
    QQ_LAUNCH(ctx, moe_mg_kernel<1>, dim3(g2), dim3(MG_THREADS), 0, a);
    prof_end(ctx);
    QQ_HIP(ctx, hipGetLastError());
    return launch_combine(ctx, m, T, y, true, inv, w, hidden);
}

}  // namespace qq
