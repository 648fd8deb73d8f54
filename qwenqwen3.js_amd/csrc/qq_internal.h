// qq_internal.h -- shared definitions of the gfx950 MoE library (not installed).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_ext.h>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdarg>
#include <cstring>
#include <vector>

#include "../../include/qq_moe.h"

struct qq_gguf;

namespace qq {

constexpr int QK = 32;        // weights per Q8_0 block
constexpr int QBLK = 34;      // bytes per GGUF Q8_0 block {fp16 d, int8 qs[32]}
constexpr int WAVE = 64;      // CDNA wavefront width
constexpr int MAX_E = 256;    // experts supported by the router and the mask bitset
constexpr int MAX_K = 16;     // experts used per token
// Decode router exchange: SYNC_REPLICAS device-coherent copies of the router
// logit table [MAX_E], each 4608 B apart so that the copies start in
// different DRAM channels ...
constexpr int SYNC_REPLICAS = 16;
constexpr int SYNC_REPLICA_WORDS = 576;
// ... and one table per XCD (XCC_ID < 16), 4 KiB apart.
constexpr int SYNC_LOCAL_TABLES = 16;
constexpr int SYNC_LOCAL_WORDS = 2 * MAX_E;
static_assert(SYNC_REPLICA_WORDS >= 2 * MAX_E, "slot table");
// Batch-1 decode exchange tables (64-bit tagged words): h values [K][F] in a
// group-local and a device-coherent copy, partial down sums [8][K][H], and
// one arrival word per workgroup.
constexpr int SYNC_H_WORDS = MAX_K * 4096;
constexpr int SYNC_P_WORDS = 8 * MAX_K * 2048;
constexpr int SYNC_ARRIVE_WORDS = 256;
// Stack decode (several layers in one launch): each XCD group's residual row
// after each layer, in two alternating sets of 8 tables of up to SYNC_X_WORDS
// words, group-local and device-coherent.
constexpr int SYNC_X_WORDS = 2048;
constexpr int STACK_MAX_LAYERS = 256;
// Fused routing and dispatch of a small token batch: the binary64 partial
// logits [KS][T][E] as two tagged words each (an XCD-local and a device-
// coherent copy), and the expert ids [T][K].
constexpr int SYNC_RP_WORDS = 2 * 8 * 128 * 128;
constexpr int SYNC_RI_WORDS = 1024;
// After a timed-out call the host moves the epoch on by this much: a
// workgroup of that call that started after workgroup 0 advanced the epoch
// wrote words tagged with the next call's tags (up to twice the call's layer
// count past the old epoch), which the next call must not accept.
constexpr uint32_t SYNC_EPOCH_SKIP = 1024;
// Split items of the stream kernels, after the error word and the epoch:
// for each of the two kernels, SEG_CTR_WORDS / 4 32-bit segment counters (one
// per split item, zero between launches), then its generation and a count of
// split items done; after them the segments' partial sums as tagged 64-bit
// words, at most one segment per CU in a launch.
constexpr int SEG_CTR_WORDS = 4096;
constexpr int SEG_PART_WORDS = 4096;
static_assert(SYNC_EPOCH_SKIP >= 2 * STACK_MAX_LAYERS + 2, "epoch skip");

// Expert mask passed by value to kernels (bit e set = expert e skipped).
struct MaskBits {
    uint32_t w[MAX_E / 32];
};

// The word is picked by a chain of selects over the (uniform, kernel-argument)
// words rather than by a dynamic index, which on the device would turn every
// lookup into a memory load of the argument block.
__host__ __device__ inline bool mask_has(const MaskBits &m, int e)
{
    const int i = e >> 5;
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < MAX_E / 32; k++) w = (i == k) ? m.w[k] : w;
    return (w >> (e & 31)) & 1u;
}

}  // namespace qq

// Device-resident Q8_0 matrices after the one-time repack.
//   qs: int8 [n_mats][rows][kp]   (row r = GGUF column r, kp = nb*32, k contiguous)
//   d : fp16 [n_mats][rows][nb]   (scale of block b of row r)
// The repack keeps 34 bytes per 32 weights (the GGUF byte count) but splits
// the 2-byte scale out of each block so that every row of qs is 32-byte
// aligned and a wavefront reads it as 64 lanes x 16 contiguous bytes.
//   dcm: fp16 [n_mats][rows][nbp]  the same scales row by row (nbp = nb
//        rounded up to 8, zero padded), so that one lane reads the scales of
//        8 consecutive blocks of its row in one 16-byte load (decode kernel)
struct qq_tensor {
    int in_dim;     // k (GGUF shape[0])
    int out_dim;    // rows (GGUF shape[1])
    int n_mats;     // experts (GGUF shape[2], 1 for a 2-D tensor)
    int nb;         // blocks per row = ceil(in_dim/32)
    int kp;         // nb*32
    int nbp;        // nb rounded up to a multiple of 8
    int8_t *qs;
    __half *d;
    __half *dcm;
    size_t qs_bytes, d_bytes, dcm_bytes;
};

struct qq_moe {
    int H, F, E, K;
    int router_type;           // QQ_TYPE_F32 or QQ_TYPE_Q8_0
    float *router_f32;         // [E][H] (F32 router; GGUF column e = expert e)
    qq_tensor *router_q8;      // owned copy when the router is Q8_0
    float *bias;               // [E] selection bias (zeros when absent)
    int has_bias;
    int gating;                // QQ_GATING_SIGMOID_BIAS or QQ_GATING_SOFTMAX
    const qq_tensor *gate, *up, *down;   // borrowed; the caller keeps them alive ...
    qq_tensor *owned[3];                 // ... unless the layer owns them (GGUF loader)
};

namespace qq { struct DecodeLayer; }

// Layers of one MoE stack (qq_moe_stack_create): borrowed layer handles, their
// ffn_norm weights, and the decode kernel's device table of their pointers.
struct qq_moe_stack {
    int n = 0;
    std::vector<const qq_moe *> layers;
    std::vector<const float *> norm_w;
    qq::DecodeLayer *table = nullptr;
};

struct qq_ctx {
    int device;
    int num_cus;
    hipStream_t stream;
    int own_stream;
    char err[512];
    // device scratch arena (grown on demand; one arena per context)
    void *scratch;
    size_t scratch_bytes;
    // this device's fixed scratch array (qq_moe_forward_noalloc_dev), from
    // hipGetSymbolAddress at qq_init
    char *noalloc_scratch;
    // pinned host staging for the host-pointer entry points, and its address
    // in the device's address space (the staging copies are kernels)
    void *pinned;
    char *pinned_dev;
    size_t pinned_bytes;
    // timing events of the bench entry points
    hipEvent_t ev0, ev1;
    // device words shared by the kernels of this context: the decode
    // kernel's exchange tables (router logits: SYNC_REPLICAS device-coherent
    // copies and one table per XCD group; h values, partial sums, arrivals),
    // the error word and the decode epoch (advanced on the device by every
    // decode call, so a replayed graph of decode launches sees a fresh epoch
    // each time)
    uint64_t *sync_slots;
    uint64_t *sync_local;
    uint32_t *sync_err;
    // bound on the decode kernel's device-side waits, in 100 MHz wall-clock ticks
    uint64_t dec_wait_ticks;
    uint32_t *sync_epoch;
    uint64_t *sync_hloc, *sync_hdev, *sync_part, *sync_arrive, *sync_hx, *sync_rp, *sync_ri;
    uint32_t *sync_seg;   // SEG_CTR_WORDS stream-kernel segment counters and generations
    uint64_t *seg_part;   // num_cus x SEG_PART_WORDS partial sums
    // device-side waits that timed out on this context so far (counted when
    // the error word is read); device-resident state built across calls (an
    // LFM2 model's conv states and KV cache) is invalid after one
    uint64_t timeouts;
    // set while a call must take the multi-launch path (a host-pointer
    // forward's retry after a timed-out decode launch)
    int batch_only;
    // a graph capture on `stream` is open (qq_capture_begin)
    int capturing;
    // token batches of at least this many rows take the fp16 MFMA path (0: never)
    int mfma_min_tokens;
    // per-kernel event pairs (qq_profile_*): pool of 2*prof_cap events
    int prof_on;
    int prof_kind;             // kernel id of the launches being issued, -1 none
    int prof_n, prof_cap;
    hipEvent_t *prof_ev;
    int *prof_id;
};

namespace qq {

// Kernel ids reported by qq_profile_read (names in api.hip).
enum KernelId {
    K_REPACK = 0,
    K_MATVEC,
    K_ROUTER_LOGITS,
    K_ROUTER_TOPK,
    K_DECODE,
    K_DISPATCH,
    K_GROUPED_GATEUP,
    K_GROUPED_DOWN,
    K_COMBINE,
    K_CAST_F16,
    K_MFMA_GATEUP,
    K_MFMA_DOWN,
    K_STREAM_GATEUP,
    K_STREAM_DOWN,
    K_RMSNORM,
    K_LFM2_EMBED,
    K_LFM2_MV,
    K_LFM2_ATTN,
    K_ROUTE_DISPATCH,
    K_COUNT
};

// Launches between prof_begin(ctx, id) and prof_end(ctx) are reported under
// kernel id `id`.  When profiling is on, each QQ_LAUNCH there takes the next
// event pair of the pool and hands it to hipExtLaunchKernelGGL, which stamps
// the start and end of the dispatch packet itself (no event packets between
// kernels, so the timing matches a kernel trace).
void prof_begin(qq_ctx *ctx, int id);
void prof_end(qq_ctx *ctx);
void prof_slot(qq_ctx *ctx, hipEvent_t *start, hipEvent_t *stop);

#define QQ_LAUNCH(ctx, kernel, grid, block, shm, ...)                                  \
    do {                                                                               \
        hipEvent_t qq_e0_ = nullptr, qq_e1_ = nullptr;                                 \
        ::qq::prof_slot(ctx, &qq_e0_, &qq_e1_);                                        \
        hipExtLaunchKernelGGL(kernel, grid, block, shm, (ctx)->stream, qq_e0_, qq_e1_, 0, \
                              __VA_ARGS__);                                            \
    } while (0)

int set_error(qq_ctx *ctx, const char *fmt, ...);
int check_hip(qq_ctx *ctx, hipError_t e, const char *what);
// Wait for the context stream and report a device-side wait that timed out
// (the decode kernel's error word), in one synchronisation: the word is
// copied to the pinned header by a small kernel behind the enqueued work, or
// already was by the caller's last staging copy (`staged`).
int check_device_error(qq_ctx *ctx, bool staged = false);
// QQ_E_ARG while a graph capture is open on the context's stream.
int no_capture(qq_ctx *ctx, const char *what);
int ensure_scratch(qq_ctx *ctx, size_t bytes);
// The pinned staging buffer: a PIN_HDR-byte header (word 0: the device error
// word as of the last staging copy), then `bytes` of staging from PIN_HDR on.
constexpr size_t PIN_HDR = 256;
int ensure_pinned(qq_ctx *ctx, size_t bytes);
// Copy `bytes` (a multiple of 16) between the pinned staging buffer and
// device memory with one small kernel on the context stream (device
// addresses: ctx->pinned_dev + offset on the host side).
int launch_stage_copy(qq_ctx *ctx, const void *src, void *dst, size_t bytes);

#define QQ_HIP(ctx, call)                                          \
    do {                                                           \
        hipError_t e_ = (call);                                    \
        if (e_ != hipSuccess) return ::qq::check_hip(ctx, e_, #call); \
    } while (0)

// kernel entry wrappers (defined in the .hip files)
int launch_repack_q8_0(qq_ctx *ctx, const uint8_t *gguf_dev, qq_tensor *t);
int launch_q8_0_matvec(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, int ldx,
                       float *y, int ldy, int rows);
// Router of a token batch: binary64 partial logits (router_work_bytes of
// scratch at `part`), then top-K.
constexpr int ROUTER_MAX_SPLIT = 8;
size_t router_work_bytes(const qq_moe *m, int T);
// With xh (T x H fp16) the F32 matrix-core router also stores x rounded to
// fp16 there and sets *xh_done.  With norm, x holds residual rows and the
// router forms rmsnorm(x) itself, bit-equal to launch_rmsnorm's rows (needs
// router_norm_supported and xh).
struct NormArgs;
bool router_norm_supported(const qq_moe *m, const float *hidden, const float *norm_w);
int launch_router_topk(qq_ctx *ctx, const qq_moe *m, const float *x, int T, double *part,
                       int32_t *idx, double *w, float *probs, void *xh = nullptr,
                       bool *xh_done = nullptr, const NormArgs *norm = nullptr);
// Router, top-K and dispatch of a small batch in one launch (all workgroups
// resident, tagged-word exchange through the context's sync area); writes
// what launch_router_topk and launch_dispatch together write.
bool route_dispatch_supported(const qq_ctx *ctx, const qq_moe *m, int T, const float *x);
struct DispatchTiles;
int launch_route_dispatch(qq_ctx *ctx, const qq_moe *m, const float *x, int T, const MaskBits &mask,
                          int32_t *idx, double *w, float *probs, int32_t *counts, int32_t *offsets,
                          int32_t *perm, int32_t *inv, const DispatchTiles &tiles);
// Batch-1 decode in one launch (decode.hip); its exchange tables live in the
// context's sync area, so it needs no scratch.
bool decode_supported(const qq_ctx *ctx, const qq_moe *m, int T);
// ... and a whole stack of such layers in one launch
bool stack_decode_supported(const qq_ctx *ctx, const qq_moe *m);
// ffn_norm folded into a forward: x = rmsnorm(x) * w (w NULL: unit weight).
struct NormArgs {
    const float *w;
    double eps;
};

// The weights of one layer of the batch-1 decode kernel (a stack launch
// reads them from a device table of these).
struct DecodeLayer {
    const float *rf32;    // F32 router [E][H], or
    const int8_t *rq;     // Q8_0 router (block-major)
    const __half *rd;
    const float *bias;
    const int8_t *gq;
    const __half *gdcm;   // gate/up scales row by row (qq_tensor.dcm), nbpH per row
    const int8_t *uq;
    const __half *udcm;
    const int8_t *dq;
    const __half *dd;     // down scales, block-major
    const float *norm_w;  // ffn_norm weight; NULL: unit weight
};
DecodeLayer decode_layer_of(const qq_moe *m, const float *norm_w);
// L layers of equal shape and gating on one residual row in one launch:
// hidden = hidden + MoE_l(rmsnorm(hidden) * norm_w_l) for l = 0 .. L-1
// (layers_dev: a device table of L entries); routing outputs at l K / l E.
int launch_moe_stack_decode(qq_ctx *ctx, const qq_moe *m0, const DecodeLayer *layers_dev, int L, float *hidden,
                            double eps, const MaskBits &mask, int32_t *out_idx, double *out_w, float *out_probs);
int launch_moe_decode(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden,
                      const MaskBits &mask, int32_t *out_idx, double *out_w, float *out_probs,
                      const NormArgs *norm = nullptr, float *out_rec = nullptr);
// The routing record of T rows, rec[t * (2K + E) + ...] = [K idx as float |
// K w rounded to fp32 | E probs], from the router's outputs.
int launch_route_record(qq_ctx *ctx, const int32_t *idx, const double *w, const float *probs, int T,
                        int K, int E, float *rec);
size_t grouped_work_bytes(const qq_moe *m, int T);

// LFM2 single-token forward (lfm2.hip).  Matvec modes: y = W x; hidden +=
// W x; silu(gate x) * (up x); in_proj + short-conv; raw q and k rows with v
// stored into the KV cache.
enum { LM_PLAIN = 0, LM_RESID = 1, LM_SWIGLU = 2, LM_CONV = 3, LM_QKV = 4 };
struct LmLaunch {
    const float *x = nullptr;
    const qq_tensor *mats[3] = {nullptr, nullptr, nullptr};
    int norm = 0;
    const float *norm_w = nullptr;
    double eps = 0.0;
    float *y = nullptr;
    float *state = nullptr;
    const float *kern = nullptr;
    int L = 0, H = 0;
    float *q = nullptr, *kraw = nullptr, *kc = nullptr, *vc = nullptr;
    const float *qn = nullptr, *kn = nullptr;
    int n_heads = 0, n_kv_heads = 0, pos = 0, max_ctx = 0;
    const double *freq = nullptr;
};
int launch_lfm2_mv(qq_ctx *ctx, int mode, const LmLaunch &l);
// Contexts beyond 256 positions run in chunks; `work` holds
// lfm2_attn_work_bytes(n_heads) of per-chunk partials.
size_t lfm2_attn_work_bytes(int n_heads);
// q and kraw are the raw rows of this call (the attention forms the per-head
// norms and RoPE and stores the new k row at position n - 1).
int launch_lfm2_attn(qq_ctx *ctx, const float *q, const float *kraw, const float *qn, const float *kn,
                     const double *freq, double eps, float *kc, const float *vc, int n_heads,
                     int n_kv_heads, int max_ctx, int n, double scale, float *out, double *work);
int launch_lfm2_embed(qq_ctx *ctx, const qq_tensor *t, int token, float *out);
int launch_lfm2_zero(qq_ctx *ctx, float *p, size_t n);
// First byte of a GGUF reader's file (gguf.cpp).
const uint8_t *gguf_base(const ::qq_gguf *g);
// Optional row-tile table written by the dispatch kernel: tile i covers slots
// [m0[i], m0[i] + bm) of expert e[i] (clipped to the expert's count); *n = tiles.
struct DispatchTiles {
    int bm = 0;            // 0: no table
    int cap = 0;           // capacity of e[] / m0[]
    int32_t *e = nullptr;
    int32_t *m0 = nullptr;
    int32_t *n = nullptr;
};
int launch_dispatch(qq_ctx *ctx, const qq_moe *m, const int32_t *idx, int P, const MaskBits &mask,
                    int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                    const DispatchTiles &tiles);
// hidden[t] += sum_k w[t,k] * y[inv[t,k]] (ranks in order, fp32 steps); y rows
// fp32, or fp16 when y_f16 (the MFMA path's outputs).
int launch_combine(qq_ctx *ctx, const qq_moe *m, int T, const void *y, bool y_f16,
                   const int32_t *inv, const double *w, float *hidden);
// fp16 MFMA grouped GEMMs for prefill chunks (mfma.hip); needs H and F
// multiples of 32 and 16-byte aligned activations.
bool mfma_supported(const qq_moe *m);
size_t mfma_work_bytes(const qq_moe *m, int T);
int launch_moe_mfma(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                    const MaskBits &mask, const int32_t *idx, const double *w, char *work,
                    bool x_cast = false);
// Where launch_moe_mfma keeps the fp16 activations in `work` (x_cast: the
// router launch filled them).
void *mfma_xh(const qq_moe *m, int T, char *work);
// Split-fp16 MFMA kernels with weights streamed into registers, for decode
// batches at fp32 accuracy (stream.hip); same shape needs as the MFMA path.
size_t stream_work_bytes(const qq_moe *m, int T);
// The stream path's dispatch outputs inside `work`.
struct StreamDispatch {
    int32_t *counts, *offsets, *perm, *inv;
    DispatchTiles tiles;
};
StreamDispatch stream_dispatch(const qq_moe *m, int T, char *work);
// dispatched: `work` already holds the dispatch of idx (stream_dispatch)
int launch_moe_stream(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                      const MaskBits &mask, const int32_t *idx, const double *w, char *work,
                      bool dispatched = false);
int launch_rmsnorm(qq_ctx *ctx, const float *x, const float *w, float *out, int T, int H,
                   double eps);
int launch_moe_grouped(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                       const MaskBits &mask, const int32_t *idx, const double *w, char *work);

}  // namespace qq
