// api.hip -- the extern "C" boundary declared in include/qq_moe.h.
#include "qq_internal.h"

#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

// Scratch of qq_moe_forward_noalloc_dev: one array per GPU, held until the
// process ends.  Host code reaches it only through the address that
// hipGetSymbolAddress gave for that device (qq_ctx::noalloc_scratch).
static __device__ __align__(256) char scratch[QQ_NOALLOC_SCRATCH_BYTES];

namespace qq {

static thread_local char g_init_err[512] = "";

// 64-bit exchange words of a context's sync area, ahead of the error word
// and the epoch.
static size_t sync_table_words()
{
    return (size_t)SYNC_REPLICAS * SYNC_REPLICA_WORDS + (size_t)SYNC_LOCAL_TABLES * SYNC_LOCAL_WORDS +
           2 * (size_t)SYNC_H_WORDS + SYNC_P_WORDS + SYNC_ARRIVE_WORDS + 4 * 8 * (size_t)SYNC_X_WORDS +
           2 * (size_t)SYNC_RP_WORDS + SYNC_RI_WORDS;
}

int set_error(qq_ctx *ctx, const char *fmt, ...)
{
    char *dst = ctx ? ctx->err : g_init_err;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(dst, 512, fmt, ap);
    va_end(ap);
    return QQ_E_ARG;
}

int check_hip(qq_ctx *ctx, hipError_t e, const char *what)
{
    char *dst = ctx ? ctx->err : g_init_err;
    snprintf(dst, 512, "HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
    return (e == hipErrorOutOfMemory) ? QQ_E_NOMEM : QQ_E_HIP;
}

int ensure_scratch(qq_ctx *ctx, size_t bytes)
{
    if (bytes <= ctx->scratch_bytes) return QQ_OK;
    if (ctx->capturing)
        return set_error(ctx, "call needs %zu scratch bytes, the context holds %zu: run it once "
                              "before capturing", bytes, ctx->scratch_bytes);
    // in-flight kernels may still use the old arena
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    const size_t sz = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    QQ_HIP(ctx, hipMalloc(&ctx->scratch, sz));
    ctx->scratch_bytes = sz;
    return QQ_OK;
}

int ensure_pinned(qq_ctx *ctx, size_t bytes)
{
    bytes += PIN_HDR;
    if (bytes <= ctx->pinned_bytes) return QQ_OK;
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->pinned) (void)hipHostFree(ctx->pinned);
    ctx->pinned = nullptr;
    ctx->pinned_bytes = 0;
    ctx->pinned_dev = nullptr;
    const size_t sz = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    // coherent: the staging kernels read and write it across calls, so no GPU
    // cache may keep an old copy of a line
    QQ_HIP(ctx, hipHostMalloc(&ctx->pinned, sz, hipHostMallocMapped | hipHostMallocCoherent));
    void *d = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&d, ctx->pinned, 0);
    if (e != hipSuccess) {
        (void)hipHostFree(ctx->pinned);
        ctx->pinned = nullptr;
        return check_hip(ctx, e, "hipHostGetDevicePointer");
    }
    ctx->pinned_dev = static_cast<char *>(d);
    ctx->pinned_bytes = sz;
    return QQ_OK;
}

// Small host <-> device transfers (the 8-16 KB rows of a decode call) as one
// copy kernel over the mapped pinned buffer: the GPU reads or writes host
// memory over PCIe directly instead of a DMA-engine transfer.
// The device error word rides along to the pinned header, so the host learns
// of a timed-out device wait from the same synchronisation.
__global__ __launch_bounds__(256) void stage_copy_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                         size_t n, const uint32_t *__restrict__ err,
                                                         uint32_t *__restrict__ err_dst)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
    if (blockIdx.x == 0 && threadIdx.x == 0) *err_dst = *err;
}

int launch_stage_copy(qq_ctx *ctx, const void *src, void *dst, size_t bytes)
{
    if (bytes % 16) return set_error(ctx, "stage_copy: %zu bytes is not a multiple of 16", bytes);
    if (!ctx->pinned_dev) return set_error(ctx, "stage_copy: no pinned staging buffer");
    const size_t n = bytes / 16;
    const unsigned g = (unsigned)std::max<size_t>(std::min<size_t>((n + 255) / 256, 256), 1);
    QQ_LAUNCH(ctx, stage_copy_kernel, dim3(g), dim3(256), 0, static_cast<const uint4 *>(src),
              static_cast<uint4 *>(dst), n, static_cast<const uint32_t *>(ctx->sync_err),
              reinterpret_cast<uint32_t *>(ctx->pinned_dev));
    QQ_HIP(ctx, hipGetLastError());
    return QQ_OK;
}

// Entry points that copy to or from the host, synchronise or allocate cannot
// be recorded into a graph.
int no_capture(qq_ctx *ctx, const char *what)
{
    if (ctx && ctx->capturing)
        return set_error(ctx, "%s cannot run while a graph capture is open", what);
    return QQ_OK;
}

static const char *const kKernelNames[K_COUNT] = {
    "repack_q8_0",      "q8_0_matvec",    "router_logits",  "router_topk",   "moe_decode",
    "dispatch",       "grouped_gateup", "grouped_down",  "combine",
    "cast_f16",         "mfma_gateup",    "mfma_down",      "stream_gateup", "stream_down",
    "rmsnorm", "lfm2_embed", "lfm2_matvec", "lfm2_attention", "route_dispatch",
};

// After a timed-out call: clear the error word and move the epoch on by
// SYNC_EPOCH_SKIP, so no exchange word that call left behind carries a tag a
// later call accepts.  (A workgroup of the failed launch that started after
// workgroup 0 advanced the epoch used the next call's tags.)  The stream has
// drained, so no workgroup of that launch still runs.
__global__ void sync_recover_kernel(uint32_t *err, uint32_t *epoch)
{
    *err = 0;
    *epoch = *epoch + SYNC_EPOCH_SKIP;
}

// Every exchange word of the context (test hook qq_debug_plant_words).
__global__ void sync_plant_kernel(uint64_t *w, size_t n, uint64_t word)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        w[i] = word;
}

// Read and clear the device error word; non-zero means a bounded device-side
// wait expired (the results of that call are not valid).
int check_device_error(qq_ctx *ctx, bool staged)
{
    if (!staged) {   // the error word alone, behind the enqueued work
        int rc = ensure_pinned(ctx, 0);
        if (!rc) rc = launch_stage_copy(ctx, nullptr, nullptr, 0);
        if (rc) return rc;
    }
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    volatile uint32_t *word = static_cast<volatile uint32_t *>(ctx->pinned);
    const uint32_t e = *word;
    if (e) {
        *word = 0;
        ctx->timeouts++;
        hipLaunchKernelGGL(sync_recover_kernel, dim3(1), dim3(1), 0, ctx->stream, ctx->sync_err, ctx->sync_epoch);
        QQ_HIP(ctx, hipGetLastError());
        QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        snprintf(ctx->err, sizeof ctx->err,
                 "a device-side wait of the decode, fused routing or split-item exchange timed out (code %u)", e);
        return QQ_E_HIP;
    }
    return QQ_OK;
}

void prof_begin(qq_ctx *ctx, int id) { ctx->prof_kind = id; }

void prof_end(qq_ctx *ctx) { ctx->prof_kind = -1; }

void prof_slot(qq_ctx *ctx, hipEvent_t *start, hipEvent_t *stop)
{
    *start = *stop = nullptr;
    if (!ctx->prof_on || ctx->prof_kind < 0 || ctx->prof_n >= ctx->prof_cap) return;
    const int i = ctx->prof_n++;
    ctx->prof_id[i] = ctx->prof_kind;
    *start = ctx->prof_ev[2 * i];
    *stop = ctx->prof_ev[2 * i + 1];
}

static void prof_free(qq_ctx *ctx)
{
    for (int i = 0; i < 2 * ctx->prof_cap; i++) (void)hipEventDestroy(ctx->prof_ev[i]);
    free(ctx->prof_ev);
    free(ctx->prof_id);
    ctx->prof_ev = nullptr;
    ctx->prof_id = nullptr;
    ctx->prof_cap = ctx->prof_n = 0;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

static int mask_from_bytes(qq_ctx *ctx, const uint8_t *mask, int E, MaskBits *out)
{
    memset(out, 0, sizeof(*out));
    if (!mask) return QQ_OK;
    if (E > MAX_E) return set_error(ctx, "expert count %d exceeds %d", E, MAX_E);
    for (int e = 0; e < E; e++)
        if (mask[e]) out->w[e >> 5] |= 1u << (e & 31);
    return QQ_OK;
}

static int tensor_alloc(qq_ctx *ctx, int in_dim, int out_dim, int n_mats, qq_tensor **out)
{
    if (in_dim <= 0 || out_dim <= 0 || n_mats <= 0)
        return set_error(ctx, "bad Q8_0 shape [%d, %d, %d]", in_dim, out_dim, n_mats);
    qq_tensor *t = new (std::nothrow) qq_tensor();
    if (!t) return set_error(ctx, "host allocation failed");
    t->in_dim = in_dim;
    t->out_dim = out_dim;
    t->n_mats = n_mats;
    t->nb = (in_dim + QK - 1) / QK;
    t->kp = t->nb * QK;
    const size_t rows = (size_t)n_mats * out_dim;
    t->nbp = (t->nb + 7) & ~7;
    t->qs_bytes = rows * t->kp;
    t->d_bytes = rows * t->nb * sizeof(__half);
    // + 128 bytes: a 16-byte scale load of the last row may start up to 56
    // blocks past its end (the blocks it covers there are masked)
    t->dcm_bytes = rows * t->nbp * sizeof(__half) + 128;
    hipError_t e = hipMalloc(&t->qs, t->qs_bytes);
    if (e == hipSuccess) e = hipMalloc(&t->d, t->d_bytes);
    if (e == hipSuccess) e = hipMalloc(&t->dcm, t->dcm_bytes);
    // the padding stays zero (same stream as the repack that fills the rest)
    if (e == hipSuccess) e = hipMemsetAsync(t->dcm, 0, t->dcm_bytes, ctx->stream);
    if (e != hipSuccess) {
        if (t->qs) (void)hipFree(t->qs);
        if (t->d) (void)hipFree(t->d);
        if (t->dcm) (void)hipFree(t->dcm);
        delete t;
        return check_hip(ctx, e, "hipMalloc(Q8_0 tensor)");
    }
    *out = t;
    return QQ_OK;
}

}  // namespace qq

using namespace qq;

extern "C" {

int qq_init(int device, qq_ctx **out)
{
    if (!out) return set_error(nullptr, "qq_init: out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        snprintf(g_init_err, sizeof g_init_err, "no HIP device available (%s)",
                 e == hipSuccess ? "0 devices" : hipGetErrorString(e));
        return QQ_E_NODEV;
    }
    if (device < 0 || device >= n) {
        snprintf(g_init_err, sizeof g_init_err, "device %d out of range (%d devices)", device, n);
        return QQ_E_NODEV;
    }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return check_hip(nullptr, e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_init_err, sizeof g_init_err, "device %d is %s, this library is built for gfx950",
                 device, prop.gcnArchName);
        return QQ_E_NODEV;
    }
    if ((e = hipSetDevice(device)) != hipSuccess) return check_hip(nullptr, e, "hipSetDevice");
    qq_ctx *ctx = new (std::nothrow) qq_ctx();
    if (!ctx) return set_error(nullptr, "host allocation failed");
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    // this device's copy of the fixed scratch array (the device is current)
    void *fixed = nullptr;
    if ((e = hipGetSymbolAddress(&fixed, HIP_SYMBOL(scratch))) != hipSuccess || !fixed) {
        delete ctx;
        return check_hip(nullptr, e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    }
    ctx->noalloc_scratch = static_cast<char *>(fixed);
    if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete ctx;
        return check_hip(nullptr, e, "hipStreamCreate");
    }
    ctx->own_stream = 1;
    ctx->prof_kind = -1;
    ctx->mfma_min_tokens = QQ_MFMA_MIN_TOKENS_DEFAULT;
    ctx->dec_wait_ticks = (uint64_t)QQ_WAIT_LIMIT_US_DEFAULT * 100;
    if ((e = hipEventCreate(&ctx->ev0)) != hipSuccess || (e = hipEventCreate(&ctx->ev1)) != hipSuccess) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return check_hip(nullptr, e, "hipEventCreate");
    }
    void *sync = nullptr;
    const size_t sync_bytes = sync_table_words() * sizeof(uint64_t) + 512 + SEG_CTR_WORDS * 4 + 256 +
                              (size_t)ctx->num_cus * SEG_PART_WORDS * 8;
    if ((e = hipMalloc(&sync, sync_bytes)) != hipSuccess || (e = hipMemset(sync, 0, sync_bytes)) != hipSuccess) {
        if (sync) (void)hipFree(sync);
        (void)hipEventDestroy(ctx->ev0);
        (void)hipEventDestroy(ctx->ev1);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return check_hip(nullptr, e, "sync area");
    }
    ctx->sync_slots = static_cast<uint64_t *>(sync);
    ctx->sync_local = ctx->sync_slots + SYNC_REPLICAS * SYNC_REPLICA_WORDS;
    ctx->sync_hloc = ctx->sync_local + SYNC_LOCAL_TABLES * SYNC_LOCAL_WORDS;
    ctx->sync_hdev = ctx->sync_hloc + SYNC_H_WORDS;
    ctx->sync_part = ctx->sync_hdev + SYNC_H_WORDS;
    ctx->sync_arrive = ctx->sync_part + SYNC_P_WORDS;
    ctx->sync_hx = ctx->sync_arrive + SYNC_ARRIVE_WORDS;
    ctx->sync_rp = ctx->sync_hx + 4 * 8 * SYNC_X_WORDS;
    ctx->sync_ri = ctx->sync_rp + 2 * SYNC_RP_WORDS;   // after the XCD-local and device copies
    // error word and epoch each on a 128-byte line of their own
    ctx->sync_err = reinterpret_cast<uint32_t *>(ctx->sync_ri + SYNC_RI_WORDS);
    ctx->sync_epoch = ctx->sync_err + 32;
    ctx->sync_seg = ctx->sync_err + 128;
    ctx->seg_part = reinterpret_cast<uint64_t *>(((uintptr_t)(ctx->sync_seg + SEG_CTR_WORDS) + 255) & ~(uintptr_t)255);
    ctx->capturing = 0;
    *out = ctx;
    return QQ_OK;
}

void qq_destroy(qq_ctx *ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->capturing) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(ctx->stream, &g);
        if (g) (void)hipGraphDestroy(g);
    }
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->pinned) (void)hipHostFree(ctx->pinned);
    (void)hipEventDestroy(ctx->ev0);
    (void)hipEventDestroy(ctx->ev1);
    if (ctx->sync_slots) (void)hipFree(ctx->sync_slots);
    prof_free(ctx);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char *qq_last_error(const qq_ctx *ctx) { return ctx ? ctx->err : g_init_err; }

int qq_set_stream(qq_ctx *ctx, void *hip_stream)
{
    if (!ctx) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_set_stream")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    if (hip_stream) {
        ctx->stream = static_cast<hipStream_t>(hip_stream);
        ctx->own_stream = 0;
    } else {
        QQ_HIP(ctx, hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
        ctx->own_stream = 1;
    }
    return QQ_OK;
}

int qq_synchronize(qq_ctx *ctx)
{
    if (!ctx) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_synchronize")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    return check_device_error(ctx);
}

// ---- Q8_0 tensors ---------------------------------------------------------

static int upload_common(qq_ctx *ctx, const void *src, bool src_on_device, size_t nbytes,
                         int in_dim, int out_dim, int n_mats, qq_tensor **out)
{
    if (!ctx || !out || !src) return set_error(ctx, "qq_q8_0_upload: NULL argument");
    if (int rc = no_capture(ctx, "qq_q8_0_upload")) return rc;
    *out = nullptr;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    qq_tensor *t = nullptr;
    int rc = tensor_alloc(ctx, in_dim, out_dim, n_mats, &t);
    if (rc) return rc;
    const size_t need = (size_t)n_mats * out_dim * t->nb * QBLK;
    if (nbytes < need) {
        qq_tensor_release(ctx, t);
        return set_error(ctx, "Q8_0 tensor [%d, %d, %d] needs %zu bytes, got %zu", in_dim, out_dim,
                         n_mats, need, nbytes);
    }
    const uint8_t *dev_src = static_cast<const uint8_t *>(src);
    void *staging = nullptr;
    if (!src_on_device) {
        hipError_t e = hipMalloc(&staging, need);
        if (e != hipSuccess) {
            qq_tensor_release(ctx, t);
            return check_hip(ctx, e, "hipMalloc(upload staging)");
        }
        e = hipMemcpyAsync(staging, src, need, hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(staging);
            qq_tensor_release(ctx, t);
            return check_hip(ctx, e, "hipMemcpy(upload)");
        }
        dev_src = static_cast<const uint8_t *>(staging);
    }
    rc = launch_repack_q8_0(ctx, dev_src, t);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (staging) (void)hipFree(staging);
    if (rc == QQ_OK && e != hipSuccess) rc = check_hip(ctx, e, "repack");
    if (rc) {
        qq_tensor_release(ctx, t);
        return rc;
    }
    *out = t;
    return QQ_OK;
}

int qq_q8_0_upload(qq_ctx *ctx, const void *gguf_bytes, size_t nbytes, int in_dim, int out_dim,
                   int n_mats, qq_tensor **out)
{
    return upload_common(ctx, gguf_bytes, false, nbytes, in_dim, out_dim, n_mats, out);
}

int qq_q8_0_upload_dev(qq_ctx *ctx, const void *gguf_bytes_dev, size_t nbytes, int in_dim,
                       int out_dim, int n_mats, qq_tensor **out)
{
    return upload_common(ctx, gguf_bytes_dev, true, nbytes, in_dim, out_dim, n_mats, out);
}

int qq_tensor_release(qq_ctx *ctx, qq_tensor *t)
{
    if (!t) return QQ_OK;
    if (int rc = no_capture(ctx, "qq_tensor_release")) return rc;
    if (ctx) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    if (t->qs) (void)hipFree(t->qs);
    if (t->d) (void)hipFree(t->d);
    if (t->dcm) (void)hipFree(t->dcm);
    delete t;
    return QQ_OK;
}

static int matvec_check(qq_ctx *ctx, const qq_tensor *t, int mat, int rows)
{
    if (!ctx) return QQ_E_ARG;
    if (!t) return set_error(ctx, "matvec: NULL tensor");
    if (mat < 0 || mat >= t->n_mats) return set_error(ctx, "matvec: matrix %d of %d", mat, t->n_mats);
    if (rows < 0) return set_error(ctx, "matvec: rows %d", rows);
    return QQ_OK;
}

int qq_q8_0_matvec_dev(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x_dev, float *y_dev,
                       int rows)
{
    int rc = matvec_check(ctx, t, mat, rows);
    if (rc) return rc;
    if (rows == 0) return QQ_OK;
    if (!x_dev || !y_dev) return set_error(ctx, "matvec: NULL buffer");
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    return launch_q8_0_matvec(ctx, t, mat, x_dev, t->in_dim, y_dev, t->out_dim, rows);
}

int qq_q8_0_matvec(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, float *y, int rows)
{
    int rc = matvec_check(ctx, t, mat, rows);
    if (rc) return rc;
    if (rows == 0) return QQ_OK;
    if (!x || !y) return set_error(ctx, "matvec: NULL buffer");
    if ((rc = no_capture(ctx, "qq_q8_0_matvec"))) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    const size_t xb = (size_t)rows * t->in_dim * 4, yb = (size_t)rows * t->out_dim * 4;
    if ((rc = ensure_scratch(ctx, align256(xb) + yb))) return rc;
    if ((rc = ensure_pinned(ctx, align256(xb) + yb))) return rc;   // staging: x in, y out
    char *ph = static_cast<char *>(ctx->pinned) + PIN_HDR;
    char *pd = ctx->pinned_dev + PIN_HDR;
    float *dx = static_cast<float *>(ctx->scratch);
    float *dy = reinterpret_cast<float *>(static_cast<char *>(ctx->scratch) + align256(xb));
    memcpy(ph, x, xb);
    if ((rc = launch_stage_copy(ctx, pd, dx, align256(xb)))) return rc;
    if ((rc = launch_q8_0_matvec(ctx, t, mat, dx, t->in_dim, dy, t->out_dim, rows))) return rc;
    if ((rc = launch_stage_copy(ctx, dy, pd + align256(xb), (yb + 15) & ~(size_t)15))) return rc;
    if ((rc = check_device_error(ctx, true))) return rc;
    memcpy(y, ph + align256(xb), yb);
    return QQ_OK;
}

// ---- MoE layer --------------------------------------------------------------

int qq_moe_create(qq_ctx *ctx, const void *router_bytes, int router_type, const float *bias,
                  const qq_tensor *gate, const qq_tensor *up, const qq_tensor *down, int H, int F,
                  int E, int K, qq_moe **out)
{
    if (!ctx || !out) return QQ_E_ARG;
    *out = nullptr;
    if (!router_bytes || !gate || !up || !down) return set_error(ctx, "qq_moe_create: NULL tensor");
    if (H <= 0 || F <= 0 || E <= 0 || K <= 0 || K > E || E > MAX_E || K > MAX_K)
        return set_error(ctx, "qq_moe_create: bad dims H=%d F=%d E=%d K=%d (E<=%d, K<=%d)", H, F, E, K,
                         MAX_E, MAX_K);
    if (H > 4096 || F > 4096) return set_error(ctx, "qq_moe_create: H and F must be <= 4096");
    if (gate->in_dim != H || gate->out_dim != F || gate->n_mats != E || up->in_dim != H ||
        up->out_dim != F || up->n_mats != E)
        return set_error(ctx, "qq_moe_create: gate/up must be [%d, %d, %d]", H, F, E);
    if (down->in_dim != F || down->out_dim != H || down->n_mats != E)
        return set_error(ctx, "qq_moe_create: down must be [%d, %d, %d]", F, H, E);
    if (router_type != QQ_TYPE_F32 && router_type != QQ_TYPE_Q8_0)
        return set_error(ctx, "Unsupported tensor type for matmul: %d", router_type);
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    qq_moe *m = new (std::nothrow) qq_moe();
    if (!m) return set_error(ctx, "host allocation failed");
    m->H = H;
    m->F = F;
    m->E = E;
    m->K = K;
    m->router_type = router_type;
    m->gate = gate;
    m->up = up;
    m->down = down;
    m->has_bias = bias != nullptr;
    m->gating = QQ_GATING_SIGMOID_BIAS;
    int rc = QQ_OK;
    hipError_t e = hipMalloc(&m->bias, (size_t)E * 4);
    if (e == hipSuccess) {
        e = bias ? hipMemcpy(m->bias, bias, (size_t)E * 4, hipMemcpyHostToDevice)
                 : hipMemset(m->bias, 0, (size_t)E * 4);
    }
    if (e != hipSuccess) rc = check_hip(ctx, e, "router bias");
    if (rc == QQ_OK) {
        if (router_type == QQ_TYPE_F32) {
            e = hipMalloc(&m->router_f32, (size_t)E * H * 4);
            if (e == hipSuccess) e = hipMemcpy(m->router_f32, router_bytes, (size_t)E * H * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = check_hip(ctx, e, "router upload");
        } else {
            const size_t nb = (size_t)(H + QK - 1) / QK;
            rc = qq_q8_0_upload(ctx, router_bytes, (size_t)E * nb * QBLK, H, E, 1, &m->router_q8);
        }
    }
    if (rc) {
        qq_moe_release(ctx, m);
        return rc;
    }
    *out = m;
    return QQ_OK;
}

int qq_moe_set_gating(qq_ctx *ctx, qq_moe *m, int gating)
{
    if (!ctx) return QQ_E_ARG;
    if (!m) return set_error(ctx, "moe_set_gating: NULL layer");
    if (gating != QQ_GATING_SIGMOID_BIAS && gating != QQ_GATING_SOFTMAX)
        return set_error(ctx, "moe_set_gating: unknown gating %d", gating);
    m->gating = gating;
    return QQ_OK;
}

int qq_moe_release(qq_ctx *ctx, qq_moe *m)
{
    if (!m) return QQ_OK;
    if (int rc = no_capture(ctx, "qq_moe_release")) return rc;
    if (ctx) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    if (m->bias) (void)hipFree(m->bias);
    if (m->router_f32) (void)hipFree(m->router_f32);
    if (m->router_q8) qq_tensor_release(ctx, m->router_q8);
    for (qq_tensor *t : m->owned) qq_tensor_release(ctx, t);
    delete m;
    return QQ_OK;
}

// Scratch of one forward.  Decode (T == 1): the decode kernels' own area.
// Token batches: logits | idx | w | grouped work, per chunk of tokens.
constexpr int T_CHUNK = 4096;

// Path of one chunk of tn tokens: the fp16 MFMA GEMMs for chunks of at least
// ctx->mfma_min_tokens rows; below that the split-fp16 streaming kernels
// (fp32 accuracy); the fp32 vector-unit grouped kernels for shapes neither
// takes (H or F not a multiple of 32, unaligned activations).
enum Path { PATH_MFMA, PATH_STREAM, PATH_GROUPED };

// The one-launch decode kernel for this call (the host-pointer forward turns
// it off for its retry after a timed-out wait).
static bool use_decode(const qq_ctx *ctx, const qq_moe *m, int T)
{
    return !ctx->batch_only && decode_supported(ctx, m, T);
}

// The one-launch router + top-K + dispatch for a stream-path chunk (off for
// the host-pointer forward's retry, like the decode kernel).
static bool use_route_fused(const qq_ctx *ctx, const qq_moe *m, int T, const float *x)
{
    return !ctx->batch_only && route_dispatch_supported(ctx, m, T, x);
}

static Path chunk_path(const qq_ctx *ctx, const qq_moe *m, int tn, const float *x)
{
    if (!mfma_supported(m) || ((uintptr_t)x & 15) != 0) return PATH_GROUPED;
    if (ctx->mfma_min_tokens > 0 && tn >= ctx->mfma_min_tokens) return PATH_MFMA;
    return PATH_STREAM;
}

static size_t forward_scratch(const qq_ctx *ctx, const qq_moe *m, int T)
{
    if (use_decode(ctx, m, T)) return 0;
    const int Tc = T < T_CHUNK ? T : T_CHUNK;
    size_t work = grouped_work_bytes(m, Tc);
    if (mfma_supported(m)) {
        // the first chunk is the largest; a last, smaller chunk may take another path
        work = std::max(work, stream_work_bytes(m, Tc));
        if (ctx->mfma_min_tokens > 0 && Tc >= ctx->mfma_min_tokens)
            work = std::max(work, mfma_work_bytes(m, Tc));
    }
    return align256(router_work_bytes(m, Tc)) + align256((size_t)Tc * m->K * 4) +
           align256((size_t)Tc * m->K * 8) + align256(work);
}

// x, hidden (and the optional outputs) are device pointers; s holds
// forward_scratch(ctx, m, T) bytes (256-byte aligned).  Allocates nothing.
// With norm, x = rmsnorm(hidden) of each chunk is formed first: by the
// router launch itself on the MFMA path (router_norm_supported), else into
// xn (T x H floats) and x is ignored.
static int forward_run(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                       const MaskBits &mask, int32_t *idx, double *w, float *probs, char *s,
                       const NormArgs *norm = nullptr, float *xn = nullptr)
{
    int rc = QQ_OK;
    if (use_decode(ctx, m, T))
        return launch_moe_decode(ctx, m, norm ? hidden : x, hidden, mask, idx, w, probs, norm);
    const size_t Tc = (size_t)(T < T_CHUNK ? T : T_CHUNK);
    double *part = reinterpret_cast<double *>(s);
    int32_t *sidx = reinterpret_cast<int32_t *>(s + align256(router_work_bytes(m, (int)Tc)));
    double *sw = reinterpret_cast<double *>(reinterpret_cast<char *>(sidx) + align256(Tc * m->K * 4));
    char *work = reinterpret_cast<char *>(sw) + align256(Tc * m->K * 8);
    for (int t0 = 0; t0 < T; t0 += T_CHUNK) {
        const int tn = (T - t0 < T_CHUNK) ? T - t0 : T_CHUNK;
        int32_t *ci = idx ? idx + (size_t)t0 * m->K : sidx;
        double *cw = w ? w + (size_t)t0 * m->K : sw;
        float *cp = probs ? probs + (size_t)t0 * m->E : nullptr;
        const float *cx = (norm ? xn : x) + (size_t)t0 * m->H;
        float *ch = hidden + (size_t)t0 * m->H;
        const Path path = chunk_path(ctx, m, tn, cx);
        // on the MFMA path the router launch also writes the fp16 rows
        void *xh = path == PATH_MFMA ? mfma_xh(m, tn, work) : nullptr;
        bool xh_done = false;
        const bool nfused = norm && path == PATH_MFMA && router_norm_supported(m, ch, norm->w);
        if (norm && !nfused &&
            (rc = launch_rmsnorm(ctx, ch, norm->w, xn + (size_t)t0 * m->H, tn, m->H, norm->eps)))
            return rc;
        if (path == PATH_STREAM && use_route_fused(ctx, m, tn, cx)) {
            const StreamDispatch d = stream_dispatch(m, tn, work);
            if ((rc = launch_route_dispatch(ctx, m, cx, tn, mask, ci, cw, cp, d.counts, d.offsets, d.perm,
                                            d.inv, d.tiles)))
                return rc;
            if ((rc = launch_moe_stream(ctx, m, cx, ch, tn, mask, ci, cw, work, true))) return rc;
            continue;
        }
        if ((rc = launch_router_topk(ctx, m, nfused ? ch : cx, tn, part, ci, cw, cp, xh, &xh_done,
                                     nfused ? norm : nullptr)))
            return rc;
        switch (path) {
        case PATH_MFMA: rc = launch_moe_mfma(ctx, m, cx, ch, tn, mask, ci, cw, work, xh_done); break;
        case PATH_STREAM: rc = launch_moe_stream(ctx, m, cx, ch, tn, mask, ci, cw, work); break;
        default: rc = launch_moe_grouped(ctx, m, cx, ch, tn, mask, ci, cw, work); break;
        }
        if (rc) return rc;
    }
    return QQ_OK;
}

// The same with the context's arena as scratch, from `base` on.
static int forward_impl(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                        const MaskBits &mask, int32_t *idx, double *w, float *probs, size_t base)
{
    const int rc = ensure_scratch(ctx, base + forward_scratch(ctx, m, T));
    if (rc) return rc;
    return forward_run(ctx, m, x, hidden, T, mask, idx, w, probs, static_cast<char *>(ctx->scratch) + base);
}

static int forward_check(qq_ctx *ctx, const qq_moe *m, int T)
{
    if (!ctx) return QQ_E_ARG;
    if (!m) return set_error(ctx, "moe_forward: NULL layer");
    if (T < 0) return set_error(ctx, "moe_forward: T=%d", T);
    return QQ_OK;
}

int qq_moe_forward_dev(qq_ctx *ctx, const qq_moe *m, const float *x_dev, float *hidden_dev, int T,
                       const uint8_t *mask, int32_t *idx_dev, double *w_dev, float *probs_dev)
{
    int rc = forward_check(ctx, m, T);
    if (rc || T == 0) return rc;
    if (!x_dev || !hidden_dev) return set_error(ctx, "moe_forward: NULL buffer");
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    MaskBits mb;
    if ((rc = mask_from_bytes(ctx, mask, m->E, &mb))) return rc;
    return forward_impl(ctx, m, x_dev, hidden_dev, T, mb, idx_dev, w_dev, probs_dev, 0);
}

int qq_moe_forward_noalloc_dev(qq_ctx *ctx, const qq_moe *m, const float *x_dev, float *hidden_dev, int T,
                               const uint8_t *mask, int32_t *idx_dev, double *w_dev, float *probs_dev)
{
    int rc = forward_check(ctx, m, T);
    if (rc || T == 0) return rc;
    if (!x_dev || !hidden_dev) return set_error(ctx, "moe_forward_noalloc: NULL buffer");
    const size_t need = forward_scratch(ctx, m, T);
    if (need > QQ_NOALLOC_SCRATCH_BYTES)
        return set_error(ctx, "moe_forward_noalloc: T=%d needs %zu scratch bytes, the fixed array holds %zu", T,
                         need, (size_t)QQ_NOALLOC_SCRATCH_BYTES);
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    MaskBits mb;
    if ((rc = mask_from_bytes(ctx, mask, m->E, &mb))) return rc;
    return forward_run(ctx, m, x_dev, hidden_dev, T, mb, idx_dev, w_dev, probs_dev, ctx->noalloc_scratch);
}

int qq_moe_forward_norm_dev(qq_ctx *ctx, const qq_moe *m, float *hidden_dev, const float *norm_w_dev,
                            double eps, int T, const uint8_t *mask, int32_t *idx_dev,
                            double *w_dev, float *probs_dev)
{
    int rc = forward_check(ctx, m, T);
    if (rc || T == 0) return rc;
    if (!hidden_dev) return set_error(ctx, "moe_forward_norm: NULL buffer");
    if (!(eps >= 0.0)) return set_error(ctx, "moe_forward_norm: eps %g", eps);
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    MaskBits mb;
    if ((rc = mask_from_bytes(ctx, mask, m->E, &mb))) return rc;
    const NormArgs norm{norm_w_dev, eps};
    if (decode_supported(ctx, m, T)) {
        // every workgroup of the decode kernel normalises the row itself
        return launch_moe_decode(ctx, m, hidden_dev, hidden_dev, mb, idx_dev, w_dev, probs_dev, &norm);
    }
    // x = rmsnorm(hidden), chunk by chunk, at the start of the scratch (or
    // formed by the router launch), then the forward
    const size_t xb = align256((size_t)T * m->H * 4);
    if ((rc = ensure_scratch(ctx, xb + forward_scratch(ctx, m, T)))) return rc;
    float *x = static_cast<float *>(ctx->scratch);
    return forward_run(ctx, m, x, hidden_dev, T, mb, idx_dev, w_dev, probs_dev,
                       static_cast<char *>(ctx->scratch) + xb, &norm, x);
}

// ---- MoE stacks ------------------------------------------------------------

int qq_moe_stack_create(qq_ctx *ctx, const qq_moe *const *layers, const float *const *norm_w_dev, int n,
                        qq_moe_stack **out)
{
    if (!ctx || !out) return QQ_E_ARG;
    *out = nullptr;
    if (int rc = no_capture(ctx, "qq_moe_stack_create")) return rc;
    if (!layers || n < 1 || n > STACK_MAX_LAYERS)
        return set_error(ctx, "moe_stack_create: %d layers (1 .. %d)", n, STACK_MAX_LAYERS);
    const qq_moe *m0 = layers[0];
    for (int l = 0; l < n; l++) {
        const qq_moe *m = layers[l];
        if (!m) return set_error(ctx, "moe_stack_create: layer %d is NULL", l);
        if (m->H != m0->H || m->F != m0->F || m->E != m0->E || m->K != m0->K || m->gating != m0->gating ||
            m->router_type != m0->router_type)
            return set_error(ctx, "moe_stack_create: layer %d differs from layer 0 in shape, gating or router type", l);
    }
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    qq_moe_stack *st = new (std::nothrow) qq_moe_stack();
    if (!st) return set_error(ctx, "host allocation failed");
    st->n = n;
    st->layers.assign(layers, layers + n);
    st->norm_w.assign((size_t)n, nullptr);
    if (norm_w_dev) st->norm_w.assign(norm_w_dev, norm_w_dev + n);
    std::vector<DecodeLayer> table((size_t)n);
    for (int l = 0; l < n; l++) table[l] = decode_layer_of(layers[l], st->norm_w[l]);
    hipError_t e = hipMalloc(&st->table, sizeof(DecodeLayer) * n);
    if (e == hipSuccess) e = hipMemcpy(st->table, table.data(), sizeof(DecodeLayer) * n, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (st->table) (void)hipFree(st->table);
        delete st;
        return check_hip(ctx, e, "moe_stack_create: layer table");
    }
    *out = st;
    return QQ_OK;
}

int qq_moe_stack_release(qq_ctx *ctx, qq_moe_stack *st)
{
    if (!ctx) return QQ_E_ARG;
    if (!st) return QQ_OK;
    if (int rc = no_capture(ctx, "qq_moe_stack_release")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (st->table) (void)hipFree(st->table);
    delete st;
    return QQ_OK;
}

int qq_moe_stack_forward_dev(qq_ctx *ctx, const qq_moe_stack *st, float *hidden_dev, double eps, int T,
                             const uint8_t *mask, int32_t *idx_dev, double *w_dev, float *probs_dev)
{
    if (!ctx) return QQ_E_ARG;
    if (!st) return set_error(ctx, "moe_stack_forward: NULL stack");
    if (T < 0) return set_error(ctx, "moe_stack_forward: T=%d", T);
    if (T == 0) return QQ_OK;
    if (!hidden_dev) return set_error(ctx, "moe_stack_forward: NULL buffer");
    if (!(eps >= 0.0)) return set_error(ctx, "moe_stack_forward: eps %g", eps);
    const qq_moe *m0 = st->layers[0];
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    MaskBits mb;
    if (int rc = mask_from_bytes(ctx, mask, m0->E, &mb)) return rc;
    if (T == 1 && stack_decode_supported(ctx, m0))   // one launch for the whole stack
        return launch_moe_stack_decode(ctx, m0, st->table, st->n, hidden_dev, eps, mb, idx_dev, w_dev, probs_dev);
    // layer by layer (routing outputs of layer l at l T K resp. l T E)
    const size_t TK = (size_t)T * m0->K, TE = (size_t)T * m0->E;
    for (int l = 0; l < st->n; l++) {
        if (int rc = qq_moe_forward_norm_dev(ctx, st->layers[l], hidden_dev, st->norm_w[l], eps, T, mask,
                                             idx_dev ? idx_dev + l * TK : nullptr, w_dev ? w_dev + l * TK : nullptr,
                                             probs_dev ? probs_dev + l * TE : nullptr))
            return rc;
    }
    return QQ_OK;
}

int qq_moe_forward(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                   const uint8_t *mask, int32_t *idx, double *w, float *probs)
{
    int rc = forward_check(ctx, m, T);
    if (rc || T == 0) return rc;
    if (!x || !hidden) return set_error(ctx, "moe_forward: NULL buffer");
    if ((rc = no_capture(ctx, "qq_moe_forward"))) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    MaskBits mb;
    if ((rc = mask_from_bytes(ctx, mask, m->E, &mb))) return rc;
    // device copies: x | hidden | idx | w | probs, then the forward's scratch.
    // The same span is staged in the context's pinned host buffer, so each
    // direction is one DMA copy: x | hidden in, hidden .. probs out.
    const size_t xb = (size_t)T * m->H * 4;
    const size_t ib = (size_t)T * m->K * 4, wb = (size_t)T * m->K * 8, pb = (size_t)T * m->E * 4;
    const size_t xa = align256(xb), ia = align256(ib), wa = align256(wb);
    const size_t io = 2 * xa + ia + wa + align256(pb);
    if ((rc = ensure_pinned(ctx, io))) return rc;
    char *ph = static_cast<char *>(ctx->pinned) + PIN_HDR;
    char *pd = ctx->pinned_dev + PIN_HDR;
    // hidden .. the last routing output wanted, in whole 16-byte words (the
    // regions are 256-byte aligned, so the rounding stays inside them)
    const size_t out_span = (xa + ia + (probs ? wa + pb : (w ? wb : 0)) + 15) & ~(size_t)15;
    // A batch-1 call runs the one-launch decode kernel and a small batch the
    // one-launch routing kernel, whose workgroups must all be resident at
    // once.  When one of their waits timed out (the CUs were held by other
    // work), the call is run again through the multi-launch path, which
    // needs no co-residency: the caller's rows are untouched
    // until the results are copied back, so the retry starts from them.
    for (int attempt = 0;; attempt++) {
        ctx->batch_only = attempt > 0;
        rc = ensure_scratch(ctx, io + forward_scratch(ctx, m, T));
        char *s = static_cast<char *>(ctx->scratch);
        float *dx = reinterpret_cast<float *>(s);
        float *dh = reinterpret_cast<float *>(s + xa);
        int32_t *didx = reinterpret_cast<int32_t *>(s + 2 * xa);
        double *dw = reinterpret_cast<double *>(s + 2 * xa + ia);
        float *dp = reinterpret_cast<float *>(s + 2 * xa + ia + wa);
        memcpy(ph, x, xb);
        memcpy(ph + xa, hidden, xb);
        const uint64_t timeouts = ctx->timeouts;
        if (!rc) rc = launch_stage_copy(ctx, pd, dx, 2 * xa);
        if (!rc) rc = forward_impl(ctx, m, dx, dh, T, mb, didx, dw, probs ? dp : nullptr, io);
        if (!rc) rc = launch_stage_copy(ctx, dh, pd + xa, out_span);
        if (!rc) rc = check_device_error(ctx, true);
        ctx->batch_only = 0;
        if (rc && attempt == 0 && ctx->timeouts != timeouts) continue;
        if (rc) return rc;
        break;
    }
    memcpy(hidden, ph + xa, xb);
    if (idx) memcpy(idx, ph + 2 * xa, ib);
    if (w) memcpy(w, ph + 2 * xa + ia, wb);
    if (probs) memcpy(probs, ph + 2 * xa + ia + wa, pb);
    return QQ_OK;
}

// ---- device buffers and the routing record ---------------------------------

int qq_buffer_alloc(qq_ctx *ctx, size_t nbytes, void **dev)
{
    if (!ctx || !dev) return QQ_E_ARG;
    *dev = nullptr;
    if (int rc = no_capture(ctx, "qq_buffer_alloc")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    const size_t n = nbytes ? nbytes : 1;
    void *p = nullptr;
    QQ_HIP(ctx, hipMalloc(&p, n));
    hipError_t e = hipMemsetAsync(p, 0, n, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return check_hip(ctx, e, "buffer_alloc: clear");
    }
    *dev = p;
    return QQ_OK;
}

int qq_buffer_free(qq_ctx *ctx, void *dev)
{
    if (!ctx) return QQ_E_ARG;
    if (!dev) return QQ_OK;
    if (int rc = no_capture(ctx, "qq_buffer_free")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    QQ_HIP(ctx, hipFree(dev));
    return QQ_OK;
}

int qq_buffer_write(qq_ctx *ctx, void *dev, const void *host, size_t nbytes)
{
    if (!ctx) return QQ_E_ARG;
    if (nbytes == 0) return QQ_OK;
    if (!dev || !host) return set_error(ctx, "buffer_write: NULL pointer");
    if (int rc = no_capture(ctx, "qq_buffer_write")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipMemcpyAsync(dev, host, nbytes, hipMemcpyHostToDevice, ctx->stream));
    return check_device_error(ctx);
}

int qq_buffer_read(qq_ctx *ctx, const void *dev, void *host, size_t nbytes)
{
    if (!ctx) return QQ_E_ARG;
    if (nbytes == 0) return QQ_OK;
    if (!dev || !host) return set_error(ctx, "buffer_read: NULL pointer");
    if (int rc = no_capture(ctx, "qq_buffer_read")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipMemcpyAsync(host, dev, nbytes, hipMemcpyDeviceToHost, ctx->stream));
    return check_device_error(ctx);
}

int qq_moe_forward_record_dev(qq_ctx *ctx, const qq_moe *m, const float *x_dev, float *hidden_dev, int T,
                              const uint8_t *mask, float *record_dev)
{
    int rc = forward_check(ctx, m, T);
    if (rc || T == 0) return rc;
    if (!x_dev || !hidden_dev) return set_error(ctx, "moe_forward_record: NULL buffer");
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    MaskBits mb;
    if ((rc = mask_from_bytes(ctx, mask, m->E, &mb))) return rc;
    if (decode_supported(ctx, m, T))   // the decode kernel writes the record itself
        return launch_moe_decode(ctx, m, x_dev, hidden_dev, mb, nullptr, nullptr, nullptr, nullptr, record_dev);
    if (!record_dev) return forward_impl(ctx, m, x_dev, hidden_dev, T, mb, nullptr, nullptr, nullptr, 0);
    // idx | w | probs ahead of the forward's scratch, then the record from them
    const size_t ib = align256((size_t)T * m->K * 4), wb = align256((size_t)T * m->K * 8);
    const size_t pb = align256((size_t)T * m->E * 4);
    if ((rc = ensure_scratch(ctx, ib + wb + pb + forward_scratch(ctx, m, T)))) return rc;
    char *s = static_cast<char *>(ctx->scratch);
    int32_t *idx = reinterpret_cast<int32_t *>(s);
    double *w = reinterpret_cast<double *>(s + ib);
    float *probs = reinterpret_cast<float *>(s + ib + wb);
    if ((rc = forward_impl(ctx, m, x_dev, hidden_dev, T, mb, idx, w, probs, ib + wb + pb))) return rc;
    return launch_route_record(ctx, idx, w, probs, T, m->K, m->E, record_dev);
}

int qq_set_wait_limit(qq_ctx *ctx, int microseconds)
{
    if (!ctx) return QQ_E_ARG;
    if (microseconds < 0) return set_error(ctx, "set_wait_limit: %d us < 0", microseconds);
    ctx->dec_wait_ticks = (uint64_t)microseconds * 100;   // the 100 MHz wall clock
    return QQ_OK;
}

int qq_debug_epoch(qq_ctx *ctx, uint32_t *epoch)
{
    if (!ctx || !epoch) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_debug_epoch")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    QQ_HIP(ctx, hipMemcpy(epoch, ctx->sync_epoch, 4, hipMemcpyDeviceToHost));
    return QQ_OK;
}

int qq_debug_plant_words(qq_ctx *ctx, uint32_t tag)
{
    if (!ctx) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_debug_plant_words")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    // 1e30f: a logit, h value, partial or row that a call accepted would show
    const uint64_t word = ((uint64_t)tag << 32) | 0x7149f2cau;
    const size_t n = sync_table_words();
    hipLaunchKernelGGL(sync_plant_kernel, dim3(256), dim3(256), 0, ctx->stream, ctx->sync_slots, n, word);
    QQ_HIP(ctx, hipGetLastError());
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return QQ_OK;
}

int qq_set_mfma_min_tokens(qq_ctx *ctx, int tokens)
{
    if (!ctx) return QQ_E_ARG;
    if (tokens < 0) return set_error(ctx, "set_mfma_min_tokens: %d < 0", tokens);
    ctx->mfma_min_tokens = tokens;
    return QQ_OK;
}

int qq_rmsnorm_dev(qq_ctx *ctx, const float *x_dev, const float *weight_dev, float *out_dev, int T,
                   int H, double eps)
{
    if (!ctx) return QQ_E_ARG;
    if (T < 0 || H <= 0) return set_error(ctx, "rmsnorm: bad shape T=%d H=%d", T, H);
    if (T == 0) return QQ_OK;
    if (!x_dev || !out_dev) return set_error(ctx, "rmsnorm: NULL buffer");
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    return launch_rmsnorm(ctx, x_dev, weight_dev, out_dev, T, H, eps);
}

// ---- measurement ------------------------------------------------------------

int qq_timer_start(qq_ctx *ctx)
{
    if (!ctx) return QQ_E_ARG;
    QQ_HIP(ctx, hipEventRecord(ctx->ev0, ctx->stream));
    return QQ_OK;
}

int qq_timer_stop(qq_ctx *ctx, float *ms)
{
    if (!ctx || !ms) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_timer_stop")) return rc;
    QQ_HIP(ctx, hipEventRecord(ctx->ev1, ctx->stream));
    QQ_HIP(ctx, hipEventSynchronize(ctx->ev1));
    QQ_HIP(ctx, hipEventElapsedTime(ms, ctx->ev0, ctx->ev1));
    return QQ_OK;
}

int qq_profile_enable(qq_ctx *ctx, int max_launches)
{
    if (!ctx) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_profile_enable")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ctx->prof_on = 0;
    ctx->prof_n = 0;
    if (max_launches <= 0) return QQ_OK;
    if (max_launches > ctx->prof_cap) {
        prof_free(ctx);
        ctx->prof_ev = static_cast<hipEvent_t *>(calloc(2 * (size_t)max_launches, sizeof(hipEvent_t)));
        ctx->prof_id = static_cast<int *>(calloc((size_t)max_launches, sizeof(int)));
        if (!ctx->prof_ev || !ctx->prof_id) {
            prof_free(ctx);
            return set_error(ctx, "profile: host allocation failed");
        }
        for (int i = 0; i < 2 * max_launches; i++) {
            hipError_t e = hipEventCreate(&ctx->prof_ev[i]);
            if (e != hipSuccess) {
                ctx->prof_cap = i / 2;
                return check_hip(ctx, e, "hipEventCreate(profile)");
            }
            ctx->prof_cap = (i + 1) / 2;
        }
    }
    ctx->prof_on = 1;
    return QQ_OK;
}

int qq_profile_read(qq_ctx *ctx, float *ms_sum, int *count, int n)
{
    if (!ctx || !ms_sum || !count) return QQ_E_ARG;
    if (int rc = no_capture(ctx, "qq_profile_read")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int i = 0; i < n; i++) {
        ms_sum[i] = 0.0f;
        count[i] = 0;
    }
    for (int i = 0; i < ctx->prof_n; i++) {
        float ms = 0.0f;
        QQ_HIP(ctx, hipEventElapsedTime(&ms, ctx->prof_ev[2 * i], ctx->prof_ev[2 * i + 1]));
        const int id = ctx->prof_id[i];
        if (id >= 0 && id < n) {
            ms_sum[id] += ms;
            count[id]++;
        }
    }
    ctx->prof_n = 0;
    return QQ_OK;
}

const char *qq_profile_name(int id)
{
    return (id >= 0 && id < K_COUNT) ? kKernelNames[id] : "";
}

int qq_profile_kernel_count(void) { return K_COUNT; }

// ---- graphs -------------------------------------------------------------------

struct qq_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

int qq_capture_begin(qq_ctx *ctx)
{
    if (!ctx) return QQ_E_ARG;
    if (ctx->capturing) return set_error(ctx, "qq_capture_begin: a capture is already open");
    if (ctx->prof_on) return set_error(ctx, "qq_capture_begin: per-launch profiling is on");
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = 1;
    return QQ_OK;
}

int qq_capture_end(qq_ctx *ctx, qq_graph **out)
{
    if (!ctx || !out) return QQ_E_ARG;
    *out = nullptr;
    if (!ctx->capturing) return set_error(ctx, "qq_capture_end: no capture is open");
    ctx->capturing = 0;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return check_hip(ctx, e, "hipStreamEndCapture (a call inside the capture failed?)");
    }
    qq_graph *qg = new (std::nothrow) qq_graph();
    if (!qg) {
        (void)hipGraphDestroy(g);
        return set_error(ctx, "host allocation failed");
    }
    qg->graph = g;
    e = hipGraphInstantiate(&qg->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete qg;
        return check_hip(ctx, e, "hipGraphInstantiate");
    }
    *out = qg;
    return QQ_OK;
}

int qq_graph_launch(qq_ctx *ctx, const qq_graph *g)
{
    if (!ctx) return QQ_E_ARG;
    if (!g) return set_error(ctx, "qq_graph_launch: NULL graph");
    if (int rc = no_capture(ctx, "qq_graph_launch")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    QQ_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return QQ_OK;
}

int qq_graph_release(qq_ctx *ctx, qq_graph *g)
{
    if (!g) return QQ_OK;
    if (int rc = no_capture(ctx, "qq_graph_release")) return rc;
    if (ctx) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
    return QQ_OK;
}

}  // extern "C"
