/*
 * qq_moe.h -- C ABI of the MI355X (gfx950) LFM2-MoE Q8_0 MoE feed-forward path.
 *
 * Plain C: opaque handles, host or device pointers, sizes, int status codes.
 * Every entry point returns QQ_OK (0) or a negative QQ_E* code; the message of
 * the last failure on a context is qq_last_error(ctx) (qq_last_error(NULL)
 * reports a failed qq_init).  A binding turns a non-zero status into an
 * exception, as the reference does with `throw new Error(...)`
 * (src/tensor.js:494).
 *
 * Entry points whose pointers are host memory (suffix-free names) are
 * synchronous, like the JavaScript functions they replace.  The *_dev
 * variants take device pointers, enqueue on the context's stream and return
 * without waiting.
 *
 * Reference interfaces replaced (kishida/QwenQwen3.js):
 *   matmulQ80xF32(meta, input)          src/tensor.js:26-53
 *   matmulGeneric(meta, input)          src/tensor.js:485-496 (type 8 branch)
 *   Lfm2Engine.prototype._moEFFN        src/lfm2-engine.js:413-487
 *   Lfm2GPUEngine.prototype._moEFFNGPU  src/webgpu.js:1882-1917 (device-resident peer)
 */
#ifndef QQ_MOE_H
#define QQ_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QQ_OK            0
#define QQ_E_ARG        -1   /* bad argument, shape or type            */
#define QQ_E_HIP        -2   /* HIP runtime error                      */
#define QQ_E_NODEV      -3   /* no usable gfx950 device                */
#define QQ_E_NOMEM      -4   /* device or pinned allocation failed     */
#define QQ_E_STATE      -5   /* device-resident state invalid: reset it */

/* GGUF tensor type codes (src/gguf.js TENSOR_TYPES) accepted on this path. */
#define QQ_TYPE_F32      0
#define QQ_TYPE_Q8_0     8

typedef struct qq_ctx qq_ctx;
typedef struct qq_tensor qq_tensor;
typedef struct qq_moe qq_moe;
typedef struct qq_graph qq_graph;
typedef struct qq_moe_stack qq_moe_stack;

/* ---- context --------------------------------------------------------- */

/* Open device `device` (HIP ordinal) and create a stream.  Fails with
 * QQ_E_NODEV when the device is absent or not gfx950.  No reference
 * counterpart: the reference's device setup is GPUDevice.init
 * (src/webgpu.js:349-489). */
int qq_init(int device, qq_ctx **out);
void qq_destroy(qq_ctx *ctx);
const char *qq_last_error(const qq_ctx *ctx);

/* Use `hip_stream` (a hipStream_t, or NULL for the context's own stream) for
 * every later launch on this context. */
int qq_set_stream(qq_ctx *ctx, void *hip_stream);
int qq_synchronize(qq_ctx *ctx);

/* ---- Q8_0 tensors ---------------------------------------------------- */

/* Repack `n_mats` GGUF Q8_0 matrices of shape [in_dim, out_dim] into device
 * memory once.  `gguf_bytes` points at the first block (meta.buffer +
 * meta.offset, src/gguf.js:235-261) and holds n_mats*out_dim*ceil(in_dim/32)
 * 34-byte blocks; n_mats = 1 for a 2-D tensor and E for the 3-D expert
 * tensors ffn_{gate,up,down}_exps (src/lfm2-engine.js:131-136), whose expert
 * e is sliced by _expertSlice (src/lfm2-engine.js:489-505). */
int qq_q8_0_upload(qq_ctx *ctx, const void *gguf_bytes, size_t nbytes, int in_dim,
                   int out_dim, int n_mats, qq_tensor **out);
/* Same, from GGUF bytes already in device memory. */
int qq_q8_0_upload_dev(qq_ctx *ctx, const void *gguf_bytes_dev, size_t nbytes, int in_dim,
                       int out_dim, int n_mats, qq_tensor **out);
int qq_tensor_release(qq_ctx *ctx, qq_tensor *t);

/* matmulQ80xF32 (src/tensor.js:26-53) for `rows` input vectors:
 * y[r][c] = sum_k x[r][k] * W_mat[k][c], W_mat = matrix `mat` of t.
 * x is rows*in_dim floats, y is rows*out_dim floats (host memory). */
int qq_q8_0_matvec(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x, float *y,
                   int rows);
/* Device-pointer variant; enqueued, not waited for. */
int qq_q8_0_matvec_dev(qq_ctx *ctx, const qq_tensor *t, int mat, const float *x_dev,
                       float *y_dev, int rows);

/* ---- MoE layer ------------------------------------------------------- */

/* Bind one LFM2-MoE MoE layer (src/lfm2-engine.js:129-137).
 *   router_bytes  ffn_gate_inp.weight [H, E]: F32 (E columns of H floats) or Q8_0
 *   bias          exp_probs_b.bias as E floats (_readWeightF32, src/tensor.js:80-100),
 *                 or NULL when the layer has none
 *   gate, up      ffn_gate_exps / ffn_up_exps tensors [H, F, E]
 *   down          ffn_down_exps tensor [F, H, E]
 * The router and bias are copied; gate/up/down are borrowed and must outlive
 * the layer handle. */
int qq_moe_create(qq_ctx *ctx, const void *router_bytes, int router_type, const float *bias,
                  const qq_tensor *gate, const qq_tensor *up, const qq_tensor *down,
                  int H, int F, int E, int K, qq_moe **out);

/* Router gating of the layer (default QQ_GATING_SIGMOID_BIAS):
 *   QQ_GATING_SIGMOID_BIAS  LFM2-MoE (src/lfm2-engine.js:417-447): sigmoid
 *                           probabilities, selection by probability + bias,
 *                           weights p_k / (1e-6 + sum p).
 *   QQ_GATING_SOFTMAX       Qwen3-MoE (src/qwen3-engine.js:304-325):
 *                           softmaxInPlace (src/tensor.js:150-164) over the
 *                           router logits, selection by probability, weights
 *                           p_k / sum p (0 when the sum is 0); bias unused.
 * probs outputs carry the sigmoid resp. softmax probabilities. */
#define QQ_GATING_SIGMOID_BIAS 0
#define QQ_GATING_SOFTMAX      1
int qq_moe_set_gating(qq_ctx *ctx, qq_moe *m, int gating);
int qq_moe_release(qq_ctx *ctx, qq_moe *m);

/* Lfm2Engine._moEFFN (src/lfm2-engine.js:413-487) over T tokens, each row
 * independent (the reference runs T sequential calls, src/lfm2-engine.js:550-555):
 *   x       [T*H]  ffn_norm output (bufNormed), read only
 *   hidden  [T*H]  residual stream (bufHidden), updated in place: hidden += MoE(x)
 *   mask    [E]    expertMask membership (nonzero = skip that expert) or NULL;
 *                  masked weights are not renormalised (src/lfm2-engine.js:464)
 *   idx     [T*K]  selected experts in rank order, or NULL
 *   w       [T*K]  normalised weights p_k/(1e-6 + sum p), binary64 as the
 *                  onRouterUpdate payload carries them, or NULL
 *   probs   [T*E]  sigmoid probabilities, or NULL
 * Host pointers; synchronous. */
int qq_moe_forward(qq_ctx *ctx, const qq_moe *m, const float *x, float *hidden, int T,
                   const uint8_t *mask, int32_t *idx, double *w, float *probs);
/* Device-pointer variant (mask stays a host array of E bytes or NULL;
 * idx/w/probs device pointers or NULL); enqueued, not waited for. */
int qq_moe_forward_dev(qq_ctx *ctx, const qq_moe *m, const float *x_dev, float *hidden_dev,
                       int T, const uint8_t *mask, int32_t *idx_dev, double *w_dev,
                       float *probs_dev);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The same as qq_moe_forward_dev, but the forward's
 * scratch is a fixed array of QQ_NOALLOC_SCRATCH_BYTES per GPU (32 MiB,
 * held until the process ends) instead of the context's arena, so the call
 * allocates nothing.  A T whose scratch does not fit (about 500 rows at
 * LFM2-8B-A1B shapes; batch-1 decode needs none) is rejected with
 * QQ_E_ARG before anything is enqueued.  Every call on one GPU shares that
 * GPU's array (the kernels write all of it that they read, so nothing needs
 * clearing between calls): calls that overlap on one GPU -- two streams, two
 * contexts -- race. */
#define QQ_NOALLOC_SCRATCH_BYTES (32u << 20)
int qq_moe_forward_noalloc_dev(qq_ctx *ctx, const qq_moe *m, const float *x_dev, float *hidden_dev,
                               int T, const uint8_t *mask, int32_t *idx_dev, double *w_dev,
                               float *probs_dev);

/* The FFN sub-block of an MoE layer (src/lfm2-engine.js:250-257): the
 * ffn_norm RMSNorm of the residual row (src/tensor.js:103-114), then the MoE
 * block on it:
 *   x = rmsnorm(hidden) * norm_w     (norm_w_dev NULL: unit weight)
 *   hidden += MoE(x)
 * for T rows, with the same routing outputs as qq_moe_forward_dev.  A
 * single row is normalised inside the decode kernel, and the rows of a chunk
 * on the fp16 MFMA path inside its router launch (F32 router, hidden_dev and
 * norm_w_dev 16-byte aligned; no separate launch); the result equals
 * qq_rmsnorm_dev followed by qq_moe_forward_dev bit for bit.  Device
 * pointers; enqueued, not waited for. */
int qq_moe_forward_norm_dev(qq_ctx *ctx, const qq_moe *m, float *hidden_dev,
                            const float *norm_w_dev, double eps, int T, const uint8_t *mask,
                            int32_t *idx_dev, double *w_dev, float *probs_dev);

/* ---- MoE stacks: a token through many layers in one launch ----------------
 * Lfm2Engine.forward runs, per block, the FFN sub-block `x = rmsnorm(hidden)
 * * ffn_norm; hidden += _moEFFN(x)` (src/lfm2-engine.js:232-258, :250-257),
 * and the WebGPU engine records a token's blocks into one command encoder
 * (src/webgpu.js:1954-2034).  A stack binds n MoE layers of equal shape,
 * gating and router type (borrowed; they must outlive the stack), with their
 * ffn_norm weights (norm_w_dev: n device pointers of H floats, entries or
 * the whole array NULL for unit weights), 1 <= n <= 256. */
int qq_moe_stack_create(qq_ctx *ctx, const qq_moe *const *layers, const float *const *norm_w_dev, int n,
                        qq_moe_stack **out);
int qq_moe_stack_release(qq_ctx *ctx, qq_moe_stack *s);
/* For l = 0 .. n-1, on T rows: x = rmsnorm(hidden) * norm_w[l];
 * hidden += MoE_l(x) -- qq_moe_forward_norm_dev layer after layer, with the
 * same results.  Routing outputs of layer l at idx_dev + l*T*K,
 * w_dev + l*T*K, probs_dev + l*T*E (each NULL or device memory).  A single
 * row (T = 1) runs the whole stack in one launch of the decode kernel: the
 * residual row passes from layer to layer inside the launch, and each
 * layer's router rows are read while the previous layer's down weights
 * stream in.  Device pointers; enqueued, not waited for. */
int qq_moe_stack_forward_dev(qq_ctx *ctx, const qq_moe_stack *s, float *hidden_dev, double eps, int T,
                             const uint8_t *mask, int32_t *idx_dev, double *w_dev, float *probs_dev);

/* ---- The WebGPU engines' device-resident MoE block ------------------------
 * Lfm2GPUEngine and Qwen3GPUEngine keep the residual stream in device
 * buffers and run the block with no host round trip, leaving each MoE
 * layer's routing in a buffer that is read back in one batch after the token
 * (src/webgpu.js:1882-1945, :878-990).
 *
 * Device buffers, standing for GPUDevice.createBuffer / uploadBuffer,
 * queue.writeBuffer and readF32 (src/webgpu.js:349-430): alloc returns
 * zeroed device memory; write copies host bytes in and returns once they
 * are copied; read waits for the work enqueued before it, then copies out.
 * Not allowed while a capture is open. */
int qq_buffer_alloc(qq_ctx *ctx, size_t nbytes, void **dev);
int qq_buffer_free(qq_ctx *ctx, void *dev);
int qq_buffer_write(qq_ctx *ctx, void *dev, const void *host, size_t nbytes);
int qq_buffer_read(qq_ctx *ctx, const void *dev, void *host, size_t nbytes);

/* _moEFFNGPU (src/webgpu.js:1882-1917 for LFM2, :878-915 for Qwen3):
 * hidden += MoE(x) for T rows on device pointers, enqueued, and per row the
 * routing record the engines' top-K shaders write for the batched readback
 * (src/webgpu.js:1236-1240, :1175-1178):
 *   record_dev[t*(2K+E) + k]        selected expert of rank k, as a float
 *   record_dev[t*(2K+E) + K + k]    its weight, the w of qq_moe_forward
 *                                   rounded to fp32
 *   record_dev[t*(2K+E) + 2K + e]   probability of expert e
 * (record_dev NULL: no record).  mask as in qq_moe_forward_dev (the WebGPU
 * engines have none; NULL matches them).  The values are the CPU engine's
 * (binary64 routing math, as qq_moe_forward), not the shaders' fp32
 * arithmetic: the selection equals the CPU engine's. */
int qq_moe_forward_record_dev(qq_ctx *ctx, const qq_moe *m, const float *x_dev, float *hidden_dev,
                              int T, const uint8_t *mask, float *record_dev);

/* No reference counterpart.  The workgroups of the batch-1 decode kernel,
 * and of the one-launch routing and dispatch of small batches, wait on each
 * other through memory (the routing, the h values, the partial sums, the
 * partial logits and expert ids), and the last workgroup of a split item in
 * the decode-batch kernels reads the other segments' partial sums; every
 * such wait gives up after
 * `microseconds` (default QQ_WAIT_LIMIT_US_DEFAULT, 50 ms), the kernel then
 * finishes with what it has, and the call's error surfaces at the next
 * synchronising call as QQ_E_HIP ("a device-side wait ... timed out")
 * rather than the kernel waiting on.  0: a wait gives up at its first poll
 * that misses a word (for tests of that path).
 * qq_moe_forward (host pointers) recovers by itself: when such a launch's
 * wait times out, the call runs again through the multi-launch path, which
 * needs no co-residency, and returns its result.
 * What a failed call leaves: each row of hidden holds either its value
 * before the call or its correct new value (a decode workgroup writes its
 * rows only when all of its waits succeeded; a failed batch routing writes
 * an empty dispatch, so hidden keeps its old value); idx/w/probs are not
 * valid.  (The exception: a split item whose partial-sum read expired --
 * its segments stored their words before counting themselves in, so this
 * takes a memory system that lost them -- leaves its rows of hidden
 * unspecified.)  When the
 * error is read, the host moves the device epoch past every tag the failed
 * launch can have written, so later calls are unaffected by it.  Device-
 * resident state built across calls is invalid after such a call: an LFM2
 * model's forward then fails with QQ_E_STATE until qq_lfm2_reset. */
#define QQ_WAIT_LIMIT_US_DEFAULT 50000
int qq_set_wait_limit(qq_ctx *ctx, int microseconds);

/* Test hooks, no reference counterpart (they wait for the stream; not
 * allowed while a capture is open): the device epoch that tags the decode
 * and batch-routing kernels' exchange words (a call uses the tags after it and advances it),
 * and a fill of every exchange table of the context with words carrying
 * `tag`, standing for what a workgroup of a failed call may have left. */
int qq_debug_epoch(qq_ctx *ctx, uint32_t *epoch);
int qq_debug_plant_words(qq_ctx *ctx, uint32_t tag);

/* Token batches (T > 1) of at least `tokens` rows per chunk run their expert
 * products as fp16 MFMA grouped GEMMs (fp16 activations and dequantised
 * weights, fp32 accumulation: ~1e-3 relative L2 on the layer output);
 * smaller batches, and every batch when `tokens` is 0, keep the fp32 path
 * (~1e-7).  Routing (top-K indices, weights, probs) is exact on both paths.
 * Default QQ_MFMA_MIN_TOKENS_DEFAULT.  No reference counterpart: the
 * reference's prefill is T sequential fp32 calls (src/lfm2-engine.js:550-555). */
#define QQ_MFMA_MIN_TOKENS_DEFAULT 512
int qq_set_mfma_min_tokens(qq_ctx *ctx, int tokens);

/* rmsnorm (src/tensor.js:103-114) of T rows of H floats, the ffn_norm step
 * that produces the MoE input (src/lfm2-engine.js:251-252):
 *   out[i] = w[i] * x[i] / sqrt(sum_j x[j]^2 / H + eps)   (binary64 math)
 * weight_dev: H floats (_readWeightF32 of ffn_norm.weight) or NULL for 1.
 * Device pointers; enqueued, not waited for; out may equal x. */
int qq_rmsnorm_dev(qq_ctx *ctx, const float *x_dev, const float *weight_dev, float *out_dev, int T,
                   int H, double eps);

/* ---- measurement ------------------------------------------------------ */

/* Record a HIP event pair around work enqueued between qq_timer_start and
 * qq_timer_stop on the context's stream; qq_timer_stop waits and returns the
 * elapsed milliseconds. */
int qq_timer_start(qq_ctx *ctx);
int qq_timer_stop(qq_ctx *ctx, float *ms);

/* Per-kernel timing: while enabled, every kernel launch on the context
 * carries its own start/stop event pair, stamped by the dispatch itself
 * (hipExtLaunchKernelGGL), up to max_launches launches; 0 disables.  qq_profile_read waits for the stream and returns,
 * for each kernel id < n, the summed milliseconds and the launch count, then
 * clears the record.  qq_profile_name(id) names the kernel. */
int qq_profile_enable(qq_ctx *ctx, int max_launches);
int qq_profile_read(qq_ctx *ctx, float *ms_sum, int *count, int n);
const char *qq_profile_name(int id);
int qq_profile_kernel_count(void);

/* ---- graphs ------------------------------------------------------------ */

/* Record the device-pointer calls (qq_moe_forward_dev, qq_q8_0_matvec_dev,
 * qq_rmsnorm_dev) made between qq_capture_begin and qq_capture_end on the
 * context's stream into a HIP graph, and replay it with qq_graph_launch
 * (enqueued, not waited for).  A replay runs the same kernels on the same
 * pointers; every decode call draws a fresh router epoch on the device, so
 * replays are independent.  While a capture is open, entry points that copy
 * host memory, synchronise, allocate or profile fail with QQ_E_ARG, and a
 * call whose scratch exceeds what the context already holds fails: run each
 * call once before capturing it.  No reference counterpart: the reference
 * records WebGPU command encoders per token (src/webgpu.js:1954-2034); this
 * is the serving-loop form of the same idea. */
int qq_capture_begin(qq_ctx *ctx);
int qq_capture_end(qq_ctx *ctx, qq_graph **out);
int qq_graph_launch(qq_ctx *ctx, const qq_graph *g);
int qq_graph_release(qq_ctx *ctx, qq_graph *g);

#ifdef __cplusplus
}
#endif
#endif /* QQ_MOE_H */
