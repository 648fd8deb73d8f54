/*
 * qq_lfm2.h -- the LFM2 single-token forward on the device.
 *
 * Replaces Lfm2Engine.forward (src/lfm2-engine.js:228-280) and the state it
 * keeps between tokens (conv states, KV cache: :183-224, src/kv-cache.js):
 * one call runs embedding lookup, every block (short-conv or GQA attention,
 * then dense SwiGLU or MoE FFN) and the output norm and head for one token,
 * with every buffer resident in device memory -- no host round trip between
 * blocks.  Part of libqqmoe.so.
 *
 * Supported files: the tensors Lfm2Engine binds (src/lfm2-engine.js:78-144),
 * with Q8_0 matrices (token_embd / output, in_proj, out_proj, attn_q/k/v/
 * output, ffn_gate/up/down, expert tensors), F32 or Q8_0 norm weights, an F32,
 * F16 or Q8_0 conv kernel with l_cache = 3, head_dim 64, rows of at most 8192
 * inputs, and MoE blocks the batch-1 decode kernel takes (embedding length
 * at most 2048, at most 256 experts).  Anything else fails at creation with a
 * message naming the tensor, key or block.
 *
 * Numerics: matrix products accumulate in fp32 (the reference: binary64);
 * the elementwise steps round to fp32 where the reference stores into a
 * Float32Array.  The MoE blocks run the batch-1 decode path of qq_moe.h.
 */
#ifndef QQ_LFM2_H
#define QQ_LFM2_H
#include <stdint.h>
#include "qq_moe.h"
#include "qq_gguf.h"
#ifdef __cplusplus
extern "C" {
#endif

typedef struct qq_lfm2 qq_lfm2;

/* The configuration Lfm2Engine's constructor derives (src/lfm2-engine.js:15-76). */
typedef struct qq_lfm2_info {
    int n_layers;          /* <arch>.block_count || 24 */
    int n_embd;            /* <arch>.embedding_length || 2048 */
    int n_heads;           /* <arch>.attention.head_count || 32 */
    int n_head_kv;         /* max of the positive per-layer head_count_kv, or the scalar || 8 */
    int head_dim;          /* attn_q rows / n_heads of the first attention block */
    int n_vocab;           /* token_embd.weight shape[1] */
    int n_ff;              /* ffn_gate rows of the first dense block (7168 if none) */
    int n_experts;         /* <arch>.expert_count || 32 */
    int n_experts_used;    /* <arch>.expert_used_count || 4 */
    int n_dense_lead;      /* <arch>.leading_dense_block_count || 2 */
    int l_cache;           /* <arch>.shortconv.l_cache || 3 */
    int max_ctx;           /* min(<arch>.context_length || 4096, 4096) */
    int n_attn_layers;     /* blocks without shortconv.conv.weight */
    double eps;            /* <arch>.attention.layer_norm_rms_epsilon || 1e-5 */
    double rope_freq_base; /* <arch>.rope.freq_base (or rope_freq_base) || 5e6 */
} qq_lfm2_info;

/* new Lfm2Engine(gguf) minus the tokenizer (src/lfm2-engine.js:15-76):
 * binds and uploads every tensor of an open reader (qq_gguf_open) and
 * allocates the conv states and the KV cache, zeroed.  The reader may be
 * closed afterwards. */
int qq_lfm2_create(qq_ctx *ctx, const qq_gguf *g, qq_lfm2 **out);
int qq_lfm2_get_info(const qq_lfm2 *m, qq_lfm2_info *out);

/* resetState (src/lfm2-engine.js:216-222): zero the KV cache and conv states.
 * Also required after a device-side wait on the context timed out (the
 * forward calls fail with QQ_E_STATE until then: that call may have left the
 * hidden row, conv states and KV cache half written). */
int qq_lfm2_reset(qq_ctx *ctx, qq_lfm2 *m);

/* forward(tokenId, position, skipLogits) (src/lfm2-engine.js:228-280) on
 * device memory: logits_dev receives n_vocab floats, or is NULL to skip the
 * output head (skipLogits).  idx_dev, when not NULL, receives each MoE
 * block's selected experts (int32 [n_layers][n_experts_used]; dense blocks'
 * rows are left as they are) -- the onRouterUpdate telemetry of _moEFFN.
 * Enqueued on the context's stream, not waited for.  token must lie in
 * [0, n_vocab) and position in [0, max_ctx). */
int qq_lfm2_forward_dev(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits_dev,
                        int32_t *idx_dev);

/* Same with host logits (n_vocab floats, or NULL); waits for the result. */
int qq_lfm2_forward(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits);

/* forward with the engine's expertMask and the whole onRouterUpdate payload
 * of every MoE block (src/lfm2-engine.js:449-464):
 *   mask   [n_experts] bytes, nonzero = the expert is skipped in every MoE
 *          block (its weight is not renormalised away), or NULL;
 *   idx    [n_layers][n_experts_used] int32  selected experts, rank order;
 *   w      [n_layers][n_experts_used] binary64  p_k / (1e-6 + sum p);
 *   probs  [n_layers][n_experts] fp32  sigmoid probabilities;
 * each NULL or filled for the MoE blocks (rows of dense blocks are left as
 * they are).  The _dev form takes device pointers (mask stays a host array)
 * and is enqueued, not waited for; the host form waits. */
int qq_lfm2_forward_routed_dev(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits_dev,
                               const uint8_t *mask, int32_t *idx_dev, double *w_dev, float *probs_dev);
int qq_lfm2_forward_routed(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits,
                           const uint8_t *mask, int32_t *idx, double *w, float *probs);

void qq_lfm2_release(qq_ctx *ctx, qq_lfm2 *m);

#ifdef __cplusplus
}
#endif
#endif /* QQ_LFM2_H */
