/*
 * qq_oracle.h -- CPU restatement of the LFM2-MoE Q8_0 MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * HIP product path never does.
 *
 * Every function follows one reference function (file:line in
 * kishida/QwenQwen3.js) with the same operation order and the same
 * float64 arithmetic as the JavaScript it restates (a JS Number is an IEEE
 * binary64; a Float32Array store is one round-to-nearest-even to binary32).
 */
#ifndef QQ_ORACLE_H
#define QQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type codes used on this path (src/gguf.js TENSOR_TYPES). */
#define QO_TYPE_F32  0
#define QO_TYPE_Q8_0 8

/* Exact binary16 -> binary64 decode, as DataView.getFloat16(off, true)
 * (src/tensor.js:21-23).  Closed form, no table. */
double qo_f16_to_f64(uint16_t h);

/* Round-to-nearest-even binary32 -> binary16 (synthetic-scale generator). */
uint16_t qo_f32_to_f16(float f);

/* matmulQ80xF32 (src/tensor.js:26-53).  `base + offset` is the first Q8_0
 * block of a GGUF [in_dim, out_dim] tensor (column-major: column c holds
 * ceil(in_dim/32) blocks of 34 bytes {fp16 d, int8 qs[32]}).
 * y[c] = fp32( sum_b sum_i (x[32b+i] * q) * d ), sequential in float64. */
void qo_matmul_q8_0(const uint8_t *base, size_t offset, int in_dim, int out_dim,
                    const float *x, float *y);

/* matmulF32xF32 (src/tensor.js:469-482): column c at offset + c*in_dim*4. */
void qo_matmul_f32(const uint8_t *base, size_t offset, int in_dim, int out_dim,
                   const float *x, float *y);

/* matmulGeneric (src/tensor.js:485-496) restricted to the types this path
 * carries.  Returns 0, or -1 for a type the reference would reject with
 * `throw new Error(...)` (k-quants are outside this path and also -1). */
int qo_matmul_generic(int type, const uint8_t *base, size_t offset, int in_dim,
                      int out_dim, const float *x, float *y);

/* _readWeightF32 (src/tensor.js:80-100): 1-D F32 view or Q8_0 dequant.
 * Returns -1 for other types (the reference throws). */
int qo_read_weight_f32(int type, const uint8_t *base, size_t offset, int n, float *out);

/* siluInPlace / mulInPlace / addVec (src/tensor.js:167-185). */
void qo_silu_inplace(float *a, int n);
void qo_mul_inplace(float *a, const float *b, int n);
void qo_add_vec(float *a, const float *b, int n);

/* One LFM2-MoE MoE layer as Lfm2Engine binds it (src/lfm2-engine.js:129-137). */
typedef struct {
    int H;              /* embedding_length (2048)            */
    int F;              /* expert_feed_forward_length (1792)  */
    int E;              /* expert_count (32)                  */
    int K;              /* expert_used_count (4)              */
    int router_type;    /* ffn_gate_inp.weight: F32 or Q8_0, shape [H, E]  */
    const uint8_t *router;  size_t router_off;
    int bias_type;      /* exp_probs_b.bias type, or -1 when the tensor is absent */
    const uint8_t *bias;    size_t bias_off;
    /* ffn_{gate,up}_exps [H, F, E] and ffn_down_exps [F, H, E], Q8_0 */
    const uint8_t *gate;    size_t gate_off;
    const uint8_t *up;      size_t up_off;
    const uint8_t *down;    size_t down_off;
    int gating;         /* QO_GATING_SIGMOID_BIAS (LFM2) or QO_GATING_SOFTMAX (Qwen3) */
} qo_moe_layer;

/* Router gating functions: LFM2's sigmoid with expert-bias selection and
 * 1e-6-seeded renormalisation (src/lfm2-engine.js:417-447), Qwen3-MoE's
 * softmax with renormalisation from 0 (src/qwen3-engine.js:304-325). */
#define QO_GATING_SIGMOID_BIAS 0
#define QO_GATING_SOFTMAX      1

/* Lfm2Engine._moEFFN (src/lfm2-engine.js:413-487) applied to T independent
 * tokens in order (the reference's prefill is T sequential single-token
 * calls, src/lfm2-engine.js:550-555).
 *   x      [T*H]  ffn_norm output (bufNormed), read only
 *   hidden [T*H]  residual stream (bufHidden), updated in place
 *   mask   [E]    expertMask membership (nonzero = masked) or NULL
 *   idx    [T*K]  selected experts in rank order, or NULL
 *   w      [T*K]  normalised weights as reported to onRouterUpdate (binary64), or NULL
 *   probs  [T*E]  sigmoid probabilities (binary32), or NULL
 * Returns 0, or -1 on an unsupported tensor type / bad shape. */
int qo_moe_ffn(const qo_moe_layer *L, const float *x, float *hidden, int T,
               const uint8_t *mask, int32_t *idx, double *w, float *probs);

/* Steps 1-5 of _moEFFN only (router, sigmoid, bias, top-K, renormalise;
 * src/lfm2-engine.js:417-447) for T tokens: the routing a full call would
 * make, at a fraction of the cost.  Outputs as qo_moe_ffn. */
int qo_moe_route(const qo_moe_layer *L, const float *x, int T, int32_t *idx, double *w,
                 float *probs);

/* RMSNorm with unit weight, as src/tensor.js:103-114 with an all-ones
 * ffn_norm (the 22-layer stack workload between MoE layers). */
void qo_rmsnorm_unit(const float *in, float *out, int n, double eps);

#ifdef __cplusplus
}
#endif
#endif
