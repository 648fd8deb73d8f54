// lfm2_model.cpp -- binding an LFM2-MoE GGUF file to device memory and the
// per-token launch sequence of the device forward (include/qq_lfm2.h).
//
// Reference: Lfm2Engine (src/lfm2-engine.js): constructor and _loadWeights
// :15-144 (config keys and defaults, block kinds, derived sizes),
// _dequantConvKernel :146-180, resetState :216-222, forward :228-280.
// Kernels: lfm2.hip (matvecs with fused norm / residual / short-conv /
// q-k-v epilogues, attention, embedding) and decode.hip (MoE blocks).
#include <algorithm>
#include <cmath>
#include <new>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/qq_gguf.h"
#include "../../include/qq_lfm2.h"
#include "qq_internal.h"

namespace {

constexpr int kHeadDim = 64;    // the attention kernels' head size
constexpr int kMaxIn = 8192;    // longest matvec input row
constexpr int kMaxCtx = 4096;   // src/lfm2-engine.js:33

struct LmLayer {
    bool rec = false, moe = false;
    int cache_idx = -1, conv_idx = -1;
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    qq_tensor *in_proj = nullptr, *out_proj = nullptr;
    float *kern = nullptr;                       // [H][l_cache]
    qq_tensor *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
    float *qn = nullptr, *kn = nullptr;
    qq_tensor *gate = nullptr, *up = nullptr, *down = nullptr;
    qq_moe *ffn_moe = nullptr;
};

float half_bits_to_float(uint16_t h)
{
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) {
        v = std::ldexp((float)m, -24);
        return s ? -v : v;
    }
    uint32_t bits;
    if (e == 31) bits = s | 0x7f800000u | (m << 13);
    else bits = s | ((e + 112) << 23) | (m << 13);
    std::memcpy(&v, &bits, 4);
    return v;
}

}  // namespace

struct qq_lfm2 {
    qq_lfm2_info info{};
    qq_tensor *embd = nullptr, *output = nullptr;
    float *out_norm = nullptr;
    std::vector<LmLayer> layers;
    float *conv_state = nullptr;
    size_t conv_floats = 0;            // per short-conv block: (l_cache - 1) * H
    float *kc = nullptr, *vc = nullptr;
    size_t kv_floats = 0;              // per attention block: n_head_kv * max_ctx * 64
    float *hidden = nullptr, *ybuf = nullptr, *q = nullptr, *kraw = nullptr, *attn = nullptr,
          *ffn = nullptr, *logits = nullptr;
    double *freq = nullptr;
    double *attn_work = nullptr;       // per-chunk attention partials (long contexts)
    // routing record staging of qq_lfm2_forward_routed: [n_layers][K] indices
    // and weights, [n_layers][E] probabilities
    int32_t *r_idx = nullptr;
    double *r_w = nullptr;
    float *r_probs = nullptr;
    std::vector<void *> dev;
    std::vector<qq_tensor *> tens;
    std::vector<qq_moe *> moes;
    // the context's timeout count when the conv states and KV cache were
    // last cleared: a later timed-out call may have left them half written
    uint64_t timeouts_at_reset = 0;
};

namespace {

using qq::set_error;

struct Binder {
    qq_ctx *ctx;
    const qq_gguf *g;
    qq_lfm2 *m;
    std::string arch;
    uint64_t file_size = 0;

    bool tensor(const std::string &name, qq_gguf_tensor *t)
    {
        const int64_t i = qq_gguf_find_tensor(g, name.c_str());
        return i >= 0 && qq_gguf_tensor_info(g, (uint64_t)i, t) == QQ_OK;
    }
    // Bytes of a tensor, `need` of them checked against the file.
    const uint8_t *bytes(const qq_gguf_tensor &t, uint64_t need)
    {
        if (t.offset > file_size || need > file_size - t.offset) return nullptr;
        return qq::gguf_base(g) + t.offset;
    }
    // Number(getKeyValue(key)) || dflt (src/lfm2-engine.js:19-35)
    double num(const std::string &key, double dflt)
    {
        const int64_t i = qq_gguf_find_key(g, key.c_str());
        double v;
        if (i < 0 || qq_gguf_kv_number(g, (uint64_t)i, &v) != QQ_OK) return dflt;
        return (v != 0.0 && v == v) ? v : dflt;
    }
    int alloc(size_t bytes, void **p)
    {
        *p = nullptr;
        if (hipMalloc(p, bytes ? bytes : 4) != hipSuccess) {
            *p = nullptr;
            return set_error(ctx, "lfm2: device allocation of %zu bytes failed", bytes);
        }
        m->dev.push_back(*p);
        return QQ_OK;
    }
    int upload(const void *host, size_t bytes, void **p)
    {
        if (int rc = alloc(bytes, p)) return rc;
        QQ_HIP(ctx, hipMemcpy(*p, host, bytes, hipMemcpyHostToDevice));
        return QQ_OK;
    }
    // _readWeightF32 (src/tensor.js:80-100): F32, or Q8_0 dequantised.
    int vec_f32(const std::string &name, uint64_t n, float **out)
    {
        qq_gguf_tensor t;
        if (!tensor(name, &t)) return set_error(ctx, "lfm2: tensor %s is missing", name.c_str());
        std::vector<float> v(n);
        if (t.type == QQ_TYPE_F32) {
            const uint8_t *b = bytes(t, n * 4);
            if (!b) return set_error(ctx, "lfm2: tensor %s runs past the file", name.c_str());
            std::memcpy(v.data(), b, n * 4);
        } else if (t.type == QQ_TYPE_Q8_0) {
            const uint8_t *b = bytes(t, (n + 31) / 32 * 34);
            if (!b) return set_error(ctx, "lfm2: tensor %s runs past the file", name.c_str());
            for (uint64_t i = 0; i < n; i++) {
                const uint8_t *blk = b + (i / 32) * 34;
                uint16_t h;
                std::memcpy(&h, blk, 2);
                v[i] = (float)((int8_t)blk[2 + i % 32] * (double)half_bits_to_float(h));
            }
        } else {
            return set_error(ctx, "lfm2: unsupported weight type %u for %s", t.type, name.c_str());
        }
        return upload(v.data(), n * 4, reinterpret_cast<void **>(out));
    }
    // A 2-D Q8_0 matrix [in_dim, out_dim], repacked on the device.
    int mat(const std::string &name, int in_dim, int out_dim, qq_tensor **out)
    {
        qq_gguf_tensor t;
        if (!tensor(name, &t)) return set_error(ctx, "lfm2: tensor %s is missing", name.c_str());
        if (t.type != QQ_TYPE_Q8_0)
            return set_error(ctx, "lfm2: tensor %s has type %u (Q8_0 supported)", name.c_str(), t.type);
        if ((in_dim > 0 && t.shape[0] != (uint64_t)in_dim) || (out_dim > 0 && t.shape[1] != (uint64_t)out_dim) ||
            t.shape[2] != 1 || t.shape[0] > (uint64_t)kMaxIn || t.shape[1] > (1u << 24))
            return set_error(ctx, "lfm2: tensor %s has shape [%llu, %llu, %llu]", name.c_str(),
                             (unsigned long long)t.shape[0], (unsigned long long)t.shape[1],
                             (unsigned long long)t.shape[2]);
        const uint64_t nbytes = (t.shape[0] + 31) / 32 * 34 * t.shape[1];
        const uint8_t *b = bytes(t, nbytes);
        if (!b) return set_error(ctx, "lfm2: tensor %s runs past the file", name.c_str());
        if (int rc = qq_q8_0_upload(ctx, b, nbytes, (int)t.shape[0], (int)t.shape[1], 1, out)) return rc;
        m->tens.push_back(*out);
        return QQ_OK;
    }
    // _dequantConvKernel (src/lfm2-engine.js:146-180): [L, H] -> floats d * L + k.
    int conv_kernel(const qq_gguf_tensor &t, const std::string &name, int L, int H, float **out)
    {
        const uint64_t n = (uint64_t)L * H;
        if (t.shape[0] != (uint64_t)L || t.shape[1] != (uint64_t)H)
            return set_error(ctx, "lfm2: tensor %s is not [%d, %d]", name.c_str(), L, H);
        std::vector<float> v(n);
        if (t.type == QQ_TYPE_F32) {
            const uint8_t *b = bytes(t, n * 4);
            if (!b) return set_error(ctx, "lfm2: tensor %s runs past the file", name.c_str());
            std::memcpy(v.data(), b, n * 4);
        } else if (t.type == 1) {   // F16
            const uint8_t *b = bytes(t, n * 2);
            if (!b) return set_error(ctx, "lfm2: tensor %s runs past the file", name.c_str());
            for (uint64_t i = 0; i < n; i++) {
                uint16_t h;
                std::memcpy(&h, b + 2 * i, 2);
                v[i] = half_bits_to_float(h);
            }
        } else if (t.type == QQ_TYPE_Q8_0) {
            const uint64_t per = (uint64_t)((L + 31) / 32) * 34;
            const uint8_t *b = bytes(t, per * H);
            if (!b) return set_error(ctx, "lfm2: tensor %s runs past the file", name.c_str());
            for (int d = 0; d < H; d++) {
                const uint8_t *col = b + (uint64_t)d * per;
                uint16_t h;
                std::memcpy(&h, col, 2);
                const double sc = (double)half_bits_to_float(h);
                for (int k = 0; k < L; k++) v[(size_t)d * L + k] = (float)((int8_t)col[2 + k] * sc);
            }
        } else {
            return set_error(ctx, "lfm2: unsupported conv kernel type %u", t.type);
        }
        return upload(v.data(), n * 4, reinterpret_cast<void **>(out));
    }
};

int bind(Binder &B)
{
    qq_lfm2 *m = B.m;
    qq_lfm2_info &I = m->info;
    {
        const int64_t k = qq_gguf_find_key(B.g, "general.architecture");
        const char *s;
        uint64_t len;
        B.arch = (k >= 0 && qq_gguf_kv_string(B.g, (uint64_t)k, &s, &len) == QQ_OK) ? std::string(s, len)
                                                                                   : std::string("lfm2moe");
    }
    const std::string p = B.arch + ".";
    I.n_layers = (int)B.num(p + "block_count", 24);
    I.n_embd = (int)B.num(p + "embedding_length", 2048);
    I.n_heads = (int)B.num(p + "attention.head_count", 32);
    I.eps = B.num(p + "attention.layer_norm_rms_epsilon", 1e-5);
    I.n_experts = (int)B.num(p + "expert_count", 32);
    I.n_experts_used = (int)B.num(p + "expert_used_count", 4);
    // the forward writes n_experts_used indices per MoE block into idx_dev
    if (I.n_experts_used < 1 || I.n_experts_used > qq::MAX_K)
        return set_error(B.ctx, "lfm2: %sexpert_used_count = %d, supported 1..%d", p.c_str(), I.n_experts_used,
                         qq::MAX_K);
    I.n_dense_lead = (int)B.num(p + "leading_dense_block_count", 2);
    I.l_cache = (int)B.num(p + "shortconv.l_cache", 3);
    I.max_ctx = (int)std::min(B.num(p + "context_length", 4096), (double)kMaxCtx);
    I.rope_freq_base = B.num(p + "rope.freq_base", 0.0);
    if (I.rope_freq_base == 0.0) I.rope_freq_base = B.num(p + "rope_freq_base", 5000000.0);
    {
        // per-layer array (short-conv blocks 0): the largest positive entry
        const int64_t k = qq_gguf_find_key(B.g, (p + "attention.head_count_kv").c_str());
        uint32_t et;
        uint64_t n;
        if (k >= 0 && qq_gguf_kv_array(B.g, (uint64_t)k, &et, &n) == QQ_OK) {
            double best = -1.0;
            for (uint64_t i = 0; i < n; i++) {
                double v;
                if (qq_gguf_kv_array_number(B.g, (uint64_t)k, i, &v) == QQ_OK && v > 0 && v > best) best = v;
            }
            if (best <= 0) return set_error(B.ctx, "lfm2: %sattention.head_count_kv has no positive entry", p.c_str());
            I.n_head_kv = (int)best;
        } else {
            I.n_head_kv = (int)B.num(p + "attention.head_count_kv", 8);
        }
    }
    const int H = I.n_embd;
    if (I.n_layers < 1 || I.n_layers > 4096 || H < 1 || H > kMaxIn || I.n_heads < 1 || I.n_head_kv < 1 ||
        I.max_ctx < 1 || !(I.eps >= 0.0))
        return set_error(B.ctx, "lfm2: unsupported configuration (%d blocks, %d embd, %d/%d heads, ctx %d)",
                         I.n_layers, H, I.n_heads, I.n_head_kv, I.max_ctx);
    if (I.l_cache != 3)
        return set_error(B.ctx, "lfm2: shortconv.l_cache %d (the short-conv block is written for 3)", I.l_cache);

    // token embedding [H, vocab] (also the output head when output.weight is absent)
    qq_gguf_tensor te;
    if (!B.tensor("token_embd.weight", &te)) return set_error(B.ctx, "lfm2: tensor token_embd.weight is missing");
    I.n_vocab = (int)te.shape[1];
    if (int rc = B.mat("token_embd.weight", H, -1, &m->embd)) return rc;
    qq_gguf_tensor to;
    if (B.tensor("output.weight", &to)) {
        if (int rc = B.mat("output.weight", H, I.n_vocab, &m->output)) return rc;
    } else {
        m->output = m->embd;
    }
    if (int rc = B.vec_f32("token_embd_norm.weight", H, &m->out_norm)) return rc;

    m->layers.resize(I.n_layers);
    int n_conv = 0, n_attn = 0;
    I.head_dim = kHeadDim;
    I.n_ff = 7168;
    bool seen_attn = false, seen_dense = false;
    for (int i = 0; i < I.n_layers; i++) {
        LmLayer &L = m->layers[i];
        const std::string b = "blk." + std::to_string(i) + ".";
        qq_gguf_tensor ct;
        L.rec = B.tensor(b + "shortconv.conv.weight", &ct);
        L.moe = i >= I.n_dense_lead;
        if (int rc = B.vec_f32(b + "attn_norm.weight", H, &L.attn_norm)) return rc;
        if (int rc = B.vec_f32(b + "ffn_norm.weight", H, &L.ffn_norm)) return rc;
        if (L.rec) {
            L.conv_idx = n_conv++;
            if (int rc = B.conv_kernel(ct, b + "shortconv.conv.weight", I.l_cache, H, &L.kern)) return rc;
            if (int rc = B.mat(b + "shortconv.in_proj.weight", H, 3 * H, &L.in_proj)) return rc;
            if (int rc = B.mat(b + "shortconv.out_proj.weight", H, H, &L.out_proj)) return rc;
        } else {
            L.cache_idx = n_attn++;
            qq_gguf_tensor tq;
            if (!B.tensor(b + "attn_q.weight", &tq)) return set_error(B.ctx, "lfm2: tensor %sattn_q.weight is missing", b.c_str());
            if (!seen_attn) {
                // headDim from the first attention block (src/lfm2-engine.js:55-57)
                I.head_dim = (int)(tq.shape[1] / (uint64_t)I.n_heads);
                seen_attn = true;
            }
            if (I.head_dim != kHeadDim || tq.shape[1] != (uint64_t)I.n_heads * kHeadDim ||
                I.n_heads % I.n_head_kv != 0)
                return set_error(B.ctx, "lfm2: attention of %d heads x %d (head_dim 64 supported)", I.n_heads,
                                 I.head_dim);
            const int nq = I.n_heads * kHeadDim, nkv = I.n_head_kv * kHeadDim;
            if (int rc = B.mat(b + "attn_q.weight", H, nq, &L.wq)) return rc;
            if (int rc = B.mat(b + "attn_k.weight", H, nkv, &L.wk)) return rc;
            if (int rc = B.mat(b + "attn_v.weight", H, nkv, &L.wv)) return rc;
            if (int rc = B.mat(b + "attn_output.weight", nq, H, &L.wo)) return rc;
            if (int rc = B.vec_f32(b + "attn_q_norm.weight", kHeadDim, &L.qn)) return rc;
            if (int rc = B.vec_f32(b + "attn_k_norm.weight", kHeadDim, &L.kn)) return rc;
        }
        if (L.moe) {
            // Lfm2Engine gates with sigmoid + bias and its own nExpertsUsed
            // (src/lfm2-engine.js:417-447), whatever the architecture string
            if (int rc = qq_gguf_moe_layer(B.ctx, B.g, i, I.n_experts_used, QQ_GATING_SIGMOID_BIAS, &L.ffn_moe))
                return rc;
            m->moes.push_back(L.ffn_moe);
            if (!qq::decode_supported(B.ctx, L.ffn_moe, 1))
                return set_error(B.ctx, "lfm2: MoE block %d is outside the batch-1 decode kernel's shapes", i);
        } else {
            qq_gguf_tensor tg;
            if (!B.tensor(b + "ffn_gate.weight", &tg)) return set_error(B.ctx, "lfm2: tensor %sffn_gate.weight is missing", b.c_str());
            if (!seen_dense) {
                I.n_ff = (int)tg.shape[1];
                seen_dense = true;
            }
            if (int rc = B.mat(b + "ffn_gate.weight", H, -1, &L.gate)) return rc;
            if (int rc = B.mat(b + "ffn_up.weight", H, L.gate->out_dim, &L.up)) return rc;
            if (int rc = B.mat(b + "ffn_down.weight", L.gate->out_dim, H, &L.down)) return rc;
        }
    }
    I.n_attn_layers = n_attn;

    // state and activations
    m->conv_floats = (size_t)(I.l_cache - 1) * H;
    m->kv_floats = (size_t)I.n_head_kv * I.max_ctx * kHeadDim;
    void *v;
    if (int rc = B.alloc(std::max<size_t>(1, n_conv * m->conv_floats) * 4, &v)) return rc;
    m->conv_state = static_cast<float *>(v);
    if (int rc = B.alloc(std::max<size_t>(1, n_attn * m->kv_floats) * 4, &v)) return rc;
    m->kc = static_cast<float *>(v);
    if (int rc = B.alloc(std::max<size_t>(1, n_attn * m->kv_floats) * 4, &v)) return rc;
    m->vc = static_cast<float *>(v);
    int max_ff = I.n_ff;
    for (const LmLayer &L : m->layers)
        if (L.gate) max_ff = std::max(max_ff, L.gate->out_dim);
    const size_t nq = (size_t)I.n_heads * kHeadDim;
    float **bufs[] = {&m->hidden, &m->ybuf, &m->q, &m->kraw, &m->attn, &m->ffn, &m->logits};
    const size_t lens[] = {(size_t)H, (size_t)H, nq, (size_t)I.n_head_kv * kHeadDim, nq, (size_t)max_ff,
                           (size_t)I.n_vocab};
    for (int i = 0; i < 7; i++) {
        if (int rc = B.alloc(lens[i] * 4, &v)) return rc;
        *bufs[i] = static_cast<float *>(v);
    }
    if (int rc = B.alloc(qq::lfm2_attn_work_bytes(I.n_heads), &v)) return rc;
    m->attn_work = static_cast<double *>(v);
    const size_t nlk = (size_t)I.n_layers * I.n_experts_used;
    if (int rc = B.alloc(nlk * 4, &v)) return rc;
    m->r_idx = static_cast<int32_t *>(v);
    if (int rc = B.alloc(nlk * 8, &v)) return rc;
    m->r_w = static_cast<double *>(v);
    if (int rc = B.alloc((size_t)I.n_layers * I.n_experts * 4, &v)) return rc;
    m->r_probs = static_cast<float *>(v);
    // applyRoPE's frequencies 1 / base^(i / half) (src/tensor.js:135-137)
    double fr[kHeadDim / 2];
    for (int i = 0; i < kHeadDim / 2; i++) fr[i] = 1.0 / std::pow(I.rope_freq_base, (double)i / (kHeadDim / 2));
    if (int rc = B.upload(fr, sizeof fr, &v)) return rc;
    m->freq = static_cast<double *>(v);
    return qq_lfm2_reset(B.ctx, m);
}

}  // namespace

extern "C" {

void qq_lfm2_release(qq_ctx *ctx, qq_lfm2 *m)
{
    if (!m) return;
    if (ctx) (void)hipSetDevice(ctx->device);
    for (qq_moe *x : m->moes) qq_moe_release(ctx, x);
    for (qq_tensor *t : m->tens) qq_tensor_release(ctx, t);
    for (void *p : m->dev) (void)hipFree(p);
    delete m;
}

int qq_lfm2_create(qq_ctx *ctx, const qq_gguf *g, qq_lfm2 **out)
{
    if (!ctx) return QQ_E_ARG;
    if (!g || !out) return set_error(ctx, "lfm2_create: NULL argument");
    *out = nullptr;
    if (int rc = qq::no_capture(ctx, "qq_lfm2_create")) return rc;
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    qq_lfm2 *m = new (std::nothrow) qq_lfm2();
    if (!m) return set_error(ctx, "lfm2_create: out of host memory");
    qq_gguf_header_info hi;
    if (qq_gguf_header(g, &hi) != QQ_OK) {
        delete m;
        return set_error(ctx, "lfm2_create: %s", qq_gguf_last_error());
    }
    Binder B{ctx, g, m, std::string(), hi.file_size};
    int rc = bind(B);
    if (!rc) {
        const hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) rc = qq::check_hip(ctx, e, "hipStreamSynchronize");
    }
    if (rc) {
        qq_lfm2_release(ctx, m);
        return rc;
    }
    *out = m;
    return QQ_OK;
}

int qq_lfm2_get_info(const qq_lfm2 *m, qq_lfm2_info *out)
{
    if (!m || !out) return QQ_E_ARG;
    *out = m->info;
    return QQ_OK;
}

int qq_lfm2_reset(qq_ctx *ctx, qq_lfm2 *m)
{
    if (!ctx) return QQ_E_ARG;
    if (!m) return set_error(ctx, "lfm2_reset: NULL model");
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    m->timeouts_at_reset = ctx->timeouts;
    int n_conv = 0;
    for (const LmLayer &L : m->layers) n_conv += L.rec ? 1 : 0;
    if (int rc = qq::launch_lfm2_zero(ctx, m->conv_state, (size_t)n_conv * m->conv_floats)) return rc;
    if (int rc = qq::launch_lfm2_zero(ctx, m->kc, (size_t)m->info.n_attn_layers * m->kv_floats)) return rc;
    return qq::launch_lfm2_zero(ctx, m->vc, (size_t)m->info.n_attn_layers * m->kv_floats);
}

static int lfm2_forward(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits_dev, const uint8_t *mask,
                 int32_t *idx_dev, double *w_dev, float *probs_dev)
{
    if (!ctx) return QQ_E_ARG;
    if (!m) return set_error(ctx, "lfm2_forward: NULL model");
    const qq_lfm2_info &I = m->info;
    if (token < 0 || token >= I.n_vocab)
        return set_error(ctx, "lfm2_forward: token %d outside [0, %d)", token, I.n_vocab);
    if (position < 0 || position >= I.max_ctx)
        return set_error(ctx, "lfm2_forward: position %d outside [0, %d)", position, I.max_ctx);
    if (ctx->timeouts != m->timeouts_at_reset) {
        set_error(ctx, "lfm2_forward: a device-side wait on this context timed out since the model's "
                       "last reset, so its hidden row, conv states and KV cache are not valid: call "
                       "qq_lfm2_reset first");
        return QQ_E_STATE;
    }
    QQ_HIP(ctx, hipSetDevice(ctx->device));
    const int H = I.n_embd;
    if (int rc = qq::launch_lfm2_embed(ctx, m->embd, token, m->hidden)) return rc;
    for (int i = 0; i < I.n_layers; i++) {
        const LmLayer &L = m->layers[i];
        // operator block: attn_norm, then short-conv or attention, residual
        if (L.rec) {
            qq::LmLaunch c;
            c.x = m->hidden;
            c.mats[0] = L.in_proj;
            c.norm = 1;
            c.norm_w = L.attn_norm;
            c.eps = I.eps;
            c.y = m->ybuf;
            c.state = m->conv_state + (size_t)L.conv_idx * m->conv_floats;
            c.kern = L.kern;
            c.L = I.l_cache;
            c.H = H;
            if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_CONV, c)) return rc;
            qq::LmLaunch r;
            r.x = m->ybuf;
            r.mats[0] = L.out_proj;
            r.y = m->hidden;
            if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_RESID, r)) return rc;
        } else {
            float *kc = m->kc + (size_t)L.cache_idx * m->kv_floats;
            float *vc = m->vc + (size_t)L.cache_idx * m->kv_floats;
            qq::LmLaunch a;
            a.x = m->hidden;
            a.mats[0] = L.wq;
            a.mats[1] = L.wk;
            a.mats[2] = L.wv;
            a.norm = 1;
            a.norm_w = L.attn_norm;
            a.eps = I.eps;
            a.q = m->q;
            a.kraw = m->kraw;
            a.kc = kc;
            a.vc = vc;
            a.qn = L.qn;
            a.kn = L.kn;
            a.n_heads = I.n_heads;
            a.n_kv_heads = I.n_head_kv;
            a.pos = position;
            a.max_ctx = I.max_ctx;
            a.freq = m->freq;
            if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_QKV, a)) return rc;
            if (int rc = qq::launch_lfm2_attn(ctx, m->q, m->kraw, L.qn, L.kn, m->freq, I.eps, kc, vc, I.n_heads,
                                              I.n_head_kv, I.max_ctx, position + 1,
                                              1.0 / std::sqrt((double)kHeadDim), m->attn, m->attn_work))
                return rc;
            qq::LmLaunch r;
            r.x = m->attn;
            r.mats[0] = L.wo;
            r.y = m->hidden;
            if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_RESID, r)) return rc;
        }
        // FFN block: ffn_norm, then dense SwiGLU or MoE, residual
        if (L.moe) {
            const size_t rk = (size_t)i * I.n_experts_used, re = (size_t)i * I.n_experts;
            if (int rc = qq_moe_forward_norm_dev(ctx, L.ffn_moe, m->hidden, L.ffn_norm, I.eps, 1, mask,
                                                 idx_dev ? idx_dev + rk : nullptr, w_dev ? w_dev + rk : nullptr,
                                                 probs_dev ? probs_dev + re : nullptr))
                return rc;
        } else {
            qq::LmLaunch s;
            s.x = m->hidden;
            s.mats[0] = L.gate;
            s.mats[1] = L.up;
            s.norm = 1;
            s.norm_w = L.ffn_norm;
            s.eps = I.eps;
            s.y = m->ffn;
            if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_SWIGLU, s)) return rc;
            qq::LmLaunch r;
            r.x = m->ffn;
            r.mats[0] = L.down;
            r.y = m->hidden;
            if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_RESID, r)) return rc;
        }
    }
    if (logits_dev) {
        // output norm ("token_embd_norm.weight") and head
        qq::LmLaunch o;
        o.x = m->hidden;
        o.mats[0] = m->output;
        o.norm = 1;
        o.norm_w = m->out_norm;
        o.eps = I.eps;
        o.y = logits_dev;
        if (int rc = qq::launch_lfm2_mv(ctx, qq::LM_PLAIN, o)) return rc;
    }
    return QQ_OK;
}

int qq_lfm2_forward_dev(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits_dev,
                        int32_t *idx_dev)
{
    return lfm2_forward(ctx, m, token, position, logits_dev, nullptr, idx_dev, nullptr, nullptr);
}

int qq_lfm2_forward_routed_dev(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits_dev,
                               const uint8_t *mask, int32_t *idx_dev, double *w_dev, float *probs_dev)
{
    return lfm2_forward(ctx, m, token, position, logits_dev, mask, idx_dev, w_dev, probs_dev);
}

int qq_lfm2_forward_routed(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits,
                           const uint8_t *mask, int32_t *idx, double *w, float *probs)
{
    if (!ctx) return QQ_E_ARG;
    if (int rc = qq::no_capture(ctx, "qq_lfm2_forward")) return rc;
    if (!m) return set_error(ctx, "lfm2_forward: NULL model");
    if (int rc = lfm2_forward(ctx, m, token, position, logits ? m->logits : nullptr, mask, idx ? m->r_idx : nullptr,
                              w ? m->r_w : nullptr, probs ? m->r_probs : nullptr))
        return rc;
    const qq_lfm2_info &I = m->info;
    if (logits)
        QQ_HIP(ctx, hipMemcpyAsync(logits, m->logits, (size_t)I.n_vocab * 4, hipMemcpyDeviceToHost, ctx->stream));
    // the MoE blocks' rows (blocks n_dense_lead .. n_layers - 1); dense rows stay as they are
    const size_t l0 = (size_t)I.n_dense_lead, nm = (size_t)(I.n_layers - I.n_dense_lead);
    const size_t K = (size_t)I.n_experts_used, E = (size_t)I.n_experts;
    if (idx && nm)
        QQ_HIP(ctx, hipMemcpyAsync(idx + l0 * K, m->r_idx + l0 * K, nm * K * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (w && nm)
        QQ_HIP(ctx, hipMemcpyAsync(w + l0 * K, m->r_w + l0 * K, nm * K * 8, hipMemcpyDeviceToHost, ctx->stream));
    if (probs && nm)
        QQ_HIP(ctx, hipMemcpyAsync(probs + l0 * E, m->r_probs + l0 * E, nm * E * 4, hipMemcpyDeviceToHost,
                                   ctx->stream));
    return qq::check_device_error(ctx);
}

int qq_lfm2_forward(qq_ctx *ctx, qq_lfm2 *m, int token, int position, float *logits)
{
    return qq_lfm2_forward_routed(ctx, m, token, position, logits, nullptr, nullptr, nullptr, nullptr);
}

}  // extern "C"
