// GGUF v3 reader and direct-to-device MoE layer loader (host code).
//
// Parses a GGUF file the way GGUFReader does (src/gguf.js:1-94 header, KV and
// tensor-info tables; 96-131 value sizes; 177-226 value reads and key
// lookup; 235-261 tensor metas; 302-343 byte sizes) over a read-only memory
// map, so an 8.9 GB LFM2-8B-A1B file needs no whole-file buffer (the
// reference slices the File per tensor for the same reason, gguf.js:350-374).
// qq_gguf_moe_layer binds one MoE block the way the engines do
// (src/lfm2-engine.js:129-137, src/qwen3-engine.js:48-73) and repacks its
// Q8_0 expert tensors from the mapping straight into device memory.
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qq_gguf.h"
#include "qq_internal.h"

namespace {

// KV value types (gguf.js:17-22)
enum : uint32_t {
    KV_U8 = 0, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL,
    KV_STRING, KV_ARRAY, KV_U64, KV_I64, KV_F64,
};

constexpr int MAX_DIMS = 8;         // GGUF files hold at most 4; garbage counts stop here
constexpr int MAX_ARRAY_DEPTH = 16; // nested arrays

thread_local char g_err[512] = "";

int fail(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return QQ_E_ARG;
}

struct Kv {
    std::string key;
    uint32_t type;
    uint64_t val;   // file offset of the value
};

struct Tensor {
    std::string name;
    int n_dims;
    uint64_t ne[MAX_DIMS];
    uint32_t type;
    uint64_t offset;   // absolute
    uint64_t nbytes;   // rounded up to 256 (gguf.js:78-79)
};

}  // namespace

struct qq_gguf {
    const uint8_t *base = nullptr;
    uint64_t size = 0;
    size_t map_len = 0;        // 0: caller-owned bytes
    uint32_t version = 0;
    uint64_t data_start = 0;
    uint64_t alignment = 0;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_by_name;   // first of equal names
    std::unordered_map<std::string, size_t> kv_by_key;
};

namespace {

// Bounds-checked little-endian reads; `ok` turns false past the end.
struct Cursor {
    const qq_gguf *g;
    bool ok = true;
    uint64_t bad_at = 0;
    int64_t bad_type = -1;   // unknown value type met by skip_value
    bool too_deep = false;

    bool have(uint64_t off, uint64_t n)
    {
        if (off > g->size || n > g->size - off) {
            if (ok) bad_at = off;
            ok = false;
            return false;
        }
        return true;
    }
    template <typename T> T rd(uint64_t off)
    {
        T v{};
        if (have(off, sizeof(T))) memcpy(&v, g->base + off, sizeof(T));
        return v;
    }
};

uint64_t scalar_size(uint32_t t)
{
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    default: return 0;
    }
}

// _skipValue (gguf.js:96-131): offset just past a value of type t at off;
// UINT64_MAX on an unknown type or a read past the end.
uint64_t skip_value(Cursor &c, uint32_t t, uint64_t off, int depth)
{
    if (const uint64_t n = scalar_size(t)) return c.have(off, n) ? off + n : UINT64_MAX;
    if (t == KV_STRING) {
        const uint64_t len = c.rd<uint64_t>(off);
        if (!c.ok || !c.have(off + 8, len)) return UINT64_MAX;
        return off + 8 + len;
    }
    if (t == KV_ARRAY) {
        if (depth >= MAX_ARRAY_DEPTH) {
            c.too_deep = true;
            return UINT64_MAX;
        }
        const uint32_t et = c.rd<uint32_t>(off);
        const uint64_t n = c.rd<uint64_t>(off + 4);
        if (!c.ok) return UINT64_MAX;
        uint64_t p = off + 12;
        if (const uint64_t es = scalar_size(et)) {   // fixed-size elements: one bounds check
            if (n > (c.g->size - std::min(p, c.g->size)) / es) {
                c.have(p, UINT64_MAX);
                return UINT64_MAX;
            }
            return p + n * es;
        }
        for (uint64_t i = 0; i < n; i++) {
            p = skip_value(c, et, p, depth + 1);
            if (p == UINT64_MAX) return p;
        }
        return p;
    }
    c.bad_type = t;
    return UINT64_MAX;
}

// _tensorNbytes (gguf.js:302-343), before the 256-byte rounding
uint64_t tensor_nbytes(const Tensor &t)
{
    uint64_t n = 1;
    for (int d = 0; d < t.n_dims; d++) n *= t.ne[d];
    switch (t.type) {
    case 0: return n * 4;                      // F32
    case 1: return n * 2;                      // F16
    case 8: case 2: return (n + 31) / 32 * 34; // Q8_0, Q4_0
    case 3: return (n + 31) / 32 * 36;         // Q4_1
    case 6: return (n + 31) / 32 * 42;         // Q5_0
    case 7: return (n + 31) / 32 * 44;         // Q5_1
    case 10: return (n + 255) / 256 * 84;      // Q2_K
    case 11: return (n + 255) / 256 * 110;     // Q3_K
    case 12: return (n + 255) / 256 * 144;     // Q4_K
    case 13: return (n + 255) / 256 * 176;     // Q5_K
    case 14: return (n + 255) / 256 * 210;     // Q6_K
    default: return n * 4;                     // unknown: taken as F32, as the reference does
    }
}

bool kv_is_number(uint32_t t) { return scalar_size(t) != 0; }

double kv_scalar(const qq_gguf *g, uint32_t t, uint64_t off)
{
    const uint8_t *p = g->base + off;
    switch (t) {
    case KV_U8: return *p;
    case KV_I8: return (int8_t)*p;
    case KV_BOOL: return *p != 0;
    case KV_U16: { uint16_t v; memcpy(&v, p, 2); return v; }
    case KV_I16: { int16_t v; memcpy(&v, p, 2); return v; }
    case KV_U32: { uint32_t v; memcpy(&v, p, 4); return v; }
    case KV_I32: { int32_t v; memcpy(&v, p, 4); return v; }
    case KV_F32: { float v; memcpy(&v, p, 4); return v; }
    case KV_U64: { uint64_t v; memcpy(&v, p, 8); return (double)v; }
    case KV_I64: { int64_t v; memcpy(&v, p, 8); return (double)v; }
    case KV_F64: { double v; memcpy(&v, p, 8); return v; }
    }
    return NAN;
}

// Number(getKeyValue(key)) with JS conversion rules for the value kinds a
// GGUF key holds: numbers and bools as themselves, strings parsed as decimal
// numbers (NaN otherwise), absent keys and arrays NaN.
double kv_js_number(const qq_gguf *g, const char *key)
{
    const auto it = g->kv_by_key.find(key);
    if (it == g->kv_by_key.end()) return NAN;
    const Kv &kv = g->kvs[it->second];
    if (kv_is_number(kv.type)) return kv_scalar(g, kv.type, kv.val);
    if (kv.type == KV_STRING) {
        uint64_t len;
        memcpy(&len, g->base + kv.val, 8);
        std::string s((const char *)g->base + kv.val + 8, len);
        const size_t b = s.find_first_not_of(" \t\n\r");
        if (b == std::string::npos) return 0.0;   // Number("") === 0
        const size_t e = s.find_last_not_of(" \t\n\r");
        s = s.substr(b, e - b + 1);
        char *end = nullptr;
        const double v = strtod(s.c_str(), &end);
        return (end && *end == 0) ? v : NAN;
    }
    return NAN;
}

int parse(qq_gguf *g)
{
    Cursor c{g};
    if (g->size < 4 || memcmp(g->base, "GGUF", 4) != 0) {
        char sig[5] = {0};
        memcpy(sig, g->base, g->size < 4 ? g->size : 4);
        for (char &ch : sig)
            if (ch && (ch < 32 || ch > 126)) ch = '?';
        return fail("Invalid signature: %s", sig);
    }
    g->version = c.rd<uint32_t>(4);
    const uint64_t n_tensors = c.rd<uint64_t>(8);
    const uint64_t n_kv = c.rd<uint64_t>(16);
    if (!c.ok) return fail("GGUF header truncated (%llu bytes)", (unsigned long long)g->size);
    // (a version other than 3 is read on, as gguf.js:44-46 does after a warning)
    uint64_t off = 24;
    for (uint64_t i = 0; i < n_kv; i++) {
        const uint64_t klen = c.rd<uint64_t>(off);
        if (!c.ok || !c.have(off + 8, klen)) break;
        Kv kv;
        kv.key.assign((const char *)g->base + off + 8, klen);
        kv.type = c.rd<uint32_t>(off + 8 + klen);
        kv.val = off + 8 + klen + 4;
        if (!c.ok) break;
        const uint64_t next = skip_value(c, kv.type, kv.val, 0);
        if (next == UINT64_MAX) {
            if (c.bad_type >= 0) return fail("Unknown KV type: %lld", (long long)c.bad_type);
            if (c.too_deep) return fail("GGUF KV '%s': arrays nested deeper than %d", kv.key.c_str(),
                                        MAX_ARRAY_DEPTH);
            break;
        }
        g->kv_by_key.emplace(kv.key, g->kvs.size());   // first of equal keys, as findKey
        g->kvs.push_back(std::move(kv));
        off = next;
    }
    if (!c.ok) return fail("GGUF KV table truncated at offset %llu", (unsigned long long)c.bad_at);
    for (uint64_t i = 0; i < n_tensors; i++) {
        const uint64_t nlen = c.rd<uint64_t>(off);
        if (!c.ok || !c.have(off + 8, nlen)) break;
        Tensor t;
        t.name.assign((const char *)g->base + off + 8, nlen);
        off += 8 + nlen;
        const uint32_t nd = c.rd<uint32_t>(off);
        off += 4;
        if (!c.ok) break;
        if (nd > MAX_DIMS) return fail("GGUF tensor '%s' has %u dimensions", t.name.c_str(), nd);
        t.n_dims = (int)nd;
        for (int d = 0; d < MAX_DIMS; d++) t.ne[d] = 1;
        for (uint32_t d = 0; d < nd; d++, off += 8) t.ne[d] = c.rd<uint64_t>(off);
        t.type = c.rd<uint32_t>(off);
        t.offset = c.rd<uint64_t>(off + 4);   // relative until the data start is known
        off += 12;
        if (!c.ok) break;
        t.nbytes = (tensor_nbytes(t) + 255) / 256 * 256;
        g->tensor_by_name.emplace(t.name, g->tensors.size());
        g->tensors.push_back(std::move(t));
    }
    if (!c.ok) return fail("GGUF tensor table truncated at offset %llu", (unsigned long long)c.bad_at);
    // tensor data start (gguf.js:83-93): general.alignment, or 32 when absent or 0/NaN
    const double a = kv_js_number(g, "general.alignment");
    g->alignment = (std::isfinite(a) && a >= 1.0 && a < 1e18) ? (uint64_t)a : 32;
    g->data_start = off + (g->alignment - off % g->alignment) % g->alignment;
    for (Tensor &t : g->tensors) t.offset += g->data_start;
    return QQ_OK;
}

int finish_open(qq_gguf *g, qq_gguf **out)
{
    const int rc = parse(g);
    if (rc) {
        qq_gguf_close(g);
        return rc;
    }
    *out = g;
    return QQ_OK;
}

const Tensor *find(const qq_gguf *g, const char *name)
{
    const auto it = g->tensor_by_name.find(name);
    return it == g->tensor_by_name.end() ? nullptr : &g->tensors[it->second];
}

// The data of t, checked against the file (the reference reads past a short
// file into the next tensor or throws on the typed-array view).
const uint8_t *tensor_bytes(const qq_gguf *g, const Tensor &t, uint64_t need, qq_ctx *ctx)
{
    if (t.offset > g->size || need > g->size - t.offset) {
        fail("GGUF tensor '%s': %llu bytes at offset %llu run past the end of the file (%llu bytes)",
             t.name.c_str(), (unsigned long long)need, (unsigned long long)t.offset,
             (unsigned long long)g->size);
        (void)ctx;
        return nullptr;
    }
    return g->base + t.offset;
}

std::string arch_of(const qq_gguf *g)
{
    const auto it = g->kv_by_key.find("general.architecture");
    if (it == g->kv_by_key.end() || g->kvs[it->second].type != KV_STRING) return "";
    const Kv &kv = g->kvs[it->second];
    uint64_t len;
    memcpy(&len, g->base + kv.val, 8);
    return std::string((const char *)g->base + kv.val + 8, len);
}

// Q8_0 block with an fp16 scale -> float (the reference's _readF16 is exact)
float half_to_float(uint16_t h)
{
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(1024 + m), e - 25);
    return (float)(s ? -v : v);
}

}  // namespace

extern "C" {

const char *qq_gguf_last_error(void) { return g_err; }

int qq_gguf_open(const char *path, qq_gguf **out)
{
    if (!out) return fail("qq_gguf_open: out is NULL");
    *out = nullptr;
    if (!path) return fail("qq_gguf_open: path is NULL");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail("cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return fail("cannot read %s (empty or not a file)", path);
    }
    void *p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return fail("cannot map %s", path);
    qq_gguf *g = new (std::nothrow) qq_gguf();
    if (!g) {
        munmap(p, (size_t)st.st_size);
        return fail("host allocation failed");
    }
    g->base = (const uint8_t *)p;
    g->size = (uint64_t)st.st_size;
    g->map_len = (size_t)st.st_size;
    return finish_open(g, out);
}

int qq_gguf_open_memory(const void *bytes, size_t nbytes, qq_gguf **out)
{
    if (!out) return fail("qq_gguf_open_memory: out is NULL");
    *out = nullptr;
    if (!bytes && nbytes) return fail("qq_gguf_open_memory: NULL bytes");
    qq_gguf *g = new (std::nothrow) qq_gguf();
    if (!g) return fail("host allocation failed");
    static const uint8_t empty = 0;
    g->base = bytes ? (const uint8_t *)bytes : &empty;
    g->size = nbytes;
    return finish_open(g, out);
}

void qq_gguf_close(qq_gguf *g)
{
    if (!g) return;
    if (g->map_len) munmap((void *)g->base, g->map_len);
    delete g;
}

int qq_gguf_header(const qq_gguf *g, qq_gguf_header_info *h)
{
    if (!g || !h) return fail("qq_gguf_header: NULL argument");
    h->version = g->version;
    h->tensor_count = g->tensors.size();
    h->kv_count = g->kvs.size();
    h->file_size = g->size;
    h->alignment = g->alignment;
    h->data_offset = g->data_start;
    return QQ_OK;
}

int64_t qq_gguf_find_tensor(const qq_gguf *g, const char *name)
{
    if (!g || !name) return -1;
    const auto it = g->tensor_by_name.find(name);
    return it == g->tensor_by_name.end() ? -1 : (int64_t)it->second;
}

int qq_gguf_tensor_info(const qq_gguf *g, uint64_t index, qq_gguf_tensor *t)
{
    if (!g || !t) return fail("qq_gguf_tensor_info: NULL argument");
    if (index >= g->tensors.size()) return fail("tensor index %llu out of range", (unsigned long long)index);
    const Tensor &s = g->tensors[index];
    t->name = s.name.c_str();
    t->n_dims = s.n_dims;
    for (int d = 0; d < 4; d++) t->shape[d] = d < s.n_dims ? s.ne[d] : 1;
    t->type = s.type;
    t->offset = s.offset;
    t->nbytes = s.nbytes;
    return QQ_OK;
}

int64_t qq_gguf_find_key(const qq_gguf *g, const char *key)
{
    if (!g || !key) return -1;
    const auto it = g->kv_by_key.find(key);
    return it == g->kv_by_key.end() ? -1 : (int64_t)it->second;
}

int qq_gguf_kv_info(const qq_gguf *g, uint64_t index, const char **key, uint32_t *type)
{
    if (!g) return fail("qq_gguf_kv_info: NULL reader");
    if (index >= g->kvs.size()) return fail("KV index %llu out of range", (unsigned long long)index);
    if (key) *key = g->kvs[index].key.c_str();
    if (type) *type = g->kvs[index].type;
    return QQ_OK;
}

int qq_gguf_kv_number(const qq_gguf *g, uint64_t index, double *v)
{
    if (!g || !v) return fail("qq_gguf_kv_number: NULL argument");
    if (index >= g->kvs.size()) return fail("KV index %llu out of range", (unsigned long long)index);
    const Kv &kv = g->kvs[index];
    if (!kv_is_number(kv.type)) return fail("KV '%s' (type %u) is not a number", kv.key.c_str(), kv.type);
    *v = kv_scalar(g, kv.type, kv.val);
    return QQ_OK;
}

int qq_gguf_kv_string(const qq_gguf *g, uint64_t index, const char **s, uint64_t *len)
{
    if (!g || !s || !len) return fail("qq_gguf_kv_string: NULL argument");
    if (index >= g->kvs.size()) return fail("KV index %llu out of range", (unsigned long long)index);
    const Kv &kv = g->kvs[index];
    if (kv.type != KV_STRING) return fail("KV '%s' (type %u) is not a string", kv.key.c_str(), kv.type);
    memcpy(len, g->base + kv.val, 8);
    *s = (const char *)g->base + kv.val + 8;
    return QQ_OK;
}

int qq_gguf_kv_array(const qq_gguf *g, uint64_t index, uint32_t *elem_type, uint64_t *n)
{
    if (!g || !elem_type || !n) return fail("qq_gguf_kv_array: NULL argument");
    if (index >= g->kvs.size()) return fail("KV index %llu out of range", (unsigned long long)index);
    const Kv &kv = g->kvs[index];
    if (kv.type != KV_ARRAY) return fail("KV '%s' (type %u) is not an array", kv.key.c_str(), kv.type);
    memcpy(elem_type, g->base + kv.val, 4);
    memcpy(n, g->base + kv.val + 4, 8);
    return QQ_OK;
}

int qq_gguf_kv_array_number(const qq_gguf *g, uint64_t index, uint64_t i, double *v)
{
    uint32_t et;
    uint64_t n;
    if (int rc = qq_gguf_kv_array(g, index, &et, &n)) return rc;
    if (!v) return fail("qq_gguf_kv_array_number: NULL argument");
    if (i >= n) return fail("array index %llu of %llu", (unsigned long long)i, (unsigned long long)n);
    if (!kv_is_number(et)) return fail("array of type %u is not numeric", et);
    *v = kv_scalar(g, et, g->kvs[index].val + 12 + i * scalar_size(et));
    return QQ_OK;
}

int qq_gguf_moe_params(const qq_gguf *g, int block, int K, int gating, qq_gguf_moe_info *info)
{
    if (!g || !info) return fail("qq_gguf_moe_params: NULL argument");
    memset(info, 0, sizeof *info);
    const std::string arch = arch_of(g);
    // engine choice of html/chat.html:206-207: lfm2moe / lfm2 -> Lfm2Engine, else Qwen3Engine
    const bool lfm2 = arch.empty() || arch == "lfm2moe" || arch == "lfm2";
    if (gating < 0) gating = lfm2 ? QQ_GATING_SIGMOID_BIAS : QQ_GATING_SOFTMAX;
    if (gating != QQ_GATING_SIGMOID_BIAS && gating != QQ_GATING_SOFTMAX)
        return fail("unknown gating %d", gating);
    if (K <= 0) {
        // expert_used_count, else the engine default (lfm2-engine.js:24, qwen3-engine.js:41)
        const std::string p = (arch.empty() ? std::string("lfm2moe") : arch) + ".expert_used_count";
        const double k = kv_js_number(g, p.c_str());
        if (std::isnan(k) || k == 0.0) K = lfm2 ? 4 : 8;   // Number(x) || default
        else if (k >= 1.0 && k <= 1e6) K = (int)k;
        else return fail("%s = %g is not a usable top-K", p.c_str(), k);
    }
    char name[160];
    snprintf(name, sizeof name, "blk.%d.ffn_gate_inp.weight", block);
    const Tensor *r = find(g, name);
    snprintf(name, sizeof name, "blk.%d.ffn_gate_exps.weight", block);
    const Tensor *ge = find(g, name);
    snprintf(name, sizeof name, "blk.%d.ffn_up_exps.weight", block);
    const Tensor *ue = find(g, name);
    snprintf(name, sizeof name, "blk.%d.ffn_down_exps.weight", block);
    const Tensor *de = find(g, name);
    snprintf(name, sizeof name, "blk.%d.exp_probs_b.bias", block);
    const Tensor *b = find(g, name);
    if (!r) return fail("block %d has no MoE router (blk.%d.ffn_gate_inp.weight)", block, block);
    if (!ge || !ue || !de) return fail("block %d: expert tensors ffn_{gate,up,down}_exps missing", block);
    if (ge->type != QQ_TYPE_Q8_0 || ue->type != QQ_TYPE_Q8_0 || de->type != QQ_TYPE_Q8_0)
        return fail("block %d: expert tensors must be Q8_0 (types %u %u %u)", block, ge->type, ue->type, de->type);
    if (ge->n_dims != 3 || ue->n_dims != 3 || de->n_dims != 3 || r->n_dims != 2)
        return fail("block %d: expert tensors must be 3-D and the router 2-D", block);
    const uint64_t H = ge->ne[0], F = ge->ne[1], E = ge->ne[2];
    if (ue->ne[0] != H || ue->ne[1] != F || ue->ne[2] != E || de->ne[0] != F || de->ne[1] != H ||
        de->ne[2] != E || r->ne[0] != H || r->ne[1] != E)
        return fail("block %d: shapes do not match [H, F, E] / [F, H, E] / [H, E]", block);
    if (H > 1u << 20 || F > 1u << 20 || E > 1u << 20) return fail("block %d: implausible shape", block);
    if (r->type != QQ_TYPE_F32 && r->type != QQ_TYPE_Q8_0)
        return fail("Unsupported tensor type for matmul: %u", r->type);
    info->H = (int)H;
    info->F = (int)F;
    info->E = (int)E;
    info->K = K;
    info->gating = gating;
    info->router_type = (int)r->type;
    info->has_bias = (gating == QQ_GATING_SIGMOID_BIAS && b) ? 1 : 0;
    if (info->has_bias && b->type != QQ_TYPE_F32 && b->type != QQ_TYPE_Q8_0)
        return fail("Unsupported weight type for norm: %u", b->type);
    return QQ_OK;
}

int qq_gguf_moe_layer(qq_ctx *ctx, const qq_gguf *g, int block, int K, int gating, qq_moe **out)
{
    if (!ctx || !out) return QQ_E_ARG;
    *out = nullptr;
    qq_gguf_moe_info p;
    if (qq_gguf_moe_params(g, block, K, gating, &p)) return qq::set_error(ctx, "%s", g_err);
    const uint64_t H = p.H, F = p.F, E = p.E;
    char name[160];
    auto bytes_of = [&](const char *fmt, uint64_t need) -> const uint8_t * {
        snprintf(name, sizeof name, fmt, block);
        return tensor_bytes(g, *find(g, name), need, ctx);
    };
    const uint64_t nbH = (H + 31) / 32, nbF = (F + 31) / 32;
    const uint8_t *rb = bytes_of("blk.%d.ffn_gate_inp.weight",
                                 p.router_type == QQ_TYPE_F32 ? E * H * 4 : E * nbH * 34);
    const uint8_t *gb = rb ? bytes_of("blk.%d.ffn_gate_exps.weight", E * F * nbH * 34) : nullptr;
    const uint8_t *ub = gb ? bytes_of("blk.%d.ffn_up_exps.weight", E * F * nbH * 34) : nullptr;
    const uint8_t *db = ub ? bytes_of("blk.%d.ffn_down_exps.weight", E * H * nbF * 34) : nullptr;
    if (!db) return qq::set_error(ctx, "%s", g_err);
    // selection bias through _readWeightF32 (src/tensor.js:80-100)
    std::vector<float> bias;
    if (p.has_bias) {
        snprintf(name, sizeof name, "blk.%d.exp_probs_b.bias", block);
        const Tensor &bt = *find(g, name);
        const uint8_t *bb = tensor_bytes(g, bt, bt.type == QQ_TYPE_F32 ? E * 4 : (E + 31) / 32 * 34, ctx);
        if (!bb) return qq::set_error(ctx, "%s", g_err);
        bias.resize(E);
        if (bt.type == QQ_TYPE_F32) {
            memcpy(bias.data(), bb, E * 4);
        } else {
            for (uint64_t e = 0; e < E; e++) {
                const uint8_t *blk = bb + (e / 32) * 34;
                uint16_t h;
                memcpy(&h, blk, 2);
                bias[e] = (float)((int8_t)blk[2 + e % 32] * (double)half_to_float(h));
            }
        }
    }
    qq_tensor *t[3] = {nullptr, nullptr, nullptr};
    int rc = qq_q8_0_upload(ctx, gb, E * F * nbH * 34, (int)H, (int)F, (int)E, &t[0]);
    if (!rc) rc = qq_q8_0_upload(ctx, ub, E * F * nbH * 34, (int)H, (int)F, (int)E, &t[1]);
    if (!rc) rc = qq_q8_0_upload(ctx, db, E * H * nbF * 34, (int)F, (int)H, (int)E, &t[2]);
    qq_moe *m = nullptr;
    if (!rc)
        rc = qq_moe_create(ctx, rb, p.router_type, p.has_bias ? bias.data() : nullptr, t[0], t[1], t[2],
                           (int)H, (int)F, (int)E, p.K, &m);
    if (!rc) rc = qq_moe_set_gating(ctx, m, p.gating);
    if (!rc) {
        for (int i = 0; i < 3; i++) m->owned[i] = t[i];   // released with the layer
        *out = m;
        return QQ_OK;
    }
    {
        if (m) qq_moe_release(ctx, m);
        for (qq_tensor *x : t) qq_tensor_release(ctx, x);
        return rc;
    }
}

}  // extern "C"

const uint8_t *qq::gguf_base(const qq_gguf *g) { return g ? g->base : nullptr; }
