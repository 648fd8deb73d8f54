/*
 * qq_gguf.h -- GGUF v3 reader and direct-to-device MoE layer loader.
 *
 * Host-side part of libqqmoe.so.  The reader follows GGUFReader
 * (src/gguf.js) over a read-only memory map of the file, so a model larger
 * than one ArrayBuffer (an 8.9 GB LFM2-8B-A1B Q8_0 file) is read without
 * copying; qq_gguf_moe_layer repacks one block's expert tensors from that
 * mapping into device memory and returns a ready qq_moe layer.
 *
 * Context-free calls (everything but qq_gguf_moe_layer) report failures
 * through qq_gguf_last_error() (per thread); qq_gguf_moe_layer reports
 * through qq_last_error(ctx).
 */
#ifndef QQ_GGUF_H
#define QQ_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "qq_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qq_gguf qq_gguf;

/* getHeader (src/gguf.js:157-165) plus where the tensor data starts. */
typedef struct qq_gguf_header_info {
    uint32_t version;       /* read on when it is not 3, as gguf.js:44-46 does */
    uint64_t tensor_count;
    uint64_t kv_count;
    uint64_t file_size;
    uint64_t alignment;     /* general.alignment, 32 when absent (gguf.js:84) */
    uint64_t data_offset;   /* first byte of the tensor data section */
} qq_gguf_header_info;

/* getTensorMeta (src/gguf.js:235-255) for the whole-file buffer:
 * offset is absolute in the file, nbytes is the byte size rounded up to 256
 * (gguf.js:77-79), shape is GGUF order (shape[0] = input dim), padded with 1. */
typedef struct qq_gguf_tensor {
    const char *name;       /* owned by the reader */
    int n_dims;
    uint64_t shape[4];
    uint32_t type;          /* GGUF tensor type (gguf.js:25-33) */
    uint64_t offset;
    uint64_t nbytes;
} qq_gguf_tensor;

/* The MoE block parameters qq_gguf_moe_layer derives. */
typedef struct qq_gguf_moe_info {
    int H, F, E, K;
    int gating;             /* QQ_GATING_* */
    int router_type;        /* QQ_TYPE_F32 or QQ_TYPE_Q8_0 */
    int has_bias;           /* exp_probs_b.bias present and used */
} qq_gguf_moe_info;

/* new GGUFReader(buffer) (src/gguf.js:2-11, header parse 37-94).  Fails on a
 * bad signature ("Invalid signature: ..."), an unknown KV type ("Unknown KV
 * type: N") or a table that runs past the end of the file. */
int qq_gguf_open(const char *path, qq_gguf **out);
/* Same over caller bytes, which must outlive the reader (not copied). */
int qq_gguf_open_memory(const void *bytes, size_t nbytes, qq_gguf **out);
void qq_gguf_close(qq_gguf *g);
const char *qq_gguf_last_error(void);

int qq_gguf_header(const qq_gguf *g, qq_gguf_header_info *out);

/* getTensorMetaByName (src/gguf.js:256-261): index of the first tensor of
 * that name, -1 when there is none (the reference returns null). */
int64_t qq_gguf_find_tensor(const qq_gguf *g, const char *name);
int qq_gguf_tensor_info(const qq_gguf *g, uint64_t index, qq_gguf_tensor *out);

/* findKey (src/gguf.js:215-220): index of the first KV of that key, or -1. */
int64_t qq_gguf_find_key(const qq_gguf *g, const char *key);
/* getKVKey / getKVType (src/gguf.js:174-175); *key is owned by the reader. */
int qq_gguf_kv_info(const qq_gguf *g, uint64_t index, const char **key, uint32_t *type);
/* getKVValue (src/gguf.js:177-212) by kind: a number (integer, float or
 * bool types, 64-bit integers rounded to double as Number() does), a string
 * (UTF-8 bytes in the file, not NUL-terminated), or an array's element type
 * and length plus its numeric elements. */
int qq_gguf_kv_number(const qq_gguf *g, uint64_t index, double *out);
int qq_gguf_kv_string(const qq_gguf *g, uint64_t index, const char **s, uint64_t *len);
int qq_gguf_kv_array(const qq_gguf *g, uint64_t index, uint32_t *elem_type, uint64_t *n);
int qq_gguf_kv_array_number(const qq_gguf *g, uint64_t index, uint64_t i, double *out);

/* Parameters of MoE block `block` as the engines bind it
 * (src/lfm2-engine.js:129-137, src/qwen3-engine.js:41-73):
 *   tensors blk.N.ffn_gate_inp.weight [H, E] (F32 or Q8_0),
 *   blk.N.ffn_{gate,up}_exps.weight [H, F, E], blk.N.ffn_down_exps.weight
 *   [F, H, E] (Q8_0), blk.N.exp_probs_b.bias [E] (optional, sigmoid only);
 *   K <= 0: <arch>.expert_used_count, else 4 (LFM2) or 8 (Qwen3);
 *   gating < 0: by general.architecture as html/chat.html:206-207 picks the
 *   engine: lfm2moe / lfm2 -> QQ_GATING_SIGMOID_BIAS, others -> QQ_GATING_SOFTMAX.
 * Needs no device. */
int qq_gguf_moe_params(const qq_gguf *g, int block, int K, int gating, qq_gguf_moe_info *out);

/* Upload MoE block `block` (parameters as qq_gguf_moe_params) and create its
 * layer.  The layer owns its expert tensors: qq_moe_release frees them.  The
 * reader may be closed afterwards. */
int qq_gguf_moe_layer(qq_ctx *ctx, const qq_gguf *g, int block, int K, int gating, qq_moe **out);

#ifdef __cplusplus
}
#endif

#endif /* QQ_GGUF_H */
