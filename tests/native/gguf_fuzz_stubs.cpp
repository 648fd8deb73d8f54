// The device-side entry points the GGUF reader links against, for the host
// fuzz build of qwenqwen3.js_amd/csrc/gguf.cpp.  The fuzz driver never binds
// a layer (qq_gguf_moe_layer), so each of these only reports that it was
// reached.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../include/qq_moe.h"

namespace qq {
int set_error(qq_ctx *, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    return QQ_E_ARG;
}
}  // namespace qq

static int unreachable(const char *what)
{
    fprintf(stderr, "gguf_fuzz: %s reached\n", what);
    abort();
}

extern "C" {
int qq_q8_0_upload(qq_ctx *, const void *, size_t, int, int, int, qq_tensor **) { return unreachable("qq_q8_0_upload"); }
int qq_moe_create(qq_ctx *, const void *, int, const float *, const qq_tensor *, const qq_tensor *, const qq_tensor *,
                  int, int, int, int, qq_moe **)
{
    return unreachable("qq_moe_create");
}
int qq_moe_set_gating(qq_ctx *, qq_moe *, int) { return unreachable("qq_moe_set_gating"); }
int qq_moe_release(qq_ctx *, qq_moe *) { return unreachable("qq_moe_release"); }
int qq_tensor_release(qq_ctx *, qq_tensor *) { return unreachable("qq_tensor_release"); }
}
