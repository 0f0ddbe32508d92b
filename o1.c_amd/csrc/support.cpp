// Error buffer, launch stream, host bf16 helpers and the weight-store
// lookup. Mirrors the conventions of the reference's support.cu:12-44 and
// model.c:13-20 (process-global error strings, RNE bf16 conversion).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "hd_common.hpp"
#include "../../include/hd_hip.h"
#include "../../include/hd_weights.h"

static char g_cuda_err[512] = "";
static char g_err[1024] = "";
static hipStream_t g_stream = nullptr;

extern "C" char *hd_cuda_errbuf(void) { return g_cuda_err; }
extern "C" const char *hd_cuda_last_error(void) { return g_cuda_err; }
extern "C" void hd_cuda_clear_error(void) { g_cuda_err[0] = '\0'; }

extern "C" const char *hd_last_error(void) { return g_err; }
extern "C" void hd_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

hipStream_t hd_stream(void) { return g_stream; }
extern "C" void hd_hip_set_stream(void *s) { g_stream = (hipStream_t)s; }
extern "C" void *hd_hip_get_stream(void) { return (void *)g_stream; }
extern "C" int hd_hip_sync(void) { return (int)hipStreamSynchronize(g_stream); }

void hd_check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        snprintf(g_cuda_err, sizeof(g_cuda_err), "%s: launch failed: %s", what,
                 hipGetErrorString(e));
}

extern "C" uint16_t hd_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
extern "C" float hd_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
extern "C" void hd_bf16_buf_to_f32(const void *src, float *dst, size_t n) {
    const uint16_t *s = (const uint16_t *)src;
    for (size_t i = 0; i < n; i++) dst[i] = hd_bf16_to_f32(s[i]);
}
extern "C" void hd_f32_buf_to_bf16(const float *src, void *dst, size_t n) {
    uint16_t *d = (uint16_t *)dst;
    for (size_t i = 0; i < n; i++) d[i] = hd_f32_to_bf16(src[i]);
}

extern "C" const void *hd_weight_store_find(const hd_weight_store *s, const char *name) {
    if (!s || !name || !s->allocs) return nullptr;
    for (int64_t i = 0; i < s->n_allocs; i++)
        if (s->allocs[i].name[0] && strcmp(s->allocs[i].name, name) == 0)
            return s->allocs[i].dev_ptr;
    return nullptr;
}
