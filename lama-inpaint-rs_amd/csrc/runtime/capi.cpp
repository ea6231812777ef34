// extern "C" entry points of liblama_hip.so (include/lama_hip.h) and the
// embedded gfx950 code object.
#include <cstdio>
#include <cstring>
#include <string>

#include "engine.h"
#include "lama_hip.h"

// The code object built by `hipcc --genco --offload-arch=gfx950`, linked in
// verbatim so the library is self-contained.
__asm__(".section .rodata\n"
        ".balign 4096\n"
        ".global lama_hsaco_start\n"
        "lama_hsaco_start:\n"
        ".incbin \"" LAMA_HSACO_PATH "\"\n"
        ".global lama_hsaco_end\n"
        "lama_hsaco_end:\n"
        ".byte 0\n"
        ".balign 4096\n"
        ".global lama_scratch_hsaco_start\n"
        "lama_scratch_hsaco_start:\n"
        ".incbin \"" LAMA_SCRATCH_HSACO_PATH "\"\n"
        ".byte 0\n"
        ".previous\n");

struct lama_hip_ctx {
    lama::Engine eng;
};

namespace {
int fail(char *err, size_t len, const std::string &m)
{
    if (err && len) snprintf(err, len, "%s", m.c_str());
    return 1;
}
}  // namespace

// Every entry point with a context: a null context is an error, and no C++
// exception crosses the C boundary.
#define GUARD(expr)                          \
    do {                                     \
        if (!ctx) return fail(err, errlen, "lama_hip: null context"); \
        std::string e_;                      \
        try {                                \
            if (!(expr)) return fail(err, errlen, e_); \
        } catch (const std::exception &x) {  \
            return fail(err, errlen, x.what()); \
        }                                    \
        return 0;                            \
    } while (0)

extern "C" int lama_hip_open(lama_hip_ctx **out, char *err, size_t errlen)
{
    if (!out) return fail(err, errlen, "lama_hip_open: null output pointer");
    *out = nullptr;
    try {
        auto *c = new lama_hip_ctx;
        std::string e;
        if (!c->eng.open(e)) {
            delete c;
            return fail(err, errlen, e);
        }
        *out = c;
    } catch (const std::exception &x) {
        return fail(err, errlen, x.what());
    }
    return 0;
}

extern "C" void lama_hip_close(lama_hip_ctx *ctx) { delete ctx; }

extern "C" const char *lama_hip_plan_signature(void)
{
    // model::describe (model.rs:260-274) of the one plan this engine runs:
    // ReflectPad, model.1-4, 18 resblocks, Concat, 3 upsamples, ReflectPad,
    // OutConv; 4 + 2 * 18 FFC_BN_ACT calls
    return "29 steps, 40 FFC_BN_ACT calls, 18 resblocks";
}

extern "C" int lama_hip_load_weights(lama_hip_ctx *ctx, const void *blob, size_t blob_len,
                                     const lama_tensor_info *table, size_t n, char *err, size_t errlen)
{
    GUARD(ctx->eng.load_weights((const uint8_t *)blob, blob_len, table, n, e_));
}

extern "C" int lama_hip_forward(lama_hip_ctx *ctx, const float *input, int h, int w, float *output, char *err,
                                size_t errlen)
{
    GUARD(ctx->eng.forward_host(input, h, w, output, nullptr, e_));
}

extern "C" int lama_hip_forward_device(lama_hip_ctx *ctx, const float *d_input, int h, int w, float *d_output,
                                       void *stream, char *err, size_t errlen)
{
    GUARD(ctx->eng.forward_device(d_input, h, w, d_output, (hipStream_t)stream, e_));
}

extern "C" int lama_hip_forward_device_noalloc(lama_hip_ctx *ctx, const float *d_input, int h, int w,
                                               float *d_output, void *stream, char *err, size_t errlen)
{
    if (ctx && (!d_input || !d_output)) return fail(err, errlen, "lama_hip_forward_device_noalloc: null buffer");
    GUARD(ctx->eng.forward_device_noalloc(d_input, h, w, d_output, (hipStream_t)stream, e_));
}

extern "C" int lama_hip_forward_steps(lama_hip_ctx *ctx, const float *input, int h, int w, float *output,
                                      float *const *steps, char *err, size_t errlen)
{
    GUARD(ctx->eng.forward_host(input, h, w, output, steps, e_));
}

extern "C" int lama_hip_vram(uint64_t *free_bytes, uint64_t *total_bytes, char *name, size_t namelen, char *err,
                             size_t errlen)
{
    std::string e;
    const lama::HipApi *h = lama::hip_api(e);
    if (!h) return fail(err, errlen, e);
    int dev = getenv("LAMA_HIP_DEVICE") ? atoi(getenv("LAMA_HIP_DEVICE")) : 0;
    hipError_t r = h->hipInit(0);
    if (r == hipSuccess) r = h->hipSetDevice(dev);
    size_t f = 0, t = 0;
    if (r == hipSuccess) r = h->hipMemGetInfo(&f, &t);
    if (r != hipSuccess) return fail(err, errlen, lama::hip_error(*h, r, "hipMemGetInfo"));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    if (name && namelen) {
        char buf[256] = {0};
        if (h->hipDeviceGetName(buf, sizeof buf, dev) != hipSuccess) snprintf(buf, sizeof buf, "the GPU");
        snprintf(name, namelen, "%s", buf);
    }
    return 0;
}

extern "C" int lama_hip_profile(lama_hip_ctx *ctx, uint32_t mask)
{
    if (!ctx) return 1;
    ctx->eng.set_profile(mask);
    return 0;
}

extern "C" void lama_hip_profile_reset(lama_hip_ctx *ctx)
{
    if (ctx) ctx->eng.profile_reset();
}

extern "C" int lama_hip_profile_read(lama_hip_ctx *ctx, int i, char *name, size_t namelen, uint64_t *launches,
                                     double *ms, double *flops, double *bytes)
{
    std::string n;
    uint64_t l = 0;
    double m = 0, f = 0, b = 0;
    if (!ctx || !ctx->eng.profile_read(i, n, l, m, f, b)) return 0;
    if (name && namelen) snprintf(name, namelen, "%s", n.c_str());
    if (launches) *launches = l;
    if (ms) *ms = m;
    if (flops) *flops = f;
    if (bytes) *bytes = b;
    return 1;
}

extern "C" int lama_hip_profile_read_clock(lama_hip_ctx *ctx, int i, uint64_t *launches, double *ms)
{
    uint64_t l = 0;
    double m = 0;
    if (!ctx || !ctx->eng.profile_read_clock(i, l, m)) return 0;
    if (launches) *launches = l;
    if (ms) *ms = m;
    return 1;
}

extern "C" int lama_hip_timeline(lama_hip_ctx *ctx, int enable)
{
    std::string e;
    return ctx && ctx->eng.set_timeline(enable != 0, e) ? 0 : 1;
}

extern "C" int lama_hip_timeline_read(lama_hip_ctx *ctx, lama_launch_time *out, int max)
{
    std::string e;
    return ctx && out && max >= 0 ? ctx->eng.timeline_read(out, max, e) : -1;
}

extern "C" void lama_hip_print_stats(lama_hip_ctx *ctx)
{
    if (ctx) ctx->eng.print_stats();
}

extern "C" int lama_hip_plan_bytes(lama_hip_ctx *ctx, int h, int w, uint64_t *arena_bytes, uint64_t *weight_bytes,
                                   char *err, size_t errlen)
{
    GUARD(([&] {
        uint64_t a = 0, wb = 0;
        if (!ctx->eng.plan_bytes(h, w, a, wb, e_)) return false;
        if (arena_bytes) *arena_bytes = a;
        if (weight_bytes) *weight_bytes = wb;
        return true;
    })());
}

extern "C" int lama_hip_launch_count(lama_hip_ctx *ctx, int h, int w) { return ctx ? ctx->eng.launch_count(h, w) : -1; }

extern "C" int lama_hip_kernel_name(lama_hip_ctx *ctx, int h, int w, int family, char *name, size_t namelen)
{
    const char *n = ctx ? ctx->eng.kernel_name(h, w, family) : nullptr;
    if (!n || !name || std::strlen(n) + 1 > namelen) return 1;
    std::memcpy(name, n, std::strlen(n) + 1);
    return 0;
}

extern "C" int lama_hip_malloc(lama_hip_ctx *ctx, size_t bytes, void **ptr, char *err, size_t errlen)
{
    GUARD(ctx->eng.check(ctx->eng.hip()->hipMalloc(ptr, bytes), "hipMalloc", e_));
}

extern "C" int lama_hip_free(lama_hip_ctx *ctx, void *ptr)
{
    return ctx && ctx->eng.hip()->hipFree(ptr) == hipSuccess ? 0 : 1;
}

extern "C" int lama_hip_memcpy(lama_hip_ctx *ctx, void *dst, const void *src, size_t bytes, int kind, char *err,
                               size_t errlen)
{
    hipMemcpyKind k = kind == 1 ? hipMemcpyHostToDevice : kind == 2 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    GUARD(ctx->eng.check(ctx->eng.hip()->hipMemcpy(dst, src, bytes, k), "hipMemcpy", e_));
}

extern "C" int lama_hip_synchronize(lama_hip_ctx *ctx, char *err, size_t errlen)
{
    GUARD(ctx->eng.synchronize(e_));
}

extern "C" int lama_hip_inpaint(lama_hip_ctx *ctx, const uint8_t *rgb, const uint8_t *mask, int h, int w,
                                uint8_t *out_rgb, float *net_out, char *err, size_t errlen)
{
    if (ctx && (!rgb || !mask || !out_rgb)) return fail(err, errlen, "lama_hip_inpaint: null buffer");
    GUARD(ctx->eng.inpaint_host(rgb, mask, h, w, out_rgb, net_out, e_));
}

extern "C" int lama_hip_inpaint_device(lama_hip_ctx *ctx, const uint8_t *d_rgb, const uint8_t *d_mask, int h, int w,
                                       uint8_t *d_out_rgb, void *stream, char *err, size_t errlen)
{
    if (ctx && (!d_rgb || !d_mask || !d_out_rgb)) return fail(err, errlen, "lama_hip_inpaint_device: null buffer");
    GUARD(ctx->eng.inpaint_device(d_rgb, d_mask, h, w, d_out_rgb, (hipStream_t)stream, e_));
}

extern "C" int lama_hip_spectral(lama_hip_ctx *ctx, int ffc, const float *x, int h, int w, float *out,
                                 float *const *stages, char *err, size_t errlen)
{
    if (ctx && (!x || !out)) return fail(err, errlen, "lama_hip_spectral: null buffer");
    GUARD(ctx->eng.spectral_host(ffc, x, h, w, out, stages, e_));
}

extern "C" int lama_hip_spectral_device(lama_hip_ctx *ctx, int ffc, const float *d_x, int h, int w, float *d_out,
                                        void *stream, char *err, size_t errlen)
{
    if (ctx && (!d_x || !d_out)) return fail(err, errlen, "lama_hip_spectral_device: null buffer");
    GUARD(ctx->eng.spectral_device(ffc, d_x, h, w, d_out, (hipStream_t)stream, e_));
}

extern "C" int lama_hip_op_conv2d(lama_hip_ctx *ctx, const float *x, int cin, int h, int w, const float *wt,
                                  const float *bias, int cout, int k, int stride, const float *scale,
                                  const float *shift, int relu, float *out, char *err, size_t errlen)
{
    GUARD(ctx->eng.op_conv2d(x, cin, h, w, wt, bias, cout, k, stride, scale, shift, relu, out, e_));
}

extern "C" int lama_hip_op_conv_transpose(lama_hip_ctx *ctx, const float *x, int cin, int h, int w,
                                          const float *wt, const float *bias, int cout, const float *scale,
                                          const float *shift, int relu, float *out, char *err, size_t errlen)
{
    GUARD(ctx->eng.op_convt(x, cin, h, w, wt, bias, cout, scale, shift, relu, out, e_));
}

extern "C" int lama_hip_op_rfft2(lama_hip_ctx *ctx, const float *x, int c, int h, int w, float *out, char *err,
                                 size_t errlen)
{
    GUARD(ctx->eng.op_fft(false, x, nullptr, c, h, w, out, e_));
}

extern "C" int lama_hip_op_irfft2(lama_hip_ctx *ctx, const float *spec, const float *feat, int c, int h, int w,
                                  float *out, char *err, size_t errlen)
{
    GUARD(ctx->eng.op_fft(true, spec, feat, c, h, w, out, e_));
}

extern "C" int lama_hip_op_tail(lama_hip_ctx *ctx, const float *x, int cin, int h, int w, const float *wt,
                                const float *bias, float *out, char *err, size_t errlen)
{
    GUARD(ctx->eng.op_tail(x, cin, h, w, wt, bias, out, e_));
}
