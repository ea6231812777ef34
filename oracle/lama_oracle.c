/*
 * lama_oracle.c -- CPU restatement of the reference CPU engine, as a checker.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls this
 * file: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may use it, and only as the checker (or the timed CPU baseline), never as a
 * compute path of the product.
 *
 * It restates, loop for loop, the arithmetic of jacobsparts/lama-inpaint-rs
 * v0.2.4 `lama-rs/src/cpu.rs` (plus the plan of `model.rs`, `reflect_index` of
 * `image.rs` and the input/composite rules of `main.rs`).  Every function cites
 * the reference lines it follows.  Rules kept so the result is the reference's
 * own, not merely close to it:
 *   - f32 arithmetic with no contraction (built with -ffp-contract=off; Rust
 *     never fuses a*b+c), accumulation in the reference's order per output;
 *   - the FFT in f64 with the reference's twiddle recurrence (radix-2) and its
 *     Bluestein chirp for other lengths -- including the fact, verified
 *     numerically, that its Bluestein path computes the opposite-sign DFT of the
 *     radix-2 path (forward on a non-power-of-two length equals n*ifft);
 *   - no parallel reductions: OpenMP splits only independent outputs (the same
 *     units rayon splits), so results do not depend on the thread count.
 *
 * Where a loop is reordered for speed (the convolutions vectorise across
 * output columns), the per-output sequence of operations is unchanged, which
 * keeps every output bit-identical to the literal loop order.
 *
 * Pinning: tests/test_oracle.py checks each function against torch/numpy
 * library routines, brute-force DFTs, closed forms and invariants, and against
 * the committed golden vectors in tests/golden/.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ helpers */

/* image.rs:159-169 -- PyTorch 'reflect' index (edge sample not repeated). */
OR_EXPORT size_t or_reflect_index(long i, size_t n)
{
    if (n == 1) return 0;
    long period = 2 * ((long)n - 1);
    long m = i % period;
    if (m < 0) m += period; /* rem_euclid */
    if (m >= (long)n) m = period - m;
    return (size_t)m;
}

typedef struct {
    int c, h, w;
    float *data; /* [c][h][w] */
} Acts;

static Acts acts_new(int c, int h, int w)
{
    Acts a = {c, h, w, NULL};
    size_t n = (size_t)c * h * w;
    a.data = (float *)calloc(n ? n : 1, sizeof(float));
    return a;
}
static void acts_free(Acts *a) { free(a->data); a->data = NULL; }
static Acts acts_clone(const Acts *a)
{
    Acts b = acts_new(a->c, a->h, a->w);
    memcpy(b.data, a->data, (size_t)a->c * a->h * a->w * sizeof(float));
    return b;
}

/* -------------------------------------------------------------- BatchNorm */

/* cpu.rs:58-62 -- eval BatchNorm folded to scale/shift, f32 throughout. */
OR_EXPORT void or_bn_fold(const float *w, const float *b, const float *mean, const float *var,
                          int n, float *scale, float *shift)
{
    for (int i = 0; i < n; ++i) {
        float s = w[i] / sqrtf(var[i] + 1e-5f);
        scale[i] = s;
        float ms = mean[i] * s;
        shift[i] = b[i] - ms;
    }
}

/* cpu.rs:66-76 -- x*s + t per channel (no fusion). */
static void bn_apply(const float *scale, const float *shift, Acts *a)
{
    long plane = (long)a->h * a->w;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < a->c; ++c) {
        float s = scale[c], t = shift[c];
        float *p = a->data + (long)c * plane;
        for (long i = 0; i < plane; ++i) {
            float v = p[i] * s;
            p[i] = v + t;
        }
    }
}

/* cpu.rs:376-382 */
static void relu_inplace(Acts *a)
{
    long n = (long)a->c * a->h * a->w;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i)
        if (a->data[i] < 0.0f) a->data[i] = 0.0f;
}

/* cpu.rs:384-388 -- 1/(1+exp(-x)) in f32. */
static void sigmoid_inplace(Acts *a)
{
    long n = (long)a->c * a->h * a->w;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) {
        float e = expf(-a->data[i]);
        a->data[i] = 1.0f / (1.0f + e);
    }
}

/* cpu.rs:702-708 */
static void add_inplace(Acts *dst, const Acts *src)
{
    long n = (long)dst->c * dst->h * dst->w;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) dst->data[i] += src->data[i];
}

/* ---------------------------------------------------------- convolutions */

/* cpu.rs:110-168 -- k x k convolution, stride, reflect or zero padding.
 * Weights [cout][cin][kh][kw], optional bias.  Per output: acc = bias, then
 * + w*x over ci, ky, kx in that order.  The loop nest below walks ox
 * innermost; each output still sees exactly that sequence of adds. */
OR_EXPORT void or_conv2d(const float *src, int cin, int h, int w, const float *wt, const float *bias,
                         int cout, int kh, int kw, int pad, int stride, int reflect, float *dst)
{
    int oh = (h + 2 * pad - kh) / stride + 1;
    int ow = (w + 2 * pad - kw) / stride + 1;
    int k = kh * kw;
    /* per-kx source column (or -1 = skipped tap, zero padding) */
    long *sxt = (long *)malloc(sizeof(long) * (size_t)kw * ow);
    for (int kx = 0; kx < kw; ++kx)
        for (int ox = 0; ox < ow; ++ox) {
            long ix = (long)ox * stride + kx;
            long sx;
            if (ix < pad || ix - pad >= w)
                sx = reflect ? (long)or_reflect_index(ix - pad, (size_t)w) : -1;
            else
                sx = ix - pad;
            sxt[(long)kx * ow + ox] = sx;
        }
#pragma omp parallel for schedule(dynamic, 4)
    for (long row = 0; row < (long)cout * oh; ++row) {
        int co = (int)(row / oh), oy = (int)(row % oh);
        const float *wp = wt + (long)co * cin * k;
        float b = bias ? bias[co] : 0.0f;
        float *acc = dst + ((long)co * oh + oy) * ow;
        for (int ox = 0; ox < ow; ++ox) acc[ox] = b;
        for (int ci = 0; ci < cin; ++ci) {
            const float *sp = src + (long)ci * h * w;
            const float *kp = wp + (long)ci * k;
            for (int ky = 0; ky < kh; ++ky) {
                long iy = (long)oy * stride + ky;
                long sy;
                if (iy < pad || iy - pad >= h) {
                    if (!reflect) continue;
                    sy = (long)or_reflect_index(iy - pad, (size_t)h);
                } else {
                    sy = iy - pad;
                }
                const float *srow = sp + sy * w;
                const float *krow = kp + (long)ky * kw;
                for (int kx = 0; kx < kw; ++kx) {
                    float kv = krow[kx];
                    const long *sx = sxt + (long)kx * ow;
                    for (int ox = 0; ox < ow; ++ox) {
                        long s = sx[ox];
                        if (s < 0) continue;
                        float prod = kv * srow[s];
                        acc[ox] += prod;
                    }
                }
            }
        }
    }
    free(sxt);
}

/* cpu.rs:171-191 -- 1x1 convolution: acc = bias, + w[ci]*x[ci] in ci order. */
OR_EXPORT void or_conv1x1(const float *src, int cin, long plane, const float *wt, const float *bias,
                          int cout, float *dst)
{
#pragma omp parallel for schedule(dynamic, 1)
    for (int co = 0; co < cout; ++co) {
        const float *wp = wt + (long)co * cin;
        float b = bias ? bias[co] : 0.0f;
        float *d = dst + (long)co * plane;
        for (long i = 0; i < plane; ++i) d[i] = b;
        for (int ci = 0; ci < cin; ++ci) {
            float kv = wp[ci];
            const float *s = src + (long)ci * plane;
            for (long i = 0; i < plane; ++i) {
                float prod = kv * s[i];
                d[i] += prod;
            }
        }
    }
}

/* cpu.rs:328-374 -- ConvTranspose2d k3 s2 p1 op1 as the reference's scatter.
 * Weights [cin][cout][3][3], bias [cout]; zero inputs are skipped as there. */
OR_EXPORT void or_conv_transpose(const float *src, int cin, int h, int w, const float *wt,
                                 const float *bias, int cout, float *dst)
{
    int oh = h * 2, ow = w * 2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int co = 0; co < cout; ++co) {
        float *d = dst + (long)co * oh * ow;
        float b = bias[co];
        for (long i = 0; i < (long)oh * ow; ++i) d[i] = b;
        for (int ci = 0; ci < cin; ++ci) {
            const float *sp = src + (long)ci * h * w;
            const float *kp = wt + ((long)ci * cout + co) * 9;
            for (int iy = 0; iy < h; ++iy) {
                const float *row = sp + (long)iy * w;
                for (int ix = 0; ix < w; ++ix) {
                    float v = row[ix];
                    if (v == 0.0f) continue;
                    for (int ky = 0; ky < 3; ++ky) {
                        int oy = iy * 2 + ky;
                        if (oy == 0 || oy > oh) continue;
                        float *drow = d + (long)(oy - 1) * ow;
                        for (int kx = 0; kx < 3; ++kx) {
                            int ox = ix * 2 + kx;
                            if (ox == 0 || ox > ow) continue;
                            float prod = v * kp[ky * 3 + kx];
                            drow[ox - 1] += prod;
                        }
                    }
                }
            }
        }
    }
}

/* cpu.rs:718-738 */
static Acts reflect_pad_acts(const Acts *a, int pad)
{
    if (pad == 0) return acts_clone(a);
    Acts out = acts_new(a->c, a->h + 2 * pad, a->w + 2 * pad);
    int oh = out.h, ow = out.w;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < a->c; ++c) {
        const float *sp = a->data + (long)c * a->h * a->w;
        float *d = out.data + (long)c * oh * ow;
        for (int y = 0; y < oh; ++y) {
            size_t sy = or_reflect_index(y - pad, (size_t)a->h);
            for (int x = 0; x < ow; ++x) {
                size_t sx = or_reflect_index(x - pad, (size_t)a->w);
                d[(long)y * ow + x] = sp[sy * a->w + sx];
            }
        }
    }
    return out;
}

/* OR_EXPORT wrapper used by the tests (ReflectionPad2d). */
OR_EXPORT void or_reflect_pad(const float *src, int c, int h, int w, int pad, float *dst)
{
    Acts a = {c, h, w, (float *)src};
    Acts o = reflect_pad_acts(&a, pad);
    memcpy(dst, o.data, (size_t)c * o.h * o.w * sizeof(float));
    acts_free(&o);
}

/* ------------------------------------------------------------------ FFT */

static int is_pow2(size_t n) { return n && !(n & (n - 1)); }

/* cpu.rs:888-927 -- iterative radix-2, bit reversal then stages with the
 * twiddle advanced by complex multiplication. */
static void fft_radix2(double *re, double *im, size_t n, int inverse)
{
    size_t j = 0;
    for (size_t i = 1; i < n; ++i) {
        size_t bit = n >> 1;
        while (j & bit) {
            j ^= bit;
            bit >>= 1;
        }
        j |= bit;
        if (i < j) {
            double t = re[i]; re[i] = re[j]; re[j] = t;
            t = im[i]; im[i] = im[j]; im[j] = t;
        }
    }
    double sign = inverse ? 1.0 : -1.0;
    for (size_t len = 2; len <= n; len <<= 1) {
        double ang = sign * 2.0 * M_PI / (double)len;
        double wr = cos(ang), wi = sin(ang);
        size_t half = len / 2;
        for (size_t i = 0; i < n; i += len) {
            double cr = 1.0, ci = 0.0;
            for (size_t k = 0; k < half; ++k) {
                double ur = re[i + k], ui = im[i + k];
                double xr = re[i + k + half], xi = im[i + k + half];
                double a1 = xr * cr, a2 = xi * ci;
                double vr = a1 - a2;
                double b1 = xr * ci, b2 = xi * cr;
                double vi = b1 + b2;
                re[i + k] = ur + vr;
                im[i + k] = ui + vi;
                re[i + k + half] = ur - vr;
                im[i + k + half] = ui - vi;
                double c1 = cr * wr, c2 = ci * wi;
                double ncr = c1 - c2;
                double d1 = cr * wi, d2 = ci * wr;
                ci = d1 + d2;
                cr = ncr;
            }
        }
    }
}

/* cpu.rs:947-980 -- Bluestein tables: chirp exp(sign*i*pi*(j^2 mod 2n)/n),
 * m = next power of two >= 2n-1, b = chirp wrapped at both ends, FFT'd. */
typedef struct {
    size_t n, m;
    int inverse;
    double *wr, *wi, *br, *bi;
} Blue;

static void blue_build(Blue *t, size_t n, int inverse)
{
    double sign = inverse ? 1.0 : -1.0;
    t->n = n;
    t->inverse = inverse;
    t->wr = (double *)malloc(sizeof(double) * n);
    t->wi = (double *)malloc(sizeof(double) * n);
    for (size_t j = 0; j < n; ++j) {
        double jm = (double)(((long long)j * (long long)j) % (2 * (long long)n));
        double ang = sign * M_PI * jm / (double)n;
        t->wr[j] = cos(ang);
        t->wi[j] = sin(ang);
    }
    size_t m = 1;
    while (m < 2 * n - 1) m <<= 1;
    t->m = m;
    t->br = (double *)calloc(m, sizeof(double));
    t->bi = (double *)calloc(m, sizeof(double));
    t->br[0] = t->wr[0];
    t->bi[0] = t->wi[0];
    for (size_t j = 1; j < n; ++j) {
        t->br[j] = t->wr[j];
        t->bi[j] = t->wi[j];
        t->br[m - j] = t->wr[j];
        t->bi[m - j] = t->wi[j];
    }
    fft_radix2(t->br, t->bi, m, 0);
}

static void blue_free(Blue *t)
{
    free(t->wr); free(t->wi); free(t->br); free(t->bi);
}

/* cpu.rs:984-1011 -- a = x*conj(w); A = FFT(a); A *= B; a = IFFT(A)/m;
 * X = a*conj(w).  (This is the transform of opposite sign to fft_radix2.) */
static void fft_bluestein(double *re, double *im, size_t n, const Blue *t)
{
    size_t m = t->m;
    double *ar = (double *)calloc(m, sizeof(double));
    double *ai = (double *)calloc(m, sizeof(double));
    for (size_t j = 0; j < n; ++j) {
        double p1 = re[j] * t->wr[j], p2 = im[j] * t->wi[j];
        ar[j] = p1 + p2;
        double q1 = im[j] * t->wr[j], q2 = re[j] * t->wi[j];
        ai[j] = q1 - q2;
    }
    fft_radix2(ar, ai, m, 0);
    for (size_t i = 0; i < m; ++i) {
        double a1 = ar[i] * t->br[i], a2 = ai[i] * t->bi[i];
        double xr = a1 - a2;
        double b1 = ar[i] * t->bi[i], b2 = ai[i] * t->br[i];
        double xi = b1 + b2;
        ar[i] = xr;
        ai[i] = xi;
    }
    fft_radix2(ar, ai, m, 1);
    double inv_m = 1.0 / (double)m;
    for (size_t j = 0; j < n; ++j) {
        double cr = ar[j] * inv_m, ci = ai[j] * inv_m;
        double p1 = cr * t->wr[j], p2 = ci * t->wi[j];
        re[j] = p1 + p2;
        double q1 = ci * t->wr[j], q2 = cr * t->wi[j];
        im[j] = q1 - q2;
    }
    free(ar);
    free(ai);
}

/* cpu.rs:875-885 -- length dispatch. `blue` holds tables for this length. */
static void fft1(double *re, double *im, size_t n, int inverse, const Blue *blue)
{
    if (n <= 1) return;
    if (is_pow2(n))
        fft_radix2(re, im, n, inverse);
    else
        fft_bluestein(re, im, n, blue);
}

/* cpu.rs:846-871 -- rows first, then columns (gathered into a scratch). */
static void fft2(double *re, double *im, size_t h, size_t w, int inverse)
{
    Blue bw = {0}, bh = {0};
    if (w > 1 && !is_pow2(w)) blue_build(&bw, w, inverse);
    if (h > 1 && !is_pow2(h)) blue_build(&bh, h, inverse);
    for (size_t y = 0; y < h; ++y) fft1(re + y * w, im + y * w, w, inverse, &bw);
    double *cr = (double *)malloc(sizeof(double) * h);
    double *ci = (double *)malloc(sizeof(double) * h);
    for (size_t x = 0; x < w; ++x) {
        for (size_t y = 0; y < h; ++y) {
            cr[y] = re[y * w + x];
            ci[y] = im[y * w + x];
        }
        fft1(cr, ci, h, inverse, &bh);
        for (size_t y = 0; y < h; ++y) {
            re[y * w + x] = cr[y];
            im[y * w + x] = ci[y];
        }
    }
    free(cr);
    free(ci);
    if (bw.wr) blue_free(&bw);
    if (bh.wr) blue_free(&bh);
}

/* cpu.rs:769-783 -- rfft2 with norm='ortho'; dst = [2][h][w/2+1] (re, im). */
OR_EXPORT void or_rfft2_ortho(const float *src, int h, int w, float *dst)
{
    size_t hw = (size_t)w / 2 + 1;
    size_t n = (size_t)h * w;
    double *re = (double *)malloc(sizeof(double) * n);
    double *im = (double *)calloc(n, sizeof(double));
    for (size_t i = 0; i < n; ++i) re[i] = (double)src[i];
    fft2(re, im, (size_t)h, (size_t)w, 0);
    double scale = 1.0 / sqrt((double)n);
    for (size_t y = 0; y < (size_t)h; ++y)
        for (size_t x = 0; x < hw; ++x) {
            dst[y * hw + x] = (float)(re[y * w + x] * scale);
            dst[(size_t)h * hw + y * hw + x] = (float)(im[y * w + x] * scale);
        }
    free(re);
    free(im);
}

/* cpu.rs:801-837 -- inverse with the 2-D Hermitian completion
 * F[(h-y)%h][w-x] = conj(X[y][x]) for the missing columns, real part kept. */
OR_EXPORT void or_irfft2_ortho(const float *src, int h, int w, float *dst)
{
    size_t hw = (size_t)w / 2 + 1;
    size_t n = (size_t)h * w;
    double *re = (double *)calloc(n, sizeof(double));
    double *im = (double *)calloc(n, sizeof(double));
    for (size_t y = 0; y < (size_t)h; ++y)
        for (size_t x = 0; x < hw; ++x) {
            re[y * w + x] = (double)src[y * hw + x];
            im[y * w + x] = (double)src[(size_t)h * hw + y * hw + x];
        }
    for (size_t y = 0; y < (size_t)h; ++y)
        for (size_t x = hw; x < (size_t)w; ++x) {
            size_t xm = (size_t)w - x;
            if (xm >= hw) continue;
            size_t ym = ((size_t)h - y) % (size_t)h;
            re[y * w + x] = re[ym * w + xm];
            im[y * w + x] = -im[ym * w + xm];
        }
    fft2(re, im, (size_t)h, (size_t)w, 1);
    double scale = 1.0 / sqrt((double)n);
    for (size_t i = 0; i < n; ++i) dst[i] = (float)(re[i] * scale);
    free(re);
    free(im);
}

/* ------------------------------------------------------- the weights table */

typedef struct {
    const char *name;
    const float *data;
    int ndim;
    long shape[4];
} or_tensor;

typedef struct {
    const or_tensor *t;
    int n;
    char err[512];
} Store;

static const or_tensor *store_get(Store *s, const char *name)
{
    for (int i = 0; i < s->n; ++i)
        if (strcmp(s->t[i].name, name) == 0) return &s->t[i];
    snprintf(s->err, sizeof s->err, "missing tensor in weight blob: %s", name);
    return NULL;
}

/* ------------------------------------------------------------- the network */

typedef struct {
    int present;
    const float *w;
    const float *bias;
    int cin, cout, kh, kw;
} Conv;

typedef struct {
    int present;
    float *scale, *shift;
    int n;
    char prefix[128];
    const float *gamma, *beta; /* for calibration */
    float *cal_mean, *cal_var; /* set by a calibrating forward */
} Bn;

/* When set, every BN is re-fitted to the statistics of its own input during
 * the forward (test fixture generation only: the "calibrated-BN" weights). */
static int g_calibrate = 0;

typedef struct {
    Conv conv1, conv2, fu_conv;
    Bn bn1, fu_bn;
    int half, stride;
} Spectral;

typedef struct {
    int kernel, stride, pad, reflect;
    int in_local, in_global, out_local, out_global;
    Conv l2l, l2g, g2l;
    int has_spectral;
    Spectral sp;
    Bn bn_l, bn_g;
} Ffc;

enum { ST_PAD, ST_FFC, ST_RES, ST_CONCAT, ST_UP, ST_OUT };

typedef struct {
    int kind;
    int pad;          /* ST_PAD */
    Ffc ffc, ffc2;    /* ST_FFC: ffc; ST_RES: ffc (conv1), ffc2 (conv2) */
    Conv convt;       /* ST_UP: weight [cin][cout][3][3] + bias */
    Bn up_bn;
    Conv out;         /* ST_OUT */
} Step;

typedef struct {
    Step steps[40];
    int n;
} Net;

static int load_conv(Store *s, const char *prefix, Conv *c)
{
    char nm[256];
    snprintf(nm, sizeof nm, "%s.weight", prefix);
    const or_tensor *t = store_get(s, nm);
    if (!t) return -1;
    c->present = 1;
    c->w = t->data;
    c->cout = (int)t->shape[0];
    c->cin = (int)t->shape[1];
    c->kh = t->ndim > 2 ? (int)t->shape[2] : 1;
    c->kw = t->ndim > 3 ? (int)t->shape[3] : 1;
    snprintf(nm, sizeof nm, "%s.bias", prefix);
    c->bias = NULL;
    for (int i = 0; i < s->n; ++i)
        if (strcmp(s->t[i].name, nm) == 0) c->bias = s->t[i].data;
    return 0;
}

/* cpu.rs:45-64 */
static int load_bn(Store *s, const char *prefix, int channels, Bn *bn)
{
    char nm[256];
    const char *parts[4] = {"weight", "bias", "running_mean", "running_var"};
    const or_tensor *t[4];
    for (int i = 0; i < 4; ++i) {
        snprintf(nm, sizeof nm, "%s.%s", prefix, parts[i]);
        t[i] = store_get(s, nm);
        if (!t[i]) return -1;
        long n = 1;
        for (int d = 0; d < t[i]->ndim; ++d) n *= t[i]->shape[d];
        if (n != channels) {
            snprintf(s->err, sizeof s->err, "BatchNorm %s: expected %d channels", prefix, channels);
            return -1;
        }
    }
    bn->present = 1;
    bn->n = channels;
    snprintf(bn->prefix, sizeof bn->prefix, "%s", prefix);
    bn->gamma = t[0]->data;
    bn->beta = t[1]->data;
    bn->scale = (float *)malloc(sizeof(float) * channels);
    bn->shift = (float *)malloc(sizeof(float) * channels);
    or_bn_fold(t[0]->data, t[1]->data, t[2]->data, t[3]->data, channels, bn->scale, bn->shift);
    return 0;
}

/* model.rs:211-257 (the split rule) + cpu.rs:561-616 (the names). */
static int load_ffc(Store *s, int index, int sub, int cin, int cout, int kernel, int stride,
                    int pad, float ratio_gin, float ratio_gout, Ffc *f)
{
    memset(f, 0, sizeof *f);
    int in_global = (int)((float)cin * ratio_gin);
    int out_global = (int)((float)cout * ratio_gout);
    f->in_global = in_global;
    f->out_global = out_global;
    f->in_local = cin - in_global;
    f->out_local = cout - out_global;
    f->kernel = kernel;
    f->stride = stride;
    f->pad = pad;
    f->reflect = 1;
    char fp[128], part[128], nm[256];
    if (sub == 0) {
        snprintf(fp, sizeof fp, "model.%d.ffc", index);
        snprintf(part, sizeof part, "model.%d", index);
    } else {
        snprintf(fp, sizeof fp, "model.%d.conv%d.ffc", index, sub);
        snprintf(part, sizeof part, "model.%d.conv%d", index, sub);
    }
    if (f->in_local && f->out_local) {
        snprintf(nm, sizeof nm, "%s.convl2l", fp);
        if (load_conv(s, nm, &f->l2l)) return -1;
    }
    if (f->in_local && f->out_global) {
        snprintf(nm, sizeof nm, "%s.convl2g", fp);
        if (load_conv(s, nm, &f->l2g)) return -1;
    }
    if (f->in_global && f->out_local) {
        snprintf(nm, sizeof nm, "%s.convg2l", fp);
        if (load_conv(s, nm, &f->g2l)) return -1;
    }
    if (in_global > 0 && out_global > 0) {
        /* cpu.rs:218-236 */
        f->has_spectral = 1;
        Spectral *sp = &f->sp;
        sp->half = out_global / 2;
        sp->stride = stride;
        snprintf(nm, sizeof nm, "%s.convg2g.conv1.0", fp);
        if (load_conv(s, nm, &sp->conv1)) return -1;
        snprintf(nm, sizeof nm, "%s.convg2g.conv1.1", fp);
        if (load_bn(s, nm, sp->half, &sp->bn1)) return -1;
        snprintf(nm, sizeof nm, "%s.convg2g.conv2", fp);
        if (load_conv(s, nm, &sp->conv2)) return -1;
        snprintf(nm, sizeof nm, "%s.convg2g.fu.conv_layer", fp);
        if (load_conv(s, nm, &sp->fu_conv)) return -1;
        snprintf(nm, sizeof nm, "%s.convg2g.fu.bn", fp);
        if (load_bn(s, nm, 2 * sp->half, &sp->fu_bn)) return -1;
    }
    if (f->out_local > 0) {
        snprintf(nm, sizeof nm, "%s.bn_l", part);
        if (load_bn(s, nm, f->out_local, &f->bn_l)) return -1;
    }
    if (f->out_global > 0) {
        snprintf(nm, sizeof nm, "%s.bn_g", part);
        if (load_bn(s, nm, f->out_global, &f->bn_g)) return -1;
    }
    return 0;
}

static void bn_release(Bn *b)
{
    free(b->scale);
    free(b->shift);
    free(b->cal_mean);
    free(b->cal_var);
    b->scale = b->shift = NULL;
    b->cal_mean = b->cal_var = NULL;
}

/* Calibration (fixture generation, not a reference function): set the BN's
 * running statistics to the per-channel mean / biased variance of `a`, and
 * refold.  Values are kept so the caller can write them into a container. */
static void bn_calibrate(Bn *bn, const Acts *a)
{
    if (!g_calibrate) return;
    long plane = (long)a->h * a->w;
    if (!bn->cal_mean) {
        bn->cal_mean = (float *)malloc(sizeof(float) * bn->n);
        bn->cal_var = (float *)malloc(sizeof(float) * bn->n);
    }
    for (int c = 0; c < a->c; ++c) {
        const float *p = a->data + (long)c * plane;
        double m = 0, v = 0;
        for (long i = 0; i < plane; ++i) m += p[i];
        m /= (double)plane;
        for (long i = 0; i < plane; ++i) v += (p[i] - m) * (p[i] - m);
        v /= (double)plane;
        bn->cal_mean[c] = (float)m;
        bn->cal_var[c] = (float)v;
    }
    or_bn_fold(bn->gamma, bn->beta, bn->cal_mean, bn->cal_var, bn->n, bn->scale, bn->shift);
}

static Bn *net_bn(void *p, int i);

static void ffc_release(Ffc *f)
{
    bn_release(&f->bn_l);
    bn_release(&f->bn_g);
    if (f->has_spectral) {
        bn_release(&f->sp.bn1);
        bn_release(&f->sp.fu_bn);
    }
}

/* model.rs:135-207 + cpu.rs:460-482 -- the 29-step plan with weights. */
OR_EXPORT void *or_net_load(const or_tensor *tensors, int n, char *err, int errlen)
{
    Store s = {tensors, n, {0}};
    Net *net = (Net *)calloc(1, sizeof(Net));
    int k = 0;
    const float R = 0.75f;
#define FAIL()                                                   \
    do {                                                         \
        if (err && errlen > 0) snprintf(err, errlen, "%s", s.err); \
        free(net);                                               \
        return NULL;                                             \
    } while (0)
    net->steps[k].kind = ST_PAD;
    net->steps[k++].pad = 3;
    net->steps[k].kind = ST_FFC;
    if (load_ffc(&s, 1, 0, 4, 64, 7, 1, 0, 0.0f, 0.0f, &net->steps[k++].ffc)) FAIL();
    net->steps[k].kind = ST_FFC;
    if (load_ffc(&s, 2, 0, 64, 128, 3, 2, 1, 0.0f, 0.0f, &net->steps[k++].ffc)) FAIL();
    net->steps[k].kind = ST_FFC;
    if (load_ffc(&s, 3, 0, 128, 256, 3, 2, 1, 0.0f, 0.0f, &net->steps[k++].ffc)) FAIL();
    net->steps[k].kind = ST_FFC;
    if (load_ffc(&s, 4, 0, 256, 512, 3, 2, 1, 0.0f, R, &net->steps[k++].ffc)) FAIL();
    for (int idx = 5; idx <= 22; ++idx) {
        net->steps[k].kind = ST_RES;
        if (load_ffc(&s, idx, 1, 512, 512, 3, 1, 1, R, R, &net->steps[k].ffc)) FAIL();
        if (load_ffc(&s, idx, 2, 512, 512, 3, 1, 1, R, R, &net->steps[k].ffc2)) FAIL();
        ++k;
    }
    net->steps[k++].kind = ST_CONCAT;
    const int up_idx[3] = {24, 27, 30}, up_cout[3] = {256, 128, 64};
    for (int u = 0; u < 3; ++u) {
        char nm[64];
        net->steps[k].kind = ST_UP;
        snprintf(nm, sizeof nm, "model.%d", up_idx[u]);
        if (load_conv(&s, nm, &net->steps[k].convt)) FAIL();
        /* ConvTranspose2d weights are [cin][cout][3][3] (cpu.rs:321-326) */
        {
            Conv *ct = &net->steps[k].convt;
            int t = ct->cin;
            ct->cin = ct->cout;
            ct->cout = t;
        }
        if (!net->steps[k].convt.bias) {
            snprintf(s.err, sizeof s.err, "missing tensor in weight blob: model.%d.bias", up_idx[u]);
            FAIL();
        }
        snprintf(nm, sizeof nm, "model.%d", up_idx[u] + 1);
        if (load_bn(&s, nm, up_cout[u], &net->steps[k].up_bn)) FAIL();
        ++k;
    }
    net->steps[k].kind = ST_PAD;
    net->steps[k++].pad = 3;
    net->steps[k].kind = ST_OUT;
    if (load_conv(&s, "model.34", &net->steps[k++].out)) FAIL();
#undef FAIL
    net->n = k;
    return net;
}

OR_EXPORT void or_net_free(void *p)
{
    Net *net = (Net *)p;
    if (!net) return;
    for (int i = 0; i < net->n; ++i) {
        Step *st = &net->steps[i];
        if (st->kind == ST_FFC) ffc_release(&st->ffc);
        if (st->kind == ST_RES) {
            ffc_release(&st->ffc);
            ffc_release(&st->ffc2);
        }
        if (st->kind == ST_UP) bn_release(&st->up_bn);
    }
    free(net);
}

/* cpu.rs:623-629 */
static Acts ffc_conv(const Ffc *f, const Conv *c, const Acts *src)
{
    if (f->kernel == 1) {
        Acts o = acts_new(c->cout, src->h, src->w);
        or_conv1x1(src->data, c->cin, (long)src->h * src->w, c->w, c->bias, c->cout, o.data);
        return o;
    }
    int oh = (src->h + 2 * f->pad - c->kh) / f->stride + 1;
    int ow = (src->w + 2 * f->pad - c->kw) / f->stride + 1;
    Acts o = acts_new(c->cout, oh, ow);
    or_conv2d(src->data, c->cin, src->h, src->w, c->w, c->bias, c->cout, c->kh, c->kw, f->pad,
              f->stride, f->reflect, o.data);
    return o;
}

static Acts conv1x1_acts(const Conv *c, const Acts *src)
{
    Acts o = acts_new(c->cout, src->h, src->w);
    or_conv1x1(src->data, c->cin, (long)src->h * src->w, c->w, c->bias, c->cout, o.data);
    return o;
}

/* cpu.rs:390-411 (only reached by a strided spectral block, absent here) */
static Acts avg_pool2x2(const Acts *x)
{
    int oh = x->h / 2, ow = x->w / 2;
    Acts o = acts_new(x->c, oh, ow);
    for (int c = 0; c < x->c; ++c) {
        const float *sp = x->data + (long)c * x->h * x->w;
        float *d = o.data + (long)c * oh * ow;
        for (int oy = 0; oy < oh; ++oy)
            for (int ox = 0; ox < ow; ++ox) {
                float a = sp[(2 * oy) * x->w + 2 * ox], b = sp[(2 * oy) * x->w + 2 * ox + 1];
                float cc = sp[(2 * oy + 1) * x->w + 2 * ox], dd = sp[(2 * oy + 1) * x->w + 2 * ox + 1];
                float s = a + b;
                s = s + cc;
                s = s + dd;
                d[oy * ow + ox] = s * 0.25f;
            }
    }
    return o;
}

/* The LAMA_DUMP_SPECTRAL stages (cpu.rs:242-257) of the next
 * spectral_forward, when set: [0] conv1 + BN + ReLU, [1] the stacked
 * spectrum, [2] the FU conv after BN + ReLU, [3] f + FU(f).  Test hook only. */
static float *const *g_spec_dump = NULL;

static void spec_dump(int i, const Acts *a)
{
    if (g_spec_dump && g_spec_dump[i])
        memcpy(g_spec_dump[i], a->data, sizeof(float) * (size_t)a->c * a->h * a->w);
}

/* cpu.rs:270-308 -- FourierUnit: per-channel rfft2 (stacked re/im planes,
 * channel-major pairs), 1x1 conv + BN + ReLU, per-channel irfft2. */
static Acts fourier_unit(Spectral *sp, const Acts *x)
{
    int h = x->h, w = x->w, hw = w / 2 + 1;
    long cplane = (long)h * hw;
    Acts spec = acts_new(2 * sp->half, h, hw);
#pragma omp parallel for schedule(dynamic, 1)
    for (int c = 0; c < sp->half; ++c)
        or_rfft2_ortho(x->data + (long)c * h * w, h, w, spec.data + 2 * c * cplane);
    spec_dump(1, &spec);
    Acts conv = conv1x1_acts(&sp->fu_conv, &spec);
    acts_free(&spec);
    bn_calibrate((Bn *)&sp->fu_bn, &conv);
    bn_apply(sp->fu_bn.scale, sp->fu_bn.shift, &conv);
    relu_inplace(&conv);
    spec_dump(2, &conv);
    Acts out = acts_new(sp->half, h, w);
#pragma omp parallel for schedule(dynamic, 1)
    for (int c = 0; c < sp->half; ++c)
        or_irfft2_ortho(conv.data + 2 * c * cplane, h, w, out.data + (long)c * h * w);
    acts_free(&conv);
    return out;
}

/* cpu.rs:239-265 -- SpectralTransform: conv2(f + FU(f)), f = ReLU(BN(conv1(x))). */
static Acts spectral_forward(Spectral *sp, const Acts *x)
{
    Acts pooled = sp->stride == 2 ? avg_pool2x2(x) : acts_clone(x);
    Acts feat = conv1x1_acts(&sp->conv1, &pooled);
    acts_free(&pooled);
    bn_calibrate((Bn *)&sp->bn1, &feat);
    bn_apply(sp->bn1.scale, sp->bn1.shift, &feat);
    relu_inplace(&feat);
    spec_dump(0, &feat);
    Acts fu = fourier_unit(sp, &feat);
    Acts sum = acts_new(sp->half, feat.h, feat.w);
    long n = (long)sp->half * feat.h * feat.w;
    for (long i = 0; i < n; ++i) sum.data[i] = feat.data[i] + fu.data[i];
    spec_dump(3, &sum);
    acts_free(&feat);
    acts_free(&fu);
    Acts out = conv1x1_acts(&sp->conv2, &sum);
    acts_free(&sum);
    return out;
}

/* cpu.rs:635-688 -- FFC: local = l2l(x_l) + g2l(x_g), global = l2g(x_l) +
 * ST(x_g), each BN + ReLU.  `gl` may be NULL (no global branch yet). */
static void run_ffc(Ffc *f, const Acts *local, const Acts *gl, Acts *out_l, int *has_l,
                    Acts *out_g, int *has_g)
{
    *has_l = *has_g = 0;
    if (f->out_local > 0) {
        Acts acc = {0, local->h, local->w, NULL};
        int have = 0;
        if (f->l2l.present) {
            acc = ffc_conv(f, &f->l2l, local);
            have = 1;
        }
        if (f->g2l.present) {
            Acts o = ffc_conv(f, &f->g2l, gl);
            if (!have) {
                acc = o;
                have = 1;
            } else {
                add_inplace(&acc, &o);
                acts_free(&o);
            }
        }
        bn_calibrate((Bn *)&f->bn_l, &acc);
        bn_apply(f->bn_l.scale, f->bn_l.shift, &acc);
        relu_inplace(&acc);
        *out_l = acc;
        *has_l = 1;
    }
    if (f->out_global > 0) {
        Acts acc = {0, local->h, local->w, NULL};
        int have = 0;
        if (f->l2g.present) {
            acc = ffc_conv(f, &f->l2g, local);
            have = 1;
        }
        if (f->has_spectral) {
            Acts o = spectral_forward(&f->sp, gl);
            if (!have) {
                acc = o;
                have = 1;
            } else {
                add_inplace(&acc, &o);
                acts_free(&o);
            }
        }
        bn_calibrate((Bn *)&f->bn_g, &acc);
        bn_apply(f->bn_g.scale, f->bn_g.shift, &acc);
        relu_inplace(&acc);
        *out_g = acc;
        *has_g = 1;
    }
}

/* Size in floats of the reference's LAMA_DUMP_STEP dump after `step`
 * (local planes then global planes, cpu.rs:536-546), for an h x w input. */
OR_EXPORT long or_step_numel(int step, int h, int w)
{
    long h8 = h / 8, w8 = w / 8;
    if (step == 0) return 4L * (h + 6) * (w + 6);
    if (step == 1) return 64L * h * w;
    if (step == 2) return 128L * (h / 2) * (w / 2);
    if (step == 3) return 256L * (h / 4) * (w / 4);
    if (step >= 4 && step <= 23) return 512L * h8 * w8;
    if (step == 24) return 256L * (h / 4) * (w / 4);
    if (step == 25) return 128L * (h / 2) * (w / 2);
    if (step == 26) return 64L * h * w;
    if (step == 27) return 64L * (h + 6) * (w + 6);
    if (step == 28) return 3L * h * w;
    return 0;
}

/* cpu.rs:485-558 -- the step walk.  `input` [4][h][w]; `out` [3][h][w].
 * steps[i] (if non-NULL) receives the dump of step i, as LAMA_DUMP_STEP
 * would write it.  Stride-2 stages need h, w multiples of 8. */
OR_EXPORT int or_net_forward(void *p, const float *input, int h, int w, float *out, float **steps)
{
    Net *net = (Net *)p;
    Acts local = acts_new(4, h, w);
    memcpy(local.data, input, sizeof(float) * 4 * h * w);
    Acts global = {0, 0, 0, NULL};
    int has_global = 0;
    for (int si = 0; si < net->n; ++si) {
        Step *st = &net->steps[si];
        switch (st->kind) {
        case ST_PAD: {
            Acts nl = reflect_pad_acts(&local, st->pad);
            acts_free(&local);
            local = nl;
            if (has_global) {
                Acts ng = reflect_pad_acts(&global, st->pad);
                acts_free(&global);
                global = ng;
            }
            break;
        }
        case ST_FFC: {
            Acts nl, ng;
            int hl, hg;
            run_ffc(&st->ffc, &local, has_global ? &global : NULL, &nl, &hl, &ng, &hg);
            acts_free(&local);
            if (hl) {
                local = nl;
            } else { /* cpu.rs:682-686: empty local of the output geometry */
                local = acts_new(0, hg ? ng.h : local.h, hg ? ng.w : local.w);
            }
            if (has_global) acts_free(&global);
            has_global = hg;
            if (hg) global = ng;
            break;
        }
        case ST_RES: {
            Acts l1, g1, l2, g2;
            int hl1, hg1, hl2, hg2;
            run_ffc(&st->ffc, &local, has_global ? &global : NULL, &l1, &hl1, &g1, &hg1);
            run_ffc(&st->ffc2, &l1, hg1 ? &g1 : NULL, &l2, &hl2, &g2, &hg2);
            acts_free(&l1);
            if (hg1) acts_free(&g1);
            add_inplace(&local, &l2); /* cpu.rs:512 */
            acts_free(&l2);
            if (has_global && hg2) {
                add_inplace(&global, &g2);
                acts_free(&g2);
            } else if (!has_global && hg2) {
                global = g2;
                has_global = 1;
            }
            break;
        }
        case ST_CONCAT: {
            if (has_global) {
                Acts cat = acts_new(local.c + global.c, local.h, local.w);
                size_t nl = (size_t)local.c * local.h * local.w;
                memcpy(cat.data, local.data, nl * sizeof(float));
                memcpy(cat.data + nl, global.data, (size_t)global.c * global.h * global.w * sizeof(float));
                acts_free(&local);
                acts_free(&global);
                has_global = 0;
                local = cat;
            }
            break;
        }
        case ST_UP: {
            Acts a = acts_new(st->convt.cout, local.h * 2, local.w * 2);
            or_conv_transpose(local.data, local.c, local.h, local.w, st->convt.w, st->convt.bias,
                              st->convt.cout, a.data);
            bn_calibrate(&st->up_bn, &a);
            bn_apply(st->up_bn.scale, st->up_bn.shift, &a);
            relu_inplace(&a);
            acts_free(&local);
            local = a;
            if (has_global) acts_free(&global);
            has_global = 0;
            break;
        }
        case ST_OUT: {
            int oh = local.h - st->out.kh + 1, ow = local.w - st->out.kw + 1;
            Acts o = acts_new(st->out.cout, oh, ow);
            or_conv2d(local.data, local.c, local.h, local.w, st->out.w, st->out.bias, st->out.cout,
                      st->out.kh, st->out.kw, 0, 1, 0, o.data);
            sigmoid_inplace(&o);
            acts_free(&local);
            local = o;
            break;
        }
        }
        if (steps && steps[si]) {
            size_t nl = (size_t)local.c * local.h * local.w;
            memcpy(steps[si], local.data, nl * sizeof(float));
            if (has_global)
                memcpy(steps[si] + nl, global.data,
                       (size_t)global.c * global.h * global.w * sizeof(float));
        }
    }
    memcpy(out, local.data, sizeof(float) * (size_t)local.c * local.h * local.w);
    acts_free(&local);
    if (has_global) acts_free(&global);
    return 0;
}

/* The SpectralTransform of FFC k (0..35: resblock k/2, its conv1 or conv2
 * FFC) alone over x [384][h][w] -> out [384][h][w] (Spectral::forward,
 * cpu.rs:239-265), with the stages of g_spec_dump when `stages` is non-NULL.
 * Returns nonzero for an index past the net's FFCs. */
OR_EXPORT int or_net_spectral(void *p, int k, const float *x, int h, int w, float *out, float *const *stages)
{
    Net *net = (Net *)p;
    int r = 0;
    for (int si = 0; si < net->n; ++si) {
        Step *st = &net->steps[si];
        if (st->kind != ST_RES) continue;
        if (r++ != k / 2) continue;
        Ffc *f = k % 2 ? &st->ffc2 : &st->ffc;
        if (!f->has_spectral) return 1;
        Acts xa = acts_new(f->sp.conv1.cin, h, w);
        memcpy(xa.data, x, sizeof(float) * (size_t)xa.c * h * w);
        g_spec_dump = stages;
        Acts o = spectral_forward(&f->sp, &xa);
        g_spec_dump = NULL;
        memcpy(out, o.data, sizeof(float) * (size_t)o.c * o.h * o.w);
        acts_free(&xa);
        acts_free(&o);
        return 0;
    }
    return 1;
}

/* ------------------------------------------------- input and composite */

/* main.rs:175-196 -- [4][h+pad_h][w+pad_w]: rgb/255*(1-m), m = mask/255 > 0,
 * bottom/right reflect padding.  rgb is HWC u8, mask HW u8. */
OR_EXPORT void or_build_input(const uint8_t *rgb, const uint8_t *mask, int h, int w, int pad_h,
                              int pad_w, float *out)
{
    int oh = h + pad_h, ow = w + pad_w;
    long plane = (long)oh * ow;
    for (int y = 0; y < oh; ++y) {
        size_t sy = or_reflect_index(y, (size_t)h);
        for (int x = 0; x < ow; ++x) {
            size_t sx = or_reflect_index(x, (size_t)w);
            float m = (float)mask[sy * w + sx] / 255.0f;
            m = m > 0.0f ? 1.0f : 0.0f;
            long o = (long)y * ow + x;
            for (int c = 0; c < 3; ++c) {
                float v = (float)rgb[(sy * w + sx) * 3 + c] / 255.0f;
                out[c * plane + o] = v * (1.0f - m);
            }
            out[3 * plane + o] = m;
        }
    }
}

/* main.rs:272-307 -- u8 composite: hole pixels take trunc(clamp(v,0,1)*255+0.5),
 * the rest copy the source bytes.  `net` is [3][h+pad_h][w+pad_w]. */
OR_EXPORT void or_composite(const uint8_t *rgb, const uint8_t *mask, int h, int w, int pad_h,
                            int pad_w, const float *net, uint8_t *out)
{
    int ow = w + pad_w;
    long plane = (long)(h + pad_h) * ow;
    for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x) {
            long pi = (long)y * ow + x;
            /* the padded mask at (y, x) with y < h, x < w is the mask itself */
            int hole = mask[(long)y * w + x] > 0;
            long o = ((long)y * w + x) * 3;
            if (!hole) {
                out[o] = rgb[o];
                out[o + 1] = rgb[o + 1];
                out[o + 2] = rgb[o + 2];
                continue;
            }
            for (int c = 0; c < 3; ++c) {
                float v = net[c * plane + pi];
                v = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
                v = v * 255.0f;
                out[o + c] = (uint8_t)(v + 0.5f);
            }
        }
}

OR_EXPORT int or_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------- calibrated-BN fixtures */

static Bn *net_bn(void *p, int i)
{
    Net *net = (Net *)p;
    int k = 0;
    for (int si = 0; si < net->n; ++si) {
        Step *st = &net->steps[si];
        Ffc *fs[2] = {NULL, NULL};
        if (st->kind == ST_FFC) fs[0] = &st->ffc;
        if (st->kind == ST_RES) {
            fs[0] = &st->ffc;
            fs[1] = &st->ffc2;
        }
        for (int j = 0; j < 2; ++j) {
            Ffc *f = fs[j];
            if (!f) continue;
            Bn *list[4] = {f->has_spectral ? &f->sp.bn1 : NULL, f->has_spectral ? &f->sp.fu_bn : NULL,
                           &f->bn_l, &f->bn_g};
            for (int q = 0; q < 4; ++q)
                if (list[q] && list[q]->present && k++ == i) return list[q];
        }
        if (st->kind == ST_UP && k++ == i) return &st->up_bn;
    }
    return NULL;
}

/* Runs one forward with every BN re-fitted to its input statistics. */
OR_EXPORT int or_net_calibrate(void *p, const float *input, int h, int w, float *out)
{
    g_calibrate = 1;
    int r = or_net_forward(p, input, h, w, out, NULL);
    g_calibrate = 0;
    return r;
}

/* BN i of the net (container order): its prefix and calibrated statistics.
 * Returns the channel count, or 0 past the end. */
OR_EXPORT int or_net_bn(void *p, int i, char *prefix, int prefix_len, float *mean, float *var)
{
    Bn *b = net_bn(p, i);
    if (!b) return 0;
    if (prefix) snprintf(prefix, prefix_len, "%s", b->prefix);
    if (mean && b->cal_mean) memcpy(mean, b->cal_mean, sizeof(float) * b->n);
    if (var && b->cal_var) memcpy(var, b->cal_var, sizeof(float) * b->n);
    return b->n;
}

/* Thread count of the OpenMP regions (tests check thread-count independence). */
OR_EXPORT void or_set_threads(int n)
{
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}
