// FourierUnit transforms: rfft2 / irfft2 with norm='ortho' over one channel
// plane per block, resident in LDS.
//
// rfft2 (cpu.rs:769-783): rows are real, so two rows ride in one complex
// transform (z = a + i b) and are split afterwards with the Hermitian
// identities; then the W/2+1 kept columns are transformed along y.  The
// result is scaled by 1/sqrt(HW) and written straight into the stacked
// layout the FourierUnit's 1x1 convolution reads: plane 2c = real part,
// plane 2c+1 = imaginary part, each [H][W/2+1].
//
// irfft2 (cpu.rs:801-837): the reference completes the full plane with
// F[(h-y)%h][w-x] = conj(X[y][x]) and keeps the real part of the 2-D inverse.
// Transforming the stored columns along y first makes every row of the
// result Hermitian, so the x pass is a complex-to-real transform that ignores
// the imaginary parts of the DC and Nyquist columns; two rows again share one
// complex transform.  The output is scaled and added to `feat` (f + FU(f)).
//
// 1-D transforms are Stockham auto-sort passes with radix 8, 4, 2, 3, 5 (or a
// direct DFT for other prime factors), ping-ponging between two LDS buffers.
// Twiddles come from a per-length table exp(-2 pi i k/n) built in f64 on the
// host.  The exponent sign per length follows the reference CPU engine: a
// power-of-two length uses the usual sign, any other length the opposite one
// (its Bluestein path computes the opposite-sign DFT); `sign_fwd` carries it.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"

namespace {

__device__ __forceinline__ float2 cmul(float2 a, float2 b)
{
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
// multiply by s*i (s = +-1)
__device__ __forceinline__ float2 mul_si(float2 a, int s)
{
    return s > 0 ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
}
// exp(sign * 2 pi i idx / n) from the table exp(-2 pi i k / n)
__device__ __forceinline__ float2 twd(const float2 *tw, int idx, int sign)
{
    float2 w = tw[idx];
    if (sign > 0) w.y = -w.y;
    return w;
}

// One value of a K-split producer's output plane (FftArgs: np partials
// pstride apart, in-order sum, BN, ReLU); np <= 1 reads the plain value.
struct KsIn {
    int np;
    long ps;
    float sc, sh;
};
__device__ __forceinline__ KsIn ks_in(int np, long ps, const float *scale, const float *shift, int ch)
{
    KsIn k{np, ps, 1.f, 0.f};
    if (np > 1) {
        k.sc = gp(scale)[ch];
        k.sh = gp(shift)[ch];
    }
    return k;
}
// (up to LAMA_PW_KSPLIT_MAX partials: every load is issued before the sum)
__device__ __forceinline__ float ks_ld(const LAMA_GLOBAL float *p, long i, const KsIn &k)
{
    if (k.np <= 1) return p[i];
    float u[LAMA_PW_KSPLIT_MAX];
    u[0] = p[i];
#pragma unroll
    for (int j = 1; j < LAMA_PW_KSPLIT_MAX; ++j) u[j] = j < k.np ? p[i + j * k.ps] : 0.f;
    float v = u[0];
#pragma unroll
    for (int j = 1; j < LAMA_PW_KSPLIT_MAX; ++j)
        if (j < k.np) v += u[j];
    return fmaxf(v * k.sc + k.sh, 0.f);
}
__device__ __forceinline__ float4 ks_ld4(const LAMA_GLOBAL float *p, long i, const KsIn &k)
{
    if (k.np <= 1) return *reinterpret_cast<const LAMA_GLOBAL float4 *>(p + i);
    float4 u[LAMA_PW_KSPLIT_MAX];
    u[0] = *reinterpret_cast<const LAMA_GLOBAL float4 *>(p + i);
#pragma unroll
    for (int j = 1; j < LAMA_PW_KSPLIT_MAX; ++j)
        u[j] = j < k.np ? float4(*reinterpret_cast<const LAMA_GLOBAL float4 *>(p + i + j * k.ps))
                        : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 v = u[0];
#pragma unroll
    for (int j = 1; j < LAMA_PW_KSPLIT_MAX; ++j)
        if (j < k.np) {
            v.x += u[j].x;
            v.y += u[j].y;
            v.z += u[j].z;
            v.w += u[j].w;
        }
    return make_float4(fmaxf(v.x * k.sc + k.sh, 0.f), fmaxf(v.y * k.sc + k.sh, 0.f), fmaxf(v.z * k.sc + k.sh, 0.f),
                       fmaxf(v.w * k.sc + k.sh, 0.f));
}

template <int R>
__device__ __forceinline__ void dft(float2 (&v)[R], int sign);

template <>
__device__ __forceinline__ void dft<2>(float2 (&v)[2], int)
{
    float2 a = v[0], b = v[1];
    v[0] = cadd(a, b);
    v[1] = csub(a, b);
}

template <>
__device__ __forceinline__ void dft<4>(float2 (&v)[4], int s)
{
    float2 t0 = cadd(v[0], v[2]), t1 = csub(v[0], v[2]);
    float2 t2 = cadd(v[1], v[3]), t3 = mul_si(csub(v[1], v[3]), s);
    v[0] = cadd(t0, t2);
    v[2] = csub(t0, t2);
    v[1] = cadd(t1, t3);
    v[3] = csub(t1, t3);
}

template <>
__device__ __forceinline__ void dft<3>(float2 (&v)[3], int s)
{
    const float s3 = s * 0.86602540378443864676f;
    float2 t1 = cadd(v[1], v[2]), t2 = csub(v[1], v[2]);
    float2 m = make_float2(v[0].x - 0.5f * t1.x, v[0].y - 0.5f * t1.y);
    float2 q = make_float2(-s3 * t2.y, s3 * t2.x);
    v[0] = cadd(v[0], t1);
    v[1] = cadd(m, q);
    v[2] = csub(m, q);
}

template <>
__device__ __forceinline__ void dft<5>(float2 (&v)[5], int s)
{
    const float c1 = 0.30901699437494742410f, c2 = -0.80901699437494742410f;
    const float s1 = s * 0.95105651629515357212f, s2 = s * 0.58778525229247312917f;
    float2 a1 = cadd(v[1], v[4]), b1 = csub(v[1], v[4]);
    float2 a2 = cadd(v[2], v[3]), b2 = csub(v[2], v[3]);
    float2 x0 = v[0];
    float2 m1 = make_float2(x0.x + c1 * a1.x + c2 * a2.x, x0.y + c1 * a1.y + c2 * a2.y);
    float2 m2 = make_float2(x0.x + c2 * a1.x + c1 * a2.x, x0.y + c2 * a1.y + c1 * a2.y);
    // i * (s1 b1 + s2 b2) and i * (s2 b1 - s1 b2)
    float2 n1 = make_float2(-(s1 * b1.y + s2 * b2.y), s1 * b1.x + s2 * b2.x);
    float2 n2 = make_float2(-(s2 * b1.y - s1 * b2.y), s2 * b1.x - s1 * b2.x);
    v[0] = make_float2(x0.x + a1.x + a2.x, x0.y + a1.y + a2.y);
    v[1] = cadd(m1, n1);
    v[4] = csub(m1, n1);
    v[2] = cadd(m2, n2);
    v[3] = csub(m2, n2);
}

// Radix 8 as two radix-4 DFTs (even and odd inputs) joined by the powers of
// w = exp(s 2 pi i / 8): X[q] = E[q%4] + w^q O[q%4], w^(q+4) = -w^q.
template <>
__device__ __forceinline__ void dft<8>(float2 (&v)[8], int s)
{
    const float h = 0.70710678118654752440f;
    float2 e[4] = {v[0], v[2], v[4], v[6]}, o[4] = {v[1], v[3], v[5], v[7]};
    dft<4>(e, s);
    dft<4>(o, s);
    const float2 o1 = make_float2(h * (o[1].x - s * o[1].y), h * (o[1].y + s * o[1].x));  // * (1 + s i)/sqrt 2
    const float2 o2 = mul_si(o[2], s);                                                    // * s i
    const float2 o3 = make_float2(h * (-o[3].x - s * o[3].y), h * (-o[3].y + s * o[3].x));  // * (-1 + s i)/sqrt 2
    v[0] = cadd(e[0], o[0]);
    v[4] = csub(e[0], o[0]);
    v[1] = cadd(e[1], o1);
    v[5] = csub(e[1], o1);
    v[2] = cadd(e[2], o2);
    v[6] = csub(e[2], o2);
    v[3] = cadd(e[3], o3);
    v[7] = csub(e[3], o3);
}

// Butterfly (b, j) of a radix-R Stockham pass over `count` transforms of
// length n; element e of transform b sits at b*bstride + e*estride.
struct Pass {
    const float2 *in;
    float2 *out;
    int n, Ns, count, bstride, estride, sign;
    const float2 *tw;
};

__device__ __forceinline__ void split_idx(const Pass &P, int m, int idx, int &b, int &j)
{
    // Columns (estride > 1): neighbouring threads take neighbouring
    // transforms so LDS rows are read across lanes.
    if (P.estride != 1) {
        b = idx % P.count;
        j = idx / P.count;
    } else {
        b = idx / m;
        j = idx - b * m;
    }
}

template <int R>
__device__ __forceinline__ void pass_fixed(const Pass &P)
{
    const int m = P.n / R, twstep = P.n / (P.Ns * R), total = P.count * m;
    for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
        int b, j;
        split_idx(P, m, idx, b, j);
        const int k = j % P.Ns;
        const float2 *src = P.in + (long)b * P.bstride;
        float2 v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float2 x = src[(j + r * m) * P.estride];
            if (r > 0 && k > 0) x = cmul(x, twd(P.tw, k * r * twstep, P.sign));
            v[r] = x;
        }
        dft<R>(v, P.sign);
        float2 *dst = P.out + (long)b * P.bstride;
        const int base = (j / P.Ns) * P.Ns * R + k;
        if (R % 2 == 0 && P.Ns == 1 && P.estride == 1 && (P.bstride & 1) == 0) {
            // first pass of a row transform: the R outputs are adjacent, so
            // store them as 16-byte pairs (fewer, wider LDS writes)
#pragma unroll
            for (int r = 0; r < R; r += 2)
                *reinterpret_cast<float4 *>(dst + base + r) = make_float4(v[r].x, v[r].y, v[r + 1].x, v[r + 1].y);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) dst[(base + r * P.Ns) * P.estride] = v[r];
        }
    }
}

// Any other radix: a direct DFT per butterfly.
__device__ __forceinline__ void pass_generic(const Pass &P, int R)
{
    const int m = P.n / R, twstep = P.n / (P.Ns * R), total = P.count * m, unit = P.n / R;
    for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
        int b, j;
        split_idx(P, m, idx, b, j);
        const int k = j % P.Ns;
        const float2 *src = P.in + (long)b * P.bstride;
        float2 *dst = P.out + (long)b * P.bstride;
        const int base = (j / P.Ns) * P.Ns * R + k;
        for (int q = 0; q < R; ++q) {
            float2 acc = make_float2(0.f, 0.f);
            for (int r = 0; r < R; ++r) {
                float2 x = src[(j + r * m) * P.estride];
                if (r > 0 && k > 0) x = cmul(x, twd(P.tw, k * r * twstep, P.sign));
                acc = cadd(acc, cmul(x, twd(P.tw, ((r * q) % R) * unit, P.sign)));
            }
            dst[(base + q * P.Ns) * P.estride] = acc;
        }
    }
}

// All passes of one length over a batch; returns the buffer with the result.
__device__ __forceinline__ float2 *stockham(const FftLen &L, const float2 *tw, float2 *a, float2 *b, int count, int bstride,
                           int estride, int sign)
{
    Pass P{a, b, L.n, 1, count, bstride, estride, sign, tw};
    for (int s = 0; s < L.nstages; ++s) {
        const int R = L.radix[s];
        switch (R) {
        case 2: pass_fixed<2>(P); break;
        case 3: pass_fixed<3>(P); break;
        case 4: pass_fixed<4>(P); break;
        case 5: pass_fixed<5>(P); break;
        case 8: pass_fixed<8>(P); break;
        default: pass_generic(P, R); break;
        }
        __syncthreads();
        P.Ns *= R;
        float2 *t = const_cast<float2 *>(P.in);
        P.in = P.out;
        P.out = t;
    }
    return const_cast<float2 *>(P.in);
}

// Both twiddle tables into LDS (row table first), ahead of the first pass:
// thread t fetches entry t of the concatenated tables with an unconditional
// (clamped) load, so the fetch can be issued together with the plane's.
struct TwFetch {
    float2 v;
    __device__ __forceinline__ void issue(const FftArgs &A, int t)
    {
        const int n = A.W + A.H, i = min(t, n - 1);
        const LAMA_GLOBAL float2 *p = i < A.W ? gp(reinterpret_cast<const float2 *>(A.row.tw)) + i
                                              : gp(reinterpret_cast<const float2 *>(A.col.tw)) + (i - A.W);
        v = *p;
    }
};

__device__ __forceinline__ void put_twiddles(const FftArgs &A, const TwFetch &f, float2 *twr, float2 *twc)
{
    const int n = A.W + A.H, t = threadIdx.x;
    if (t < n) (t < A.W ? twr[t] : twc[t - A.W]) = f.v;
    for (int i = t + blockDim.x; i < n; i += blockDim.x) {  // tables longer than the block (rare shapes)
        TwFetch g;
        g.issue(A, i);
        (i < A.W ? twr[i] : twc[i - A.W]) = g.v;
    }
}

}  // namespace

// One block per channel: real [C][H][W] -> stacked [2C][H][W/2+1], ortho.
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    const FftArgs &A = *args;
    const int c = blockIdx.x, H = A.H, W = A.W, Wh = A.Wh, HP = (H + 1) / 2;
    const int NB = lama_fft_nb(H, W);
    float2 *b0 = sm, *b1 = sm + NB, *twr = sm + 2 * NB, *twc = twr + W;
    // Prologue: every global load (the twiddle entry, this block's plane) is
    // issued before the first LDS write; the host keeps this kernel to planes
    // of at most LAMA_FFT_NT * 8 row-pair elements (two quads per thread).
    TwFetch tw;
    tw.issue(A, threadIdx.x);
    const LAMA_GLOBAL float *src = gp(A.in) + (long)c * A.rs;
    const KsIn kin = ks_in(A.in_np, A.in_pstride, A.in_scale, A.in_shift, c);
    const int NT = LAMA_FFT_NT;
    if ((W & 3) == 0 && (H & 1) == 0) {  // row pairs as float4 quads
        const int W4 = W >> 2, nq = HP * W4;
        constexpr int RQ = 2;
        float4 qa[RQ], qb[RQ];
#pragma unroll
        for (int k = 0; k < RQ; ++k) {
            const int q = min((int)threadIdx.x + k * NT, nq - 1), p = q / W4, x = (q - p * W4) * 4;
            qa[k] = ks_ld4(src, (2 * p) * W + x, kin);
            qb[k] = ks_ld4(src, (2 * p + 1) * W + x, kin);
        }
        put_twiddles(A, tw, twr, twc);
#pragma unroll
        for (int k = 0; k < RQ; ++k) {
            const int q = threadIdx.x + k * NT;
            if (q >= nq) break;
            const int p = q / W4, x = (q - p * W4) * 4;
            float2 *d = b0 + p * W + x;
            d[0] = make_float2(qa[k].x, qb[k].x);
            d[1] = make_float2(qa[k].y, qb[k].y);
            d[2] = make_float2(qa[k].z, qb[k].z);
            d[3] = make_float2(qa[k].w, qb[k].w);
        }
    } else {
        const int ne = HP * W;
        constexpr int RS = 8;
        float sa[RS], sb[RS];
#pragma unroll
        for (int k = 0; k < RS; ++k) {
            const int idx = min((int)threadIdx.x + k * NT, ne - 1), p = idx / W, x = idx - p * W;
            sa[k] = ks_ld(src, (2 * p) * W + x, kin);
            sb[k] = ks_ld(src, min(2 * p + 1, H - 1) * W + x, kin);
        }
        put_twiddles(A, tw, twr, twc);
#pragma unroll
        for (int k = 0; k < RS; ++k) {
            const int idx = threadIdx.x + k * NT;
            if (idx >= ne) break;
            const int p = idx / W;
            b0[idx] = make_float2(sa[k], 2 * p + 1 < H ? sb[k] : 0.f);
        }
    }
    __syncthreads();
    float2 *r = stockham(A.row, twr, b0, b1, HP, W, 1, A.row.sign_fwd);
    float2 *o = r == b0 ? b1 : b0;
    // split each row pair into the two half spectra
    for (int idx = threadIdx.x; idx < H * Wh; idx += blockDim.x) {
        const int y = idx / Wh, k = idx - y * Wh, p = y >> 1;
        const float2 z = r[p * W + k], zm = r[p * W + (W - k) % W];
        o[idx] = (y & 1) ? make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x))
                         : make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y));
    }
    __syncthreads();
    float2 *q = stockham(A.col, twc, o, r, Wh, 1, Wh, A.col.sign_fwd);
    LAMA_GLOBAL float *dre = gp(A.out) + (long)(2 * c) * A.ss, *dim = dre + A.ss;
    for (int idx = threadIdx.x; idx < H * Wh; idx += blockDim.x) {
        const float2 v = q[idx];
        dre[idx] = v.x * A.scale;
        dim[idx] = v.y * A.scale;
    }
}

// One block per channel: stacked [2C][H][W/2+1] -> real [C][H][W], ortho,
// plus feat: out = feat + irfft2(in).
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    const FftArgs &A = *args;
    const int c = blockIdx.x, H = A.H, W = A.W, Wh = A.Wh, HP = (H + 1) / 2;
    const int NB = lama_fft_nb(H, W);
    float2 *b0 = sm, *b1 = sm + NB, *twr = sm + 2 * NB, *twc = twr + W;
    // Prologue: the twiddle entry, this block's spectrum (at most
    // LAMA_FFT_NT * 8 values per plane, as the host guarantees) and the `f +`
    // addend of the output are all fetched before the first LDS write; the
    // addend's latency then hides behind the transforms.
    const int NT = LAMA_FFT_NT;
    TwFetch tw;
    tw.issue(A, threadIdx.x);
    const LAMA_GLOBAL float *sre = gp(A.in) + (long)(2 * c) * A.ss, *sim = sre + A.ss;
    const LAMA_GLOBAL float *f = gp(A.feat) + (long)c * A.rs;
    const KsIn kre = ks_in(A.in_np, A.in_pstride, A.in_scale, A.in_shift, 2 * c);
    const KsIn kim = ks_in(A.in_np, A.in_pstride, A.in_scale, A.in_shift, 2 * c + 1);
    const KsIn kf = ks_in(A.feat_np, A.feat_pstride, A.feat_scale, A.feat_shift, c);
    const bool vec = (W & 3) == 0;
    const int n4 = (H * W) >> 2, ns = H * Wh;
    constexpr int FP = 2, RS = 8;
    float4 fpre[FP];
    // unaligned planes (W % 4 != 0) fetch a harmless aligned dummy instead
    const LAMA_GLOBAL float *fv = vec ? f : gp(A.feat);
#pragma unroll
    for (int k = 0; k < FP; ++k) fpre[k] = ks_ld4(fv, 4L * (vec ? min((int)threadIdx.x + k * NT, max(n4 - 1, 0)) : 0), kf);
    float re[RS], im[RS];
#pragma unroll
    for (int k = 0; k < RS; ++k) {
        const int idx = min((int)threadIdx.x + k * NT, ns - 1);
        re[k] = ks_ld(sre, idx, kre);
        im[k] = ks_ld(sim, idx, kim);
    }
    put_twiddles(A, tw, twr, twc);
#pragma unroll
    for (int k = 0; k < RS; ++k) {
        const int idx = threadIdx.x + k * NT;
        if (idx >= ns) break;
        b0[idx] = make_float2(re[k], im[k]);
    }
    __syncthreads();
    float2 *r = stockham(A.col, twc, b0, b1, Wh, 1, Wh, -A.col.sign_fwd);
    float2 *o = r == b0 ? b1 : b0;
    // Hermitian rows, two per complex transform: z = Ga + i Gb
    for (int idx = threadIdx.x; idx < HP * W; idx += blockDim.x) {
        const int p = idx / W, x = idx - p * W;
        float2 g[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int y = 2 * p + h;
            float2 v = make_float2(0.f, 0.f);
            if (y < H) {
                if (x < Wh) {
                    v = r[y * Wh + x];
                    if (x == 0 || 2 * x == W) v.y = 0.f;
                } else {
                    v = r[y * Wh + (W - x)];
                    v.y = -v.y;
                }
            }
            g[h] = v;
        }
        o[idx] = make_float2(g[0].x - g[1].y, g[0].y + g[1].x);
    }
    __syncthreads();
    float2 *q = stockham(A.row, twr, o, r, HP, W, 1, -A.row.sign_fwd);
    LAMA_GLOBAL float *d = gp(A.out) + (long)c * A.rs;
    if (vec) {
        auto emit = [&](int i4, float4 fv) {
            const int idx = i4 * 4, y = idx / W, x = idx - y * W;
            const float2 *v = q + (y >> 1) * W + x;
            float4 o;
            if (y & 1)
                o = make_float4(v[0].y, v[1].y, v[2].y, v[3].y);
            else
                o = make_float4(v[0].x, v[1].x, v[2].x, v[3].x);
            o.x = o.x * A.scale + fv.x;
            o.y = o.y * A.scale + fv.y;
            o.z = o.z * A.scale + fv.z;
            o.w = o.w * A.scale + fv.w;
            *reinterpret_cast<LAMA_GLOBAL float4 *>(d + idx) = o;
        };
#pragma unroll
        for (int k = 0; k < FP; ++k) {
            const int i4 = threadIdx.x + k * blockDim.x;
            if (i4 < n4) emit(i4, fpre[k]);
        }
        for (int i4 = threadIdx.x + FP * blockDim.x; i4 < n4; i4 += blockDim.x) emit(i4, ks_ld4(f, 4L * i4, kf));
    } else {
        for (int idx = threadIdx.x; idx < H * W; idx += blockDim.x) {
            const int y = idx / W, x = idx - y * W;
            const float2 v = q[(y >> 1) * W + x];
            d[idx] = ((y & 1) ? v.y : v.x) * A.scale + ks_ld(f, idx, kf);
        }
    }
}

// ---- split mode: row and column transforms as separate launches ----------
//
// For bottleneck planes whose two ping-pong buffers do not fit one block's
// LDS (2048x2048 inputs give 256x256 planes), each 2-D transform becomes a
// row launch and a column launch.  A row block transforms `rows_per_block`
// row pairs of one channel, a column block `cols_per_block` adjacent columns
// of one channel over all H rows; the half spectrum between the two launches
// is interleaved complex [C][H][Wh] in A.tmp.  The butterflies, twiddles and
// pass order are those of the single-block kernels above.

namespace {

__device__ __forceinline__ void load_table(const float *tw, int n, float2 *dst)
{
    const LAMA_GLOBAL float2 *g = gp(reinterpret_cast<const float2 *>(tw));
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = g[i];
}

}  // namespace

// real [C][H][W] -> tmp: x transforms of row pairs, split into half spectra.
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2_rows(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    const FftArgs &A = *args;
    const int H = A.H, W = A.W, Wh = A.Wh, HP = (H + 1) / 2, PB = A.rows_per_block;
    const int nchunk = (HP + PB - 1) / PB, c = blockIdx.x / nchunk;
    const int p0 = (blockIdx.x - c * nchunk) * PB, np = min(PB, HP - p0);
    float2 *b0 = sm, *b1 = sm + PB * W, *twr = sm + 2 * PB * W;
    load_table(A.row.tw, W, twr);
    const LAMA_GLOBAL float *src = gp(A.in) + (long)c * A.rs + (long)(2 * p0) * W;
    const int rows = min(2 * np, H - 2 * p0);  // real rows present in this block
    for (int idx = threadIdx.x; idx < np * W; idx += blockDim.x) {
        const int p = idx / W, x = idx - p * W;
        const float a = src[(2 * p) * W + x];
        const float b = 2 * p + 1 < rows ? src[(2 * p + 1) * W + x] : 0.f;
        b0[idx] = make_float2(a, b);
    }
    __syncthreads();
    const float2 *r = stockham(A.row, twr, b0, b1, np, W, 1, A.row.sign_fwd);
    LAMA_GLOBAL float2 *t = gp(reinterpret_cast<float2 *>(A.tmp)) + (long)c * H * Wh + (long)(2 * p0) * Wh;
    for (int idx = threadIdx.x; idx < rows * Wh; idx += blockDim.x) {
        const int y = idx / Wh, k = idx - y * Wh, p = y >> 1;
        const float2 z = r[p * W + k], zm = r[p * W + (W - k) % W];
        t[idx] = (y & 1) ? make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x))
                         : make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y));
    }
}

// tmp -> stacked [2C][H][Wh]: y transforms of the kept columns, ortho scale.
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2_cols(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    const FftArgs &A = *args;
    const int H = A.H, Wh = A.Wh, CB = A.cols_per_block;
    const int nchunk = (Wh + CB - 1) / CB, c = blockIdx.x / nchunk;
    const int x0 = (blockIdx.x - c * nchunk) * CB, nc = min(CB, Wh - x0);
    float2 *b0 = sm, *b1 = sm + H * CB, *twc = sm + 2 * H * CB;
    load_table(A.col.tw, H, twc);
    const LAMA_GLOBAL float2 *t = gp(reinterpret_cast<const float2 *>(A.tmp)) + (long)c * H * Wh + x0;
    for (int idx = threadIdx.x; idx < H * nc; idx += blockDim.x) {
        const int y = idx / nc, j = idx - y * nc;
        b0[idx] = t[(long)y * Wh + j];
    }
    __syncthreads();
    const float2 *q = stockham(A.col, twc, b0, b1, nc, 1, nc, A.col.sign_fwd);
    LAMA_GLOBAL float *dre = gp(A.out) + (long)(2 * c) * A.ss + x0, *dim = dre + A.ss;
    for (int idx = threadIdx.x; idx < H * nc; idx += blockDim.x) {
        const int y = idx / nc, j = idx - y * nc;
        const float2 v = q[idx];
        dre[(long)y * Wh + j] = v.x * A.scale;
        dim[(long)y * Wh + j] = v.y * A.scale;
    }
}

// stacked [2C][H][Wh] -> tmp: inverse y transforms of the stored columns.
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2_cols(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    const FftArgs &A = *args;
    const int H = A.H, Wh = A.Wh, CB = A.cols_per_block;
    const int nchunk = (Wh + CB - 1) / CB, c = blockIdx.x / nchunk;
    const int x0 = (blockIdx.x - c * nchunk) * CB, nc = min(CB, Wh - x0);
    float2 *b0 = sm, *b1 = sm + H * CB, *twc = sm + 2 * H * CB;
    load_table(A.col.tw, H, twc);
    const LAMA_GLOBAL float *sre = gp(A.in) + (long)(2 * c) * A.ss + x0, *sim = sre + A.ss;
    for (int idx = threadIdx.x; idx < H * nc; idx += blockDim.x) {
        const int y = idx / nc, j = idx - y * nc;
        b0[idx] = make_float2(sre[(long)y * Wh + j], sim[(long)y * Wh + j]);
    }
    __syncthreads();
    const float2 *q = stockham(A.col, twc, b0, b1, nc, 1, nc, -A.col.sign_fwd);
    LAMA_GLOBAL float2 *t = gp(reinterpret_cast<float2 *>(A.tmp)) + (long)c * H * Wh + x0;
    for (int idx = threadIdx.x; idx < H * nc; idx += blockDim.x) {
        const int y = idx / nc, j = idx - y * nc;
        t[(long)y * Wh + j] = q[idx];
    }
}

// tmp -> real [C][H][W]: complex-to-real x transforms of row pairs, ortho
// scale, plus feat.
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2_rows(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    const FftArgs &A = *args;
    const int H = A.H, W = A.W, Wh = A.Wh, HP = (H + 1) / 2, PB = A.rows_per_block;
    const int nchunk = (HP + PB - 1) / PB, c = blockIdx.x / nchunk;
    const int p0 = (blockIdx.x - c * nchunk) * PB, np = min(PB, HP - p0);
    float2 *b0 = sm, *b1 = sm + PB * W, *twr = sm + 2 * PB * W;
    load_table(A.row.tw, W, twr);
    const int rows = min(2 * np, H - 2 * p0);
    const LAMA_GLOBAL float2 *t = gp(reinterpret_cast<const float2 *>(A.tmp)) + (long)c * H * Wh + (long)(2 * p0) * Wh;
    for (int idx = threadIdx.x; idx < np * W; idx += blockDim.x) {
        const int p = idx / W, x = idx - p * W;
        float2 g[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int y = 2 * p + h;
            float2 v = make_float2(0.f, 0.f);
            if (y < rows) {
                if (x < Wh) {
                    v = t[y * Wh + x];
                    if (x == 0 || 2 * x == W) v.y = 0.f;
                } else {
                    v = t[y * Wh + (W - x)];
                    v.y = -v.y;
                }
            }
            g[h] = v;
        }
        b0[idx] = make_float2(g[0].x - g[1].y, g[0].y + g[1].x);
    }
    __syncthreads();
    const float2 *q = stockham(A.row, twr, b0, b1, np, W, 1, -A.row.sign_fwd);
    const long base = (long)c * A.rs + (long)(2 * p0) * W;
    const LAMA_GLOBAL float *f = gp(A.feat) + base;
    LAMA_GLOBAL float *d = gp(A.out) + base;
    for (int idx = threadIdx.x; idx < rows * W; idx += blockDim.x) {
        const int y = idx / W, x = idx - y * W;
        const float2 v = q[(y >> 1) * W + x];
        d[idx] = ((y & 1) ? v.y : v.x) * A.scale + f[idx];
    }
}

// ---- compile-time shapes: square planes --------------------------------------
//
// The bottleneck planes of 256x256, 512x512 and 600x600 inputs (32x32, 64x64,
// 75x75) use the single-block algorithm above with every length, count and
// stride a compile-time constant, so no index arithmetic is left in the
// kernels but shifts, masks and multiplies-high by constants.  This matters
// beside the FFC GEMM: its FP32 MFMAs hold the SIMDs' math pipes, and every
// VALU instruction of these kernels then waits its turn, so the runtime
// integer divisions of the generic path (about half of its instructions)
// cost more than the butterflies themselves.  The radix plan is the host's
// (Engine::fft_len): 8s, then 4s, 2s, 3s and 5s (64 = 8*8, 32 = 8*4,
// 75 = 3*5*5).  The exponent sign follows the same per-length rule as the
// runtime-shaped kernels: -1 forward for powers of two, +1 otherwise.  Planes
// whose side is a multiple of 4 move rows as float4 quads; others (75) load
// and store the plane linearly, one float per lane.

namespace {

// the radix of the next pass, as Engine::fft_len orders them
constexpr int ct_radix(int rem)
{
    return rem % 8 == 0 ? 8 : rem % 4 == 0 ? 4 : rem % 2 == 0 ? 2 : rem % 3 == 0 ? 3 : rem % 5 == 0 ? 5 : 0;
}

// Shape constants of a compile-time N x N plane.
template <int N>
struct CtPlane {
    static constexpr int H = N, W = N, Wh = N / 2 + 1, HP = (N + 1) / 2, NB = lama_fft_nb(N, N), NT = LAMA_FFT_NT;
    static constexpr int SF = (N & (N - 1)) == 0 ? -1 : 1;  // forward exponent sign
    static constexpr bool VEC = N % 4 == 0;                  // rows as float4 quads
    static constexpr int NE = H * W, RL = (NE + NT - 1) / NT;  // linear plane floats per thread
};

// Butterfly idx of a radix-R pass: its R inputs, twiddled and transformed
// (ct_bfly_in), then stored (ct_bfly_out).  Rows: a transform's butterflies
// on neighbouring lanes; columns: neighbouring transforms on neighbouring
// lanes.
template <int N, int R, int NS, int COUNT, int BSTRIDE, int ESTRIDE, int SIGN>
struct CtBfly {
    static constexpr int M = N / R, TWSTEP = N / (NS * R), TOTAL = COUNT * M;
    static constexpr int IT = (TOTAL + LAMA_FFT_NT - 1) / LAMA_FFT_NT;  // butterflies per thread
    static __device__ __forceinline__ void in(int idx, const float2 *buf, const float2 *tw, float2 (&v)[R])
    {
        const int b = ESTRIDE == 1 ? idx / M : idx % COUNT;
        const int j = ESTRIDE == 1 ? idx % M : idx / COUNT;
        const int k = j % NS;
        const float2 *src = buf + b * BSTRIDE;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float2 x = src[(j + r * M) * ESTRIDE];
            if (NS > 1 && r > 0) x = cmul(x, twd(tw, k * r * TWSTEP, SIGN));
            v[r] = x;
        }
        dft<R>(v, SIGN);
    }
    static __device__ __forceinline__ void out(int idx, float2 *buf, const float2 (&v)[R])
    {
        const int b = ESTRIDE == 1 ? idx / M : idx % COUNT;
        const int j = ESTRIDE == 1 ? idx % M : idx / COUNT;
        const int k = j % NS;
        float2 *dst = buf + b * BSTRIDE;
        const int base = (j / NS) * NS * R + k;
        if constexpr (NS == 1 && ESTRIDE == 1 && R % 2 == 0 && BSTRIDE % 2 == 0) {
#pragma unroll
            for (int r = 0; r < R; r += 2)
                *reinterpret_cast<float4 *>(dst + base + r) = make_float4(v[r].x, v[r].y, v[r + 1].x, v[r + 1].y);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) dst[(base + r * NS) * ESTRIDE] = v[r];
        }
    }
};

template <int N, int R, int NS, int COUNT, int BSTRIDE, int ESTRIDE, int SIGN>
__device__ __forceinline__ void ct_pass(const float2 *in, float2 *out, const float2 *tw)
{
    using B = CtBfly<N, R, NS, COUNT, BSTRIDE, ESTRIDE, SIGN>;
#pragma unroll
    for (int it = 0; it < B::IT; ++it) {
        const int idx = threadIdx.x + it * LAMA_FFT_NT;
        if (B::TOTAL % LAMA_FFT_NT != 0 && idx >= B::TOTAL) break;
        float2 v[R];
        B::in(idx, in, tw, v);
        B::out(idx, out, v);
    }
}

// The pass in place: the thread's butterflies are all read and transformed
// before a barrier and stored after it, so one buffer serves as both.
template <int N, int R, int NS, int COUNT, int BSTRIDE, int ESTRIDE, int SIGN>
__device__ __forceinline__ void ct_pass_ip(float2 *buf, const float2 *tw)
{
    using B = CtBfly<N, R, NS, COUNT, BSTRIDE, ESTRIDE, SIGN>;
    float2 v[B::IT][R];
#pragma unroll
    for (int it = 0; it < B::IT; ++it) {
        const int idx = threadIdx.x + it * LAMA_FFT_NT;
        if (B::TOTAL % LAMA_FFT_NT != 0 && idx >= B::TOTAL) break;
        B::in(idx, buf, tw, v[it]);
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < B::IT; ++it) {
        const int idx = threadIdx.x + it * LAMA_FFT_NT;
        if (B::TOTAL % LAMA_FFT_NT != 0 && idx >= B::TOTAL) break;
        B::out(idx, buf, v[it]);
    }
}

// All passes of a length-N transform; returns the buffer holding the result
// (ping-ponging between a and b, or in a alone when IP).
template <int N, int NS, int COUNT, int BSTRIDE, int ESTRIDE, int SIGN, bool IP = false>
__device__ __forceinline__ float2 *ct_stockham(float2 *a, float2 *b, const float2 *tw)
{
    if constexpr (NS >= N) {
        return a;
    } else {
        constexpr int R = ct_radix(N / NS);
        static_assert(R != 0, "lengths of factors 2, 3 and 5 only");
        if constexpr (IP) {
            ct_pass_ip<N, R, NS, COUNT, BSTRIDE, ESTRIDE, SIGN>(a, tw);
            __syncthreads();
            return ct_stockham<N, NS * R, COUNT, BSTRIDE, ESTRIDE, SIGN, IP>(a, b, tw);
        } else {
            ct_pass<N, R, NS, COUNT, BSTRIDE, ESTRIDE, SIGN>(a, b, tw);
            __syncthreads();
            return ct_stockham<N, NS * R, COUNT, BSTRIDE, ESTRIDE, SIGN, IP>(b, a, tw);
        }
    }
}

template <int N>
__device__ __forceinline__ void ct_twiddles(const FftArgs &A, float2 *twr, float2 *twc, float2 &v)
{
    // both tables (row then column, N entries each): one entry per thread
    const int t = threadIdx.x;
    if (t < 2 * N) (t < N ? twr[t] : twc[t - N]) = v;
}

template <int N>
__device__ __forceinline__ float2 ct_twiddle_fetch(const FftArgs &A)
{
    const int t = min((int)threadIdx.x, 2 * N - 1);
    const LAMA_GLOBAL float2 *p = t < N ? gp(reinterpret_cast<const float2 *>(A.row.tw)) + t
                                        : gp(reinterpret_cast<const float2 *>(A.col.tw)) + (t - N);
    return *p;
}

// IP: one plane buffer instead of two (passes and reorderings in place
// through registers), for planes whose two buffers would keep a block from
// sharing a CU with two FFC GEMM workgroups
// ---- 64-point rows as wavefront-shuffle FFTs --------------------------------
//
// lama_rfft2_64s / lama_irfft2_64s (the plan takes them with LAMA_FFT64_SHFL=1;
// the default keeps the LDS passes, which measured faster beside the FFC GEMM:
// 286.5 against 285.0 passes/s at 512 x 512, while alone these are 7% and 13%
// faster -- the lane moves are VALU instructions, which wait behind the GEMM's
// MFMAs, where LDS accesses do not).  A row pair's 64-point transform runs in the
// registers of 16 lanes of one wave, four values per lane, with no LDS pass
// and no barrier: the index is split as x = 4 l + m (lane l, register m).
// Forward (natural input): a 16-point DIF transform across the 16 lanes for
// each m, radix 2, the partner value fetched with DPP lane moves (xor 1 and 2:
// quad_perm; xor 4: row_shl / row_shr 4 by bank; xor 8: row_ror 8), leaves
// lane l with Y_m[brev4(l)]; the twiddles W64^(m k1) and a radix-4 DFT over m
// in registers give X[brev4(l) + 16 k2] in register k2.  Inverse: lane l
// starts from x[brev4(l) + 16 m] and runs the same steps in the reverse order
// (radix 4, twiddles, 16-point DIT across the lanes), ending with the natural
// quad X[4 l .. 4 l + 3].  Twiddles come from the row table (exp(-2 pi i k/64),
// f64-built, read from global memory in the prologue); the exponent sign
// follows the plane's rule as in the LDS passes.

__device__ __forceinline__ int brev4(int l) { return ((l & 1) << 3) | ((l & 2) << 1) | ((l & 4) >> 1) | ((l & 8) >> 3); }

// the value of lane l ^ D of the same 16-lane row
template <int D>
__device__ __forceinline__ float row_xor(float v)
{
    const int x = __float_as_int(v);
    int r;
    if constexpr (D == 1)
        r = __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    else if constexpr (D == 2)
        r = __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    else if constexpr (D == 4) {
        r = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);  // row_shl 4 into banks 0, 2
        r = __builtin_amdgcn_update_dpp(r, x, 0x114, 0xF, 0xA, false);  // row_shr 4 into banks 1, 3
    } else {
        static_assert(D == 8, "lane distance 1, 2, 4 or 8");
        r = __builtin_amdgcn_update_dpp(x, x, 0x128, 0xF, 0xF, false);  // row_ror 8
    }
    return __int_as_float(r);
}
template <int D>
__device__ __forceinline__ float2 row_xor2(float2 v)
{
    return make_float2(row_xor<D>(v.x), row_xor<D>(v.y));
}

// A lane's twiddles of the 64-point row transform: W16^((l mod D) 8 / D) for
// the stages of half-span D = 8, 4, 2 (D = 1 needs none) and W64^(m k) for
// m = 1, 2, 3 (k = brev4(l)), read from the row table in global memory before
// the data arrive, so the transform waits on no barrier.
struct Tw64 {
    float2 s[3], m[3];
};
template <int SIGN>
__device__ __forceinline__ Tw64 tw64_load(const FftArgs &A, int l)
{
    const LAMA_GLOBAL float2 *g = gp(reinterpret_cast<const float2 *>(A.row.tw));
    const int k = brev4(l);
    const int e[6] = {4 * (l % 8), 8 * (l % 4), 16 * (l % 2), k, 2 * k, 3 * k};
    float2 v[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        v[i] = g[e[i]];
        if (SIGN > 0) v[i].y = -v[i].y;
    }
    return Tw64{{v[0], v[1], v[2]}, {v[3], v[4], v[5]}};
}

// one radix-2 DIF stage of half-span D across the lanes (z: the lane's four
// sequences; w: W16^((l mod D) 8 / D))
template <int D>
__device__ __forceinline__ void dif16_stage(float2 (&z)[4], int l, float2 w)
{
    const bool hi = (l & D) != 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float2 o = z[m], p = row_xor2<D>(o);
        z[m] = hi ? (D == 1 ? csub(p, o) : cmul(csub(p, o), w)) : cadd(o, p);
    }
}

// one radix-2 DIT stage of half-span D across the lanes
template <int D>
__device__ __forceinline__ void dit16_stage(float2 (&z)[4], int l, float2 w)
{
    const bool hi = (l & D) != 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float2 o = z[m], t = D == 1 ? o : cmul(o, w);
        const float2 r = row_xor2<D>(hi ? t : o);
        z[m] = hi ? csub(r, t) : cadd(o, r);
    }
}

// forward: z[m] = x[4 l + m] in, z[k2] = X[brev4(l) + 16 k2] out
template <int SIGN>
__device__ __forceinline__ void row64_fwd(float2 (&z)[4], int l, const Tw64 &w)
{
    dif16_stage<8>(z, l, w.s[0]);
    dif16_stage<4>(z, l, w.s[1]);
    dif16_stage<2>(z, l, w.s[2]);
    dif16_stage<1>(z, l, make_float2(1.f, 0.f));
#pragma unroll
    for (int m = 1; m < 4; ++m) z[m] = cmul(z[m], w.m[m - 1]);
    dft<4>(z, SIGN);
}

// inverse direction of the same split: z[m] = x[brev4(l) + 16 m] in, z[m] = X[4 l + m] out
template <int SIGN>
__device__ __forceinline__ void row64_inv(float2 (&z)[4], int l, const Tw64 &w)
{
    dft<4>(z, SIGN);
#pragma unroll
    for (int m = 1; m < 4; ++m) z[m] = cmul(z[m], w.m[m - 1]);
    dit16_stage<1>(z, l, make_float2(1.f, 0.f));
    dit16_stage<2>(z, l, w.s[2]);
    dit16_stage<4>(z, l, w.s[1]);
    dit16_stage<8>(z, l, w.s[0]);
}

template <int N, bool IP, bool SH = false>
__device__ __forceinline__ void rfft2_ct(const FftArgs &A, float2 *sm)
{
    using P = CtPlane<N>;
    constexpr int H = P::H, W = P::W, Wh = P::Wh, HP = P::HP, NB = P::NB, NT = P::NT, SF = P::SF;
    static_assert(2 * N <= NT, "one twiddle entry per thread");
    float2 *b0 = sm, *b1 = IP ? sm : sm + NB, *twr = sm + (IP ? 1 : 2) * NB, *twc = twr + W;
    const int c = blockIdx.x;
    // prologue: every global load before the first LDS write
    float2 tv = ct_twiddle_fetch<N>(A);
    Tw64 tw64{};
    if constexpr (SH) tw64 = tw64_load<SF>(A, threadIdx.x & 15);
    const LAMA_GLOBAL float *src = gp(A.in) + (long)c * A.rs;
    const KsIn kin = ks_in(A.in_np, A.in_pstride, A.in_scale, A.in_shift, c);
    if constexpr (P::VEC) {
        constexpr int W4 = W / 4, NQ = HP * W4, RQ = (NQ + NT - 1) / NT;
        static_assert(RQ <= 2, "at most two quads per thread");
        float4 qa[RQ], qb[RQ];
#pragma unroll
        for (int k = 0; k < RQ; ++k) {
            const int q = min((int)threadIdx.x + k * NT, NQ - 1), p = q / W4, x = (q % W4) * 4;
            qa[k] = ks_ld4(src, (2 * p) * W + x, kin);
            qb[k] = ks_ld4(src, (2 * p + 1) * W + x, kin);
        }
        ct_twiddles<N>(A, twr, twc, tv);
        if constexpr (SH) {
            // each thread's quad is lanes l = t mod 16 of row pair t / 16:
            // the row transform in registers, the spectrum row to LDS
            static_assert(RQ == 1 && W4 == 16, "one quad per thread, 16 lanes per row pair");
            const int t = threadIdx.x, p = t >> 4, l = t & 15;
            float2 z[4] = {make_float2(qa[0].x, qb[0].x), make_float2(qa[0].y, qb[0].y), make_float2(qa[0].z, qb[0].z),
                           make_float2(qa[0].w, qb[0].w)};
            row64_fwd<SF>(z, l, tw64);
            const int k1 = brev4(l);
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) b0[p * W + k1 + 16 * k2] = z[k2];
        } else {
#pragma unroll
            for (int k = 0; k < RQ; ++k) {
                const int q = threadIdx.x + k * NT;
                if (NQ % NT != 0 && q >= NQ) break;
                const int p = q / W4, x = (q % W4) * 4;
                float2 *d = b0 + p * W + x;
                d[0] = make_float2(qa[k].x, qb[k].x);
                d[1] = make_float2(qa[k].y, qb[k].y);
                d[2] = make_float2(qa[k].z, qb[k].z);
                d[3] = make_float2(qa[k].w, qb[k].w);
            }
        }
    } else {
        // the plane in memory order; value (y, x) goes to part y & 1 of row
        // pair y / 2, and an odd plane's last pair has a zero second row
        constexpr int NE = P::NE, RL = P::RL;
        static_assert(RL <= 12, "prologue register budget");
        float xs[RL];
#pragma unroll
        for (int k = 0; k < RL; ++k) xs[k] = ks_ld(src, min((int)threadIdx.x + k * NT, NE - 1), kin);
        ct_twiddles<N>(A, twr, twc, tv);
        float *bf = reinterpret_cast<float *>(b0);
#pragma unroll
        for (int k = 0; k < RL; ++k) {
            const int e = threadIdx.x + k * NT;
            if (NE % NT != 0 && e >= NE) break;
            const int y = e / W, x = e % W;
            bf[2 * ((y >> 1) * W + x) + (y & 1)] = xs[k];
        }
        if constexpr (H & 1)
            for (int x = threadIdx.x; x < W; x += NT) b0[(HP - 1) * W + x].y = 0.f;
    }
    __syncthreads();
    float2 *r;
    if constexpr (SH)
        r = b0;  // the rows are transformed already
    else
        r = ct_stockham<W, 1, HP, W, 1, SF, IP>(b0, b1, twr);
    float2 *o = r == b0 ? b1 : b0;
    // split each row pair into the two half spectra
    auto split = [&](int idx) {
        const int y = idx / Wh, k = idx % Wh, p = y >> 1;
        const float2 z = r[p * W + k], zm = r[p * W + (k == 0 ? 0 : W - k)];
        return (y & 1) ? make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x))
                       : make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y));
    };
    if constexpr (IP) {
        constexpr int IO = (H * Wh + NT - 1) / NT;
        float2 sv[IO];
#pragma unroll
        for (int it = 0; it < IO; ++it) {
            const int idx = threadIdx.x + it * NT;
            if ((H * Wh) % NT != 0 && idx >= H * Wh) break;
            sv[it] = split(idx);
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < IO; ++it) {
            const int idx = threadIdx.x + it * NT;
            if ((H * Wh) % NT != 0 && idx >= H * Wh) break;
            o[idx] = sv[it];
        }
    } else {
        for (int idx = threadIdx.x; idx < H * Wh; idx += NT) o[idx] = split(idx);
    }
    __syncthreads();
    float2 *q = ct_stockham<H, 1, Wh, 1, Wh, SF, IP>(o, r, twc);
    LAMA_GLOBAL float *dre = gp(A.out) + (long)(2 * c) * A.ss, *dim = dre + A.ss;
    for (int idx = threadIdx.x; idx < H * Wh; idx += NT) {
        const float2 v = q[idx];
        dre[idx] = v.x * A.scale;
        dim[idx] = v.y * A.scale;
    }
}

template <int N, bool IP, bool SH = false>
__device__ __forceinline__ void irfft2_ct(const FftArgs &A, float2 *sm)
{
    using P = CtPlane<N>;
    constexpr int H = P::H, W = P::W, Wh = P::Wh, HP = P::HP, NB = P::NB, NT = P::NT, SF = P::SF;
    constexpr int NS = H * Wh, RS = (NS + NT - 1) / NT;
    constexpr int FP = P::VEC ? (H * W / 4 + NT - 1) / NT : P::RL;  // addend float4s or floats per thread
    static_assert(2 * N <= NT && RS <= 8 && (P::VEC ? FP <= 2 : FP <= 12), "prologue register budget");
    float2 *b0 = sm, *b1 = IP ? sm : sm + NB, *twr = sm + (IP ? 1 : 2) * NB, *twc = twr + W;
    const int c = blockIdx.x;
    // prologue: twiddles, this block's spectrum and the `f +` addend
    float2 tv = ct_twiddle_fetch<N>(A);
    Tw64 tw64{};
    if constexpr (SH) tw64 = tw64_load<-SF>(A, threadIdx.x & 15);
    const LAMA_GLOBAL float *sre = gp(A.in) + (long)(2 * c) * A.ss, *sim = sre + A.ss;
    const LAMA_GLOBAL float *f = gp(A.feat) + (long)c * A.rs;
    const KsIn kre = ks_in(A.in_np, A.in_pstride, A.in_scale, A.in_shift, 2 * c);
    const KsIn kim = ks_in(A.in_np, A.in_pstride, A.in_scale, A.in_shift, 2 * c + 1);
    const KsIn kf = ks_in(A.feat_np, A.feat_pstride, A.feat_scale, A.feat_shift, c);
    using FT = typename std::conditional<P::VEC, float4, float>::type;
    FT fpre[FP];
    if constexpr (SH) {
        // the quads this thread stores: rows 2p, 2p + 1 of its row pair p at x = 4 l
        static_assert(FP == 2, "two quads per thread");
        const int t = threadIdx.x, p = t >> 4, l = t & 15;
#pragma unroll
        for (int k = 0; k < FP; ++k) fpre[k] = ks_ld4(f, (long)(2 * p + k) * W + 4 * l, kf);
    } else if constexpr (P::VEC) {
        constexpr int N4 = H * W / 4;
#pragma unroll
        for (int k = 0; k < FP; ++k) fpre[k] = ks_ld4(f, 4L * min((int)threadIdx.x + k * NT, N4 - 1), kf);
    } else {
#pragma unroll
        for (int k = 0; k < FP; ++k) fpre[k] = ks_ld(f, min((int)threadIdx.x + k * NT, P::NE - 1), kf);
    }
    float re[RS], im[RS];
#pragma unroll
    for (int k = 0; k < RS; ++k) {
        const int idx = min((int)threadIdx.x + k * NT, NS - 1);
        re[k] = ks_ld(sre, idx, kre);
        im[k] = ks_ld(sim, idx, kim);
    }
    ct_twiddles<N>(A, twr, twc, tv);
#pragma unroll
    for (int k = 0; k < RS; ++k) {
        const int idx = threadIdx.x + k * NT;
        if (NS % NT != 0 && idx >= NS) break;
        b0[idx] = make_float2(re[k], im[k]);
    }
    __syncthreads();
    float2 *r = ct_stockham<H, 1, Wh, 1, Wh, -SF, IP>(b0, b1, twc);
    float2 *o = r == b0 ? b1 : b0;
    // Hermitian rows, two per complex transform: z = Ga + i Gb (an odd
    // plane's last pair has no second row)
    auto herm = [&](int idx) {
        const int p = idx / W, x = idx % W;
        float2 g[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int y = 2 * p + h;
            float2 v = make_float2(0.f, 0.f);
            if (!(H & 1) || y < H) {
                if (x < Wh) {
                    v = r[y * Wh + x];
                    if (x == 0 || 2 * x == W) v.y = 0.f;
                } else {
                    v = r[y * Wh + (W - x)];
                    v.y = -v.y;
                }
            }
            g[h] = v;
        }
        return make_float2(g[0].x - g[1].y, g[0].y + g[1].x);
    };
    if constexpr (IP) {
        constexpr int IO = (HP * W + NT - 1) / NT;
        float2 hv[IO];
#pragma unroll
        for (int it = 0; it < IO; ++it) {
            const int idx = threadIdx.x + it * NT;
            if ((HP * W) % NT != 0 && idx >= HP * W) break;
            hv[it] = herm(idx);
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < IO; ++it) {
            const int idx = threadIdx.x + it * NT;
            if ((HP * W) % NT != 0 && idx >= HP * W) break;
            o[idx] = hv[it];
        }
    } else {
        for (int idx = threadIdx.x; idx < HP * W; idx += NT) o[idx] = herm(idx);
    }
    __syncthreads();
    if constexpr (SH) {
        // row pair p in lanes l = t mod 16: x[brev4(l) + 16 m] in, the quad X[4 l ..] out
        const int t = threadIdx.x, p = t >> 4, l = t & 15, x1 = brev4(l);
        float2 z[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) z[m] = o[p * W + x1 + 16 * m];
        row64_inv<-SF>(z, l, tw64);
        LAMA_GLOBAL float4 *d4 = reinterpret_cast<LAMA_GLOBAL float4 *>(gp(A.out) + (long)c * A.rs);
        const float4 re = make_float4(z[0].x * A.scale + fpre[0].x, z[1].x * A.scale + fpre[0].y,
                                      z[2].x * A.scale + fpre[0].z, z[3].x * A.scale + fpre[0].w);
        const float4 im = make_float4(z[0].y * A.scale + fpre[1].x, z[1].y * A.scale + fpre[1].y,
                                      z[2].y * A.scale + fpre[1].z, z[3].y * A.scale + fpre[1].w);
        d4[(2 * p) * (W / 4) + l] = re;
        d4[(2 * p + 1) * (W / 4) + l] = im;
        return;
    }
    float2 *q = ct_stockham<W, 1, HP, W, 1, -SF, IP>(o, r, twr);
    if constexpr (P::VEC) {
        constexpr int N4 = H * W / 4;
        LAMA_GLOBAL float4 *d4 = reinterpret_cast<LAMA_GLOBAL float4 *>(gp(A.out) + (long)c * A.rs);
#pragma unroll
        for (int k = 0; k < FP; ++k) {
            const int i4 = threadIdx.x + k * NT;
            if (N4 % NT != 0 && i4 >= N4) break;
            const int idx = i4 * 4, y = idx / W, x = idx % W;
            const float2 *v = q + (y >> 1) * W + x;
            float4 o4 = (y & 1) ? make_float4(v[0].y, v[1].y, v[2].y, v[3].y) : make_float4(v[0].x, v[1].x, v[2].x, v[3].x);
            o4.x = o4.x * A.scale + fpre[k].x;
            o4.y = o4.y * A.scale + fpre[k].y;
            o4.z = o4.z * A.scale + fpre[k].z;
            o4.w = o4.w * A.scale + fpre[k].w;
            d4[i4] = o4;
        }
    } else {
        LAMA_GLOBAL float *d = gp(A.out) + (long)c * A.rs;
        const float *qf = reinterpret_cast<const float *>(q);
#pragma unroll
        for (int k = 0; k < FP; ++k) {
            const int e = threadIdx.x + k * NT;
            if (P::NE % NT != 0 && e >= P::NE) break;
            const int y = e / W, x = e % W;
            d[e] = qf[2 * ((y >> 1) * W + x) + (y & 1)] * A.scale + fpre[k];
        }
    }
}

}  // namespace

// IP (in place) must match the host's LDS size for the kernel
// (Engine::fft_geom: kFftCtInPlace)
#define LAMA_FFT_CT(N, IP, SFX, SH)                                                                              \
    extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2_##N##SFX(const FftArgs *__restrict__ args,      \
                                                                                  LAMA_STAMP_PARAMS)                     \
    {                                                                                                           \
        side_priority();                                                                                        \
        LAMA_STAMP_SCOPE;                                                                                       \
        extern __shared__ float2 sm[];                                                                          \
        rfft2_ct<N, IP, SH>(*args, sm);                                                                         \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2_##N##SFX(const FftArgs *__restrict__ args,     \
                                                                                   LAMA_STAMP_PARAMS)                    \
    {                                                                                                           \
        side_priority();                                                                                        \
        LAMA_STAMP_SCOPE;                                                                                       \
        extern __shared__ float2 sm[];                                                                          \
        irfft2_ct<N, IP, SH>(*args, sm);                                                                        \
    }
LAMA_FFT_CT(64, false, , false)
LAMA_FFT_CT(32, false, , false)
LAMA_FFT_CT(75, LAMA_FFT75_IP, , false)
// the 64 x 64 transforms with wavefront-shuffle rows (LAMA_FFT64_SHFL=1 at plan time)
LAMA_FFT_CT(64, false, s, true)
#undef LAMA_FFT_CT

// ---- split mode with compile-time shapes: square power-of-two planes -------
//
// The 128x128 and 256x256 bottleneck planes (1024^2 and 2048^2 inputs) take
// the row/column split launches above, with the plane shape, the row pairs per
// row block and the columns per column block compiled in.  Both counts are
// LAMA_FFT_SPLIT_LDS / (16 N): the two ping-pong buffers fill that many
// bytes, as in the host's split geometry for these planes.  Each row block's 2*PB real rows are contiguous in memory and
// are read as float4s.  The W/2+1 kept columns are CB-wide column blocks
// plus one block holding the Nyquist column alone.  Butterflies, twiddles and
// pass order are those of the kernels above (sign -1 forward, +1 inverse).

namespace {

template <int N>
struct SplitCt {
    static constexpr int W = N, H = N, Wh = N / 2 + 1, HP = N / 2, NT = LAMA_FFT_NT;
    static constexpr int PB = LAMA_FFT_SPLIT_LDS / 8 / (2 * N), CB = PB;  // row pairs / columns per block
    static constexpr int RCH = HP / PB;                             // row blocks per channel
    static constexpr int CCH = (Wh + CB - 1) / CB;                  // column blocks per channel
    static_assert(HP % PB == 0 && Wh == (CCH - 1) * CB + 1, "whole row blocks; the last column block is Nyquist");
    static_assert(W <= NT && (PB * W / 4) % NT == 0 && (PB * W) % NT == 0, "whole per-thread shares");
};

// real [C][H][W] -> tmp: x transforms of PB row pairs of one channel
template <int N>
__device__ __forceinline__ void rfft2_rows_ct(const FftArgs &A, float2 *sm)
{
    using S = SplitCt<N>;
    constexpr int W = S::W, Wh = S::Wh, PB = S::PB, NT = S::NT, W4 = W / 4, RQ = PB * W4 / NT;
    float2 *b0 = sm, *b1 = sm + PB * W, *twr = sm + 2 * PB * W;
    const int c = blockIdx.x / S::RCH, p0 = (blockIdx.x % S::RCH) * PB;
    const float2 tv = gp(reinterpret_cast<const float2 *>(A.row.tw))[min((int)threadIdx.x, W - 1)];
    const LAMA_GLOBAL float4 *src =
        reinterpret_cast<const LAMA_GLOBAL float4 *>(gp(A.in) + (long)c * A.rs + (long)(2 * p0) * W);
    float4 qa[RQ], qb[RQ];
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
        const int q = threadIdx.x + k * NT, p = q / W4, x4 = q % W4;
        qa[k] = src[(2 * p) * W4 + x4];
        qb[k] = src[(2 * p + 1) * W4 + x4];
    }
    if (threadIdx.x < W) twr[threadIdx.x] = tv;
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
        const int q = threadIdx.x + k * NT, p = q / W4, x = (q % W4) * 4;
        float2 *d = b0 + p * W + x;
        d[0] = make_float2(qa[k].x, qb[k].x);
        d[1] = make_float2(qa[k].y, qb[k].y);
        d[2] = make_float2(qa[k].z, qb[k].z);
        d[3] = make_float2(qa[k].w, qb[k].w);
    }
    __syncthreads();
    const float2 *r = ct_stockham<W, 1, PB, W, 1, -1>(b0, b1, twr);
    LAMA_GLOBAL float2 *t = gp(reinterpret_cast<float2 *>(A.tmp)) + ((long)c * N + 2 * p0) * Wh;
    for (int idx = threadIdx.x; idx < 2 * PB * Wh; idx += NT) {
        const int y = idx / Wh, k = idx % Wh, p = y >> 1;
        const float2 z = r[p * W + k], zm = r[p * W + ((W - k) & (W - 1))];
        t[idx] = (y & 1) ? make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x))
                         : make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y));
    }
}

// tmp -> stacked [2C][H][Wh]: y transforms of NC columns x0.. of channel c
template <int N, int NC>
__device__ __forceinline__ void rfft2_cols_ct(const FftArgs &A, float2 *sm, int c, int x0)
{
    using S = SplitCt<N>;
    constexpr int H = S::H, Wh = S::Wh, CB = S::CB, NT = S::NT, L = (H * NC + NT - 1) / NT;
    float2 *b0 = sm, *b1 = sm + H * CB, *twc = sm + 2 * H * CB;
    const float2 tv = gp(reinterpret_cast<const float2 *>(A.col.tw))[min((int)threadIdx.x, H - 1)];
    const LAMA_GLOBAL float2 *t = gp(reinterpret_cast<const float2 *>(A.tmp)) + (long)c * H * Wh + x0;
    float2 v[L];
#pragma unroll
    for (int k = 0; k < L; ++k) {
        const int idx = min((int)threadIdx.x + k * NT, H * NC - 1), y = idx / NC, j = idx % NC;
        v[k] = t[y * Wh + j];
    }
    if (threadIdx.x < H) twc[threadIdx.x] = tv;
#pragma unroll
    for (int k = 0; k < L; ++k) {
        const int idx = threadIdx.x + k * NT;
        if ((H * NC) % NT != 0 && idx >= H * NC) break;
        b0[idx] = v[k];
    }
    __syncthreads();
    const float2 *q = ct_stockham<H, 1, NC, 1, NC, -1>(b0, b1, twc);
    LAMA_GLOBAL float *dre = gp(A.out) + (long)(2 * c) * A.ss + x0, *dim = dre + A.ss;
    for (int idx = threadIdx.x; idx < H * NC; idx += NT) {
        const int y = idx / NC, j = idx % NC;
        const float2 u = q[idx];
        dre[y * Wh + j] = u.x * A.scale;
        dim[y * Wh + j] = u.y * A.scale;
    }
}

// stacked [2C][H][Wh] -> tmp: inverse y transforms of NC columns x0.. of channel c
template <int N, int NC>
__device__ __forceinline__ void irfft2_cols_ct(const FftArgs &A, float2 *sm, int c, int x0)
{
    using S = SplitCt<N>;
    constexpr int H = S::H, Wh = S::Wh, CB = S::CB, NT = S::NT, L = (H * NC + NT - 1) / NT;
    float2 *b0 = sm, *b1 = sm + H * CB, *twc = sm + 2 * H * CB;
    const float2 tv = gp(reinterpret_cast<const float2 *>(A.col.tw))[min((int)threadIdx.x, H - 1)];
    const LAMA_GLOBAL float *sre = gp(A.in) + (long)(2 * c) * A.ss + x0, *sim = sre + A.ss;
    float2 v[L];
#pragma unroll
    for (int k = 0; k < L; ++k) {
        const int idx = min((int)threadIdx.x + k * NT, H * NC - 1), y = idx / NC, j = idx % NC;
        v[k] = make_float2(sre[y * Wh + j], sim[y * Wh + j]);
    }
    if (threadIdx.x < H) twc[threadIdx.x] = tv;
#pragma unroll
    for (int k = 0; k < L; ++k) {
        const int idx = threadIdx.x + k * NT;
        if ((H * NC) % NT != 0 && idx >= H * NC) break;
        b0[idx] = v[k];
    }
    __syncthreads();
    const float2 *q = ct_stockham<H, 1, NC, 1, NC, 1>(b0, b1, twc);
    LAMA_GLOBAL float2 *t = gp(reinterpret_cast<float2 *>(A.tmp)) + (long)c * H * Wh + x0;
    for (int idx = threadIdx.x; idx < H * NC; idx += NT) {
        const int y = idx / NC, j = idx % NC;
        t[y * Wh + j] = q[idx];
    }
}

// tmp -> real [C][H][W]: complex-to-real x transforms of PB row pairs of one
// channel, ortho scale, plus feat
template <int N>
__device__ __forceinline__ void irfft2_rows_ct(const FftArgs &A, float2 *sm)
{
    using S = SplitCt<N>;
    constexpr int W = S::W, Wh = S::Wh, PB = S::PB, NT = S::NT;
    constexpr int NF = 2 * PB * W / 4 / NT, NZ = PB * W / NT;  // feat float4s, row-pair values per thread
    float2 *b0 = sm, *b1 = sm + PB * W, *twr = sm + 2 * PB * W;
    const int c = blockIdx.x / S::RCH, p0 = (blockIdx.x % S::RCH) * PB;
    const float2 tv = gp(reinterpret_cast<const float2 *>(A.row.tw))[min((int)threadIdx.x, W - 1)];
    const long base = (long)c * A.rs + (long)(2 * p0) * W;
    const LAMA_GLOBAL float4 *f4 = reinterpret_cast<const LAMA_GLOBAL float4 *>(gp(A.feat) + base);
    float4 fpre[NF];
#pragma unroll
    for (int k = 0; k < NF; ++k) fpre[k] = f4[threadIdx.x + k * NT];
    // the Hermitian rows 2p and 2p+1, completed from the stored half spectra
    const LAMA_GLOBAL float2 *t = gp(reinterpret_cast<const float2 *>(A.tmp)) + ((long)c * N + 2 * p0) * Wh;
    float2 g[NZ][2];
#pragma unroll
    for (int k = 0; k < NZ; ++k) {
        const int idx = threadIdx.x + k * NT, p = idx / W, x = idx % W;
        const int col = x < Wh ? x : W - x;
#pragma unroll
        for (int h = 0; h < 2; ++h) g[k][h] = t[(2 * p + h) * Wh + col];
    }
    if (threadIdx.x < W) twr[threadIdx.x] = tv;
#pragma unroll
    for (int k = 0; k < NZ; ++k) {
        const int idx = threadIdx.x + k * NT, x = idx % W;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (x >= Wh) g[k][h].y = -g[k][h].y;
            else if (x == 0 || 2 * x == W) g[k][h].y = 0.f;
        }
        b0[idx] = make_float2(g[k][0].x - g[k][1].y, g[k][0].y + g[k][1].x);
    }
    __syncthreads();
    const float2 *q = ct_stockham<W, 1, PB, W, 1, 1>(b0, b1, twr);
    LAMA_GLOBAL float4 *d4 = reinterpret_cast<LAMA_GLOBAL float4 *>(gp(A.out) + base);
#pragma unroll
    for (int k = 0; k < NF; ++k) {
        const int i4 = threadIdx.x + k * NT, idx = i4 * 4, y = idx / W, x = idx % W;
        const float2 *v = q + (y >> 1) * W + x;
        float4 o4 = (y & 1) ? make_float4(v[0].y, v[1].y, v[2].y, v[3].y) : make_float4(v[0].x, v[1].x, v[2].x, v[3].x);
        o4.x = o4.x * A.scale + fpre[k].x;
        o4.y = o4.y * A.scale + fpre[k].y;
        o4.z = o4.z * A.scale + fpre[k].z;
        o4.w = o4.w * A.scale + fpre[k].w;
        d4[i4] = o4;
    }
}

// ---- column launches of the 256 x 256 planes: four-step transforms ------
//
// Each block takes LAMA_FFT_C4 = 16 adjacent columns of one channel (the
// Nyquist column 128 has a block of its own, through rfft2_cols_ct /
// irfft2_cols_ct with one column), 16 threads per column.  Thread (column
// cc, t) holds rows t + 16 j (j = 0..15) in registers and the 256-point
// transform runs as 256 = 16 x 16 (Gentleman-Sande four-step):
//   Y_t[k1] = sum_j x[t + 16 j] W16^(j k1)     (16-point DFT in registers)
//   Y_t[k1] *= W256^(t k1)                     (twiddles from the table)
//   X[k1 + 16 k2] = sum_t Y_t[k1] W16^(t k2)   (after one exchange through
//                                               LDS, in registers again)
// with W_n = exp(sign 2 pi i / n).  Thread (cc, k1) then holds rows
// k1 + 16 k2, the same pattern as it loaded.  A wave's loads are 4 rows x 16
// columns (128-byte runs of complex values) and its stores 4 rows x 64 bytes
// per real plane, against 64- and 32-byte runs with 8-column blocks; one
// exchange replaces three Stockham passes and their barriers.

constexpr int kC4 = LAMA_FFT_C4, kC4T = 16 * kC4;  // columns per block, threads per block
static_assert(kC4T <= LAMA_FFT_NT, "the block fits the FFT launch bound");
// the twiddles follow the exchange buffer (or the Nyquist block's two buffers)
constexpr int kC4Tw = 256 * kC4 > 2 * 256 * SplitCt<256>::CB ? 256 * kC4 : 2 * 256 * SplitCt<256>::CB;
static_assert(kC4T >= 256 && 128 % kC4 == 0, "one twiddle per thread; whole blocks below the Nyquist column");

// Block i of a launch of n blocks, renumbered so that the dispatcher's
// round-robin over the eight XCDs (block i to XCD i mod 8) hands each XCD a
// contiguous range: the column blocks of one channel then share an L2, which
// holds the 128-byte lines their row runs split between them.
__device__ __forceinline__ int fft_xcd_order(int i, int n)
{
    const int x = i & 7, q = n >> 3, r = n & 7;
    return x * q + min(x, r) + (i >> 3);
}

// 16-point DFT in registers (radix 4 x 4): v[n] -> sum_n v[n] exp(s 2 pi i n k / 16)
__device__ __forceinline__ void dft16(float2 (&v)[16], int s)
{
    // W16^m for m = b * c (b, c = 0..3): exp(s 2 pi i m / 16)
    constexpr float C1 = 0.92387953251128675613f, S1 = 0.38268343236508977173f, H = 0.70710678118654752440f;
    float2 u[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        float2 q[4] = {v[b], v[b + 4], v[b + 8], v[b + 12]};
        dft<4>(q, s);
#pragma unroll
        for (int c = 0; c < 4; ++c) u[b][c] = q[c];
    }
    // twiddles W16^(b c): (b, c) = (1,1) 1, (1,2) 2, (1,3) 3, (2,1) 2, (2,2) 4, (2,3) 6, (3,1) 3, (3,2) 6, (3,3) 9
    const float2 w1 = make_float2(C1, s * S1), w2 = make_float2(H, s * H), w3 = make_float2(S1, s * C1);
    const float2 w4 = make_float2(0.f, (float)s), w6 = make_float2(-H, s * H), w9 = make_float2(-C1, -s * S1);
    u[1][1] = cmul(u[1][1], w1);
    u[1][2] = cmul(u[1][2], w2);
    u[1][3] = cmul(u[1][3], w3);
    u[2][1] = cmul(u[2][1], w2);
    u[2][2] = cmul(u[2][2], w4);
    u[2][3] = cmul(u[2][3], w6);
    u[3][1] = cmul(u[3][1], w3);
    u[3][2] = cmul(u[3][2], w6);
    u[3][3] = cmul(u[3][3], w9);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float2 q[4] = {u[0][c], u[1][c], u[2][c], u[3][c]};
        dft<4>(q, s);
#pragma unroll
        for (int d = 0; d < 4; ++d) v[c + 4 * d] = q[d];
    }
}

// The four-step transform of this block's 16 columns (v: rows t + 16 j on
// entry, rows k1 + 16 k2 on return, (cc, t) = (tid % 16, tid / 16)).  `ex`
// holds 256 x kC4 complex values, `tw` the 256 twiddles exp(-2 pi i k / 256).
__device__ __forceinline__ void col256_four_step(float2 (&v)[16], float2 *ex, const float2 *tw, int sign)
{
    const int cc = threadIdx.x % kC4, t = threadIdx.x / kC4;
    dft16(v, sign);
#pragma unroll
    for (int k1 = 1; k1 < 16; ++k1) v[k1] = cmul(v[k1], twd(tw, t * k1, sign));
    // exchange: thread (cc, t) writes Y_t[k1] at [k1][t][cc]; thread (cc, k1) reads [k1][0..15][cc]
#pragma unroll
    for (int k1 = 0; k1 < 16; ++k1) ex[(k1 * 16 + t) * kC4 + cc] = v[k1];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = ex[(t * 16 + j) * kC4 + cc];
    dft16(v, sign);
}

// tmp -> stacked [2C][256][129]: forward column transforms, ortho scale
__device__ __forceinline__ void rfft2_cols_256_c4(const FftArgs &A, float2 *sm, int c, int x0)
{
    constexpr int H = 256, Wh = 129;
    float2 *ex = sm, *tw = sm + kC4Tw;
    const int cc = threadIdx.x % kC4, t = threadIdx.x / kC4;
    const float2 tv = gp(reinterpret_cast<const float2 *>(A.col.tw))[threadIdx.x % H];
    const LAMA_GLOBAL float2 *src = gp(reinterpret_cast<const float2 *>(A.tmp)) + (long)c * H * Wh + x0 + cc;
    float2 v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = src[(t + 16 * j) * Wh];
    if (threadIdx.x < H) tw[threadIdx.x] = tv;
    __syncthreads();
    col256_four_step(v, ex, tw, -1);
    LAMA_GLOBAL float *dre = gp(A.out) + (long)(2 * c) * A.ss + x0 + cc, *dim = dre + A.ss;
#pragma unroll
    for (int k2 = 0; k2 < 16; ++k2) {
        dre[(t + 16 * k2) * Wh] = v[k2].x * A.scale;
        dim[(t + 16 * k2) * Wh] = v[k2].y * A.scale;
    }
}

// stacked [2C][256][129] -> tmp: inverse column transforms
__device__ __forceinline__ void irfft2_cols_256_c4(const FftArgs &A, float2 *sm, int c, int x0)
{
    constexpr int H = 256, Wh = 129;
    float2 *ex = sm, *tw = sm + kC4Tw;
    const int cc = threadIdx.x % kC4, t = threadIdx.x / kC4;
    const float2 tv = gp(reinterpret_cast<const float2 *>(A.col.tw))[threadIdx.x % H];
    const LAMA_GLOBAL float *sre = gp(A.in) + (long)(2 * c) * A.ss + x0 + cc, *sim = sre + A.ss;
    float2 v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = make_float2(sre[(t + 16 * j) * Wh], sim[(t + 16 * j) * Wh]);
    if (threadIdx.x < H) tw[threadIdx.x] = tv;
    __syncthreads();
    col256_four_step(v, ex, tw, 1);
    LAMA_GLOBAL float2 *dst = gp(reinterpret_cast<float2 *>(A.tmp)) + (long)c * H * Wh + x0 + cc;
#pragma unroll
    for (int k2 = 0; k2 < 16; ++k2) dst[(t + 16 * k2) * Wh] = v[k2];
}

}  // namespace

#define LAMA_FFT_SPLIT_ROWS(N)                                                                                       \
    extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2_rows_##N(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)  \
    {                                                                                                                \
        side_priority();                                                                                             \
        LAMA_STAMP_SCOPE;                                                                                            \
        extern __shared__ float2 sm[];                                                                               \
        rfft2_rows_ct<N>(*args, sm);                                                                                 \
    }                                                                                                                \
    extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2_rows_##N(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS) \
    {                                                                                                                \
        side_priority();                                                                                             \
        LAMA_STAMP_SCOPE;                                                                                            \
        extern __shared__ float2 sm[];                                                                               \
        irfft2_rows_ct<N>(*args, sm);                                                                                \
    }
LAMA_FFT_SPLIT_ROWS(256)
LAMA_FFT_SPLIT_ROWS(128)
#undef LAMA_FFT_SPLIT_ROWS

// 128 x 128 planes: Stockham column blocks of SplitCt<128>::CB columns, in
// XCD-contiguous order
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2_cols_128(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    using S = SplitCt<128>;
    const int blk = fft_xcd_order(blockIdx.x, (int)gridDim.x), c = blk / S::CCH, ch = blk % S::CCH;
    if (ch < S::CCH - 1)
        rfft2_cols_ct<128, S::CB>(*args, sm, c, ch * S::CB);
    else
        rfft2_cols_ct<128, 1>(*args, sm, c, ch * S::CB);
}
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2_cols_128(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    using S = SplitCt<128>;
    const int blk = fft_xcd_order(blockIdx.x, (int)gridDim.x), c = blk / S::CCH, ch = blk % S::CCH;
    if (ch < S::CCH - 1)
        irfft2_cols_ct<128, S::CB>(*args, sm, c, ch * S::CB);
    else
        irfft2_cols_ct<128, 1>(*args, sm, c, ch * S::CB);
}

// 256 x 256 planes: 128 / kC4 four-step blocks and the Nyquist column per
// channel, kC4T threads per block (the host's launch shape, Engine::push_fft)
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_rfft2_cols_256(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    constexpr int NB = 128 / kC4 + 1;
    const int blk = fft_xcd_order(blockIdx.x, (int)gridDim.x), c = blk / NB, ch = blk % NB;
    if (ch < NB - 1)
        rfft2_cols_256_c4(*args, sm, c, ch * kC4);
    else
        rfft2_cols_ct<256, 1>(*args, sm, c, 128);
}
extern "C" __global__ void __launch_bounds__(LAMA_FFT_NT) lama_irfft2_cols_256(const FftArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    side_priority();
    LAMA_STAMP_SCOPE;
    extern __shared__ float2 sm[];
    constexpr int NB = 128 / kC4 + 1;
    const int blk = fft_xcd_order(blockIdx.x, (int)gridDim.x), c = blk / NB, ch = blk % NB;
    if (ch < NB - 1)
        irfft2_cols_256_c4(*args, sm, c, ch * kC4);
    else
        irfft2_cols_ct<256, 1>(*args, sm, c, 128);
}
