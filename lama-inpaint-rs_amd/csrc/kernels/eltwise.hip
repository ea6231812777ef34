// Elementwise finish of the FFC local branch: the local GEMM runs as K
// ranges that write raw partial sums (l2l over the 128 local input channels,
// then g2l over the 384 global ones in four ranges of 96); this sums them in
// that order, then applies BN_l, ReLU and the
// residual (cpu.rs:650-653 and 508-512).  HBM-bound: reads the partials and
// the residual once, writes the output once.
#include <hip/hip_runtime.h>

#include "common.h"

// NP partials, a compile-time count: every load is issued before any
// arithmetic, and the partials are summed in order
template <int NP>
__device__ __forceinline__ void finalize_body(const FinalizeArgs &A)
{
    const long n = (long)A.C * A.plane;
    const long i = ((long)blockIdx.x * LAMA_NT + threadIdx.x) * 4;
    if (i >= n) return;
    long idx[4];
    int ch[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        idx[e] = min(i + e, n - 1);
        ch[e] = (int)(idx[e] / A.plane);
    }
    float part[NP][4], sc[4], sh[4], rs[4];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const LAMA_GLOBAL float *pq = gp(A.part[q]);
#pragma unroll
        for (int e = 0; e < 4; ++e) part[q][e] = pq[idx[e]];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        sc[e] = gp(A.scale)[ch[e]];
        sh[e] = gp(A.shift)[ch[e]];
    }
    if (A.res) {
#pragma unroll
        for (int e = 0; e < 4; ++e) rs[e] = gp(A.res)[idx[e]];
    }
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < NP; ++q) v += part[q][e];
        float x = fmaxf(v * sc[e] + sh[e], 0.f);
        if (A.res) x += rs[e];
        out[e] = x;
    }
    LAMA_GLOBAL float *o = gp(A.out);
    if (i + 4 <= n) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[i + e] = out[e];
    } else {
        for (int e = 0; e < (int)(n - i); ++e) o[i + e] = out[e];
    }
}

// The FFC local branch's finish over 5, 10 or 20 partials (K split 1, 2, 4),
// one kernel each so that each holds only its own partials in registers.
#define LAMA_FINALIZE(NAME, NP)                                                                                   \
    extern "C" __global__ void __launch_bounds__(LAMA_NT) NAME(const FinalizeArgs *__restrict__ args, LAMA_STAMP_PARAMS) \
    {                                                                                                            \
        LAMA_STAMP_SCOPE;                                                                                        \
        finalize_body<NP>(*args);                                                                                \
    }
LAMA_FINALIZE(lama_finalize, LAMA_FIN_PARTS)
LAMA_FINALIZE(lama_finalize10, 2 * LAMA_FIN_PARTS)
LAMA_FINALIZE(lama_finalize20, 4 * LAMA_FIN_PARTS)
#undef LAMA_FINALIZE

// build_input (main.rs:175-196) on the device: the 8-bit h x w image (HWC
// RGB) and mask to the network input [4][H][W], padded bottom/right by
// reflection (image.rs:159-169).  Per pixel: m = (mask > 0), channel c =
// (rgb_c / 255) * (1 - m) with a correctly rounded f32 division and a
// separately rounded product, as the reference computes it; plane 3 = m.
// One thread per output pixel: byte reads, four coalesced plane stores.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_build_input(const InputArgs *__restrict__ args, int h, int w, int,
                                                                unsigned long long *__restrict__ stamp)
{
    LAMA_STAMP_SCOPE;
    const InputArgs &A = *args;
    const long plane = (long)A.H * A.W;
    const long i = (long)blockIdx.x * LAMA_NT + threadIdx.x;
    if (i >= plane) return;
    const int y = (int)(i / A.W), x = (int)(i - (long)y * A.W);
    const long s = (long)lama_reflect_full(y, h) * w + lama_reflect_full(x, w);
    const float m = gp(A.mask)[s] > 0 ? 1.0f : 0.0f;
    const float keep = __fsub_rn(1.0f, m);
    LAMA_GLOBAL float *o = gp(A.out);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float v = __fdiv_rn((float)gp(A.rgb)[3 * s + c], 255.0f);
        o[c * plane + i] = __fmul_rn(v, keep);
    }
    o[3 * plane + i] = m;
}
