// Elementwise finish of the FFC local branch: the local GEMM runs as K
// ranges that write raw partial sums (l2l over the 128 local input channels,
// then g2l over the 384 global ones in four ranges of 96); this sums them in
// that order, then applies BN_l, ReLU and the
// residual (cpu.rs:650-653 and 508-512).  HBM-bound: reads the partials and
// the residual once, writes the output once.
#include <hip/hip_runtime.h>

#include "common.h"

// One block per (channel, G * 1024-element segment of its plane): the channel
// and its BN scale and shift are block-uniform (no per-element division).
// Each thread takes G groups of 4 consecutive elements, 1024 apart, with
// 16-byte accesses that need only 4-byte alignment (a plane need not be a
// multiple of 4).  A group that runs past the plane reads the plane's last 4
// elements instead (a clamped window, so every load is issued before any
// arithmetic, without branches) and stores only its own elements.  The NP
// partials are summed in order.
typedef float f4a4 __attribute__((ext_vector_type(4), aligned(4)));
template <int NP, int G>
__device__ __forceinline__ void finalize_body(const FinalizeArgs &A)
{
    constexpr int SEG = 4 * LAMA_NT * G;
    const int plane = (int)A.plane;
    const int segs = (plane + SEG - 1) / SEG;
    const int c = blockIdx.x / segs, j0 = (blockIdx.x - c * segs) * SEG + 4 * threadIdx.x;
    if (c >= A.C || j0 >= plane) return;
    const float sc = gp(A.scale)[c], sh = gp(A.shift)[c];
    const long cb = (long)c * plane;
    if (plane < 4) {  // planes of 1 to 3 pixels: one element at a time
        for (int j = j0; j < min(j0 + 4, plane); ++j) {
            float v = 0.f;
            for (int q = 0; q < NP; ++q) v += gp(A.part[q])[cb + j];
            float x = fmaxf(v * sc + sh, 0.f);
            if (A.res) x += gp(A.res)[cb + j];
            gp(A.out)[cb + j] = x;
        }
        return;
    }
    int jw[G];
    f4a4 part[G][NP], rs[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        jw[g] = min(j0 + 4 * LAMA_NT * g, plane - 4);
#pragma unroll
        for (int q = 0; q < NP; ++q) part[g][q] = *(const LAMA_GLOBAL f4a4 *)(gp(A.part[q]) + cb + jw[g]);
        if (A.res) rs[g] = *(const LAMA_GLOBAL f4a4 *)(gp(A.res) + cb + jw[g]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        f4a4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v = 0.f;
#pragma unroll
            for (int q = 0; q < NP; ++q) v += part[g][q][e];
            float x = fmaxf(v * sc + sh, 0.f);
            if (A.res) x += rs[g][e];
            out[e] = x;
        }
        const int j = j0 + 4 * LAMA_NT * g;
        LAMA_GLOBAL float *o = gp(A.out) + cb + jw[g];
        if (j + 4 <= plane) {
            *(LAMA_GLOBAL f4a4 *)o = out;
        } else if (j < plane) {  // the window's elements from j on
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (jw[g] + e >= j) o[e] = out[e];
        }
    }
}

// The FFC local branch's finish over 5, 10 or 20 partials (K split 1, 2, 4),
// one kernel each so that each holds only its own partials in registers; the
// _g2 kernels take two groups per thread (half the blocks).
#define LAMA_FINALIZE(NAME, NP, G)                                                                                \
    extern "C" __global__ void __launch_bounds__(LAMA_NT) NAME(const FinalizeArgs *__restrict__ args, LAMA_STAMP_PARAMS) \
    {                                                                                                            \
        LAMA_STAMP_SCOPE;                                                                                        \
        finalize_body<NP, G>(*args);                                                                             \
    }
LAMA_FINALIZE(lama_finalize, LAMA_FIN_PARTS, 1)
LAMA_FINALIZE(lama_finalize10, 2 * LAMA_FIN_PARTS, 1)
LAMA_FINALIZE(lama_finalize20, 4 * LAMA_FIN_PARTS, 1)
LAMA_FINALIZE(lama_finalize_g2, LAMA_FIN_PARTS, 2)
LAMA_FINALIZE(lama_finalize10_g2, 2 * LAMA_FIN_PARTS, 2)
LAMA_FINALIZE(lama_finalize20_g2, 4 * LAMA_FIN_PARTS, 2)
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
