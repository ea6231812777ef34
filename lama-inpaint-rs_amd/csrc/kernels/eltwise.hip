// Elementwise finish of the FFC local branch: the local GEMM runs as K
// ranges that write raw partial sums (l2l over the 128 local input channels,
// then g2l over the 384 global ones in four ranges of 96); this sums them in
// that order, then applies BN_l, ReLU and the
// residual (cpu.rs:650-653 and 508-512).  HBM-bound: reads the partials and
// the residual once, writes the output once.
#include <hip/hip_runtime.h>

#include "common.h"

extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_finalize(const FinalizeArgs *__restrict__ args)
{
    const FinalizeArgs &A = *args;
    const long n = (long)A.C * A.plane;
    const long i = ((long)blockIdx.x * LAMA_NT + threadIdx.x) * 4;
    if (i >= n) return;
    // every load of the four elements is issued before any arithmetic or store
    long idx[4];
    int ch[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        idx[e] = min(i + e, n - 1);
        ch[e] = (int)(idx[e] / A.plane);
    }
    float part[LAMA_FIN_PARTS][4], sc[4], sh[4], rs[4];
    const int np = A.nparts;
#pragma unroll
    for (int q = 0; q < LAMA_FIN_PARTS; ++q) {
        const LAMA_GLOBAL float *pq = gp(A.part[min(q, np - 1)]);
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
        for (int q = 0; q < LAMA_FIN_PARTS; ++q)
            if (q < np) v += part[q][e];
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
