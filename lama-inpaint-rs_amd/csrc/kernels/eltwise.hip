// Elementwise finish of the FFC local branch: the local GEMM runs as K
// quarters that write raw partial sums (one per group of 128 input
// channels); this sums them in quarter order, then applies BN_l, ReLU and the
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
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    const int m = n - i < 4 ? (int)(n - i) : 4;
    if (m == 4) {  // [C][plane] is 16-byte aligned as a whole
        for (int q = 0; q < A.nparts; ++q) {
            const float4 u = *reinterpret_cast<const LAMA_GLOBAL float4 *>(gp(A.part[q]) + i);
            v[0] += u.x;
            v[1] += u.y;
            v[2] += u.z;
            v[3] += u.w;
        }
    } else {
        for (int q = 0; q < A.nparts; ++q)
            for (int e = 0; e < m; ++e) v[e] += gp(A.part[q])[i + e];
    }
    for (int e = 0; e < m; ++e) {
        const int c = (int)((i + e) / A.plane);
        float x = fmaxf(v[e] * gp(A.scale)[c] + gp(A.shift)[c], 0.f);
        if (A.res) x += gp(A.res)[i + e];
        gp(A.out)[i + e] = x;
    }
}
