// model.34 + model.35: 7x7 convolution 64 -> 3 over the ReflectionPad2d(3)
// plane, with bias, then sigmoid (cpu.rs:531-534, 384-388).
//
// With only three output channels an MFMA tile would be >90% padding, so this
// is VALU work: a block covers 8 rows x 64 columns, each thread two adjacent
// pixels x 3 channels (6 accumulators).  All 3 x Cin x 49 weights are staged
// in LDS once (wave-uniform broadcast reads); per input channel the block
// stages the reflect-padded 14 x 70 patch, its global loads issued one
// channel ahead so they overlap the current channel's FMAs.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {
constexpr int TROWS = LAMA_TAIL_ROWS, TCOLS = LAMA_TAIL_COLS, PX = 2;
static_assert(TROWS * TCOLS / PX == LAMA_NT, "one thread per PX pixels of the tile");
constexpr int PR = TROWS + 6, PC = TCOLS + 6;

}  // namespace

extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_tail(const TailArgs *__restrict__ args)
{
    constexpr int PE = PR * PC, PK = (PE + LAMA_NT - 1) / LAMA_NT;  // patch elements per thread
    __shared__ float patch[2][PE];
    __shared__ __attribute__((aligned(16))) float wl[3 * 64 * 49];
    const TailArgs &A = *args;
    const int H = A.H, W = A.W;
    const int tiles_x = (W + TCOLS - 1) / TCOLS;
    const int oy0 = (blockIdx.x / tiles_x) * TROWS, ox0 = (blockIdx.x % tiles_x) * TCOLS;
    const int tr = threadIdx.x / (TCOLS / PX), tc = (threadIdx.x % (TCOLS / PX)) * PX;
    float acc[3][PX];
#pragma unroll
    for (int co = 0; co < 3; ++co)
#pragma unroll
        for (int p = 0; p < PX; ++p) acc[co][p] = 0.f;

    // this thread's patch elements: the same reflect-mapped offsets in every channel
    const long plane = (long)H * W;
    long off[PK];
#pragma unroll
    for (int k = 0; k < PK; ++k) {
        const int idx = min((int)threadIdx.x + k * LAMA_NT, PE - 1);
        const int r = idx / PC, c = idx - r * PC;
        off[k] = (long)reflect1(oy0 - 3 + r, H) * W + reflect1(ox0 - 3 + c, W);
    }
    const LAMA_GLOBAL float *src = gp(A.src);
    float nxt[PK];
    auto fetch = [&](int ci) {
#pragma unroll
        for (int k = 0; k < PK; ++k) nxt[k] = src[(long)ci * plane + off[k]];
    };
    auto put = [&](float *dst) {
#pragma unroll
        for (int k = 0; k < PK; ++k)
            if ((int)threadIdx.x + k * LAMA_NT < PE) dst[threadIdx.x + k * LAMA_NT] = nxt[k];
    };

    // weights (3 x Cin x 49 <= 9408 floats), four float4 loads in flight per round
    {
        const int nw = 3 * A.Cin * 49, n4 = nw >> 2;
        const LAMA_GLOBAL float4 *w4 = reinterpret_cast<const LAMA_GLOBAL float4 *>(gp(A.wt));
        fetch(0);
        for (int b = threadIdx.x; b < n4; b += 4 * LAMA_NT) {
            float4 wv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[k] = w4[min(b + k * LAMA_NT, n4 - 1)];
            // lanes past the end rewrite the last float4 with the same value
#pragma unroll
            for (int k = 0; k < 4; ++k) reinterpret_cast<float4 *>(wl)[min(b + k * LAMA_NT, n4 - 1)] = wv[k];
        }
        for (int i = 4 * n4 + threadIdx.x; i < nw; i += LAMA_NT) wl[i] = gp(A.wt)[i];
    }
    put(patch[0]);
    // one barrier per channel: channel ci+1's loads are in flight during
    // channel ci's FMAs and land in the other patch buffer afterwards
    for (int ci = 0; ci < A.Cin; ++ci) {
        if (ci + 1 < A.Cin) fetch(ci + 1);
        __syncthreads();
        const float *pp = patch[ci & 1] + tr * PC + tc;
        const float *w0 = wl + ci * 49;
        const int wstride = A.Cin * 49;
#pragma unroll
        for (int ky = 0; ky < 7; ++ky) {
            float row[PX + 6];
#pragma unroll
            for (int q = 0; q < PX + 6; ++q) row[q] = pp[ky * PC + q];
#pragma unroll
            for (int kx = 0; kx < 7; ++kx) {
#pragma unroll
                for (int co = 0; co < 3; ++co) {
                    const float wv = w0[co * wstride + ky * 7 + kx];
#pragma unroll
                    for (int p = 0; p < PX; ++p) acc[co][p] += wv * row[p + kx];
                }
            }
        }
        if (ci + 1 < A.Cin) put(patch[(ci + 1) & 1]);
    }
    const int oy = oy0 + tr;
    if (oy >= H) return;
    float bias[3];
#pragma unroll
    for (int co = 0; co < 3; ++co) bias[co] = gp(A.bias)[co];
#pragma unroll
    for (int co = 0; co < 3; ++co)
#pragma unroll
        for (int p = 0; p < PX; ++p) {
            const int ox = ox0 + tc + p;
            if (ox < W) {
                const float v = acc[co][p] + bias[co];
                gp(A.out)[co * plane + (long)oy * W + ox] = 1.0f / (1.0f + expf(-v));
            }
        }
}
