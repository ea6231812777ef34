// model.34 + model.35: 7x7 convolution 64 -> 3 over the ReflectionPad2d(3)
// plane, with bias, then sigmoid (cpu.rs:531-534, 384-388).
//
// With only three output channels an MFMA tile would be >90% padding, so this
// is VALU work: a block covers 8 rows x 64 columns, each thread two adjacent
// pixels x 3 channels (6 accumulators).  All 3 x Cin x 49 weights are staged
// in LDS once (wave-uniform broadcast reads); per input channel the block
// stages the reflect-padded 14 x 70 patch, one channel ahead.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {
constexpr int TROWS = LAMA_TAIL_ROWS, TCOLS = LAMA_TAIL_COLS, PX = 2;
static_assert(TROWS * TCOLS / PX == LAMA_NT, "one thread per PX pixels of the tile");
constexpr int PR = TROWS + 6, PC = TCOLS + 6;

}  // namespace

extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_tail(const TailArgs *__restrict__ args)
{
    __shared__ float patch[2][PR * PC];
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

    const long plane = (long)H * W;
    auto stage = [&](int ci, float *dst) {
        const float *src = A.src + (long)ci * plane;
        for (int idx = threadIdx.x; idx < PR * PC; idx += LAMA_NT) {
            const int r = idx / PC, c = idx - r * PC;
            dst[idx] = gp(src)[(long)reflect1(oy0 - 3 + r, H) * W + reflect1(ox0 - 3 + c, W)];
        }
    };
    const int nw = 3 * A.Cin * 49;  // Cin <= 64
    for (int i = threadIdx.x; i < nw; i += LAMA_NT) wl[i] = gp(A.wt)[i];
    stage(0, patch[0]);
    for (int ci = 0; ci < A.Cin; ++ci) {
        __syncthreads();
        if (ci + 1 < A.Cin) stage(ci + 1, patch[(ci + 1) & 1]);
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
    }
    const int oy = oy0 + tr;
    if (oy >= H) return;
#pragma unroll
    for (int co = 0; co < 3; ++co)
#pragma unroll
        for (int p = 0; p < PX; ++p) {
            const int ox = ox0 + tc + p;
            if (ox < W) {
                const float v = acc[co][p] + gp(A.bias)[co];
                gp(A.out)[co * plane + (long)oy * W + ox] = 1.0f / (1.0f + expf(-v));
            }
        }
}
