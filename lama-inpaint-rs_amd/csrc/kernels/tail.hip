// model.34 + model.35: 7x7 convolution 64 -> 3 over the ReflectionPad2d(3)
// plane, with bias, then sigmoid (cpu.rs:531-534, 384-388).
//
// With only three output channels an MFMA tile would be >90% padding, so this
// is VALU work: a block covers 8 rows x 64 columns, each thread two adjacent
// pixels x 3 channels (6 accumulators).  All 3 x Cin x 49 weights are staged
// in LDS once, as [ci][ky][co][8] (kx padded to 8), so the 21 weights of one
// kernel row are six wave-uniform 16-byte broadcast reads; per input channel
// the block stages the reflect-padded 14 x 70 patch, its global loads issued
// one channel ahead so they overlap the current channel's FMAs.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {
constexpr int TROWS = LAMA_TAIL_ROWS, TCOLS = LAMA_TAIL_COLS, PX = LAMA_TAIL_PX;
static_assert(TROWS * TCOLS / PX == LAMA_NT, "one thread per PX pixels of the tile");
constexpr int PR = TROWS + 6, PC = TCOLS + 6;

}  // namespace

// trunc(clamp(v, 0, 1) * 255 + 0.5) with the product and the sum each
// rounded on its own (main.rs:303-305).  This code object is built with
// -ffp-contract=fast, under which the backend fuses a multiply and an add into
// one FMA (one rounding: a different result for some v) whatever the source
// says; the empty asm statement hides the product from that combine.  NaN
// clamps to 0, as the reference's saturating cast of NaN gives 0.
__device__ __forceinline__ uint8_t composite_u8(float v)
{
    v = fminf(fmaxf(v, 0.f), 1.f);
    float p = v * 255.0f;
    __asm__ volatile("" : "+v"(p));
    return (uint8_t)(int)(p + 0.5f);
}

// U8 = false: the sigmoid plane only.  U8 = true: also the 8-bit composite of
// main.rs:272-307 over the h x w crop -- hole pixels (mask > 0) from the
// network, every other pixel copied from the source bytes.
template <bool U8>
__device__ __forceinline__ void tail_body(const TailArgs *__restrict__ args, int h, int w)
{
    constexpr int PE = PR * PC, PK = (PE + LAMA_NT - 1) / LAMA_NT;  // patch elements per thread
    __shared__ float patch[2][PE];
    constexpr int WROW = 3 * 8;  // one (ci, ky): 3 output channels x 8 (7 taps + pad)
    __shared__ __attribute__((aligned(16))) float wl[64 * 7 * WROW];
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

    // weights [3][Cin][7][7] -> LDS [Cin][7][3][8], eight loads in flight per round
    {
        const int nw = A.Cin * 7 * WROW, wstride = A.Cin * 49;
        const LAMA_GLOBAL float *w = gp(A.wt);
        fetch(0);
        for (int b = threadIdx.x; b < nw; b += 8 * LAMA_NT) {
            float wv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int i = min(b + k * LAMA_NT, nw - 1), row = i / WROW, r = i - row * WROW;
                const int co = r >> 3, kx = r & 7;  // row = ci * 7 + ky
                wv[k] = w[co * wstride + row * 7 + min(kx, 6)];
            }
            // lanes past the end rewrite the last entry; kx == 7 is padding (never read)
#pragma unroll
            for (int k = 0; k < 8; ++k) wl[min(b + k * LAMA_NT, nw - 1)] = wv[k];
        }
    }
    put(patch[0]);
    // one barrier per channel: channel ci+1's loads are in flight during
    // channel ci's FMAs and land in the other patch buffer afterwards
    for (int ci = 0; ci < A.Cin; ++ci) {
        if (ci + 1 < A.Cin) fetch(ci + 1);
        __syncthreads();
        const float *pp = patch[ci & 1] + tr * PC + tc;
#pragma unroll
        for (int ky = 0; ky < 7; ++ky) {
            float row[PX + 6];
#pragma unroll
            for (int q = 0; q < PX + 6; ++q) row[q] = pp[ky * PC + q];
            float wk[WROW];
            const float4 *w4 = reinterpret_cast<const float4 *>(wl + (ci * 7 + ky) * WROW);
#pragma unroll
            for (int q = 0; q < WROW / 4; ++q) {
                const float4 v = w4[q];
                wk[4 * q] = v.x;
                wk[4 * q + 1] = v.y;
                wk[4 * q + 2] = v.z;
                wk[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int kx = 0; kx < 7; ++kx) {
#pragma unroll
                for (int co = 0; co < 3; ++co) {
                    const float wv = wk[co * 8 + kx];
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
    float sg[3][PX];
#pragma unroll
    for (int co = 0; co < 3; ++co)
#pragma unroll
        for (int p = 0; p < PX; ++p) {
            const int ox = ox0 + tc + p;
            const float v = acc[co][p] + bias[co];
            sg[co][p] = 1.0f / (1.0f + expf(-v));
            if (ox < W) gp(A.out)[co * plane + (long)oy * W + ox] = sg[co][p];
        }
    if constexpr (U8) {
        if (oy >= h) return;
#pragma unroll
        for (int p = 0; p < PX; ++p) {
            const int ox = ox0 + tc + p;
            if (ox >= w) continue;
            const long q = (long)oy * w + ox;
            const bool hole = gp(A.mask)[q] > 0;
#pragma unroll
            for (int co = 0; co < 3; ++co)
                gp(A.out_u8)[3 * q + co] = hole ? composite_u8(sg[co][p]) : gp(A.rgb)[3 * q + co];
        }
    }
}

extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_tail(const TailArgs *__restrict__ args, LAMA_STAMP_PARAMS)
{
    LAMA_STAMP_SCOPE;
    tail_body<false>(args, 0, 0);
}

// The tail with the 8-bit composite of the h x w crop fused in.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_tail_u8(const TailArgs *__restrict__ args, int h, int w, int,
                                                            unsigned long long *__restrict__ stamp)
{
    LAMA_STAMP_SCOPE;
    tail_body<true>(args, h, w);
}
