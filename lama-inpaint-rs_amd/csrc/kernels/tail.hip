// model.34 + model.35: 7x7 convolution 64 -> 3 over the ReflectionPad2d(3)
// plane, with bias, then sigmoid (cpu.rs:531-534, 384-388).
//
// With only three output channels an MFMA tile would be >90% padding, so this
// is VALU work.  A block covers 8 rows x 64 columns with two halves of 128
// threads that split the input channels (half h takes channels h, h+2, ...);
// each thread computes four adjacent pixels x 3 channels (12 accumulators)
// and the halves' sums meet in LDS at the end.  All 3 x Cin x 49 weights are
// staged in LDS once, as [ci][ky][co][8] (kx padded to 8), so the 21 weights
// of one kernel row are six wave-uniform 16-byte broadcast reads; each half
// stages the reflect-padded 14 x 70 patch of its channel in rows of 72 floats,
// so a thread's ten inputs of a kernel row are two 16-byte and one 8-byte LDS
// reads.  Per 84 FMAs a thread issues 9 LDS reads (the kernel is bound by LDS
// instruction issue with fewer pixels per thread).  The patch loads are issued
// one channel step ahead so they overlap the current step's FMAs.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {
constexpr int TROWS = LAMA_TAIL_ROWS, TCOLS = LAMA_TAIL_COLS, PX = LAMA_TAIL_PX;
constexpr int HALF = LAMA_NT / 2;  // threads per channel half
static_assert(TROWS * TCOLS / PX == HALF, "one thread of each half per PX pixels of the tile");
static_assert(PX == 4 && TCOLS % 4 == 0, "rows read as 16-byte vectors");
constexpr int PR = TROWS + 6, PC = TCOLS + 6, PCS = TCOLS + 8;  // patch rows, columns, LDS row stride
constexpr int PE = PR * PC, PS = PR * PCS;                      // patch elements, LDS floats per patch
constexpr int PK = (PE + HALF - 1) / HALF;                      // patch elements per thread
static_assert(PS % 4 == 0 && PCS % 4 == 0, "16-byte aligned patch rows");
static_assert(3 * PX * HALF <= 4 * PS, "the halves' partial sums fit in the patch buffers");

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
    __shared__ __attribute__((aligned(16))) float patch[2][2][PS];  // [half][stage][row][PCS]
    constexpr int WROW = 3 * 8;  // one (ci, ky): 3 output channels x 8 (7 taps + pad)
    __shared__ __attribute__((aligned(16))) float wl[64 * 7 * WROW];
    const TailArgs &A = *args;
    const int H = A.H, W = A.W, Cin = A.Cin;
    const int tiles_x = (W + TCOLS - 1) / TCOLS;
    const int oy0 = (blockIdx.x / tiles_x) * TROWS, ox0 = (blockIdx.x % tiles_x) * TCOLS;
    const int half = threadIdx.x / HALF, t = threadIdx.x % HALF;  // half: wave-uniform
    const int tr = t / (TCOLS / PX), tc = (t % (TCOLS / PX)) * PX;
    float acc[3][PX];
#pragma unroll
    for (int co = 0; co < 3; ++co)
#pragma unroll
        for (int p = 0; p < PX; ++p) acc[co][p] = 0.f;

    // this thread's patch elements: the same reflect-mapped offsets in every
    // channel (below H * W, which the host bounds at 2^27), and their LDS slots
    const long plane = (long)H * W;
    int off[PK], slot[PK];
#pragma unroll
    for (int k = 0; k < PK; ++k) {
        const int idx = min(t + k * HALF, PE - 1);
        const int r = idx / PC, c = idx - r * PC;
        off[k] = reflect1(oy0 - 3 + r, H) * W + reflect1(ox0 - 3 + c, W);
        slot[k] = r * PCS + c;
    }
    const LAMA_GLOBAL float *src = gp(A.src);
    const int NS = (Cin + 1) / 2;  // channel steps; an odd count leaves half 1 idle in the last one
    float nxt[PK];
    auto fetch = [&](int s) {
        const LAMA_GLOBAL float *p = src + (long)min(2 * s + half, Cin - 1) * plane;
#pragma unroll
        for (int k = 0; k < PK; ++k) nxt[k] = p[off[k]];
    };
    auto put = [&](float *dst) {
#pragma unroll
        for (int k = 0; k < PK; ++k)
            if (t + k * HALF < PE) dst[slot[k]] = nxt[k];
    };

    // weights [3][Cin][7][7] -> LDS [Cin][7][3][8], eight loads in flight per round
    {
        const int nw = Cin * 7 * WROW, wstride = Cin * 49;
        const LAMA_GLOBAL float *wg = gp(A.wt);
        fetch(0);
        for (int b = threadIdx.x; b < nw; b += 8 * LAMA_NT) {
            float wv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int i = min(b + k * LAMA_NT, nw - 1), row = i / WROW, r = i - row * WROW;
                const int co = r >> 3, kx = r & 7;  // row = ci * 7 + ky
                wv[k] = wg[co * wstride + row * 7 + min(kx, 6)];
            }
            // lanes past the end rewrite the last entry; kx == 7 is padding (never read)
#pragma unroll
            for (int k = 0; k < 8; ++k) wl[min(b + k * LAMA_NT, nw - 1)] = wv[k];
        }
    }
    put(patch[half][0]);
    // one barrier per channel step: step s+1's loads are in flight during
    // step s's FMAs and land in the other patch buffer afterwards
    for (int s = 0; s < NS; ++s) {
        if (s + 1 < NS) fetch(s + 1);
        __syncthreads();
        const int ci = 2 * s + half;
        if (ci < Cin) {
            const float *pp = patch[half][s & 1] + tr * PCS + tc;
#pragma unroll
            for (int ky = 0; ky < 7; ++ky) {
                float row[PX + 6];
                const float4 r0 = *reinterpret_cast<const float4 *>(pp + ky * PCS);
                const float4 r1 = *reinterpret_cast<const float4 *>(pp + ky * PCS + 4);
                const float2 r2 = *reinterpret_cast<const float2 *>(pp + ky * PCS + 8);
                row[0] = r0.x;
                row[1] = r0.y;
                row[2] = r0.z;
                row[3] = r0.w;
                row[4] = r1.x;
                row[5] = r1.y;
                row[6] = r1.z;
                row[7] = r1.w;
                row[8] = r2.x;
                row[9] = r2.y;
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
        }
        if (s + 1 < NS) put(patch[half][(s + 1) & 1]);
    }
    // half 1's sums to half 0 through the (now free) patch buffers
    __syncthreads();
    float *red = &patch[0][0][0];
    if (half == 1) {
#pragma unroll
        for (int co = 0; co < 3; ++co)
#pragma unroll
            for (int p = 0; p < PX; ++p) red[(co * PX + p) * HALF + t] = acc[co][p];
    }
    __syncthreads();
    if (half == 1) return;  // no barrier follows
#pragma unroll
    for (int co = 0; co < 3; ++co)
#pragma unroll
        for (int p = 0; p < PX; ++p) acc[co][p] += red[(co * PX + p) * HALF + t];
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
