// Shared definitions of the gfx950 kernels and the host engine: launch
// descriptors live in device memory (written once per input shape), so every
// kernel takes a pointer to a small table instead of a large by-value argument.
#pragma once
#include <stdint.h>

#define LAMA_NT 256      // threads per block (4 waves of 64)
#define LAMA_CUS 256     // compute units of an MI355X (grid sizing of tile-walking kernels)
// input channels per K chunk of the pointwise (1x1) convolutions; their
// weights are packed in chunks of this many
// Pointwise convolutions over float4-aligned planes whose 64 x 64 tiles would
// give at most two workgroups per CU: 1 = the K-half kernels
// (lama_conv1x1_kh, lama_conv1x1_res_kh: 64 x 32 tiles whose waves split each
// 2 * LAMA_PW_KC-channel chunk's K slots in halves), 0 = 64 x 64 tiles there
// too.  Larger planes and those with N % 4 != 0 keep 64 x 64.
#ifndef LAMA_PW_KH
#define LAMA_PW_KH 1
#endif
#ifndef LAMA_PW_KC
#define LAMA_PW_KC 16
#endif

#define LAMA_FFT_NT 512  // threads per FFT block (8 waves)
// pointwise convolutions: all M blocks of a pixel strip on one XCD
#ifndef LAMA_PW_XCD
#define LAMA_PW_XCD 1
#endif
// Bytes of the no-allocation entry point's device array: the activation arena
// and descriptors of one forward of up to 512 x 512 (177.2 MiB at 512 x 512).
#define LAMA_SCRATCH_BYTES (192u << 20)
// LDS bytes of the two ping-pong buffers of a split-mode FFT block (row pairs
// or columns per block = this / (2 * 8 * plane side)).  32 KB rather than 64:
// a block then fits on a CU beside the FFC GEMM's two workgroups (51 KB each),
// so the side stream's transforms are not held back by that GEMM's launches.
// F(4,3) input rows as 16-byte loads in the g2l launch as well as in the l2l +
// l2g one (where the plane width is a multiple of 4).  With 64 x 64 pointwise
// tiles this made the GEMM faster but the spectral chain beside it slower
// (512x512: 270.8-270.9 passes/s against 272.3-272.4 with A alone); with the
// K-half pointwise tiles it gains (279.8-279.9 against 277.8-278.1).
#ifndef LAMA_W4_VEC_B
#define LAMA_W4_VEC_B 1
#endif
// F(4,3) weights: two MFMA steps per 16-byte load (1) or one per 8-byte load (0)
#ifndef LAMA_W4_WX4
#define LAMA_W4_WX4 1
#endif
#ifndef LAMA_FFT_SPLIT_LDS
#define LAMA_FFT_SPLIT_LDS (32 * 1024)
#endif
// Columns per block of the 256 x 256 planes' column launches (16 threads per
// column, four-step transforms; the exchange buffer is 256 x this x 8 bytes,
// at most LAMA_FFT_SPLIT_LDS).
#ifndef LAMA_FFT_C4
#define LAMA_FFT_C4 16
#endif

// The 75 x 75 single-block transforms in one LDS buffer (1: passes in place
// through registers) or two (0: ping-pong, one barrier fewer per pass)
#ifndef LAMA_FFT75_IP
#define LAMA_FFT75_IP 1
#endif

// Complex values per ping-pong buffer of the single-block FFT kernels: the
// row-pair layout [(h+1)/2][w] or the half spectrum [h][w/2+1], rounded up to
// even so the second buffer is 16-byte aligned.  (Padding the rows against
// bank conflicts would cost LDS: at 512x512 a plane's 34 KB must stay within
// what two FFC GEMM workgroups leave free on a CU -- 37 KB measured slower.)
static inline constexpr int lama_fft_nb(int h, int w)
{
    const int a = (h + 1) / 2 * w, b = h * (w / 2 + 1);
    return ((a > b ? a : b) + 1) & ~1;
}
// Input channels per K chunk of the four transposed-convolution phases
// (py, px) = (0,0), (0,1), (1,0), (1,1), which have 1, 2, 2 and 4 taps.  The
// one-tap phase takes 16 channels per chunk (8 MFMAs per wave between
// barriers), the others 8.  Measured at 512x512 (ms per pass): 8/8/8/8 4.809,
// 16/8/8/8 4.796, 16/16/16/8 4.825, 32/16/16/8 4.831 (the larger chunks
// cost a workgroup of occupancy).  Their weights are packed in chunks of
// these sizes.
// Input channels per K chunk of the stride-2 convs (lama_conv3x3s2) and of
// the two row phases of the transposed convs (lama_convt_rows); the weights
// are packed in chunks of these sizes.  Stride-2 chunks of 4 channels take
// 124 registers and 42 KB of LDS (three workgroups per CU) against 176 and
// 76 KB at 8 (two): conv3x3s2 0.286-0.293 vs 0.296-0.302 ms per pass at
// 512x512, 0.400-0.411 vs 0.445 at 600x600.  The row phases measured best at
// 8 / 8 (0.276-0.281 ms per pass; 16 / 8: 0.281-0.288, 16 / 16: 0.296,
// 8 / 4: 0.306-0.311).
#ifndef LAMA_S2_KC
#define LAMA_S2_KC 4
#endif
#ifndef LAMA_CONVT_ROWS_KC0
#define LAMA_CONVT_ROWS_KC0 8
#endif
#ifndef LAMA_CONVT_ROWS_KC1
#define LAMA_CONVT_ROWS_KC1 8
#endif
#ifndef LAMA_CONVT_KC0
#define LAMA_CONVT_KC0 16
#define LAMA_CONVT_KC1 8
#define LAMA_CONVT_KC2 8
#define LAMA_CONVT_KC3 8
#endif
static inline constexpr int lama_convt_kc(int phase)
{
    return phase == 0 ? LAMA_CONVT_KC0 : phase == 3 ? LAMA_CONVT_KC3 : phase == 1 ? LAMA_CONVT_KC1 : LAMA_CONVT_KC2;
}
// Input channels per K chunk of the Winograd FFC kernel (lama_conv3x3w);
// its weights are packed in chunks of this many
#ifndef LAMA_WINO_KC
#define LAMA_WINO_KC 4
#endif
#ifndef LAMA_W42_KC
// input channels per K chunk of the F(2x4, 3x3) kernel, 4 or 8 (4: 170
// registers, 33.5 KB of LDS; 8: 222 and 58 KB, and 3% slower at 2048x2048)
#define LAMA_W42_KC 4
#endif
#ifndef LAMA_W42_CH
#define LAMA_W42_CH 64  // output channels per F(2x4, 3x3) workgroup: 32 (4 waves) or 64 (8 waves)
#endif

// output tile of the 7x7 tail kernel (rows x columns) and the adjacent
// pixels each thread of its two channel halves computes
#ifndef LAMA_TAIL_ROWS
#define LAMA_TAIL_ROWS 8
#endif
#ifndef LAMA_TAIL_COLS
#define LAMA_TAIL_COLS 64
#endif
#ifndef LAMA_TAIL_PX
#define LAMA_TAIL_PX 4
#endif

#ifdef __HIP_DEVICE_COMPILE__
// Wave priority of the SpectralTransform chain (conv1, rfft2, FU conv,
// irfft2, conv2).  It runs on its own stream beside the FFC 3x3 GEMMs and is
// the critical path of every FFC; when its workgroups share a CU with the
// GEMM's, a higher priority lets their instructions issue first.
#ifndef LAMA_SIDE_PRIO
#define LAMA_SIDE_PRIO 3
#endif
__device__ __forceinline__ void side_priority()
{
    if (LAMA_SIDE_PRIO > 0) __builtin_amdgcn_s_setprio(LAMA_SIDE_PRIO);
}

// Pointers read out of descriptors are generic; casting them to the global
// address space lets the compiler emit global_load/global_store instead of
// flat accesses (which also count against lgkmcnt and so serialise with LDS
// waits).
#define LAMA_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const LAMA_GLOBAL T *gp(const T *p)
{
    return (const LAMA_GLOBAL T *)p;
}
template <class T>
__device__ __forceinline__ LAMA_GLOBAL T *gp(T *p)
{
    return (LAMA_GLOBAL T *)p;
}

// Kernel-clock stamps (profiling): every kernel's fifth parameter is an
// array that, when non-null, receives each workgroup's start and end on the
// constant-rate device clock (s_memrealtime), stored by thread 0 at
// [2 * blockIdx.x] and [2 * blockIdx.x + 1] with ordinary vector stores.  The
// kernels with fewer leading parameters take unused ints in their place, so
// the engine passes one parameter layout to every kernel.
#define LAMA_STAMP_PARAMS int, int, int, unsigned long long *__restrict__ stamp
struct StampScope {
    unsigned long long *p, t0;
    __device__ __forceinline__ explicit StampScope(unsigned long long *p_)
        : p(p_), t0(p_ ? __builtin_amdgcn_s_memrealtime() : 0ull)
    {
    }
    __device__ __forceinline__ ~StampScope()
    {
        if (p && threadIdx.x == 0) {
            p[2 * blockIdx.x] = t0;
            p[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
        }
    }
};
#define LAMA_STAMP_SCOPE const StampScope stamp_scope_(stamp)

// PyTorch 'reflect' index for |overshoot| < n (one reflection), clamped into
// [0, n).  Exact for every input position a stored output reads (pad < n,
// or n == 1); positions read only by out-of-range tile pixels are clamped.
__device__ __forceinline__ int reflect1(int i, int n)
{
    i = i < 0 ? -i : (i >= n ? 2 * n - 2 - i : i);
    return min(max(i, 0), n - 1);
}
#endif

// One K segment of an implicit-GEMM convolution.  `src` is planar
// [C][IH][IW] with channel planes `cs` floats apart (cs >= IH * IW; the
// bottleneck planes are padded to a multiple of 4 floats so that every plane
// is 16-byte aligned); `wt` points at row 0 of the packed weights
// [M][nchunk][taps][KC] (KC input channels per chunk, zero-padded).
struct ConvSeg {
    const float *src;
    const float *wt;
    int C, IH, IW;
    int nchunk;
    int wrow;  // floats per packed weight row = nchunk * taps * KC
    int cs;    // floats between input channel planes
};

// The first workgroup of problems 1..3 of a grouped conv launch (INT32_MAX
// where absent), passed to the kernels as three scalar arguments that the
// dispatch preloads into SGPRs, so a workgroup finds its problem without
// reading the descriptors' block counts first (that chain of dependent scalar
// loads sat at the head of every workgroup's prologue).
#define LAMA_MAX_PROBS 4
struct alignas(16) ProbStarts {
    int n;                       // number of problems (1..LAMA_MAX_PROBS)
    int s[LAMA_MAX_PROBS - 1];   // first workgroup of problems 1, 2, ...
};

// One output problem: out[co][oy'][ox'] for co < M, (oy, ox) on the OH x OW
// GEMM grid, stored at oy' = oy*oy_mul + oy_off, ox' = ox*ox_mul + ox_off
// (the conv-transpose phases interleave four grids into one plane).
// Epilogue: v = acc (+bias) (+addends) -> *scale + shift -> ReLU -> (+res)
// -> store; `addend` and `res` are indexed like `out`.
struct ConvProblem {
    ConvSeg s0, s1;  // s1.nchunk == 0 when absent; s1 is always 1x1
    int M, OH, OW;
    int tiles_x, tiles_y, mblocks, nblocks;
    const float *bias, *addend, *scale, *shift;
    int relu;
    int vec_in;  // F(4,3) kernels: the input rows as 16-byte loads (plane width a multiple of 4)
    const float *res;
    float *out;
    long out_cstride;  // floats between output channel planes
    int outW;          // output row stride
    int oy_mul, oy_off, ox_mul, ox_off;
    // K split (the F(4,3) kernels): the problem's nblocks are ksplit slices
    // of mblocks * tiles_x * tiles_y blocks; slice ks covers input channels
    // [ks * kchunks * KC, +kchunks * KC) and stores its raw partial at
    // out + ks * out_kstride.  ksplit <= 1: no split.
    int ksplit, kchunks;
    long out_kstride;
    // the epilogue adds naddend planes, addend + i * addend_kstride
    int naddend;
    long addend_kstride;
};

// FFT length descriptor.  Twiddles tw[k] = exp(-2*pi*i*k/n) in f32 (computed
// in f64 on the host).  `sign_fwd` is the exponent sign the reference CPU
// engine effectively uses for its forward transform of this length: -1 for a
// power of two (radix-2 path), +1 otherwise (its Bluestein path computes the
// opposite-sign DFT).  The inverse uses -sign_fwd.
struct FftLen {
    int n;
    int nstages;
    int radix[16];
    int sign_fwd;
    int pad_;
    const float *tw;  // float2[n]
};

struct FftArgs {
    FftLen row, col;  // row: length W, col: length H
    int C, H, W, Wh;
    const float *in;    // rfft: real [C][H][W]; irfft: stacked [2C][H][Wh]
    float *out;         // rfft: stacked [2C][H][Wh]; irfft: real [C][H][W]
    const float *feat;  // irfft only: added to the output (f + ifft)
    float scale;        // 1/sqrt(H*W)
    // Split mode (planes too large for one block's LDS): the row and column
    // transforms are separate launches and the half spectrum between them is
    // interleaved complex [C][H][Wh] in `tmp`.  `rows_per_block` row pairs,
    // `cols_per_block` columns per block.
    int rows_per_block;
    float *tmp;
    int cols_per_block;
    // K-split producers (single-block kernels only): the transform's input
    // (rfft: the SpectralTransform conv1's output; irfft: the FourierUnit
    // conv's) and irfft's `feat` (conv1's output) arrive as `np` raw partial
    // sums `pstride` floats apart; a value is then the in-order sum of its
    // partials through BN and ReLU, max(sum * scale[ch] + shift[ch], 0), with
    // ch the plane's output channel of the producer.  np <= 1: plain values.
    int in_np;    // <= LAMA_PW_KSPLIT_MAX
    int feat_np;
    int pad_;
    long in_pstride, feat_pstride;
    const float *in_scale, *in_shift, *feat_scale, *feat_shift;
    // floats between the planes of the real side (rfft input, irfft output
    // and feat; >= H * W) and of the stacked spectrum (>= H * Wh)
    long rs, ss;
};

// Most K slices of the pointwise convolutions that feed a transform.
#define LAMA_PW_KSPLIT_MAX 4

// Sum of K-partials + BN + ReLU (+ residual) over [C][plane].
#ifndef LAMA_G2L_RANGES
#define LAMA_G2L_RANGES 4  // K ranges of the FFC g2l GEMM (384 input channels)
#endif
#define LAMA_FIN_PARTS (1 + LAMA_G2L_RANGES)  // K partials of the FFC local GEMM: l2l, then g2l's K ranges
#define LAMA_KSPLIT_MAX 4                      // the F(4,3) kernels' K split of the FFC GEMMs
#define LAMA_FIN_MAX (LAMA_FIN_PARTS * LAMA_KSPLIT_MAX)
struct FinalizeArgs {
    const float *part[LAMA_FIN_MAX];
    int nparts, C;
    long plane;
    const float *scale, *shift, *res;
    float *out;
};

// The 7x7 output convolution (64 -> 3, reflect pad 3, bias, sigmoid).  The
// composite variant (lama_tail_u8) also reads the unpadded source image and
// mask, h x w with h <= H, w <= W, and writes the 8-bit composite.
struct TailArgs {
    const float *src;  // [Cin][H][W]
    const float *wt;   // [3][Cin][7][7]
    const float *bias; // [3]
    float *out;        // [3][H][W]
    int Cin, H, W;
    int pad_;
    const uint8_t *rgb;   // lama_tail_u8: source pixels, HWC [h][w][3]
    const uint8_t *mask;  // lama_tail_u8: [h][w], hole where > 0
    uint8_t *out_u8;      // lama_tail_u8: composite, HWC [h][w][3]
};

// One FFC 3x3 weight matrix W[M][C][3][3] to pack into a Winograd kernel's
// layout on the device (lama_pack_wino): input channels ci < C0 come from
// src0 [M][C0][9], the rest from src1 [M][C - C0][9] (the FFC's local GEMM
// concatenates l2l and g2l along K).  kind 4: the F(4,3) layout of
// lama_conv3x3w4*; kind 42: the F(2x4, 3x3) layout of lama_conv3x3w42.
// dst is pre-zeroed (rows past M, channels past C stay zero).
struct WinoPackJob {
    const float *src0, *src1;
    float *dst;
    int M, C, C0, nchunk, kind;
    int pad_;
};

// Device build_input: the 8-bit image and mask (h x w, HWC RGB) to the
// network input [4][H][W], H >= h, W >= w, reflect-padded bottom/right.
struct InputArgs {
    const uint8_t *rgb;
    const uint8_t *mask;
    float *out;
    int H, W;
};

// PyTorch 'reflect' index for any i >= 0 (image.rs reflect_index: period
// 2(n-1), the edge sample not repeated; n == 1 maps everything to 0).
static inline
#ifdef __HIP_DEVICE_COMPILE__
    __device__
#endif
    int lama_reflect_full(int i, int n)
{
    if (n == 1) return 0;
    const int period = 2 * (n - 1);
    int m = i % period;
    if (m < 0) m += period;
    return m >= n ? period - m : m;
}
