// Implicit-GEMM convolutions on FP32 MFMA (v_mfma_f32_32x32x2_f32).
//
// GEMM view: C[co][p] = sum_k W[co][k] * X[k][p], k = (ci, tap), p = output
// pixel.  A block computes a 64 (co) x 64 (pixel) tile with 4 waves; wave
// (wm, wn) owns the 32 x 32 sub-tile co in [wm*32, +32), tile pixels
// [wn*32, +32).  The pixel tile is a TR x TC rectangle of the output grid.
//
// K is walked in chunks of KC input channels.  Per chunk the block stages, in
// LDS: the packed weights [64 co][taps][KC] (rows padded to a stride = 4 mod
// 8 floats, so the 16-byte reads of 16 lanes fall on distinct banks) and the
// input patch [KC][PR][PC] that covers the tile's receptive field, gathered
// with PyTorch 'reflect' index mapping (or zero fill for the transposed
// convolution phases).  im2col is never materialised.  The next chunk's
// global loads are issued into registers before the MFMAs of the current one.
//
// MFMA operand mapping (32x32x2, one block): lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; the two K slots of every MFMA are given to the two lane
// halves as channels ci = g*KC/2 + c (g = lane/32) of the same tap, so each
// lane reads its KC/2 weights for a tap with one vector LDS read.  D[i][j]
// lands in lane j + 32*((i/4)%2), register (i/8)*4 + i%4.
#include <hip/hip_runtime.h>

#include "common.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

template <int KH_, int KW_, int S_, bool REFLECT_, int KC_, int TR_, int TC_>
struct Cfg {
    static constexpr int KH = KH_, KW = KW_, S = S_, KC = KC_, TR = TR_, TC = TC_;
    static constexpr bool REFLECT = REFLECT_;
    static constexpr int T = KH * KW;
    static constexpr int PAD = REFLECT ? (KH - 1) / 2 : 0;
    static constexpr int PR = (TR - 1) * S + KH;
    static constexpr int PC = (TC - 1) * S + KW;
    static constexpr int WK = T * KC;
    static constexpr int WSTR = WK + ((12 - WK % 8) % 8);  // = 4 (mod 8)
    static constexpr int W_LDS = 64 * WSTR;
    static constexpr int P_LDS = KC * PR * PC;
    static constexpr int W4 = 64 * WK / 4;
    static constexpr int WITER = (W4 + LAMA_NT - 1) / LAMA_NT;
    static constexpr int PITER = (P_LDS + LAMA_NT - 1) / LAMA_NT;
    static constexpr int LDS = W_LDS + P_LDS;
    static_assert(TR * TC == 64, "pixel tile must hold 64 pixels");
    static_assert(WK % 4 == 0, "weight chunk must be float4 aligned");
    static_assert(KC % 4 == 0 || KC == 4, "KC must be a multiple of 4");
};

constexpr int cmax(int a, int b) { return a > b ? a : b; }

// Registers holding one chunk on its way from global memory to LDS.
template <class C>
struct Stage {
    float4 w[C::WITER];
    float p[C::PITER];
};

// Issue the global loads of chunk `ck` of segment `sg`.
template <class C>
__device__ __forceinline__ void load_chunk(Stage<C> &st, const ConvSeg &sg, int ck, int m0, int M,
                                           int oy0, int ox0)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (idx < C::W4) {
            const int row = idx / (C::WK / 4), c4 = idx % (C::WK / 4);
            const int co = m0 + row;
            if (co < M)
                v = *reinterpret_cast<const LAMA_GLOBAL float4 *>(gp(sg.wt) + (long)co * sg.wrow + (long)ck * C::WK + c4 * 4);
        }
        st.w[it] = v;
    }
    const long plane = (long)sg.IH * sg.IW;
#pragma unroll
    for (int it = 0; it < C::PITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        float v = 0.f;
        if (idx < C::P_LDS) {
            const int cl = idx / (C::PR * C::PC);
            const int rem = idx - cl * (C::PR * C::PC);
            const int r = rem / C::PC, c = rem - r * C::PC;
            const int ci = ck * C::KC + cl;
            const int iy = oy0 * C::S - C::PAD + r, ix = ox0 * C::S - C::PAD + c;
            if (ci < sg.C) {
                if (C::REFLECT) {
                    v = gp(sg.src)[(long)ci * plane + (long)reflect1(iy, sg.IH) * sg.IW + reflect1(ix, sg.IW)];
                } else if (iy >= 0 && ix >= 0 && iy < sg.IH && ix < sg.IW) {
                    v = gp(sg.src)[(long)ci * plane + (long)iy * sg.IW + ix];
                }
            }
        }
        st.p[it] = v;
    }
}

template <class C>
__device__ __forceinline__ void store_chunk(const Stage<C> &st, float *wl, float *pl)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        if (idx < C::W4) {
            const int row = idx / (C::WK / 4), c4 = idx % (C::WK / 4);
            *reinterpret_cast<float4 *>(wl + row * C::WSTR + c4 * 4) = st.w[it];
        }
    }
#pragma unroll
    for (int it = 0; it < C::PITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        if (idx < C::P_LDS) pl[idx] = st.p[it];
    }
}

template <int N>
__device__ __forceinline__ void lds_vec(float (&a)[N], const float *p)
{
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
            float4 v = *reinterpret_cast<const float4 *>(p + 4 * q);
            a[4 * q] = v.x;
            a[4 * q + 1] = v.y;
            a[4 * q + 2] = v.z;
            a[4 * q + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        float2 v = *reinterpret_cast<const float2 *>(p);
        a[0] = v.x;
        a[1] = v.y;
    } else {
#pragma unroll
        for (int q = 0; q < N; ++q) a[q] = p[q];
    }
}

template <class C>
__device__ __forceinline__ void compute_chunk(f32x16 &acc, const float *wl, const float *pl)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int pr = p / C::TC, pc = p % C::TC;
    const float *wrow = wl + (wm * 32 + j) * C::WSTR + g * (C::KC / 2);
    const float *prow = pl + g * (C::KC / 2) * C::PR * C::PC + pr * C::S * C::PC + pc * C::S;
#pragma unroll
    for (int t = 0; t < C::T; ++t) {
        const int ky = t / C::KW, kx = t % C::KW;
        float a[C::KC / 2];
        lds_vec<C::KC / 2>(a, wrow + t * C::KC);
#pragma unroll
        for (int c = 0; c < C::KC / 2; ++c) {
            const float bv = prow[c * C::PR * C::PC + ky * C::PC + kx];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[c], bv, acc, 0, 0, 0);
        }
    }
}

template <class C>
__device__ __forceinline__ void run_segment(f32x16 &acc, const ConvSeg &sg, int m0, int M, int oy0, int ox0,
                                            float *lds)
{
    float *wl = lds, *pl = lds + C::W_LDS;
    Stage<C> st;
    load_chunk<C>(st, sg, 0, m0, M, oy0, ox0);
    for (int ck = 0; ck < sg.nchunk; ++ck) {
        __syncthreads();
        store_chunk<C>(st, wl, pl);
        __syncthreads();
        if (ck + 1 < sg.nchunk) load_chunk<C>(st, sg, ck + 1, m0, M, oy0, ox0);
        compute_chunk<C>(acc, wl, pl);
    }
}

template <int TR, int TC>
__device__ __forceinline__ void epilogue(const f32x16 &acc, const ConvProblem &P, int m0, int oy0, int ox0)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int oy = oy0 + p / TC, ox = ox0 + p % TC;
    if (oy >= P.OH || ox >= P.OW) return;
    const long pix = (long)(oy * P.oy_mul + P.oy_off) * P.outW + (long)ox * P.ox_mul + P.ox_off;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = 8 * (r >> 2) + 4 * g + (r & 3);
        const int co = m0 + wm * 32 + i;
        if (co < P.M) {
            float v = acc[r];
            if (P.bias) v += gp(P.bias)[co];
            if (P.scale) v = v * gp(P.scale)[co] + gp(P.shift)[co];
            if (P.relu) v = fmaxf(v, 0.f);
            const long o = (long)co * P.out_cstride + pix;
            if (P.res) v += gp(P.res)[o];
            gp(P.out)[o] = v;
        }
    }
}

// One 64 x 64 output tile of problem P: segment 0 with the template geometry,
// then (SEG1) the optional 1x1 segment over a second source.
template <class C0, bool SEG1>
__device__ __forceinline__ void conv_tile(const ConvProblem &P, int b, float *lds)
{
    const int mb = b % P.mblocks, t = b / P.mblocks;
    const int tx = t % P.tiles_x, ty = t / P.tiles_x;
    const int m0 = mb * 64, oy0 = ty * C0::TR, ox0 = tx * C0::TC;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    run_segment<C0>(acc, P.s0, m0, P.M, oy0, ox0, lds);
    if constexpr (SEG1) {
        using C1 = Cfg<1, 1, 1, false, C0::KC, C0::TR, C0::TC>;
        if (P.s1.nchunk > 0) run_segment<C1>(acc, P.s1, m0, P.M, oy0, ox0, lds);
    }
    epilogue<C0::TR, C0::TC>(acc, P, m0, oy0, ox0);
}

__device__ __forceinline__ int find_problem(const ConvProblem *probs, int nprob, int &b)
{
    int pi = 0;
    while (pi + 1 < nprob && b >= probs[pi].nblocks) {
        b -= probs[pi].nblocks;
        ++pi;
    }
    return pi;
}

using CfgHead = Cfg<7, 7, 1, true, 4, 2, 32>;
using CfgDown = Cfg<3, 3, 2, true, 8, 2, 32>;
using CfgFfc = Cfg<3, 3, 1, true, 8, 2, 32>;
using CfgFfc1 = Cfg<1, 1, 1, false, 8, 2, 32>;
using Cfg1x1 = Cfg<1, 1, 1, false, 32, 1, 64>;
using CfgT00 = Cfg<1, 1, 1, false, 8, 2, 32>;
using CfgT01 = Cfg<1, 2, 1, false, 8, 2, 32>;
using CfgT10 = Cfg<2, 1, 1, false, 8, 2, 32>;
using CfgT11 = Cfg<2, 2, 1, false, 8, 2, 32>;

}  // namespace

// model.1: 7x7, reflect pad 3 (the ReflectionPad2d(3) + valid 7x7 of the
// reference), 4 -> 64, BN + ReLU.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv7x7(const ConvProblem *__restrict__ probs, int nprob)
{
    __shared__ __attribute__((aligned(16))) float lds[CfgHead::LDS];
    int b = blockIdx.x;
    int pi = find_problem(probs, nprob, b);
    conv_tile<CfgHead, false>(probs[pi], b, lds);
}

// model.2/3/4: 3x3 stride 2, reflect pad 1, BN + ReLU.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv3x3s2(const ConvProblem *__restrict__ probs, int nprob)
{
    __shared__ __attribute__((aligned(16))) float lds[CfgDown::LDS];
    int b = blockIdx.x;
    int pi = find_problem(probs, nprob, b);
    conv_tile<CfgDown, false>(probs[pi], b, lds);
}

// FFC spatial convolutions: 3x3 stride 1 reflect pad 1, with an optional 1x1
// second K segment (the SpectralTransform's conv2, summed before BN_g).
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv3x3(const ConvProblem *__restrict__ probs, int nprob)
{
    __shared__ __attribute__((aligned(16))) float lds[cmax(CfgFfc::LDS, CfgFfc1::LDS)];
    int b = blockIdx.x;
    int pi = find_problem(probs, nprob, b);
    conv_tile<CfgFfc, true>(probs[pi], b, lds);
}

// 1x1 convolutions over flat planes (SpectralTransform conv1, FourierUnit conv).
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv1x1(const ConvProblem *__restrict__ probs, int nprob)
{
    __shared__ __attribute__((aligned(16))) float lds[Cfg1x1::LDS];
    int b = blockIdx.x;
    int pi = find_problem(probs, nprob, b);
    conv_tile<Cfg1x1, false>(probs[pi], b, lds);
}

// ConvTranspose2d k3 s2 p1 op1 as four sub-pixel phase convolutions
// (problems 0..3 = phases (py,px) = (0,0), (0,1), (1,0), (1,1)), each a valid
// (1+py) x (1+px) convolution with zero fill at the bottom/right edge.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_convt(const ConvProblem *__restrict__ probs, int nprob)
{
    __shared__ __attribute__((aligned(16))) float lds[cmax(cmax(CfgT00::LDS, CfgT01::LDS), cmax(CfgT10::LDS, CfgT11::LDS))];
    int b = blockIdx.x;
    int pi = find_problem(probs, nprob, b);
    switch (pi) {
    case 0: conv_tile<CfgT00, false>(probs[0], b, lds); break;
    case 1: conv_tile<CfgT01, false>(probs[1], b, lds); break;
    case 2: conv_tile<CfgT10, false>(probs[2], b, lds); break;
    default: conv_tile<CfgT11, false>(probs[3], b, lds); break;
    }
}
