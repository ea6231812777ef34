// FFC 3x3 convolutions (stride 1, reflect pad 1) as a one-dimensional
// Winograd F(2,3) along x, on FP32 MFMA.
//
// Each output pair (x, x+1) of a row is computed from four input columns
// d0..d3 = in[x-1 .. x+2] of each kernel row ky:
//     V = (d0 - d2, d1 + d2, d2 - d1, d1 - d3)             (input transform)
//     U = (g0, (g0 + g1 + g2) / 2, (g0 - g1 + g2) / 2, g2)   (weight transform, host)
//     m_u = sum over (ci, ky) of U_u * V_u                   (four GEMMs)
//     out[x] = m0 + m1 + m2,  out[x+1] = m1 - m2 - m3        (output transform)
// which is the same convolution with 12 instead of 18 multiplications per
// output pair and input channel (Lavin & Gray, "Fast Algorithms for
// Convolutional Neural Networks", 2016).  The transforms are exact in
// arithmetic; in FP32 they round differently from the direct sum.
//
// A workgroup computes 64 output channels x 2 output rows x 64 pixels (32
// Winograd tiles per row).  Wave (wm, wn) owns channels wm*32 .. +32 of
// output row wn, as four 32 x 32 accumulators (u = 0..3) of
// v_mfma_f32_32x32x2f32: GEMM rows are output channels, GEMM columns the 32
// tiles of the row, K = (ci, ky).  K is walked in chunks of LAMA_WINO_KC = 4
// input channels; per chunk the block stages in LDS the transformed weights
// [64 co][u][ky][4] and the transformed input [4 rows][u][32 tiles][4 (+2
// pad)], with the same two-stage pipeline as the direct kernels.  The chunk
// count is even (the host pads the packed weights with a zero chunk), so the
// K loop runs in chunk pairs with a single exit.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {

struct WCfg {
    static constexpr int KC = LAMA_WINO_KC;         // input channels per chunk
    static constexpr int NU = 4, KY = 3;            // Winograd positions, kernel rows
    static constexpr int WK = NU * KY * KC;         // weights per output channel and chunk
    static constexpr int WSTR = WK + 4;             // LDS row stride (= 4 mod 8)
    static constexpr int NT = 32;                   // tiles per output row
    static constexpr int TR = 2, TC = 2 * NT;       // output rows x pixels per block
    static constexpr int IR = TR + 2;               // input rows per block
    static constexpr int H = KC / 2;                // channels per lane half and MFMA K slot
    static constexpr int KCP = H % 4 == 0 ? KC + 4 : KC + 2;  // LDS floats per (row, u, tile)
    static constexpr int W_LDS = 64 * WSTR;
    static constexpr int V_LDS = IR * NU * NT * KCP;
    static constexpr int LDS = W_LDS + V_LDS;       // floats per stage
    static constexpr int WITER = 64 * WK / 4 / LAMA_NT;     // weight float4s per thread
    static constexpr int VITER = KC * IR * NT / LAMA_NT;    // (ci, row, tile) items per thread
    static_assert(WITER * LAMA_NT * 4 == 64 * WK, "whole weight float4s");
    static_assert(VITER * LAMA_NT == KC * IR * NT, "whole input items");
};

struct WSlots {
    int wg[WCfg::WITER], wl[WCfg::WITER];  // weights: float offset in the row, LDS offset
    unsigned po[WCfg::VITER][4];           // input: byte offsets of d0..d3 from the chunk's first plane
    int vl[WCfg::VITER];                   // input: LDS offset of V_0 (V_u at + u * NT * KCP)
};

struct WStage {
    float w[4 * WCfg::WITER];
    float d[WCfg::VITER][4];
};

__device__ __forceinline__ void wino_slots(WSlots &sl, const ConvSeg &sg, int m0, int M, int oy0, int ox0)
{
    using C = WCfg;
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const int idx = tid + it * LAMA_NT, row = idx / (C::WK / 4), c4 = idx % (C::WK / 4);
        sl.wl[it] = row * C::WSTR + c4 * 4;
        sl.wg[it] = min(m0 + row, M - 1) * sg.wrow + c4 * 4;
    }
    const unsigned cs = (unsigned)sg.cs;
#pragma unroll
    for (int it = 0; it < C::VITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        const int t = idx % C::NT, r = (idx / C::NT) % C::IR, ci = idx / (C::NT * C::IR);
        const int iy = reflect1(oy0 - 1 + r, sg.IH);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int ix = reflect1(ox0 + 2 * t - 1 + c, sg.IW);
            sl.po[it][c] = 4u * ((unsigned)ci * cs + (unsigned)(iy * sg.IW + ix));
        }
        sl.vl[it] = (r * C::NU * C::NT + t) * C::KCP + ci;
    }
}

__device__ __forceinline__ void wino_load(WStage &st, const WSlots &sl, const ConvSeg &sg, int ck)
{
    using C = WCfg;
    const LAMA_GLOBAL float *wt = gp(sg.wt) + (long)ck * C::WK;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const float4 v = *at_byte<float4>(wt, 4u * (unsigned)sl.wg[it]);
        st.w[4 * it] = v.x;
        st.w[4 * it + 1] = v.y;
        st.w[4 * it + 2] = v.z;
        st.w[4 * it + 3] = v.w;
    }
    // channels past C (zero weights) read the last float of the source; the
    // zero chunk that pads the count to even reads within channel C - 1
    const unsigned plane = (unsigned)(sg.IH * sg.IW), cs = (unsigned)sg.cs;
    const int c0 = min(ck * C::KC, sg.C - 1);
    const unsigned last = 4u * ((unsigned)(min(sg.C - c0, C::KC) - 1) * cs + plane - 1u);
    const LAMA_GLOBAL float *src = gp(sg.src) + (long)c0 * cs;
#pragma unroll
    for (int it = 0; it < C::VITER; ++it)
#pragma unroll
        for (int c = 0; c < 4; ++c) st.d[it][c] = *at_byte<float>(src, min(sl.po[it][c], last));
}

__device__ __forceinline__ void wino_store(const WStage &st, const WSlots &sl, float *lds)
{
    using C = WCfg;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it)
        *reinterpret_cast<float4 *>(lds + sl.wl[it]) =
            make_float4(st.w[4 * it], st.w[4 * it + 1], st.w[4 * it + 2], st.w[4 * it + 3]);
    float *vl = lds + C::W_LDS;
#pragma unroll
    for (int it = 0; it < C::VITER; ++it) {
        const float d0 = st.d[it][0], d1 = st.d[it][1], d2 = st.d[it][2], d3 = st.d[it][3];
        vl[sl.vl[it]] = d0 - d2;
        vl[sl.vl[it] + C::NT * C::KCP] = d1 + d2;
        vl[sl.vl[it] + 2 * C::NT * C::KCP] = d2 - d1;
        vl[sl.vl[it] + 3 * C::NT * C::KCP] = d1 - d3;
    }
}

// MFMAs of one chunk: for each (ky, u), lane half g reads its H = KC/2
// channels H*g .. H*g + H - 1 of the weights and of the input (one 8-byte
// read each at KC = 4) and feeds one of them to each of H MFMAs as the
// MFMA's K slot g; the reads of the next (ky, u) are issued before the
// current MFMAs.
__device__ __forceinline__ void wino_compute(f32x16 (&acc)[WCfg::NU], const float *lds)
{
    using C = WCfg;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const float *wrow = lds + (wm * 32 + j) * C::WSTR + C::H * g;
    const float *vrow = lds + C::W_LDS + j * C::KCP + C::H * g;
    float a[2][C::H], b[2][C::H];
    auto rd = [&](int s, int buf) {
        const int ky = s / C::NU, u = s % C::NU;
        lds_vec<C::H>(a[buf], wrow + (u * C::KY + ky) * C::KC);
        lds_vec<C::H>(b[buf], vrow + ((wn + ky) * C::NU + u) * C::NT * C::KCP);
    };
    rd(0, 0);
#pragma unroll
    for (int s = 0; s < C::KY * C::NU; ++s) {
        const int cur = s & 1;
        if (s + 1 < C::KY * C::NU) rd(s + 1, cur ^ 1);
        const int u = s % C::NU;
#pragma unroll
        for (int c = 0; c < C::H; ++c) acc[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[cur][c], b[cur][c], acc[u], 0, 0, 0);
    }
}

// One 64-channel x 2-row x 64-pixel block of problem P (s1 absent).
__device__ __forceinline__ void wino_tile(const ConvProblem &P, int b, float *lds, float *epl)
{
    using C = WCfg;
    const int mb = b % P.mblocks, t = b / P.mblocks;
    const int tx = t % P.tiles_x, ty = t / P.tiles_x;
    const int m0 = mb * 64, oy0 = ty * C::TR, ox0 = tx * C::TC;
    const float ep = epi_param_load(P, m0);
    f32x16 acc[C::NU];
#pragma unroll
    for (int u = 0; u < C::NU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
    const ConvSeg sg = P.s0;  // held in registers across the barriers
    const int n = sg.nchunk, last = n - 1;
    WSlots sl;
    wino_slots(sl, sg, m0, P.M, oy0, ox0);
    float *l0 = lds, *l1 = lds + C::LDS;
    WStage r0, r1;
    wino_load(r0, sl, sg, 0);
    wino_load(r1, sl, sg, min(1, last));
    wino_store(r0, sl, l0);
    wino_load(r0, sl, sg, min(2, last));
    __syncthreads();
    // n is even (the weights are packed in pairs of chunks), so the loop has
    // one exit and the accumulators stay in the same registers throughout
    for (int ck = 0; ck < n; ck += 2) {
        wino_compute(acc, l0);
        wino_store(r1, sl, l1);
        wino_load(r1, sl, sg, min(ck + 3, last));
        __syncthreads();
        wino_compute(acc, l1);
        wino_store(r0, sl, l0);
        wino_load(r0, sl, sg, min(ck + 4, last));
        __syncthreads();
    }
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
    // output transform, then the fused epilogue of the direct kernels
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int oy = oy0 + wn, ox = ox0 + 2 * j;
    if (oy >= P.OH || ox >= P.OW) return;
    const bool second = ox + 1 < P.OW;
    const long pix = (long)oy * P.outW + ox;
    LAMA_GLOBAL float *out = gp(P.out);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int cl = wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m0 + cl >= P.M) continue;
        const long o = (long)(m0 + cl) * P.out_cstride + pix;
        float y[2] = {acc[0][r] + acc[1][r] + acc[2][r], acc[1][r] - acc[2][r] - acc[3][r]};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            if (e == 1 && !second) break;
            float x = y[e];
            if (P.bias) x += epl[cl];
            for (int i = 0; i < P.naddend; ++i) x += gp(P.addend)[o + e + i * P.addend_kstride];
            if (P.scale) x = x * epl[64 + cl] + epl[128 + cl];
            if (P.relu) x = fmaxf(x, 0.f);
            if (P.res) x += gp(P.res)[o + e];
            out[o + e] = x;
        }
    }
}

}  // namespace

// FFC spatial convolutions (3x3, stride 1, reflect pad 1) as Winograd F(2,3)
// along x; problems of a grouped launch are found as in the direct kernels.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv3x3w(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    __shared__ __attribute__((aligned(16))) float lds[2 * WCfg::LDS];
    __shared__ float epl[192];
    int b = blockIdx.x;
    int pi = find_problem(ps, b);
    wino_tile(probs[pi], b, lds, epl);
    LAMA_STAMP_END;
}
