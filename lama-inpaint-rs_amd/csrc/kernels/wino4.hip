// FFC 3x3 convolutions (stride 1, reflect pad 1) as a one-dimensional
// Winograd F(4,3) along x, on FP32 MFMA.
//
// Each output quad (x .. x+3) of a row is computed from the six input columns
// d0..d5 = in[x-1 .. x+4] of each kernel row ky, with the interpolation points
// 0, 1, -1, 2, -2 and infinity (Lavin & Gray, "Fast Algorithms for
// Convolutional Neural Networks", 2016):
//     V = B^T d   (input transform, while the rows are staged in LDS)
//         V0 = 4 d0 - 5 d2 + d4          V3 = -2 d1 - d2 + 2 d3 + d4
//         V1 = -4 (d1 + d2) + d3 + d4    V4 = 2 d1 - d2 - 2 d3 + d4
//         V2 = 4 (d1 - d2) - d3 + d4     V5 = 4 d1 - 5 d3 + d5
//     U = G g     (weight transform in f64, once, by lama_pack_wino)
//         U = (g0/4, -(g0+g1+g2)/6, -(g0-g1+g2)/6, g0/24+g1/12+g2/6, g0/24-g1/12+g2/6, g2)
//     m_u = sum over (ci, ky) of U_u * V_u                   (six GEMMs)
//     out = A^T m (output transform, in the epilogue)
//         out0 = m0 + m1 + m2 + m3 + m4      out2 = m1 + m2 + 4 (m3 + m4)
//         out1 = m1 - m2 + 2 (m3 - m4)       out3 = m1 - m2 + 8 (m3 - m4) + m5
// 6 multiplications per 4 outputs and kernel row instead of the 12 of the
// direct sum: half the direct convolution's MFMA work, 3/4 of F(2,3)'s.
//
// A workgroup computes 64 output channels x RW rows x 4*NTR pixels (32
// Winograd tiles: RW rows of NTR tiles, NTR = 16, 8 or 4, so 64-, 32- or
// 16-pixel wide blocks).  Wave (wm, wu) owns channels wm*32 .. +32 and the
// positions u = 3*wu .. 3*wu+2 as three 32 x 32 accumulators of
// v_mfma_f32_32x32x2f32: GEMM rows are output channels, GEMM columns the
// block's 32 tiles, K = (ci, ky).  K is walked in chunks of LAMA_WINO_KC = 4
// input channels.  Each weight is an MFMA operand of exactly one wave, so the
// waves load their transformed weights straight from global memory into
// registers (the host packs them in operand order), two register sets that
// alternate by chunk, each step pair's registers reloaded for the chunk after
// next as soon as that pair's MFMAs have issued; only the
// transformed input, which the two channel halves share, is staged in LDS
// ([rows][u][tiles][4 (+2 pad)]), two stages with one barrier per chunk and
// an even chunk count.  In the epilogue the two position halves of each
// channel half swap partial sums of the output transform through LDS, so
// that each wave finishes two of the four pixels of every tile.
#include <hip/hip_runtime.h>

#include "common.h"

// Weight reloads inside the MFMA sequence (w4_compute_ld): 1, the default,
// measured 30.4 / 24.9 against 34.6 / 27.8 us per launch (l2l + l2g /
// g2l, one stream, 512x512) and 181.5 against 175.4 passes/s at 600x600;
// 0 reloads a chunk's weights after its last MFMA (w4_load_w).
#ifndef LAMA_W4_WIL
#define LAMA_W4_WIL 1
#endif

namespace {

template <int NTR_, bool V4_ = false>
struct W4Cfg {
    // V4: the plane width is a multiple of 4, so each tile's inputs d1..d4 are
    // one aligned 16-byte load (d0 and d5, reflect-mapped at the edges, two
    // scalar ones): three loads per item instead of six
    static constexpr bool V4 = V4_;
    static constexpr int KC = LAMA_WINO_KC;      // input channels per chunk
    static constexpr int NU = 6, KY = 3;         // Winograd positions, kernel rows
    static constexpr int NUW = NU / 2;           // positions per wave
    static constexpr int NS = KY * NUW;          // MFMA steps of two K slots per wave and chunk
    static constexpr int NTR = NTR_;             // tiles per output row
    static constexpr int RW = 32 / NTR;          // output rows per block
    static constexpr int TR = RW, TC = 4 * NTR;  // output rows x pixels per block
    static constexpr int IR = TR + 2;            // input rows per block
    static constexpr int WK = NU * KY * KC;      // weights per output channel and chunk (72)
    static constexpr int WCH = 64 * WK;          // packed weights per 64-channel block and chunk
    static constexpr int H = KC / 2;             // channels per lane half and MFMA K slot
    static constexpr int KCP = KC + 2;           // LDS floats per (row, u, tile)
    static constexpr int NITEM = KC * IR * NTR;  // (ci, row, tile) input items per chunk
    static constexpr int NT = LAMA_NT;           // threads per workgroup
    static constexpr int VITER = (NITEM + NT - 1) / NT;
    static constexpr int VRS = NU * NTR * KCP;   // LDS stride of an input row
    static constexpr int V_LDS = IR * VRS + NU * 64;  // per stage, + a dummy tail for items past NITEM
    // epilogue exchange: per channel half, two pixels x 16 registers x 64 lanes from each position half
    static constexpr int X_LDS = 2 * 2 * 2 * 16 * 64;
    static constexpr int LDS = 2 * V_LDS > X_LDS ? 2 * V_LDS : X_LDS;  // floats
    static_assert(NTR * RW == 32, "32 tiles per block");
    static_assert(KC == 4, "two channels per lane half");
};

template <class C>
struct W4Slots {
    unsigned po[C::VITER][6];  // byte offsets of d0..d5 from the chunk's first plane
    int vl[C::VITER];          // LDS offset of V_0 (V_u at + u * NTR * KCP)
};

template <class C>
struct W4Stage {
    float d[C::VITER][6];
};

template <class C>
__device__ __forceinline__ void w4_slots(W4Slots<C> &sl, const ConvSeg &sg, int oy0, int ox0)
{
    const int tid = threadIdx.x;
    const unsigned cs = (unsigned)sg.cs;
#pragma unroll
    for (int it = 0; it < C::VITER; ++it) {
        // items past NITEM (a partial last round) read clamped, valid
        // addresses and land in the dummy tail of the V region
        const int idx = tid + it * C::NT, q = min(idx, C::NITEM - 1);
        const int t = q % C::NTR, r = (q / C::NTR) % C::IR, ci = q / (C::NTR * C::IR);
        const int iy = reflect1(oy0 - 1 + r, sg.IH);
#pragma unroll
        for (int c = 0; c < 6; ++c) {
            const int ix = reflect1(ox0 + 4 * t - 1 + c, sg.IW);
            sl.po[it][c] = 4u * ((unsigned)ci * cs + (unsigned)(iy * sg.IW + ix));
        }
        if constexpr (C::V4) {
            // d1..d4 in place; a tile past the plane's right edge (outputs
            // dropped) reads the row's last quad instead
            const int x4 = min(ox0 + 4 * t, sg.IW - 4);
            sl.po[it][1] = 4u * ((unsigned)ci * cs + (unsigned)(iy * sg.IW + x4));
        }
        sl.vl[it] = idx < C::NITEM ? r * C::VRS + t * C::KCP + ci : C::IR * C::VRS + (idx - C::NITEM) % 64;
    }
}

// A wave's MFMA A operands of one chunk: for steps s = ky * 3 + q (position
// u = 3 wu + q) lane (g, j) holds the transformed weights of output channel
// wm * 32 + j and input channels 2g, 2g + 1 of the chunk.  LAMA_W4_WX4: steps
// 2p and 2p + 1 (p < 4) are one 16-byte load per lane (64 lanes x 16
// contiguous bytes), step 8 an 8-byte one -- five loads per chunk instead of
// nine; else 64 lanes x 8 contiguous bytes per step.  `wb` is the wave's
// first float (WX4) or its lane's.
template <class C>
__device__ __forceinline__ void w4_load_w(float (&w)[2 * C::NS], const LAMA_GLOBAL float *wb, int ck)
{
    const LAMA_GLOBAL float *p = wb + (long)ck * C::WCH;
#if LAMA_W4_WX4
    static_assert(C::NS == 9, "four step pairs and a last step");
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 v = *reinterpret_cast<const LAMA_GLOBAL float4 *>(p + q * 256 + lane * 4);
        w[4 * q] = v.x;
        w[4 * q + 1] = v.y;
        w[4 * q + 2] = v.z;
        w[4 * q + 3] = v.w;
    }
    const float2 v = *reinterpret_cast<const LAMA_GLOBAL float2 *>(p + 1024 + lane * 2);
    w[16] = v.x;
    w[17] = v.y;
#else
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
        const float2 v = *reinterpret_cast<const LAMA_GLOBAL float2 *>(p + s * 128);
        w[2 * s] = v.x;
        w[2 * s + 1] = v.y;
    }
#endif
}

// The input rows d0..d5 of each of the thread's items of chunk `ck`.
template <class C>
__device__ __forceinline__ void w4_load_d(W4Stage<C> &st, const W4Slots<C> &sl, const ConvSeg &sg, int ck)
{
    // channels past C (zero weights) read the last float of the source; the
    // zero chunk that pads the count to even reads within channel C - 1
    const unsigned plane = (unsigned)(sg.IH * sg.IW), cs = (unsigned)sg.cs;
    const int c0 = min(ck * C::KC, sg.C - 1);
    const unsigned last = 4u * ((unsigned)(min(sg.C - c0, C::KC) - 1) * cs + plane - 1u);
    const LAMA_GLOBAL float *src = gp(sg.src) + (long)c0 * cs;
    if constexpr (C::V4) {
        // the last quad: 16-byte aligned, as the plane size and stride are
        const unsigned last4 = last - 12u;
#pragma unroll
        for (int it = 0; it < C::VITER; ++it) {
            const float4 m = *at_byte<float4>(src, min(sl.po[it][1], last4));
            st.d[it][0] = *at_byte<float>(src, min(sl.po[it][0], last));
            st.d[it][1] = m.x;
            st.d[it][2] = m.y;
            st.d[it][3] = m.z;
            st.d[it][4] = m.w;
            st.d[it][5] = *at_byte<float>(src, min(sl.po[it][5], last));
        }
    } else {
#pragma unroll
        for (int it = 0; it < C::VITER; ++it)
#pragma unroll
            for (int c = 0; c < 6; ++c) st.d[it][c] = *at_byte<float>(src, min(sl.po[it][c], last));
    }
}

// V = B^T d of each item into the LDS stage `vl`.
template <class C>
__device__ __forceinline__ void w4_store_v(const W4Stage<C> &st, const W4Slots<C> &sl, float *vl)
{
    constexpr int S = C::NTR * C::KCP;  // LDS distance between positions
#pragma unroll
    for (int it = 0; it < C::VITER; ++it) {
        const float d0 = st.d[it][0], d1 = st.d[it][1], d2 = st.d[it][2], d3 = st.d[it][3], d4 = st.d[it][4],
                    d5 = st.d[it][5];
        const int o = sl.vl[it];
        // dummy items (o in the tail) write six words within the tail's 6 * 64
        const int st_ = o >= C::IR * C::VRS ? 64 : S;
        vl[o] = 4.f * d0 - 5.f * d2 + d4;
        vl[o + st_] = d3 + d4 - 4.f * (d1 + d2);
        vl[o + 2 * st_] = 4.f * (d1 - d2) - d3 + d4;
        vl[o + 3 * st_] = 2.f * (d3 - d1) - d2 + d4;
        vl[o + 4 * st_] = 2.f * (d1 - d3) - d2 + d4;
        vl[o + 5 * st_] = 4.f * d1 - 5.f * d3 + d5;
    }
}

// MFMAs of one chunk for wave (wm, wu): for each (ky, u) of the wave's three
// positions, lane half g reads its two channels of the input (one 8-byte
// read, issued a step ahead) and feeds one to each of two MFMAs as the MFMA's
// K slot g, beside the weights of that step from registers.
template <class C>
__device__ __forceinline__ void w4_compute(f32x16 (&acc)[C::NUW], const float (&w)[2 * C::NS], const float *vl)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wu = wave & 1, g = lane >> 5, j = lane & 31;
    const int r = j / C::NTR, t = j % C::NTR;  // the MFMA column's output row and tile within the block
    const float *vrow = vl + t * C::KCP + C::H * g;
    float b[2][C::H];
    auto rd = [&](int s, int buf) {
        const int ky = s / C::NUW, u = C::NUW * wu + s % C::NUW;
        lds_vec<C::H>(b[buf], vrow + (r + ky) * C::VRS + u * C::NTR * C::KCP);
    };
    rd(0, 0);
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
        const int cur = s & 1;
        if (s + 1 < C::NS) rd(s + 1, cur ^ 1);
        const int q = s % C::NUW;
#pragma unroll
        for (int c = 0; c < C::H; ++c)
            acc[q] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[2 * s + c], b[cur][c], acc[q], 0, 0, 0);
    }
}

// w4_compute, reloading the weight registers with chunk `ckn` as the steps
// that read them issue: steps 2q, 2q + 1 share one 16-byte load per lane
// (LAMA_W4_WX4), so load q follows step 2q + 1's MFMAs and has the rest of
// this chunk and the whole next one to land, instead of the next one only.
template <class C>
__device__ __forceinline__ void w4_compute_ld(f32x16 (&acc)[C::NUW], float (&w)[2 * C::NS], const float *vl,
                                              const LAMA_GLOBAL float *wb, int ckn)
{
    static_assert(C::NS == 9 && LAMA_W4_WX4, "four step pairs and a last step, 16-byte weight loads");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wu = wave & 1, g = lane >> 5, j = lane & 31;
    const int r = j / C::NTR, t = j % C::NTR;
    const float *vrow = vl + t * C::KCP + C::H * g;
    const LAMA_GLOBAL float *p = wb + (long)ckn * C::WCH;
    float b[2][C::H];
    auto rd = [&](int s, int buf) {
        const int ky = s / C::NUW, u = C::NUW * wu + s % C::NUW;
        lds_vec<C::H>(b[buf], vrow + (r + ky) * C::VRS + u * C::NTR * C::KCP);
    };
    rd(0, 0);
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
        const int cur = s & 1;
        if (s + 1 < C::NS) rd(s + 1, cur ^ 1);
        const int q = s % C::NUW;
#pragma unroll
        for (int c = 0; c < C::H; ++c)
            acc[q] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[2 * s + c], b[cur][c], acc[q], 0, 0, 0);
        if (s & 1) {
            const int h = s >> 1;
            const float4 v = *reinterpret_cast<const LAMA_GLOBAL float4 *>(p + h * 256 + lane * 4);
            w[4 * h] = v.x;
            w[4 * h + 1] = v.y;
            w[4 * h + 2] = v.z;
            w[4 * h + 3] = v.w;
            // keep the load here: the scheduler would otherwise sink it below
            // the chunk's last MFMA
            __builtin_amdgcn_sched_barrier(0);
        } else if (s == C::NS - 1) {
            const float2 v = *reinterpret_cast<const LAMA_GLOBAL float2 *>(p + 1024 + lane * 2);
            w[16] = v.x;
            w[17] = v.y;
        }
    }
}

// One 64-channel x RW-row x 4*NTR-pixel block of problem P (s1 absent).
template <class C>
__device__ __forceinline__ void w4_tile(const ConvProblem &P, int b, float *lds, float *epl)
{
    // K slice of a split problem: the blocks of slice ks follow those of ks - 1
    int ks = 0;
    if (P.ksplit > 1) {
        const int per = P.mblocks * P.tiles_x * P.tiles_y;
        ks = b / per;
        b -= ks * per;
    }
#if LAMA_W4_XCD
    // M-block-major: with the XCD-contiguous launch order, an XCD's blocks
    // cover few M blocks (each of whose weights its L2 then holds once)
    const int ntile = P.tiles_x * P.tiles_y, mb = b / ntile, tt = b - mb * ntile;
#else
    const int mb = b % P.mblocks, tt = b / P.mblocks;
#endif
    const int tx = tt % P.tiles_x, ty = tt / P.tiles_x;
    const int m0 = mb * 64, oy0 = ty * C::TR, ox0 = tx * C::TC;
    const float ep = epi_param_load(P, m0);
    f32x16 acc[C::NUW];
#pragma unroll
    for (int q = 0; q < C::NUW; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[q][r] = 0.f;
    ConvSeg sg = P.s0;  // held in registers across the barriers
    if (P.ksplit > 1) {
        const int c0 = ks * P.kchunks * C::KC;
        sg.src += (long)c0 * sg.cs;
        sg.wt += (long)ks * P.kchunks * C::WCH;
        sg.C -= c0;
        sg.nchunk = P.kchunks;
    }
    const int n = sg.nchunk, last = n - 1;
    {
        W4Slots<C> sl;
        w4_slots<C>(sl, sg, oy0, ox0);
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        // the M block's weights (64 rows of wrow floats), then this wave's and lane's operands
        const LAMA_GLOBAL float *wb =
            gp(sg.wt) + (long)mb * 64 * sg.wrow + wave * (C::NS * 128) + (LAMA_W4_WX4 ? 0 : lane * 2);
        float *l0 = lds, *l1 = lds + C::V_LDS;
        float w0[2 * C::NS], w1[2 * C::NS];
        W4Stage<C> r0, r1;
        // weights one chunk ahead, inputs two; the prefetches past the last
        // chunk re-read it (uniform control flow)
        w4_load_w<C>(w0, wb, 0);
        w4_load_d<C>(r0, sl, sg, 0);
        w4_load_w<C>(w1, wb, min(1, last));
        w4_load_d<C>(r1, sl, sg, min(1, last));
        w4_store_v<C>(r0, sl, l0);
        w4_load_d<C>(r0, sl, sg, min(2, last));
        __syncthreads();
        // n is even (the weights are packed in pairs of chunks): one loop exit
        for (int ck = 0; ck < n; ck += 2) {
#if LAMA_W4_WIL
            w4_compute_ld<C>(acc, w0, l0, wb, min(ck + 2, last));
#else
            w4_compute<C>(acc, w0, l0);
            w4_load_w<C>(w0, wb, min(ck + 2, last));
#endif
            w4_store_v<C>(r1, sl, l1);
            w4_load_d<C>(r1, sl, sg, min(ck + 3, last));
            __syncthreads();
#if LAMA_W4_WIL
            w4_compute_ld<C>(acc, w1, l1, wb, min(ck + 3, last));
#else
            w4_compute<C>(acc, w1, l1);
            w4_load_w<C>(w1, wb, min(ck + 3, last));
#endif
            w4_store_v<C>(r0, sl, l0);
            w4_load_d<C>(r0, sl, sg, min(ck + 4, last));
            __syncthreads();
        }
    }
    // output transform: wave wu = 0 holds m0..m2, wu = 1 holds m3..m5.
    // Partials  p = (m0 + m1 + m2, m1 - m2, m1 + m2, m1 - m2)   (wu = 0)
    //           q = (m3 + m4, 2 (m3 - m4), 4 (m3 + m4), 8 (m3 - m4) + m5)   (wu = 1)
    // and out_i = p_i + q_i; wave wu finishes pixels 2 wu and 2 wu + 1 of each
    // tile, after taking the other half's two partials through LDS.
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wu = wave & 1, g = lane >> 5, j = lane & 31;
    float mine[2][16], give[2][16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float a = acc[0][r], b2 = acc[1][r], c = acc[2][r];
        float v[4];
        if (wu == 0) {
            v[0] = a + b2 + c;
            v[1] = b2 - c;
            v[2] = b2 + c;
            v[3] = b2 - c;
        } else {
            v[0] = a + b2;
            v[1] = 2.f * (a - b2);
            v[2] = 4.f * (a + b2);
            v[3] = 8.f * (a - b2) + c;
        }
        mine[0][r] = v[2 * wu];
        mine[1][r] = v[2 * wu + 1];
        give[0][r] = v[2 - 2 * wu];
        give[1][r] = v[3 - 2 * wu];
    }
    // X[wm][from wu][pixel e][r][lane]: the staging buffers are free once
    // every wave has left the K loop
    float *xl = lds;
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int r = 0; r < 16; ++r) xl[(((wm * 2 + wu) * 2 + e) * 16 + r) * 64 + lane] = give[e][r];
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int r = 0; r < 16; ++r) mine[e][r] += xl[(((wm * 2 + (wu ^ 1)) * 2 + e) * 16 + r) * 64 + lane];
    // the fused epilogue of the direct kernels on pixels 4t + 2wu + e
    const int oy = oy0 + j / C::NTR, ox = ox0 + 4 * (j % C::NTR) + 2 * wu;
    if (oy >= P.OH || ox >= P.OW) return;
    const bool second = ox + 1 < P.OW;
    const long pix = (long)oy * P.outW + ox;
    LAMA_GLOBAL float *out = gp(P.out) + (long)ks * P.out_kstride;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int cl = wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m0 + cl >= P.M) continue;
        const long o = (long)(m0 + cl) * P.out_cstride + pix;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            if (e == 1 && !second) break;
            float x = mine[e][r];
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

// FFC spatial convolutions (3x3, stride 1, reflect pad 1) as Winograd F(4,3)
// along x, in 64-pixel (lama_conv3x3w4) or 32-pixel (lama_conv3x3w4n) wide
// blocks; problems of a grouped launch are found as in the direct kernels.
// Register budget of the F(4,3) kernels: at 120 the compiler keeps the
// accumulators in VGPRs and fits the kernel in 130 registers (216 with
// accumulation registers, without the bound), so three of these fit on a
// SIMD, or two beside a SpectralTransform kernel's wave.  With 33.5 KB of
// LDS three workgroups also fit on a CU; the host adds dynamic LDS to hold
// the GEMMs at two per CU where that leaves the SpectralTransform's kernels
// room.
// XCD-contiguous launch order: the dispatcher deals workgroups to the eight
// XCDs round-robin (workgroup i to XCD i mod 8), each XCD with its own L2.
// Workgroup i takes block x * q + min(x, r) + i / 8 of the launch's natural
// order (x = i mod 8; the n blocks split as q = n / 8 per XCD, the first
// r = n mod 8 XCDs one more), so that each XCD works through one contiguous
// range: with M-block-major problems that is one or two M blocks' weights
// (0.6 MB each) and one problem's input channels per L2, instead of every
// M block's weights (A: 4.7 MB against a 4 MB L2) or all 384 global input
// planes (B: 6.3 MB) in every L2.  LAMA_W4_XCD=0 keeps the natural order.
#ifndef LAMA_W4_XCD
#define LAMA_W4_XCD 1
#endif
namespace {
__device__ __forceinline__ int w4_xcd_order(int i, int n)
{
#if LAMA_W4_XCD
    const int x = i & 7, q = n >> 3, r = n & 7;
    return x * q + min(x, r) + (i >> 3);
#else
    (void)n;
    return i;
#endif
}
}  // namespace

// (the cap: 128 measured 283.6-284.5 passes/s at 512x512 against 281.1-281.9
// at 120, the same 138 registers with a different schedule; 132 to 144 gave
// two waves per SIMD and 192-265 passes/s)
#ifndef LAMA_W4_NUM_VGPR
#define LAMA_W4_NUM_VGPR 128
#endif
#if LAMA_W4_NUM_VGPR > 0
#define LAMA_W4_REGS __attribute__((amdgpu_num_vgpr(LAMA_W4_NUM_VGPR)))
#else
#define LAMA_W4_REGS
#endif
#define LAMA_W4_KERNEL(NAME, NTR)                                                          \
    extern "C" __global__ void __launch_bounds__(LAMA_NT) LAMA_W4_REGS NAME(LAMA_CONV_PARAMS) \
    {                                                                                      \
        LAMA_CONV_STARTS;                                                                  \
        LAMA_STAMP_BEGIN;                                                                  \
        using C = W4Cfg<NTR>;                                                              \
        using C4 = W4Cfg<NTR, true>;                                                       \
        static_assert(C4::LDS == C::LDS, "one LDS layout");                               \
        __shared__ __attribute__((aligned(16))) float lds[C::LDS];                         \
        __shared__ float epl[192];                                                         \
        int b = w4_xcd_order(blockIdx.x, gridDim.x);                                       \
        int pi = find_problem(ps, b);                                                      \
        if (probs[pi].vec_in && (probs[pi].s0.IW & 3) == 0)                                 \
            w4_tile<C4>(probs[pi], b, lds, epl);                                           \
        else                                                                               \
            w4_tile<C>(probs[pi], b, lds, epl);                                            \
        LAMA_STAMP_END;                                                                    \
    }
LAMA_W4_KERNEL(lama_conv3x3w4, 16)
LAMA_W4_KERNEL(lama_conv3x3w4n, 8)
LAMA_W4_KERNEL(lama_conv3x3w4q, 4)
#undef LAMA_W4_KERNEL

// ---------------------------------------------------------------------------
// FFC 3x3 convolutions as a two-dimensional Winograd F(2x4, 3x3): F(2,3)
// along y (points 0, 1, -1, infinity) times the F(4,3) above along x.  An
// output tile is 2 rows x 4 pixels, read from input rows r0..r3 x the six
// columns d0..d5 of each:
//     V_x(r) = B_x^T d(r)                        (the input transform above)
//     V(0) = V_x(r0) - V_x(r2)   V(1) = V_x(r1) + V_x(r2)
//     V(2) = V_x(r2) - V_x(r1)   V(3) = V_x(r1) - V_x(r3)       (B_y^T)
//     U(vy, u) = sum over (ky, kx) of G_y[vy][ky] G_x[u][kx] g[ky][kx]
//         G_y = (1, 0, 0; 1/2, 1/2, 1/2; 1/2, -1/2, 1/2; 0, 0, 1)   (f64, lama_pack_wino)
//     m(vy, u) = sum over ci of U(vy, u) V(vy, u)               (24 GEMMs)
//     out(row 0) = A_x^T (m(0) + m(1) + m(2)),  out(row 1) = A_x^T (m(1) - m(2) - m(3))
// 24 multiplications per 8 outputs and input channel: 2/3 of the
// one-dimensional F(4,3)'s, 1/3 of the direct sum's.
//
// A workgroup (8 waves) computes 64 output channels x 32 tiles: RP = 32 / NTR
// row pairs of NTR tiles.  Wave (wm, vy) owns channels wm*32 .. +32 and the
// six positions (vy, 0..5) as six 32 x 32 accumulators of
// v_mfma_f32_32x32x2f32 (GEMM columns: the block's 32 tiles).  The input rows
// are staged x-transformed in LDS exactly as in the one-dimensional kernel;
// each MFMA's B operand is the sum or difference of two staged rows (row vy
// of B_y^T), formed as the operands are read.  Each wave loads its own 12
// transformed weights per chunk into registers, reloading each 16-byte group
// as soon as its MFMAs have issued.  The epilogue runs in four rounds, one
// per pixel column of the tiles: every wave applies that column of A_x^T to
// its six accumulators and parks the 16 results in LDS; each wave then
// finishes four of the 16 register rows of its channel half, both output
// rows, from the four y positions.
namespace {

template <int NTR_, bool V4_ = false>
struct W42Cfg {
    static constexpr bool V4 = V4_;               // 16-byte input loads (plane width a multiple of 4)
    static constexpr int KC = LAMA_W42_KC;        // input channels per chunk
    static constexpr int NU = 6, NUY = 4;         // x positions, y positions
    static constexpr int NTR = NTR_;              // tiles per row pair
    static constexpr int RP = 32 / NTR;           // row pairs per block
    static constexpr int TR = 2 * RP, TC = 4 * NTR;  // output rows x pixels per block
    static constexpr int IR = TR + 2;             // input rows per block
    static constexpr int WK = NU * NUY * KC;      // weights per output channel and chunk (96)
    static constexpr int WCH = 64 * WK;           // packed weights per 64-channel block and chunk
    static constexpr int H = KC / 2;              // channels per lane half and MFMA K slot
    static constexpr int WW = NU * H;             // weight registers per wave and chunk (12 or 24)
    static constexpr int KCP = KC == 4 ? 6 : 12;  // LDS floats per (row, u, tile): 8- or 16-byte operand reads
    static constexpr int NITEM = KC * IR * NTR;   // (ci, row, tile) input items per chunk
    static constexpr int CH = LAMA_W42_CH;        // output channels per workgroup (32 or 64)
    static constexpr int WMS = CH / 32;           // channel halves per workgroup
    static constexpr int NT = 256 * WMS;          // threads per workgroup (4 waves per channel half)
    static constexpr int VITER = (NITEM + NT - 1) / NT;
    static constexpr int VRS = NU * NTR * KCP;    // LDS stride of an input row
    static constexpr int V_LDS = IR * VRS + NU * 64;  // per stage, + a dummy tail for items past NITEM
    static constexpr int X_LDS = 4 * WMS * 16 * 64;  // epilogue: one pixel column, 16 registers x 64 lanes per wave
    static constexpr int LDS = 2 * V_LDS > X_LDS ? 2 * V_LDS : X_LDS;  // floats
    static_assert(NTR * RP == 32, "32 tiles per block");
    static_assert(KC == 4 || KC == 8, "two or four channels per lane half");
    static_assert(CH == 32 || CH == 64, "one or two channel halves");
};

// The wave's WW weight operands of chunk `ck` (w[H u + c]: position u, K slot
// c), as WW / 4 16-byte loads per lane.
template <class C>
__device__ __forceinline__ void w42_load_w(float (&w)[C::WW], const LAMA_GLOBAL float *wb, int ck)
{
    const int lane = threadIdx.x & 63;
    const LAMA_GLOBAL float *p = wb + (long)ck * C::WCH;
#pragma unroll
    for (int h = 0; h < C::WW / 4; ++h) {
        const float4 v = *reinterpret_cast<const LAMA_GLOBAL float4 *>(p + h * 256 + lane * 4);
        w[4 * h] = v.x;
        w[4 * h + 1] = v.y;
        w[4 * h + 2] = v.z;
        w[4 * h + 3] = v.w;
    }
}

// MFMAs of one chunk for wave (wm, vy): for each x position u, lane half g
// reads its H channels of staged rows ra and rb (one 8- or 16-byte read each,
// a position ahead) and feeds ra + sb * rb -- row vy of B_y^T -- to H MFMAs
// as K slot g; each 16-byte group of the weight registers is reloaded with
// chunk `ckn` right after the last MFMA that reads it issues.
template <class C>
__device__ __forceinline__ void w42_compute_ld(f32x16 (&acc)[C::NU], float (&w)[C::WW], const float *vl,
                                               const LAMA_GLOBAL float *wb, int ckn)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int vy = wave & 3, g = lane >> 5, j = lane & 31;
    const int p = j / C::NTR, t = j % C::NTR;  // the MFMA column's row pair and tile within the block
    // B_y^T rows (1, 0, -1, 0), (0, 1, 1, 0), (0, -1, 1, 0), (0, 1, 0, -1)
    const int ra = 2 * p + (vy == 0 ? 0 : vy == 2 ? 2 : 1);
    const int rb = 2 * p + (vy == 2 ? 1 : vy == 3 ? 3 : 2);
    const float sb = vy == 1 ? 1.f : -1.f;
    const float *va = vl + ra * C::VRS + t * C::KCP + C::H * g;
    const float *vb = vl + rb * C::VRS + t * C::KCP + C::H * g;
    const LAMA_GLOBAL float *pw = wb + (long)ckn * C::WCH;
    float a[2][C::H], b[2][C::H];
    auto rd = [&](int u, int buf) {
        lds_vec<C::H>(a[buf], va + u * C::NTR * C::KCP);
        lds_vec<C::H>(b[buf], vb + u * C::NTR * C::KCP);
    };
    rd(0, 0);
#pragma unroll
    for (int u = 0; u < C::NU; ++u) {
        const int cur = u & 1;
        if (u + 1 < C::NU) rd(u + 1, cur ^ 1);
#pragma unroll
        for (int c = 0; c < C::H; ++c)
            acc[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[C::H * u + c], fmaf(sb, b[cur][c], a[cur][c]), acc[u], 0,
                                                          0, 0);
        if ((C::H * (u + 1)) % 4 == 0) {
            const int h = C::H * (u + 1) / 4 - 1;
            const float4 v = *reinterpret_cast<const LAMA_GLOBAL float4 *>(pw + h * 256 + lane * 4);
            w[4 * h] = v.x;
            w[4 * h + 1] = v.y;
            w[4 * h + 2] = v.z;
            w[4 * h + 3] = v.w;
            // keep the load here: the scheduler would otherwise sink it below
            // the chunk's last MFMA
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// One 64-channel x TR-row x TC-pixel block of problem P (s1 absent).
template <class C>
__device__ __forceinline__ void w42_tile(const ConvProblem &P, int b, float *lds, float *epl)
{
    // K slice of a split problem: the blocks of slice ks follow those of ks - 1
    int ks = 0;
    if (P.ksplit > 1) {
        const int per = P.mblocks * P.tiles_x * P.tiles_y;
        ks = b / per;
        b -= ks * per;
    }
#if LAMA_W4_XCD
    const int ntile = P.tiles_x * P.tiles_y, mb = b / ntile, tt = b - mb * ntile;
#else
    const int mb = b % P.mblocks, tt = b / P.mblocks;
#endif
    const int tx = tt % P.tiles_x, ty = tt / P.tiles_x;
    const int m0 = mb * C::CH, oy0 = ty * C::TR, ox0 = tx * C::TC;
    const float ep = epi_param_load(P, m0);
    f32x16 acc[C::NU];
#pragma unroll
    for (int u = 0; u < C::NU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
    ConvSeg sg = P.s0;  // held in registers across the barriers
    if (P.ksplit > 1) {
        const int c0 = ks * P.kchunks * C::KC;
        sg.src += (long)c0 * sg.cs;
        sg.wt += (long)ks * P.kchunks * C::WCH;
        sg.C -= c0;
        sg.nchunk = P.kchunks;
    }
    const int n = sg.nchunk, last = n - 1;
    {
        W4Slots<C> sl;
        w4_slots<C>(sl, sg, oy0, ox0);
        // the 64-row block's weights (64 rows of wrow floats), then wave
        // (wm, vy)'s WW * 64 per chunk (a 32-channel block is half wm of its
        // 64-row block)
        const int wave = threadIdx.x >> 6 | (m0 & 32) >> 3;
        const LAMA_GLOBAL float *wb = gp(sg.wt) + (long)(m0 >> 6) * 64 * sg.wrow + wave * (C::WW * 64);
        float *l0 = lds, *l1 = lds + C::V_LDS;
        float w0[C::WW], w1[C::WW];
        W4Stage<C> r0, r1;
        // weights one chunk ahead, inputs two; the prefetches past the last
        // chunk re-read it (uniform control flow)
        w42_load_w<C>(w0, wb, 0);
        w4_load_d<C>(r0, sl, sg, 0);
        w42_load_w<C>(w1, wb, min(1, last));
        w4_load_d<C>(r1, sl, sg, min(1, last));
        w4_store_v<C>(r0, sl, l0);
        w4_load_d<C>(r0, sl, sg, min(2, last));
        __syncthreads();
        // n is even (the weights are packed in pairs of chunks): one loop exit
        for (int ck = 0; ck < n; ck += 2) {
            w42_compute_ld<C>(acc, w0, l0, wb, min(ck + 2, last));
            w4_store_v<C>(r1, sl, l1);
            w4_load_d<C>(r1, sl, sg, min(ck + 3, last));
            __syncthreads();
            w42_compute_ld<C>(acc, w1, l1, wb, min(ck + 3, last));
            w4_store_v<C>(r0, sl, l0);
            w4_load_d<C>(r0, sl, sg, min(ck + 4, last));
            __syncthreads();
        }
    }
    // epilogue: four rounds, one per pixel column o of the tiles (the staging
    // buffers are free once every wave has left the K loop)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 2, vy = wave & 3, g = lane >> 5, j = lane & 31;
    const int p = j / C::NTR, t = j % C::NTR;
    const int oyp = oy0 + 2 * p, oxt = ox0 + 4 * t;
    float *xl = lds;
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    LAMA_GLOBAL float *out = gp(P.out) + (long)ks * P.out_kstride;
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        // column o of A_x^T: (1, 1, 1, 1, 1, 0), (0, 1, -1, 2, -2, 0),
        // (0, 1, 1, 4, 4, 0), (0, 1, -1, 8, -8, 1)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float m0v = acc[0][r], m1 = acc[1][r], m2 = acc[2][r], m3 = acc[3][r], m4 = acc[4][r],
                        m5 = acc[5][r];
            float v;
            if (o == 0)
                v = m0v + m1 + m2 + m3 + m4;
            else if (o == 1)
                v = m1 - m2 + 2.f * (m3 - m4);
            else if (o == 2)
                v = m1 + m2 + 4.f * (m3 + m4);
            else
                v = m1 - m2 + 8.f * (m3 - m4) + m5;
            xl[((wm * 4 + vy) * 16 + r) * 64 + lane] = v;
        }
        __syncthreads();
        const int ox = oxt + o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // register row r = 4 vy + i: output channel wm*32 + 8 vy + 4 g + i
            const int r = 4 * vy + i, cl = wm * 32 + 8 * vy + 4 * g + i;
            const float q0 = xl[((wm * 4 + 0) * 16 + r) * 64 + lane], q1 = xl[((wm * 4 + 1) * 16 + r) * 64 + lane],
                        q2 = xl[((wm * 4 + 2) * 16 + r) * 64 + lane], q3 = xl[((wm * 4 + 3) * 16 + r) * 64 + lane];
            if (m0 + cl >= P.M || ox >= P.OW) continue;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int oy = oyp + e;
                if (oy >= P.OH) continue;
                float x = e == 0 ? q0 + q1 + q2 : q1 - q2 - q3;
                const long ofs = (long)(m0 + cl) * P.out_cstride + (long)oy * P.outW + ox;
                if (P.bias) x += epl[cl];
                for (int k = 0; k < P.naddend; ++k) x += gp(P.addend)[ofs + k * P.addend_kstride];
                if (P.scale) x = x * epl[64 + cl] + epl[128 + cl];
                if (P.relu) x = fmaxf(x, 0.f);
                if (P.res) x += gp(P.res)[ofs];
                out[ofs] = x;
            }
        }
        __syncthreads();
    }
}

}  // namespace

// The F(2x4, 3x3) kernel: blocks of LAMA_W42_CH output channels x 4 rows x
// 64 pixels (16 tiles per row pair), four waves per 32 channels.
#define LAMA_W42_KERNEL(NAME, NTR)                                                          \
    extern "C" __global__ void __launch_bounds__(8 * LAMA_W42_CH) NAME(LAMA_CONV_PARAMS)  \
    {                                                                                       \
        LAMA_CONV_STARTS;                                                                   \
        LAMA_STAMP_BEGIN;                                                                   \
        using C = W42Cfg<NTR>;                                                              \
        using C4 = W42Cfg<NTR, true>;                                                       \
        static_assert(C4::LDS == C::LDS, "one LDS layout");                                \
        __shared__ __attribute__((aligned(16))) float lds[C::LDS];                          \
        __shared__ float epl[192];                                                          \
        int b = w4_xcd_order(blockIdx.x, gridDim.x);                                        \
        int pi = find_problem(ps, b);                                                       \
        if (probs[pi].vec_in && (probs[pi].s0.IW & 3) == 0)                                  \
            w42_tile<C4>(probs[pi], b, lds, epl);                                           \
        else                                                                                \
            w42_tile<C>(probs[pi], b, lds, epl);                                            \
        LAMA_STAMP_END;                                                                     \
    }
LAMA_W42_KERNEL(lama_conv3x3w42, 16)
#undef LAMA_W42_KERNEL
