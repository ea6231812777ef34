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
// input patch that covers the tile's receptive field, pixel-major
// [PR][PC][KC+4] (again 16-byte reads on distinct banks), gathered with
// PyTorch 'reflect' index mapping (or zero fill for the transposed
// convolution phases).  im2col is never materialised.  The next chunk's
// global loads are issued into registers before the MFMAs of the current one
// and land in the second of two LDS stages (one barrier per chunk).
//
// MFMA operand mapping (32x32x2, one block): lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; the two K slots of every MFMA are given to the two lane
// halves as channels ci = g*KC/2 + c (g = lane/32) of the same tap, so each
// lane reads its KC/2 weights and its KC/2 inputs for a tap with one vector
// LDS read each.  D[i][j]
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
    // patch pixel stride: the 16-byte (KC = 8) or 8-byte (KC = 4) per-lane
    // operand reads of neighbouring lanes land on distinct banks
    static constexpr int KCP = (KC / 2) % 4 == 0 ? KC + 4 : KC + 2;
    // Patch columns: stride-2 convolutions keep even and odd input columns in
    // two halves of a row (HPC each), so the operand reads of neighbouring
    // output pixels -- two input columns apart -- are one pixel apart in LDS.
    static constexpr int HPC = (PC + 1) / 2;
    static constexpr int PCP = S == 2 ? 2 * HPC : PC;  // LDS pixels per patch row
    static __device__ __forceinline__ constexpr int col(int c) { return S == 2 ? (c & 1) * HPC + (c >> 1) : c; }
    static constexpr int W4 = 64 * WK / 4;
    static constexpr int WITER = (W4 + LAMA_NT - 1) / LAMA_NT;
    // Patch staging: each 64-lane group takes 16 consecutive pixels x 4
    // consecutive channels (pixel fastest), so a wave's loads are 64-byte runs
    // and its 4-byte LDS stores, at pixel stride KCP, cover every bank once.
    static constexpr int NPIX = PR * PC;
    static constexpr int NPB = (NPIX + 15) / 16;            // 16-pixel blocks
    static constexpr int P_SLOTS = NPB * 16 * KC;
    static constexpr int PITER = (P_SLOTS + LAMA_NT - 1) / LAMA_NT;
    // staging is branch-free: weight slots past the data land in a dummy
    // tail of one float4 per lane, which every wave shares (its contents are
    // never read), so that the stages stay small enough for four
    // workgroups per CU
    static constexpr int W_LDS = 64 * WSTR + (WITER * LAMA_NT > W4 ? 64 * 4 : 0);
    static constexpr int P_LDS = PR * PCP * KCP + 64;
    static constexpr int LDS = W_LDS + P_LDS;
    static_assert(TR * TC == 64, "pixel tile must hold 64 pixels");
    static_assert(KC % 4 == 0, "KC must be a multiple of 4");
    static_assert((KC / 2) % 4 != 0 || KCP % 4 == 0, "b128 operand reads need 16-byte pixel stride");
    static_assert(S == 1 || S == 2, "stride 1 or 2");
};

constexpr int cmax(int a, int b) { return a > b ? a : b; }

// base + a 32-bit byte offset: a uniform base and a per-lane offset map to
// the scalar-base global load form (no 64-bit address arithmetic per lane)
template <class T>
__device__ __forceinline__ const LAMA_GLOBAL T *at_byte(const LAMA_GLOBAL float *base, unsigned off)
{
    return reinterpret_cast<const LAMA_GLOBAL T *>(reinterpret_cast<const LAMA_GLOBAL char *>(base) + off);
}

// Per-thread staging addresses, fixed for a block: each chunk only adds its
// channel / K offset.  Staging is branch-free (a divergent branch around a
// load makes the compiler wait for every outstanding load, which would
// serialise the prefetch): rows past M and channels past C read clamped, valid
// addresses (their weights are zero or their outputs are dropped), positions
// outside the plane of a transposed-convolution phase are zeroed by a select,
// and slots past the tile are written to a dummy LDS tail.
template <class C>
struct Slots {
    int wg[C::WITER];  // weights: float offset of the float4 within the rows
    int wl[C::WITER];  // weights: LDS float offset
    unsigned po[C::PITER];  // patch: byte offset from the chunk's first plane (channel * plane + position)
    int pl[C::PITER];       // patch: LDS float offset
    int pc[C::PITER];       // patch: channel within the chunk; < 0 marks a zero slot
};

template <class C>
__device__ __forceinline__ void make_wslots(Slots<C> &sl, const ConvSeg &sg, int m0, int M)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        const int row = idx / (C::WK / 4), c4 = idx % (C::WK / 4);
        const bool in = idx < C::W4;
        sl.wl[it] = in ? row * C::WSTR + c4 * 4 : 64 * C::WSTR + (idx & 63) * 4;
        sl.wg[it] = in ? min(m0 + row, M - 1) * sg.wrow + c4 * 4 : 0;
    }
}

// Patch slots of the tile at (oy0, ox0); the LDS side (pl) does not depend on
// the tile.
template <class C>
__device__ __forceinline__ void make_pslots(Slots<C> &sl, const ConvSeg &sg, int oy0, int ox0)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < C::PITER; ++it) {
        const int idx = tid + it * LAMA_NT;
        const int q = idx >> 6, l = idx & 63;  // 64-slot group: 16 pixels x 4 channels
        const int cl = (q % (C::KC / 4)) * 4 + (l >> 4);
        const int pix = (q / (C::KC / 4)) * 16 + (l & 15);
        const int r = min(pix, C::NPIX - 1) / C::PC, c = min(pix, C::NPIX - 1) - r * C::PC;
        const int iy = oy0 * C::S - C::PAD + r, ix = ox0 * C::S - C::PAD + c;
        const bool in = idx < C::P_SLOTS && pix < C::NPIX;
        bool zero = false;
        int g;
        if (C::REFLECT) {
            g = reflect1(iy, sg.IH) * sg.IW + reflect1(ix, sg.IW);
        } else {
            zero = !(iy >= 0 && ix >= 0 && iy < sg.IH && ix < sg.IW);
            g = zero ? 0 : iy * sg.IW + ix;
        }
        sl.pl[it] = in ? (r * C::PCP + C::col(c)) * C::KCP + cl : C::PR * C::PCP * C::KCP + l;
        sl.po[it] = 4u * (unsigned)(min(cl, C::KC - 1) * sg.cs + g);
        sl.pc[it] = (in && !zero) ? cl : -1;
    }
}

template <class C>
__device__ __forceinline__ void make_slots(Slots<C> &sl, const ConvSeg &sg, int m0, int M, int oy0, int ox0)
{
    make_wslots<C>(sl, sg, m0, M);
    make_pslots<C>(sl, sg, oy0, ox0);
}

// Registers holding one chunk on its way from global memory to LDS.
template <class C>
struct Stage {
    float w[4 * C::WITER];
    float p[C::PITER];
};

// Issue the global loads of chunk `ck`: weights, then the input patch.
template <class C>
__device__ __forceinline__ void load_w(Stage<C> &st, const Slots<C> &sl, const ConvSeg &sg, int ck)
{
    const LAMA_GLOBAL float *wt = gp(sg.wt) + (long)ck * C::WK;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const float4 v = *at_byte<float4>(wt, 4u * (unsigned)sl.wg[it]);
        st.w[4 * it] = v.x;
        st.w[4 * it + 1] = v.y;
        st.w[4 * it + 2] = v.z;
        st.w[4 * it + 3] = v.w;
    }
}

template <class C>
__device__ __forceinline__ void load_p(Stage<C> &st, const Slots<C> &sl, const ConvSeg &sg, int ck)
{
    // 32-bit byte offsets from the chunk's first plane (below 4 * KC * cs,
    // which the host bounds); slots of channels past C (zero weights) read the
    // last float of the source instead
    const unsigned plane = (unsigned)(sg.IH * sg.IW), cs = (unsigned)sg.cs;
    const int c0 = ck * C::KC;
    const unsigned last = 4u * ((unsigned)(min(sg.C - c0, C::KC) - 1) * cs + plane - 1u);
    const LAMA_GLOBAL float *src = gp(sg.src) + (long)c0 * cs;
#pragma unroll
    for (int it = 0; it < C::PITER; ++it) {
        const float v = *at_byte<float>(src, min(sl.po[it], last));
        st.p[it] = sl.pc[it] >= 0 ? v : 0.f;
    }
}

template <class C>
__device__ __forceinline__ void load_chunk(Stage<C> &st, const Slots<C> &sl, const ConvSeg &sg, int ck)
{
    load_w<C>(st, sl, sg, ck);
    load_p<C>(st, sl, sg, ck);
}

template <class C>
__device__ __forceinline__ void store_w(const Stage<C> &st, const Slots<C> &sl, float *wl)
{
#pragma unroll
    for (int it = 0; it < C::WITER; ++it)
        *reinterpret_cast<float4 *>(wl + sl.wl[it]) =
            make_float4(st.w[4 * it], st.w[4 * it + 1], st.w[4 * it + 2], st.w[4 * it + 3]);
}

template <class C>
__device__ __forceinline__ void store_p(const Stage<C> &st, const Slots<C> &sl, float *pl)
{
#pragma unroll
    for (int it = 0; it < C::PITER; ++it) pl[sl.pl[it]] = st.p[it];
}

template <class C>
__device__ __forceinline__ void store_chunk(const Stage<C> &st, const Slots<C> &sl, float *wl, float *pl)
{
    store_w<C>(st, sl, wl);
    store_p<C>(st, sl, pl);
}

template <int N>
__device__ __forceinline__ void lds_vec(float (&a)[N], const float *p)
{
    static_assert(N % 2 == 0, "vector of 2 or 4k floats");
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
            float4 v = *reinterpret_cast<const float4 *>(p + 4 * q);
            a[4 * q] = v.x;
            a[4 * q + 1] = v.y;
            a[4 * q + 2] = v.z;
            a[4 * q + 3] = v.w;
        }
    } else {
        float2 v = *reinterpret_cast<const float2 *>(p);
        a[0] = v.x;
        a[1] = v.y;
    }
}

// MFMAs of one chunk.  Both operands of a tap are KC/2 consecutive floats per
// lane (weights [co][tap][ci], patch [pixel][ci]); the reads of tap t+1 are
// issued before the MFMAs of tap t.
template <class C>
__device__ __forceinline__ void compute_chunk(f32x16 &acc, const float *wl, const float *pl)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int pr = p / C::TC, pc = p % C::TC;
    const float *wrow = wl + (wm * 32 + j) * C::WSTR + g * (C::KC / 2);
    const float *prow = pl + ((pr * C::S) * C::PCP + C::col(pc * C::S)) * C::KCP + g * (C::KC / 2);
    constexpr int H = C::KC / 2;
    float a[2][H], b[2][H];
    lds_vec<H>(a[0], wrow);
    lds_vec<H>(b[0], prow);
#pragma unroll
    for (int t = 0; t < C::T; ++t) {
        const int cur = t & 1;
        if (t + 1 < C::T) {
            const int ky = (t + 1) / C::KW, kx = (t + 1) % C::KW;
            lds_vec<H>(a[cur ^ 1], wrow + (t + 1) * C::KC);
            lds_vec<H>(b[cur ^ 1], prow + (ky * C::PCP + C::col(kx)) * C::KCP);
        }
#pragma unroll
        for (int c = 0; c < H; ++c) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[cur][c], b[cur][c], acc, 0, 0, 0);
    }
}

// Taps of a lama_convt_rows workgroup (row phase py: output rows 2m+py, both
// column phases): tap t reads the window offset (dy, dx) and feeds the
// accumulator of column phase px.  py = 0: phase (0,0) at (0,0); phase
// (0,1) at (0,0), (0,1).  py = 1: phase (1,0) at (0,0), (1,0); phase (1,1)
// at (0,0), (0,1), (1,0), (1,1).  The weights are packed in this order.
__device__ __forceinline__ constexpr int rows_tap_dy(int py, int t) { return py ? (t == 1 || t >= 4 ? 1 : 0) : 0; }
__device__ __forceinline__ constexpr int rows_tap_dx(int py, int t)
{
    return py ? (t == 3 || t == 5 ? 1 : 0) : (t == 2 ? 1 : 0);
}
__device__ __forceinline__ constexpr int rows_tap_px(int py, int t) { return py ? (t >= 2 ? 1 : 0) : (t >= 1 ? 1 : 0); }

struct RowsAcc {
    f32x16 a[2];  // column phases 0 and 1
};

// MFMAs of one chunk of a lama_convt_rows workgroup: as compute_chunk, with
// each tap into its column phase's accumulator.
template <class C>
__device__ __forceinline__ void compute_chunk(RowsAcc &acc, const float *wl, const float *pl)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int pr = p / C::TC, pc = p % C::TC;
    const float *wrow = wl + (wm * 32 + j) * C::WSTR + g * (C::KC / 2);
    const float *prow = pl + (pr * C::PCP + pc) * C::KCP + g * (C::KC / 2);
    constexpr int H = C::KC / 2;
    float a[2][H], b[2][H];
    lds_vec<H>(a[0], wrow);
    lds_vec<H>(b[0], prow + (rows_tap_dy(C::PY, 0) * C::PCP + rows_tap_dx(C::PY, 0)) * C::KCP);
#pragma unroll
    for (int t = 0; t < C::T; ++t) {
        const int cur = t & 1;
        if (t + 1 < C::T) {
            lds_vec<H>(a[cur ^ 1], wrow + (t + 1) * C::KC);
            lds_vec<H>(b[cur ^ 1],
                       prow + (rows_tap_dy(C::PY, t + 1) * C::PCP + rows_tap_dx(C::PY, t + 1)) * C::KCP);
        }
        const int px = rows_tap_px(C::PY, t);
#pragma unroll
        for (int c = 0; c < H; ++c)
            acc.a[px] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[cur][c], b[cur][c], acc.a[px], 0, 0, 0);
    }
}

// K loop of one segment.  NBUF = 2: two LDS stages and two register stages,
// one barrier per chunk.  Chunk k's global loads are issued two chunks ahead
// (during chunk k-2's MFMAs), written to LDS after chunk k-1's MFMAs and
// consumed at step k, so each load has two chunks of MFMA time to land.
// NBUF = 1 (single-chunk segments such as the 4-channel head) stages once.
template <class C, int NBUF, class Acc>
__device__ __forceinline__ void run_segment(Acc &acc, const ConvSeg &sg_mem, int m0, int M, int oy0, int ox0,
                                            float *lds)
{
    // a register copy: the barriers of the loop would otherwise make the
    // compiler re-read the descriptor from memory every chunk
    const ConvSeg sg = sg_mem;
    const int n = sg.nchunk;
    if (n <= 0) return;
    Slots<C> sl;
    make_slots<C>(sl, sg, m0, M, oy0, ox0);
    if constexpr (NBUF == 1) {
        Stage<C> st;
        for (int ck = 0; ck < n; ++ck) {
            load_chunk<C>(st, sl, sg, ck);
            __syncthreads();
            store_chunk<C>(st, sl, lds, lds + C::W_LDS);
            __syncthreads();
            compute_chunk<C>(acc, lds, lds + C::W_LDS);
        }
    } else {
        // prefetches past the last chunk re-read it (uniform control flow)
        float *l0 = lds, *l1 = lds + C::LDS;
        const int last = n - 1;
        Stage<C> r0, r1;
        load_chunk<C>(r0, sl, sg, 0);
        load_chunk<C>(r1, sl, sg, min(1, last));
        store_chunk<C>(r0, sl, l0, l0 + C::W_LDS);
        load_chunk<C>(r0, sl, sg, min(2, last));
        __syncthreads();
        // one exit: a break between the two steps made the compiler copy the
        // accumulators every iteration (and hold two sets of them)
        int ck = 0;
        for (; ck + 1 < n; ck += 2) {
            // even step: compute stage 0, stage chunk ck+1 (r1), refill r1 with ck+3
            compute_chunk<C>(acc, l0, l0 + C::W_LDS);
            store_chunk<C>(r1, sl, l1, l1 + C::W_LDS);
            load_chunk<C>(r1, sl, sg, min(ck + 3, last));
            __syncthreads();
            // odd step: compute stage 1, stage chunk ck+2 (r0), refill r0 with ck+4
            compute_chunk<C>(acc, l1, l1 + C::W_LDS);
            store_chunk<C>(r0, sl, l0, l0 + C::W_LDS);
            load_chunk<C>(r0, sl, sg, min(ck + 4, last));
            __syncthreads();
        }
        if (ck < n) {  // an odd count: the last chunk is in stage 0
            compute_chunk<C>(acc, l0, l0 + C::W_LDS);
            __syncthreads();
        }
    }
}

// Pointwise (1x1) convolution over flat planes of N pixels: 64 output
// channels x NPX pixels per block (NPX = 64 or 128), 4 waves, the two-stage
// pipeline of run_segment.  Wave (wm, wn) owns channels wm*32.. +32 and pixels
// wn*NPX/2 .. +NPX/2 as NACC = NPX/64 accumulators of 32 pixels.  The
// activations are staged channel-major, [KC][NPX], as they lie in memory:
// every thread moves whole runs of 4 pixels (one 16-byte global load and one
// 16-byte LDS store, no transpose), and each MFMA's B operand is one 4-byte
// LDS read per lane: lane half g reads 32 consecutive pixels of channel
// g*KC/2 + c.  The two halves' rows sit in separate regions whose bases
// differ by 32 banks.  Channel planes lie cs floats apart.  VW = 4: planes
// 16-byte aligned with cs % 4 == 0 (one float4 load per run; the last run of
// a plane may cover up to 3 floats of padding past N, which only feed the
// unstored columns past N); VW = 2: 8-byte aligned with N % 2 == 0, cs even
// and N >= 4 (two float2 loads); VW = 1: four clamped scalar loads.
// KH (K halves, NPX = 32): wave (wm, kh) takes channels wm*32.. +32, all 32
// pixels, and half of every chunk's K slots (kh = wave & 1); the two halves'
// sums meet in LDS after the K loop.  Half the dependent MFMA chain per wave
// and twice the workgroups of a 64-pixel tile, for the conv2 launch, which
// runs nearly alone on the FFC's critical path.
template <int KC_, int VW_, int NPX_, bool KH_ = false>
struct PwCfg {
    static constexpr int VW = VW_;  // activation load width: float4, float2 or scalar
    static constexpr bool VEC = VW_ > 1;
    static constexpr bool KH = KH_;
    static constexpr int KC = KC_, NPX = NPX_, NACC = KH ? 1 : NPX / 64;
    static constexpr int WSTR = KC + 4;              // weight row stride, = 4 (mod 8)
    static constexpr int HALF = KC / 2 * NPX + 32;   // one lane half's channel rows
    static constexpr int W_LDS = 64 * WSTR;
    static constexpr int LDS = W_LDS + 2 * HALF;
    static constexpr int WITER = 64 * KC / 4 / LAMA_NT;   // weight float4s per thread
    static constexpr int XITER = KC * NPX / 4 / LAMA_NT;  // activation runs per thread
    static_assert(KH ? NPX == 32 && KC % 16 == 0 : NPX == 64 || NPX == 128, "64 or 128 pixels per tile, 32 with KH");
    static_assert(WITER * LAMA_NT * 4 == 64 * KC && XITER * LAMA_NT * 4 == KC * NPX, "whole float4 slots");
    static_assert(KC % 8 == 0 && WSTR % 8 == 4 && HALF % 64 == 32, "bank placement");
};

template <class C>
struct PwSlots {
    int wg[C::WITER], wl[C::WITER];                // weights: global float offset in the row, LDS offset
    int xc[C::XITER], xp[C::XITER], xl[C::XITER];  // activations: channel in chunk, first pixel, LDS offset
    unsigned xo[C::XITER];                         // VEC: byte offset from the chunk's first plane
};

template <class C>
struct PwStage {
    float w[4 * C::WITER];
    float x[4 * C::XITER];
};

template <class C>
__device__ __forceinline__ void pw_make_slots(PwSlots<C> &sl, const ConvSeg &sg, int m0, int M, int ox0)
{
    const int tid = threadIdx.x, N = sg.IH * sg.IW, N4 = (N + 3) & ~3;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const int idx = tid + it * LAMA_NT, row = idx / (C::KC / 4), c4 = idx % (C::KC / 4);
        sl.wl[it] = row * C::WSTR + c4 * 4;
        sl.wg[it] = min(m0 + row, M - 1) * sg.wrow + c4 * 4;
    }
#pragma unroll
    for (int it = 0; it < C::XITER; ++it) {
        const int idx = tid + it * LAMA_NT, ci = idx / (C::NPX / 4), q = idx % (C::NPX / 4);
        sl.xc[it] = ci;
        sl.xl[it] = (ci / (C::KC / 2)) * C::HALF + (ci % (C::KC / 2)) * C::NPX + 4 * q;
        // VW = 4 (cs % 4 == 0): runs past the plane read the last whole run
        // of the padded plane (its pixels past N feed only the tile columns
        // past N, which are not stored); else clamp per float2 pair / element
        sl.xp[it] = C::VW == 4 ? min(ox0 + 4 * q, N4 - 4) : ox0 + 4 * q;
        sl.xo[it] = 4u * (unsigned)(ci * sg.cs + sl.xp[it]);
    }
}

template <class C>
__device__ __forceinline__ void pw_load_chunk(PwStage<C> &st, const PwSlots<C> &sl, const ConvSeg &sg, int ck)
{
    const LAMA_GLOBAL float *wt = gp(sg.wt) + (long)ck * C::KC;
#pragma unroll
    for (int it = 0; it < C::WITER; ++it) {
        const float4 v = *at_byte<float4>(wt, 4u * (unsigned)sl.wg[it]);
        st.w[4 * it] = v.x;
        st.w[4 * it + 1] = v.y;
        st.w[4 * it + 2] = v.z;
        st.w[4 * it + 3] = v.w;
    }
    const int N = sg.IH * sg.IW, cs = sg.cs;
    const int c0 = ck * C::KC, clast = sg.C - 1 - c0;  // channels past C read a valid plane (zero weights)
    const LAMA_GLOBAL float *src = gp(sg.src) + (long)c0 * cs;
    // VEC: runs of channels past C (zero weights) read the last valid
    // channel's last run (VW = 4: of the plane padded to a multiple of 4)
    const unsigned vlast =
        4u * ((unsigned)(min(sg.C - c0, C::KC) - 1) * (unsigned)cs + (unsigned)(C::VW == 4 ? (N + 3) & ~3 : N) - 4u);
#pragma unroll
    for (int it = 0; it < C::XITER; ++it) {
        if constexpr (C::VW == 4) {
            const float4 v = *at_byte<float4>(src, min(sl.xo[it], vlast));
            st.x[4 * it] = v.x;
            st.x[4 * it + 1] = v.y;
            st.x[4 * it + 2] = v.z;
            st.x[4 * it + 3] = v.w;
        } else if constexpr (C::VW == 2) {
            // each pair clamped to the last pair: a run starting at N - 2 keeps
            // its two valid pixels in place
            const unsigned plast = vlast + 8u;
            const float2 a = *at_byte<float2>(src, min(sl.xo[it], plast));
            const float2 b = *at_byte<float2>(src, min(sl.xo[it] + 8u, plast));
            st.x[4 * it] = a.x;
            st.x[4 * it + 1] = a.y;
            st.x[4 * it + 2] = b.x;
            st.x[4 * it + 3] = b.y;
        } else {
            const LAMA_GLOBAL float *q = src + (long)min(sl.xc[it], clast) * cs;
#pragma unroll
            for (int e = 0; e < 4; ++e) st.x[4 * it + e] = q[min(sl.xp[it] + e, N - 1)];
        }
    }
}

template <class C>
__device__ __forceinline__ void pw_store_chunk(const PwStage<C> &st, const PwSlots<C> &sl, float *lds)
{
#pragma unroll
    for (int it = 0; it < C::WITER; ++it)
        *reinterpret_cast<float4 *>(lds + sl.wl[it]) =
            make_float4(st.w[4 * it], st.w[4 * it + 1], st.w[4 * it + 2], st.w[4 * it + 3]);
#pragma unroll
    for (int it = 0; it < C::XITER; ++it)
        *reinterpret_cast<float4 *>(lds + C::W_LDS + sl.xl[it]) =
            make_float4(st.x[4 * it], st.x[4 * it + 1], st.x[4 * it + 2], st.x[4 * it + 3]);
}

template <class C>
__device__ __forceinline__ void pw_compute_chunk(f32x16 (&acc)[C::NACC], const float *lds)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    constexpr int H = C::KC / 2;
    if constexpr (C::KH) {
        // K slots g * H + wn * H/2 + c of the chunk (c < H/2): this wave's half
        constexpr int HH = H / 2;
        const float *wrow = lds + (wm * 32 + j) * C::WSTR + g * H + wn * HH;
        const float *xrow = lds + C::W_LDS + g * C::HALF + wn * HH * C::NPX + j;
        float a[HH], b[HH];
        lds_vec<HH>(a, wrow);
#pragma unroll
        for (int c = 0; c < HH; ++c) b[c] = xrow[c * C::NPX];
#pragma unroll
        for (int c = 0; c < HH; ++c) acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[c], b[c], acc[0], 0, 0, 0);
        return;
    }
    const float *wrow = lds + (wm * 32 + j) * C::WSTR + g * H;
    const float *xrow = lds + C::W_LDS + g * C::HALF + wn * (C::NPX / 2) + j;
    float a[H];
    lds_vec<H>(a, wrow);
#pragma unroll
    for (int h = 0; h < C::NACC; ++h) {
        float b[H];
#pragma unroll
        for (int c = 0; c < H; ++c) b[c] = xrow[c * C::NPX + h * 32];
#pragma unroll
        for (int c = 0; c < H; ++c) acc[h] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[c], b[c], acc[h], 0, 0, 0);
    }
}

// The K loop of a pointwise segment: two LDS stages and D register stages,
// one barrier per chunk.  Chunk c's global loads are issued D steps before it
// is written to LDS (at step c - 1) and consumed at step c, so each load has
// D chunks of MFMA time to land; these small-K GEMMs run one wave per SIMD
// and are bound by that latency.  A depth that divides the chunk counts (12
// and 24 at 16 channels) keeps the unrolled group free of early exits.  Depth
// 2 (fewer staging registers) measured fastest beside the direct-weight
// F(4,3) GEMM: 263.8 vs 262.9 (depth 4) passes/s at 512x512, 162.2 vs 161.0
// at 600x600.
#ifndef LAMA_PW_DEPTH
#define LAMA_PW_DEPTH 2
#endif
template <class C, int D>
__device__ __forceinline__ void run_segment_pw(f32x16 (&acc)[C::NACC], const ConvSeg &sg_mem, int m0, int M, int ox0,
                                               float *lds)
{
    const ConvSeg sg = sg_mem;  // held in registers across the barriers
    const int n = sg.nchunk;
    if (n <= 0) return;
    PwSlots<C> sl;
    pw_make_slots<C>(sl, sg, m0, M, ox0);
    float *l0 = lds, *l1 = lds + C::LDS;
    const int last = n - 1;
    // prefetches past the last chunk re-read it (uniform control flow)
    PwStage<C> r[D];
#pragma unroll
    for (int d = 0; d < D; ++d) pw_load_chunk<C>(r[d], sl, sg, min(d, last));
    pw_store_chunk<C>(r[0], sl, l0);
    pw_load_chunk<C>(r[0], sl, sg, min(D, last));
    __syncthreads();
    for (int ck = 0; ck < n; ck += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int k = ck + j;
            if (j > 0 && k >= n) break;
            pw_compute_chunk<C>(acc, (k & 1) ? l1 : l0);
            pw_store_chunk<C>(r[(j + 1) % D], sl, (k & 1) ? l0 : l1);
            pw_load_chunk<C>(r[(j + 1) % D], sl, sg, min(k + 1 + D, last));
            __syncthreads();
        }
    }
}

// Epilogue operands read from memory (addend, residual) are fetched before
// the K loop so their latency hides behind it.
struct EpiPre {
    float add[16], res[16];
};

template <int TR, int TC>
__device__ __forceinline__ void epilogue_prefetch(EpiPre &e, const ConvProblem &P, int m0, int oy0, int ox0)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int oy = min(oy0 + p / TC, P.OH - 1), ox = min(ox0 + p % TC, P.OW - 1);
    const long pix = (long)(oy * P.oy_mul + P.oy_off) * P.outW + (long)ox * P.ox_mul + P.ox_off;
    long o[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int co = min(m0 + wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3), P.M - 1);
        o[r] = (long)co * P.out_cstride + pix;
        e.res[r] = P.res ? gp(P.res)[o[r]] : 0.f;
        e.add[r] = 0.f;
    }
    // the addend's K slices, summed in order (uniform guards: one slice's 16
    // loads in flight at a time, 16 registers beyond the sums)
#pragma unroll
    for (int i = 0; i < LAMA_KSPLIT_MAX; ++i) {
        if (i >= P.naddend) break;
#pragma unroll
        for (int r = 0; r < 16; ++r) e.add[r] += gp(P.addend)[o[r] + i * P.addend_kstride];
    }
}

// Per-channel epilogue operands (bias, BN scale, BN shift) of the block's 64
// output channels: one value per thread for threads 0..191, loaded into a
// register before the K loop and parked in LDS after it, so the epilogue
// reads them from LDS instead of making dependent global round trips after
// its first store (which the compiler may not reorder loads above).
__device__ __forceinline__ float epi_param_load(const ConvProblem &P, int m0)
{
    const int t = threadIdx.x, row = t >> 6, c = min(m0 + (t & 63), P.M - 1);
    if (t >= 192) return 0.f;
    if (row == 0) return P.bias ? gp(P.bias)[c] : 0.f;
    if (row == 1) return P.scale ? gp(P.scale)[c] : 1.f;
    return P.scale ? gp(P.shift)[c] : 0.f;
}

template <int TR, int TC, bool PREFETCH>
__device__ __forceinline__ void epilogue(const f32x16 &acc, const EpiPre &e, const ConvProblem &P, const float *epl,
                                         int m0, int oy0, int ox0, long obase = 0)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int oy = oy0 + p / TC, ox = ox0 + p % TC;
    if (oy >= P.OH || ox >= P.OW) return;
    const long pix = (long)(oy * P.oy_mul + P.oy_off) * P.outW + (long)ox * P.ox_mul + P.ox_off;
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int cl = wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const long o = (long)min(m0 + cl, P.M - 1) * P.out_cstride + pix;
        float x = acc[r];
        if (P.bias) x += epl[cl];
        if (PREFETCH)
            x += e.add[r];
        else
            for (int i = 0; i < P.naddend; ++i) x += gp(P.addend)[o + i * P.addend_kstride];
        if (P.scale) x = x * epl[64 + cl] + epl[128 + cl];
        if (P.relu) x = fmaxf(x, 0.f);
        if (PREFETCH)
            x += e.res[r];
        else if (P.res)
            x += gp(P.res)[o];
        v[r] = x;
    }
    LAMA_GLOBAL float *out = gp(P.out) + obase;
    const int cbase = m0 + wm * 32 + 4 * g;
    if (m0 + 64 <= P.M) {
#pragma unroll
        for (int r = 0; r < 16; ++r) out[(long)(cbase + 8 * (r >> 2) + (r & 3)) * P.out_cstride + pix] = v[r];
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = cbase + 8 * (r >> 2) + (r & 3);
            if (co < P.M) out[(long)co * P.out_cstride + pix] = v[r];
        }
    }
}

// One 64 x 64 output tile of problem P: segment 0 with the template
// geometry, then (SEG1) the optional 1x1 segment over a second source.
template <class C0, bool SEG1, int NBUF = 2, bool PREFETCH = false>
__device__ __forceinline__ void conv_tile(const ConvProblem &P, int b, float *lds, float *epl)
{
    const int mb = b % P.mblocks, t = b / P.mblocks;
    const int tx = t % P.tiles_x, ty = t / P.tiles_x;
    const int m0 = mb * 64, oy0 = ty * C0::TR, ox0 = tx * C0::TC;
    const float ep = epi_param_load(P, m0);
    EpiPre pre;
    if constexpr (PREFETCH) {
        epilogue_prefetch<C0::TR, C0::TC>(pre, P, m0, oy0, ox0);
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) pre.add[r] = pre.res[r] = 0.f;
    }
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    run_segment<C0, NBUF>(acc, P.s0, m0, P.M, oy0, ox0, lds);
    if constexpr (SEG1) {
        using C1 = Cfg<1, 1, 1, false, C0::KC, C0::TR, C0::TC>;
        if (P.s1.nchunk > 0) run_segment<C1, NBUF>(acc, P.s1, m0, P.M, oy0, ox0, lds);
    }
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
    epilogue<C0::TR, C0::TC, PREFETCH>(acc, pre, P, epl, m0, oy0, ox0);
}

// One 64 x NPX tile of a pointwise problem (a flat plane: OH == 1).  The
// epilogue runs once per 32-pixel accumulator; shifting its tile origin by
// wn*(NPX/2 - 32) + h*32 places accumulator h of wave column wn.
//
// K split (P.ksplit > 1, from the host for small planes whose tiles leave
// most CUs idle): the blocks of slice ks follow those of ks - 1; slice ks
// walks input channels [ks * kchunks * KC, + kchunks * KC) and stores its raw
// partial at out + ks * out_kstride (the host clears bias, BN, ReLU, addends
// and residual; the consumer sums the partials and applies them).
template <class C, bool PREFETCH, int D>
__device__ __forceinline__ void pw_tile(const ConvProblem &P, int b, float *lds, float *epl)
{
    int ks = 0;
    if (P.ksplit > 1) {
        const int per = P.mblocks * P.tiles_x;
        ks = b / per;
        b -= ks * per;
    }
    int mb = b % P.mblocks, t = b / P.mblocks;
#if LAMA_PW_XCD
    // XCD-aware order: workgroups are dealt to the eight XCDs round-robin
    // (XCD = blockIdx.x mod 8, here b, the launch's only problem), and each
    // XCD has an L2 of its own; giving all M blocks of pixel strip t to XCD
    // t mod 8 makes each strip travel from HBM into one L2 once, instead of
    // once per M block.  The host opts in by sizing the grid for the strips
    // rounded up to a multiple of 8; blocks of the padding strips return
    // (the whole workgroup, before any barrier).
    if (P.ksplit <= 1 && P.nblocks == (P.tiles_x + 7) / 8 * 8 * P.mblocks) {
        const int j = b >> 3;
        mb = j % P.mblocks;
        t = (j / P.mblocks) * 8 + (b & 7);
        if (t >= P.tiles_x) return;
    }
#endif
    const int m0 = mb * 64, ox0 = t * C::NPX;
    const int wn = (threadIdx.x >> 6) & 1;
    const float ep = epi_param_load(P, m0);
    EpiPre pre[C::NACC];
#pragma unroll
    for (int h = 0; h < C::NACC; ++h) {
        if constexpr (PREFETCH && C::KH) {
            if (wn == 0) epilogue_prefetch<1, 32>(pre[h], P, m0, 0, ox0);  // the K-half that stores
        } else if constexpr (PREFETCH) {
            epilogue_prefetch<1, 64>(pre[h], P, m0, 0, ox0 + wn * (C::NPX / 2 - 32) + h * 32);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) pre[h].add[r] = pre[h].res[r] = 0.f;
        }
    }
    f32x16 acc[C::NACC];
#pragma unroll
    for (int h = 0; h < C::NACC; ++h)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[h][r] = 0.f;
    ConvSeg sg = P.s0;
    if (P.ksplit > 1) {
        const int c0 = ks * P.kchunks * C::KC;
        sg.src += (long)c0 * sg.cs;
        sg.wt += c0;  // 1x1 rows: chunk k at k * KC floats
        sg.C -= c0;
        sg.nchunk = P.kchunks;
    }
    run_segment_pw<C, D>(acc, sg, m0, P.M, ox0, lds);
    if constexpr (C::KH) {
        // K half 1 hands its sums to half 0 (the staging buffers are free
        // after the K loop's last barrier), which runs the epilogue
        const int lane = threadIdx.x & 63, wm = threadIdx.x >> 7;
        float *xs = lds + wm * 16 * 64 + lane;
        if (wn == 1)
#pragma unroll
            for (int r = 0; r < 16; ++r) xs[r * 64] = acc[0][r];
        if (threadIdx.x < 192) epl[threadIdx.x] = ep;
        __syncthreads();
        if (wn == 1) return;  // no barrier follows
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][r] += xs[r * 64];
        epilogue<1, 32, PREFETCH>(acc[0], pre[0], P, epl, m0, 0, ox0, (long)ks * P.out_kstride);
        return;
    }
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
#pragma unroll
    for (int h = 0; h < C::NACC; ++h)
        epilogue<1, 64, PREFETCH>(acc[h], pre[h], P, epl, m0, 0, ox0 + wn * (C::NPX / 2 - 32) + h * 32,
                                  (long)ks * P.out_kstride);
}

// Problem index of workgroup b, and b made relative to that problem's first
// workgroup.  Selects over the (already loaded) starts, not an indexed read,
// which would be one more dependent scalar load at the head of the prologue.
__device__ __forceinline__ int find_problem(const ProbStarts &ps, int &b)
{
    int pi = 0, start = 0;
#pragma unroll
    for (int i = 0; i < LAMA_MAX_PROBS - 1; ++i) {
        const bool in = b >= ps.s[i];
        pi += in;
        start = in ? ps.s[i] : start;
    }
    b -= start;
    return pi;
}

// Parameters of every conv kernel: the problem table and the first workgroup
// of problems 1..3 as separate scalars, so all of them are preloaded into
// SGPRs with the dispatch (-amdgpu-kernarg-preload-count) instead of being
// fetched from the kernarg segment at the head of the prologue.  `stamp`
// (null unless the launch is profiled) receives the workgroup's start and end
// on the constant-rate device clock (s_memrealtime), written by thread 0 to
// stamp[2 * blockIdx.x] and stamp[2 * blockIdx.x + 1] with ordinary vector
// stores: the host takes the launch's duration as the last end minus the
// first start, the window a kernel trace reports.
#define LAMA_CONV_PARAMS \
    const ConvProblem *__restrict__ probs, int ps1, int ps2, int ps3, unsigned long long *__restrict__ stamp
#define LAMA_CONV_STARTS const ProbStarts ps{0, {ps1, ps2, ps3}}
#define LAMA_STAMP_BEGIN const unsigned long long stamp_t0 = stamp ? __builtin_amdgcn_s_memrealtime() : 0ull
#define LAMA_STAMP_END                                                      \
    do {                                                                    \
        if (stamp && threadIdx.x == 0) {                                    \
            stamp[2 * blockIdx.x] = stamp_t0;                               \
            stamp[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();  \
        }                                                                   \
    } while (0)

using CfgHead = Cfg<7, 7, 1, true, 4, 2, 32>;
using CfgFfc = Cfg<3, 3, 1, true, 8, 2, 32>;
using CfgFfc1 = Cfg<1, 1, 1, false, 8, 2, 32>;
// The stride-2 and transposed convolutions also come in 4 x 16-pixel tiles
// (the _q kernels), for planes whose width leaves much of a 32-pixel tile
// row empty (75 wide: 3 x 32 columns hold 78% of the tile, 5 x 16 hold 94%).
template <int TR, int TC>
using CfgDownT = Cfg<3, 3, 2, true, LAMA_S2_KC, TR, TC>;
template <int TR, int TC>
struct CfgT {
    using P00 = Cfg<1, 1, 1, false, LAMA_CONVT_KC0, TR, TC>;
    using P01 = Cfg<1, 2, 1, false, LAMA_CONVT_KC1, TR, TC>;
    using P10 = Cfg<2, 1, 1, false, LAMA_CONVT_KC2, TR, TC>;
    using P11 = Cfg<2, 2, 1, false, LAMA_CONVT_KC3, TR, TC>;
    static constexpr int LDS = cmax(cmax(P00::LDS, P01::LDS), cmax(P10::LDS, P11::LDS));
};

// The transposed convolution by row phase (lama_convt_rows): a workgroup
// computes both column phases of output rows 2m+py for 64 channels x TR x TC
// input positions, through a (1+py) x 2 window over a (TR+py) x (TC+1)
// patch -- 3 taps for py = 0, 6 for py = 1 (rows_tap_*).  Each lane then
// holds output pixels 2n and 2n+1 of a row and stores them as one float2,
// so every output line is written whole by one workgroup.  The staging
// members follow Cfg, so the slot and stage code is shared.
template <int PY_, int TR_, int TC_>
struct CfgRows {
    static constexpr int PY = PY_, KH = 1 + PY_, KW = 2, S = 1, TR = TR_, TC = TC_, T = PY_ ? 6 : 3, PAD = 0;
    static constexpr int KC = PY_ ? LAMA_CONVT_ROWS_KC1 : LAMA_CONVT_ROWS_KC0;
    static constexpr bool REFLECT = false;
    static constexpr int PR = TR + PY, PC = TC + 1, PCP = PC;
    static constexpr int WK = T * KC;
    static constexpr int WSTR = WK + ((12 - WK % 8) % 8);
    static constexpr int KCP = (KC / 2) % 4 == 0 ? KC + 4 : KC + 2;  // as Cfg
    static __device__ __forceinline__ constexpr int col(int c) { return c; }
    static constexpr int W4 = 64 * WK / 4;
    static constexpr int WITER = (W4 + LAMA_NT - 1) / LAMA_NT;
    static constexpr int NPIX = PR * PC;
    static constexpr int NPB = (NPIX + 15) / 16;
    static constexpr int P_SLOTS = NPB * 16 * KC;
    static constexpr int PITER = (P_SLOTS + LAMA_NT - 1) / LAMA_NT;
    static constexpr int W_LDS = 64 * WSTR + (WITER * LAMA_NT > W4 ? 64 * 4 : 0);  // as Cfg
    static constexpr int P_LDS = PR * PCP * KCP + 64;
    static constexpr int LDS = W_LDS + P_LDS;
    static_assert(TR * TC == 64, "pixel tile must hold 64 positions");
    static_assert(KC % 4 == 0, "KC must be a multiple of 4");
};

}  // namespace

// model.1: 7x7, reflect pad 3 (the ReflectionPad2d(3) + valid 7x7 of the
// reference), 4 -> 64, BN + ReLU.  K = 4 x 49 is one chunk, so the 64 x 196
// weights (53 KB) would be re-fetched by every tile; instead each workgroup
// keeps them in LDS and walks tiles blockIdx.x, + gridDim.x, ..., with the
// next tile's 4-channel patch loaded into registers during this tile's MFMAs
// and parked in the other of two patch buffers.
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv7x7(LAMA_CONV_PARAMS)
{
    using C = CfgHead;
    __shared__ __attribute__((aligned(16))) float lds[C::W_LDS + 2 * C::P_LDS];
    __shared__ float epl[192];
    float *const wl = lds, *const pl0 = lds + C::W_LDS, *const pl1 = pl0 + C::P_LDS;
    LAMA_STAMP_BEGIN;
    const ConvProblem &P = probs[0];
    const ConvSeg sg = P.s0;
    const int ntiles = P.nblocks;
    int t = blockIdx.x;
    if (t >= ntiles) {  // whole workgroup
        LAMA_STAMP_END;
        return;
    }
    if (sg.nchunk != 1 || P.mblocks != 1) {
        // more than 4 input channels or 64 output channels (single-op tests):
        // one tile at a time through the generic path
        for (; t < ntiles; t += gridDim.x) conv_tile<C, false, 1>(P, t, lds, epl);
        LAMA_STAMP_END;
        return;
    }
    auto origin = [&](int tile, int &oy0, int &ox0) {
        oy0 = (tile / P.tiles_x) * C::TR;
        ox0 = (tile % P.tiles_x) * C::TC;
    };
    Slots<C> sl;
    Stage<C> cur, nxt;
    int oy0, ox0, ny0, nx0;
    origin(t, oy0, ox0);
    make_wslots<C>(sl, sg, 0, P.M);
    make_pslots<C>(sl, sg, oy0, ox0);
    load_w<C>(cur, sl, sg, 0);
    load_p<C>(cur, sl, sg, 0);
    const float ep = epi_param_load(P, 0);
    // the next tile (clamped: the last tile is re-read instead of branching)
    int tn = min(t + (int)gridDim.x, ntiles - 1);
    origin(tn, ny0, nx0);
    make_pslots<C>(sl, sg, ny0, nx0);
    load_p<C>(nxt, sl, sg, 0);
    store_w<C>(cur, sl, wl);
    store_p<C>(cur, sl, pl0);
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
    EpiPre pre;
#pragma unroll
    for (int r = 0; r < 16; ++r) pre.add[r] = pre.res[r] = 0.f;
    for (int i = 0;; ++i) {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        compute_chunk<C>(acc, wl, (i & 1) ? pl1 : pl0);
        epilogue<C::TR, C::TC, false>(acc, pre, P, epl, 0, oy0, ox0);
        t += gridDim.x;
        if (t >= ntiles) break;
        oy0 = ny0;
        ox0 = nx0;
        store_p<C>(nxt, sl, (i & 1) ? pl0 : pl1);
        tn = min(t + (int)gridDim.x, ntiles - 1);
        origin(tn, ny0, nx0);
        make_pslots<C>(sl, sg, ny0, nx0);
        load_p<C>(nxt, sl, sg, 0);
        __syncthreads();
    }
    LAMA_STAMP_END;
}

// model.1 with each wave's weights in registers (the plan's head: 4 input
// and 64 output channels, one chunk).  Lane (g, j) of wave (wm, wn) holds the
// MFMA A operands of output channel wm * 32 + j, input channels 2g and 2g + 1,
// for all 49 taps (98 registers), loaded once; LDS holds only the two patch
// buffers (15 KB instead of 68 KB with the staged weights), so three
// workgroups share a CU instead of two.  The host caps the grid at three per
// CU; each workgroup walks tiles blockIdx.x, + gridDim.x, ... as lama_conv7x7
// does, with the next tile's patch loaded into registers during this tile's
// MFMAs.
extern "C" __global__ void __launch_bounds__(LAMA_NT) __attribute__((amdgpu_waves_per_eu(3, 3)))
lama_conv7x7r(LAMA_CONV_PARAMS)
{
    using C = CfgHead;
    __shared__ __attribute__((aligned(16))) float pls[2 * C::P_LDS];
    __shared__ float epl[192];
    float *const pl0 = pls, *const pl1 = pls + C::P_LDS;
    LAMA_STAMP_BEGIN;
    const ConvProblem &P = probs[0];
    const ConvSeg sg = P.s0;
    const int ntiles = P.nblocks;
    int t = blockIdx.x;
    if (t >= ntiles) {  // whole workgroup
        LAMA_STAMP_END;
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    auto origin = [&](int tile, int &oy0, int &ox0) {
        oy0 = (tile / P.tiles_x) * C::TR;
        ox0 = (tile % P.tiles_x) * C::TC;
    };
    Slots<C> sl;
    Stage<C> cur, nxt;
    int oy0, ox0, ny0, nx0;
    origin(t, oy0, ox0);
    make_pslots<C>(sl, sg, oy0, ox0);
    load_p<C>(cur, sl, sg, 0);
    // this lane's A operands: packed row wm * 32 + j, floats tap * KC + 2g, +1
    float a[C::T][2];
    {
        const LAMA_GLOBAL float *wr = gp(sg.wt) + (long)min(wm * 32 + j, P.M - 1) * sg.wrow + g * (C::KC / 2);
#pragma unroll
        for (int tp = 0; tp < C::T; ++tp) {
            a[tp][0] = wr[tp * C::KC];
            a[tp][1] = wr[tp * C::KC + 1];
        }
    }
    const float ep = epi_param_load(P, 0);
    int tn = min(t + (int)gridDim.x, ntiles - 1);  // the last tile is re-read instead of branching
    origin(tn, ny0, nx0);
    make_pslots<C>(sl, sg, ny0, nx0);
    load_p<C>(nxt, sl, sg, 0);
    store_p<C>(cur, sl, pl0);
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
    EpiPre pre;
#pragma unroll
    for (int r = 0; r < 16; ++r) pre.add[r] = pre.res[r] = 0.f;
    const int p = wn * 32 + j, pr = p / C::TC, pc = p % C::TC;
    const int pbase = (pr * C::PCP + C::col(pc)) * C::KCP + g * (C::KC / 2);
    for (int i = 0;; ++i) {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        const float *prow = ((i & 1) ? pl1 : pl0) + pbase;
        float b[2][2];
        lds_vec<2>(b[0], prow);
#pragma unroll
        for (int tp = 0; tp < C::T; ++tp) {
            const int cb = tp & 1;
            if (tp + 1 < C::T) {
                const int ky = (tp + 1) / C::KW, kx = (tp + 1) % C::KW;
                lds_vec<2>(b[cb ^ 1], prow + (ky * C::PCP + C::col(kx)) * C::KCP);
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[tp][0], b[cb][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[tp][1], b[cb][1], acc, 0, 0, 0);
        }
        epilogue<C::TR, C::TC, false>(acc, pre, P, epl, 0, oy0, ox0);
        t += gridDim.x;
        if (t >= ntiles) break;
        oy0 = ny0;
        ox0 = nx0;
        store_p<C>(nxt, sl, (i & 1) ? pl0 : pl1);
        tn = min(t + (int)gridDim.x, ntiles - 1);
        origin(tn, ny0, nx0);
        make_pslots<C>(sl, sg, ny0, nx0);
        load_p<C>(nxt, sl, sg, 0);
        __syncthreads();
    }
    LAMA_STAMP_END;
}

// XCD-contiguous order within each problem of the stride-2 and transposed
// convolutions: the dispatcher deals workgroups to the eight XCDs
// round-robin (workgroup i to XCD i mod 8), each XCD with its own L2.  Block j
// of a problem of n blocks (which starts at a multiple of 8) is replaced by
// block x * q + min(x, r) + j / 8 (x = j mod 8, q = n / 8, r = n mod 8), so
// each XCD works through a contiguous range of tiles with all their M blocks
// (M blocks vary fastest): an input tile is fetched into one L2 instead of
// into every XCD that holds one of its M blocks (model.4's 8 M blocks fell on
// the 8 XCDs, and each XCD read the whole input).  Per problem, so that the
// four transposed-convolution phases (1, 2, 2 and 4 taps) are spread evenly
// over the XCDs, and an XCD's share of each phase covers the same input rows.
#ifndef LAMA_CONV_XCD
#define LAMA_CONV_XCD 1
#endif
__device__ __forceinline__ int conv_xcd_order(int i, int n)
{
#if LAMA_CONV_XCD
    const int x = i & 7, q = n >> 3, r = n & 7;
    return x * q + min(x, r) + (i >> 3);
#else
    (void)n;
    return i;
#endif
}

// model.2/3/4: 3x3 stride 2, reflect pad 1, BN + ReLU.
template <int TR, int TC>
__device__ __forceinline__ void conv3x3s2_body(const ConvProblem *__restrict__ probs, const ProbStarts &ps)
{
    using C = CfgDownT<TR, TC>;
    __shared__ __attribute__((aligned(16))) float lds[2 * C::LDS];
    __shared__ float epl[192];
    int b = blockIdx.x;
    int pi = find_problem(ps, b);
    b = conv_xcd_order(b, probs[pi].nblocks);
    conv_tile<C, false>(probs[pi], b, lds, epl);
}
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv3x3s2(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    conv3x3s2_body<2, 32>(probs, ps);
    LAMA_STAMP_END;
}
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv3x3s2_q(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    conv3x3s2_body<4, 16>(probs, ps);
    LAMA_STAMP_END;
}

// FFC spatial convolutions: 3x3 stride 1 reflect pad 1, with an optional 1x1
// second K segment (the SpectralTransform's conv2, summed before BN_g).
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_conv3x3(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    __shared__ __attribute__((aligned(16))) float lds[2 * cmax(CfgFfc::LDS, CfgFfc1::LDS)];
    __shared__ float epl[192];
    int b = blockIdx.x;
    int pi = find_problem(ps, b);
    conv_tile<CfgFfc, true>(probs[pi], b, lds, epl);
    LAMA_STAMP_END;
}

// 1x1 convolutions over flat planes (SpectralTransform conv1, FourierUnit
// conv): lama_conv1x1_kh in 64 x 32 K-half tiles, the others in 64 x 64
// tiles.  lama_conv1x1 and _kh need 16-byte aligned planes with a plane
// stride cs % 4 == 0 (N padded up to it), lama_conv1x1_v2 8-byte aligned
// planes with N % 2 == 0, cs even and N >= 4; lama_conv1x1_s takes any N.
#define LAMA_PW_KERNEL(NAME, KC, VW, NPX, PREFETCH, D, KH)                                                  \
    extern "C" __global__ void __launch_bounds__(LAMA_NT) NAME(LAMA_CONV_PARAMS) \
    {                                                                                                       \
        side_priority();                                                                                    \
        LAMA_CONV_STARTS;                                                                                   \
        LAMA_STAMP_BEGIN;                                                                                   \
        using C = PwCfg<KC, VW, NPX, KH>;                                                                  \
        __shared__ __attribute__((aligned(16))) float lds[2 * C::LDS];                                      \
        __shared__ float epl[192];                                                                          \
        int b = blockIdx.x;                                                                                 \
        int pi = find_problem(ps, b);                                                             \
        pw_tile<C, PREFETCH, D>(probs[pi], b, lds, epl);                                                     \
        LAMA_STAMP_END;                                                                                     \
    }
#ifndef LAMA_PW_DEPTH_RES
#define LAMA_PW_DEPTH_RES LAMA_PW_DEPTH
#endif
LAMA_PW_KERNEL(lama_conv1x1, LAMA_PW_KC, 4, 64, false, LAMA_PW_DEPTH, false)
LAMA_PW_KERNEL(lama_conv1x1_kh, 2 * LAMA_PW_KC, 4, 32, false, LAMA_PW_DEPTH, true)
LAMA_PW_KERNEL(lama_conv1x1_v2, LAMA_PW_KC, 2, 64, false, LAMA_PW_DEPTH, false)
LAMA_PW_KERNEL(lama_conv1x1_s, LAMA_PW_KC, 1, 64, false, LAMA_PW_DEPTH, false)

// The SpectralTransform conv2, whose epilogue adds the l2g partial and the
// residual (fetched before the K loop).
LAMA_PW_KERNEL(lama_conv1x1_res, LAMA_PW_KC, 4, 64, true, LAMA_PW_DEPTH_RES, false)
LAMA_PW_KERNEL(lama_conv1x1_res_kh, 2 * LAMA_PW_KC, 4, 32, true, LAMA_PW_DEPTH_RES, true)
LAMA_PW_KERNEL(lama_conv1x1_res_v2, LAMA_PW_KC, 2, 64, true, LAMA_PW_DEPTH_RES, false)
LAMA_PW_KERNEL(lama_conv1x1_res_s, LAMA_PW_KC, 1, 64, true, LAMA_PW_DEPTH_RES, false)
#undef LAMA_PW_KERNEL

// ConvTranspose2d k3 s2 p1 op1 as four sub-pixel phase convolutions
// (problems 0..3 = phases (py,px) = (0,0), (0,1), (1,0), (1,1)), each a valid
// (1+py) x (1+px) convolution with zero fill at the bottom/right edge.
template <int TR, int TC>
__device__ __forceinline__ void convt_body(const ConvProblem *__restrict__ probs, const ProbStarts &ps)
{
    using C = CfgT<TR, TC>;
    __shared__ __attribute__((aligned(16))) float lds[2 * C::LDS];
    __shared__ float epl[192];
    int b = blockIdx.x;
    int pi = find_problem(ps, b);
    b = conv_xcd_order(b, probs[pi].nblocks);
    switch (pi) {
    case 0: conv_tile<typename C::P00, false>(probs[0], b, lds, epl); break;
    case 1: conv_tile<typename C::P01, false>(probs[1], b, lds, epl); break;
    case 2: conv_tile<typename C::P10, false>(probs[2], b, lds, epl); break;
    default: conv_tile<typename C::P11, false>(probs[3], b, lds, epl); break;
    }
}
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_convt(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    convt_body<2, 32>(probs, ps);
    LAMA_STAMP_END;
}
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_convt_q(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    convt_body<4, 16>(probs, ps);
    LAMA_STAMP_END;
}

// The same convolution as two row-phase problems (problem py = 0, 1; see
// CfgRows): half the workgroups of the four-phase form, each input patch
// staged twice instead of four times, and whole output rows stored.
template <class C>
__device__ __forceinline__ void convt_rows_tile(const ConvProblem &P, int b, float *lds, float *epl)
{
    const int mb = b % P.mblocks, t = b / P.mblocks;
    const int m0 = mb * 64, y0 = (t / P.tiles_x) * C::TR, x0 = (t % P.tiles_x) * C::TC;
    const float ep = epi_param_load(P, m0);
    RowsAcc acc;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc.a[i][r] = 0.f;
    run_segment<C, 2>(acc, P.s0, m0, P.M, y0, x0, lds);
    if (threadIdx.x < 192) epl[threadIdx.x] = ep;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, j = lane & 31;
    const int p = wn * 32 + j;
    const int y = y0 + p / C::TC, x = x0 + p % C::TC;
    if (y >= P.OH || x >= P.OW) return;
    LAMA_GLOBAL float *out = gp(P.out) + (long)(2 * y + C::PY) * P.outW + 2 * x;
    // D[i][j] of a 32x32 MFMA block: lane j + 32 ((i / 4) % 2), register (i / 8) * 4 + i % 4
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int cl = wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m0 + cl >= P.M) continue;
        float e[2] = {acc.a[0][r], acc.a[1][r]};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (P.bias) e[q] += epl[cl];
            if (P.scale) e[q] = e[q] * epl[64 + cl] + epl[128 + cl];
            if (P.relu) e[q] = fmaxf(e[q], 0.f);
        }
        *reinterpret_cast<float2 *>(out + (long)(m0 + cl) * P.out_cstride) = make_float2(e[0], e[1]);
    }
}

template <int TR, int TC>
__device__ __forceinline__ void convt_rows_body(const ConvProblem *__restrict__ probs, const ProbStarts &ps)
{
    using C0 = CfgRows<0, TR, TC>;
    using C1 = CfgRows<1, TR, TC>;
    __shared__ __attribute__((aligned(16))) float lds[2 * cmax(C0::LDS, C1::LDS)];
    __shared__ float epl[192];
    int b = blockIdx.x;
    const int pi = find_problem(ps, b);
    b = conv_xcd_order(b, probs[pi].nblocks);
    if (pi == 0)
        convt_rows_tile<C0>(probs[0], b, lds, epl);
    else
        convt_rows_tile<C1>(probs[1], b, lds, epl);
}
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_convt_rows(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    convt_rows_body<2, 32>(probs, ps);
    LAMA_STAMP_END;
}
extern "C" __global__ void __launch_bounds__(LAMA_NT) lama_convt_rows_q(LAMA_CONV_PARAMS)
{
    LAMA_CONV_STARTS;
    LAMA_STAMP_BEGIN;
    convt_rows_body<4, 16>(probs, ps);
    LAMA_STAMP_END;
}
