// Winograd weight transforms of the FFC 3x3 convolutions, run once when the
// weights are loaded: each thread takes one (output channel, input channel)
// pair of one matrix, reads its nine taps and writes their transformed
// values into the layout the Winograd kernels load as MFMA operands.
//
// The transforms are evaluated in f64 and rounded once to f32, with the same
// terms summed in the same order as the host packer in engine.cpp
// (pack_wino4 / pack_wino42), and each product and sum rounded on its own, as
// on the host: this code object is built with -ffp-contract=fast, under
// which the backend fuses a multiply and an add into one FMA whatever the
// source says, so each product passes through an empty asm statement that
// hides it from that combine.  The packed floats are then identical.
//
// F(4,3) along x: U_u = sum over kx of G[u][kx] w[ky][kx], G for the points
// 0, 1, -1, 2, -2, infinity.  F(2x4, 3x3): U(vy, u) = sum over kx of
// Gx[u][kx] t[vy][kx], t = Gy w (Gy the F(2,3) transform along y, for the
// points 0, 1, -1, infinity).
#include <hip/hip_runtime.h>

#include "common.h"

namespace {

// a*x + b*y + c*z, left to right, every operation rounded on its own
__device__ __forceinline__ double dot3(double a, double x, double b, double y, double c, double z)
{
    double p = a * x, q = b * y, r = c * z;
    __asm__ volatile("" : "+v"(p), "+v"(q), "+v"(r));
    return p + q + r;
}

__device__ __forceinline__ void pack_one_w4(const WinoPackJob &J, int co, int ci, const double (&g)[9])
{
    constexpr double G[6][3] = {{0.25, 0, 0},           {-1.0 / 6, -1.0 / 6, -1.0 / 6}, {-1.0 / 6, 1.0 / 6, -1.0 / 6},
                                {1.0 / 24, 1.0 / 12, 1.0 / 6}, {1.0 / 24, -1.0 / 12, 1.0 / 6}, {0, 0, 1}};
    constexpr int KC = LAMA_WINO_KC, WK = 72;
    static_assert(KC == 4, "two channels per lane half");
    const int mb = co / 64, wm = co % 64 / 32, j = co % 32;
    const int ck = ci / KC, lg = ci % KC / 2, c = ci % 2, lane = lg * 32 + j;
    LAMA_GLOBAL float *blk = gp(J.dst) + ((long)mb * J.nchunk + ck) * 64 * WK;
#pragma unroll
    for (int u = 0; u < 6; ++u)
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
            const double v = dot3(G[u][0], g[ky * 3], G[u][1], g[ky * 3 + 1], G[u][2], g[ky * 3 + 2]);
            const int wave = wm * 2 + u / 3, st = ky * 3 + u % 3;
            const int at = LAMA_W4_WX4 ? wave * 9 * 128 + (st < 8 ? (st / 2) * 256 + lane * 4 + (st % 2) * 2
                                                                  : 1024 + lane * 2)
                                       : ((wave * 9 + st) * 64 + lane) * 2;
            blk[at + c] = (float)v;
        }
}

__device__ __forceinline__ void pack_one_w42(const WinoPackJob &J, int co, int ci, const double (&g)[9])
{
    constexpr double Gx[6][3] = {{0.25, 0, 0},           {-1.0 / 6, -1.0 / 6, -1.0 / 6}, {-1.0 / 6, 1.0 / 6, -1.0 / 6},
                                 {1.0 / 24, 1.0 / 12, 1.0 / 6}, {1.0 / 24, -1.0 / 12, 1.0 / 6}, {0, 0, 1}};
    constexpr double Gy[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    constexpr int KC = LAMA_W42_KC, H = KC / 2, WK = 24 * KC, WW = 6 * H;
    const int mb = co / 64, wm = co % 64 / 32, j = co % 32;
    const int ck = ci / KC, lg = ci % KC / H, c = ci % KC % H, lane = lg * 32 + j;
    LAMA_GLOBAL float *blk = gp(J.dst) + ((long)mb * J.nchunk + ck) * 64 * WK;
    double t[4][3];
#pragma unroll
    for (int vy = 0; vy < 4; ++vy)
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) t[vy][kx] = dot3(Gy[vy][0], g[kx], Gy[vy][1], g[3 + kx], Gy[vy][2], g[6 + kx]);
#pragma unroll
    for (int vy = 0; vy < 4; ++vy)
#pragma unroll
        for (int u = 0; u < 6; ++u) {
            const double v = dot3(Gx[u][0], t[vy][0], Gx[u][1], t[vy][1], Gx[u][2], t[vy][2]);
            const int idx = H * u + c, wave = wm * 4 + vy;
            blk[wave * WW * 64 + (idx / 4) * 256 + lane * 4 + idx % 4] = (float)v;
        }
}

}  // namespace

// grid (x: any, y: one job each), 256 threads; the (co, ci) pairs of job
// blockIdx.y are walked with a grid stride.
extern "C" __global__ void __launch_bounds__(256) lama_pack_wino(const WinoPackJob *__restrict__ jobs)
{
    const WinoPackJob J = jobs[blockIdx.y];
    const long n = (long)J.M * J.C;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const int co = (int)(i / J.C), ci = (int)(i % J.C);
        const LAMA_GLOBAL float *s = ci < J.C0 ? gp(J.src0) + ((long)co * J.C0 + ci) * 9
                                               : gp(J.src1) + ((long)co * (J.C - J.C0) + (ci - J.C0)) * 9;
        double g[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) g[k] = (double)s[k];
        if (J.kind == 42)
            pack_one_w42(J, co, ci, g);
        else
            pack_one_w4(J, co, ci, g);
    }
}
