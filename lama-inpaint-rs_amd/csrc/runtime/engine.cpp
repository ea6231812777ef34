// The HIP engine: the reference's cuda.rs host side rebuilt around a fused,
// preplanned forward.
//
//  * Weights: derived once when loaded (cuda.rs uploads the raw file and
//    derives on every call): BatchNorms folded as cpu.rs:58-62, convolution
//    weights packed for the MFMA kernels ([M][nchunk][taps][KC]), model.4's
//    l2l/l2g stacked along M, every ConvTranspose split into its sub-pixel
//    phases -- built on the host and uploaded -- and the FFC 3x3 weights in
//    the Winograd kernels' layouts, with the FFC's local convolutions
//    concatenated along K (l2l | g2l, so out_l = l2l(x_l) + g2l(x_g) is one
//    GEMM) -- transformed on the device from the raw weights.
//  * Activations: one device arena per input shape with the whole plan laid
//    out up front; local and global branches share one [512][h/8][w/8]
//    buffer (local planes first), which makes the reference's concat free.
//  * Launches: a static list per shape whose descriptors live in device
//    memory, so a forward is only kernel launches (and two copies).
#include "engine.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <chrono>
#include <cstdio>
#include <functional>

#include <atomic>
#include <mutex>
#include <system_error>
#include <thread>

namespace lama {

// The no-allocation entry point's device array, per device: the code object
// that defines it (loaded once per process, never unloaded), its address on
// that device, and whose descriptors it holds -- the engine id and shape of
// the last forward_device_noalloc on the device (0: none).
struct DeviceScratch {
    hipModule_t mod = nullptr;
    void *ptr = nullptr;
    size_t bytes = 0;
    uint64_t owner = 0;
    int h = 0, w = 0;
};
static std::mutex g_scratch_mu;
static std::map<int, DeviceScratch> g_scratch;
static std::atomic<uint64_t> g_engine_ids{0};

const char *const kFamilyName[F_COUNT] = {"conv7x7",  "conv3x3s2",  "conv3x3",    "conv1x1", "convt",
                                          "rfft2",    "irfft2",     "tail",       "finalize", "conv1x1res",
                                          "conv3x3g2l", "build_input"};

size_t step_numel(int step, int h, int w)
{
    const size_t h8 = h / 8, w8 = w / 8;
    switch (step) {
    case 0: return 4ul * (h + 6) * (w + 6);
    case 1: return 64ul * h * w;
    case 2: return 128ul * (h / 2) * (w / 2);
    case 3: return 256ul * (h / 4) * (w / 4);
    case 24: return 256ul * (h / 4) * (w / 4);
    case 25: return 128ul * (h / 2) * (w / 2);
    case 26: return 64ul * h * w;
    case 27: return 64ul * (h + 6) * (w + 6);
    case 28: return 3ul * h * w;
    default: return (step >= 4 && step <= 23) ? 512ul * h8 * w8 : 0;
    }
}

namespace {

const char *const kKernelName[F_COUNT] = {"lama_conv7x7",     "lama_conv3x3s2", "lama_conv3x3",  "lama_conv1x1",
                                          "lama_convt",       "lama_rfft2",     "lama_irfft2",   "lama_tail",
                                          "lama_finalize",    "lama_conv1x1_res", "lama_conv3x3", "lama_build_input"};

const char *const kSplitName[4] = {"lama_rfft2_rows", "lama_rfft2_cols", "lama_irfft2_cols", "lama_irfft2_rows"};
const char *const kSplitCtName[2][4] = {
    {"lama_rfft2_rows_256", "lama_rfft2_cols_256", "lama_irfft2_cols_256", "lama_irfft2_rows_256"},
    {"lama_rfft2_rows_128", "lama_rfft2_cols_128", "lama_irfft2_cols_128", "lama_irfft2_rows_128"}};

// F_CONV1 / F_CONV1R variants with per-element activation loads, for planes
// whose length is not a multiple of 4 or that are not 16-byte aligned.
const char *const kPwAnyName[2] = {"lama_conv1x1_s", "lama_conv1x1_res_s"};
const char *const kPwV2Name[2] = {"lama_conv1x1_v2", "lama_conv1x1_res_v2"};

// Single-block FFT kernels with the plane shape fixed at compile time.
// The fourth, 64 x 64 with wavefront-shuffle rows, only with LAMA_FFT64_SHFL=1.
const int kFftCtSide[4] = {64, 32, 75, 64};
// the kernel keeps one plane buffer in LDS, not two (LAMA_FFT_CT's IP)
const bool kFftCtInPlace[4] = {false, false, LAMA_FFT75_IP != 0, false};
const char *const kFftCtName[4][2] = {{"lama_rfft2_64", "lama_irfft2_64"},
                                      {"lama_rfft2_32", "lama_irfft2_32"},
                                      {"lama_rfft2_75", "lama_irfft2_75"},
                                      {"lama_rfft2_64s", "lama_irfft2_64s"}};

// The first workgroup of each problem after the first, for a grouped launch.
ProbStarts prob_starts(const ConvProblem *q, size_t n)
{
    ProbStarts ps{(int)n, {}};
    int cum = 0;
    for (int i = 0; i < LAMA_MAX_PROBS - 1; ++i) ps.s[i] = (size_t)i + 1 < n ? cum += q[i].nblocks : INT32_MAX;
    return ps;
}

// Tile geometry of each conv family (kernels/conv.hip): rows x columns.
// `narrow`: the F(4,3) kernel's 32-pixel blocks.
// Pixel tile (rows x columns) of a conv family; `w4v` is the tile variant
// (Engine::tile_variant): the F(4,3) block shape, or for the stride-2 and
// transposed convolutions 0 = 2 x 32, 1 = 4 x 16.
// Resident workgroups per CU the register-weight head kernel's grid is capped at
// (512x512: 72.8-73.6 us per pass at 3 against 78.5-80.7 at 2 or 4)
#ifndef LAMA_HEAD_WGS
#define LAMA_HEAD_WGS 3
#endif

// Channels per K chunk of the pointwise kernel a plane of tile variant v runs
// (Engine::tile_variant: 0 = the K-half kernels, 1 = the 64 x 64 ones).
int pw_kc(int v) { return v == 0 ? 2 * LAMA_PW_KC : LAMA_PW_KC; }

void tile_shape(int family, int &tr, int &tc, int wino = 0, int w4v = 0)
{
    if ((family == F_CONV3 || family == F_CONV3G) && wino == 42) {  // lama_conv3x3w42: 4 x 64
        tr = 4;
        tc = 64;
    } else if ((family == F_CONV3 || family == F_CONV3G) && wino == 4) {  // lama_conv3x3w4 / w4n / w4q
        tr = 2 << w4v;                                              // 2 x 64, 4 x 32 or 8 x 16
        tc = 128 / tr;
    } else if ((family == F_CONV3 || family == F_CONV3G) && wino) {  // lama_conv3x3w: 2 rows x 64 px
        tr = 2;
        tc = 64;
    } else if (family == F_CONV1 || family == F_CONV1R) {
        tr = 1;
        tc = w4v == 0 ? 32 : 64;  // variant 0: the K-half kernels' tiles
    } else if ((family == F_CONV3S2 || family == F_CONVT) && w4v == 1) {  // the _q kernels
        tr = 4;
        tc = 16;
    } else {
        tr = 2;
        tc = 32;
    }
}

// Pointwise launches of one problem (one row of pixel strips): the grid holds
// the strips rounded up to a multiple of 8, so that the kernel's XCD-aware
// order (all M blocks of strip t on XCD t mod 8) holds for any strip count;
// the blocks of the padding strips exit at once.
long pw_xcd_blocks(const ConvProblem &q) { return (long)(q.tiles_x + 7) / 8 * 8 * q.mblocks; }
void pw_xcd_pad(int family, ConvProblem &q)
{
    if (LAMA_PW_XCD && (family == F_CONV1 || family == F_CONV1R) && q.tiles_y == 1 && q.ksplit <= 1)
        q.nblocks = (int)pw_xcd_blocks(q);
}

struct WeightSrc {
    const uint8_t *blob;
    size_t len;
    std::map<std::string, const lama_tensor_info *> idx;

    // The tensor `name` as f32, checked against `shape`.
    bool get(const std::string &name, std::initializer_list<int64_t> shape, std::vector<float> &out,
             std::string &err) const
    {
        const lama_tensor_info *t = find(name, shape, err);
        if (!t) return false;
        out.resize(t->nbytes / 4);
        std::memcpy(out.data(), blob + t->offset, t->nbytes);
        return true;
    }
    // The tensor `name`, checked against `shape`, left in the blob.
    const lama_tensor_info *find(const std::string &name, std::initializer_list<int64_t> shape,
                                 std::string &err) const
    {
        auto it = idx.find(name);
        if (it == idx.end()) {
            err = "missing tensor in weight blob: " + name;  // weights.rs:116-120
            return nullptr;
        }
        const lama_tensor_info *t = it->second;
        bool ok = (size_t)t->ndim == shape.size();
        size_t i = 0, n = 1;
        for (int64_t d : shape) {
            ok = ok && t->shape[i++] == d;
            n *= (size_t)d;
        }
        if (!ok || t->nbytes != n * 4 || t->offset + t->nbytes > len) {
            std::string want, got;
            for (int64_t d : shape) want += (want.empty() ? "" : ",") + std::to_string(d);
            for (int d = 0; d < t->ndim; ++d) got += (d ? "," : "") + std::to_string(t->shape[d]);
            err = "tensor " + name + ": expected shape [" + want + "], found [" + got + "]";
            return nullptr;
        }
        return t;
    }
};

// The host image of a device weight arena.  add() lays regions out on
// 64-float (256-byte) boundaries of the device arena; the host side lives in
// zero-filled blocks that never move (a region never spans two), so packing
// writes each float once and a growing layout copies nothing.  The blocks
// come from calloc: their pages are zeroed when first written, by the threads
// that pack them.
struct Arena {
    static constexpr size_t BLOCK = (size_t)16 << 20;  // floats per block (64 MiB)
    struct Block {
        size_t start, cap;
        float *d;
    };
    std::vector<Block> blocks;
    size_t n = 0;  // floats laid out: the device arena's size

    Arena() = default;
    Arena(const Arena &) = delete;
    Arena &operator=(const Arena &) = delete;
    ~Arena()
    {
        for (Block &b : blocks) free(b.d);
    }
    size_t add(size_t k)
    {
        const size_t off = (n + 63) / 64 * 64;
        // block starts and capacities are multiples of 64 floats, so the
        // aligned offset never lies past the current block's end
        if (blocks.empty() || off + k > blocks.back().start + blocks.back().cap) {
            const size_t cap = (std::max(BLOCK, k) + 63) / 64 * 64;
            float *d = static_cast<float *>(calloc(cap, sizeof(float)));
            if (!d) throw std::bad_alloc();
            blocks.push_back({off, cap, d});
        }
        n = off + k;
        return off;
    }
    float *at(size_t off)
    {
        for (size_t i = blocks.size(); i-- > 0;)
            if (blocks[i].start <= off) return blocks[i].d + (off - blocks[i].start);
        return nullptr;
    }
    size_t size() const { return n; }
    // the layout into device memory of size() floats: each block up to the
    // next one's start (alignment gaps included, as zeros)
    bool upload(const HipApi *hip, float *dev, std::string &err) const
    {
        for (size_t i = 0; i < blocks.size(); ++i) {
            const size_t end = i + 1 < blocks.size() ? blocks[i + 1].start : n;
            const hipError_t e = hip->hipMemcpy(dev + blocks[i].start, blocks[i].d, (end - blocks[i].start) * 4,
                                                hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                err = hip_error(*hip, e, "hipMemcpy(weights)");
                return false;
            }
        }
        return true;
    }
};

template <class Get>
Packed pack(Arena &A, int M, int C, int T, int KC, const Get &get)
{
    Packed p;
    p.M = M;
    p.C = C;
    p.T = T;
    p.KC = KC;
    p.nchunk = (C + KC - 1) / KC;
    p.wrow = p.nchunk * T * KC;
    p.off = A.add((size_t)M * p.wrow);
    float *d = A.at(p.off);
    for (int co = 0; co < M; ++co)
        for (int ck = 0; ck < p.nchunk; ++ck)
            for (int t = 0; t < T; ++t)
                for (int kc = 0; kc < KC; ++kc) {
                    const int ci = ck * KC + kc;
                    d[(((size_t)co * p.nchunk + ck) * T + t) * KC + kc] = ci < C ? get(co, ci, t) : 0.f;
                }
    return p;
}

// ConvTranspose2d k3 s2 p1 op1 weights w [ci][co][3][3] (PyTorch layout) as
// sub-pixel phase taps.  Phase (py, px) of output pixel (2m+py, 2n+px)
// reads input (m+a, n+b) for a < 1+py, b < 1+px: kernel row ky = 1 for
// py = 0, else 2 (a = 0) or 0 (a = 1); the same for columns.
float convt_tap(const float *w, int cout, int co, int ci, int py, int px, int a, int b)
{
    const int ky = py == 0 ? 1 : (a == 0 ? 2 : 0), kx = px == 0 ? 1 : (b == 0 ? 2 : 0);
    return w[(((size_t)ci * cout + co) * 3 + ky) * 3 + kx];
}

// One phase's (1+py) x (1+px) taps, row-major (lama_convt).
Packed pack_convt_phase(Arena &A, int cout, int cin, int ph, const float *w)
{
    const int py = ph >> 1, px = ph & 1, nx = 1 + px;
    return pack(A, cout, cin, (1 + py) * nx, lama_convt_kc(ph), [&](int co, int ci, int t) {
        return convt_tap(w, cout, co, ci, py, px, t / nx, t % nx);
    });
}

// The taps of row phase py, both column phases, in K chunks of
// LAMA_CONVT_ROWS_KC0 / KC1 channels
// (lama_convt_rows): py = 0: (0,0) of phase (0,0); (0,0), (0,1) of phase
// (0,1).  py = 1: (0,0), (1,0) of phase (1,0); (0,0), (0,1), (1,0), (1,1)
// of phase (1,1).
Packed pack_convt_rows(Arena &A, int cout, int cin, int py, const float *w)
{
    static const int tap[2][6][3] = {{{0, 0, 0}, {1, 0, 0}, {1, 0, 1}},
                                     {{0, 0, 0}, {0, 1, 0}, {1, 0, 0}, {1, 0, 1}, {1, 1, 0}, {1, 1, 1}}};  // px, a, b
    return pack(A, cout, cin, py ? 6 : 3, py ? LAMA_CONVT_ROWS_KC1 : LAMA_CONVT_ROWS_KC0, [&](int co, int ci, int t) {
        return convt_tap(w, cout, co, ci, py, tap[py][t][0], tap[py][t][1], tap[py][t][2]);
    });
}

// 3x3 weights for lama_conv3x3w: per output channel and chunk of
// LAMA_WINO_KC input channels, [u][ky][ci] with U_u = sum over kx of G[u][kx] * w[ky][kx],
// G = (1, 0, 0; 1/2, 1/2, 1/2; 1/2, -1/2, 1/2; 0, 0, 1) -- the Winograd F(2,3)
// weight transform along x, evaluated in f64 and rounded once to f32.
Packed pack_wino(Arena &A, int M, int C, const std::function<float(int, int, int)> &get)
{
    static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    constexpr int KC = LAMA_WINO_KC;
    Packed p;
    p.M = M;
    p.C = C;
    p.T = 12;  // (u, ky)
    p.KC = KC;
    p.nchunk = ((C + KC - 1) / KC + 1) & ~1;  // even: the kernel runs its K loop in chunk pairs
    p.wrow = p.nchunk * 12 * KC;
    p.off = A.add((size_t)M * p.wrow);
    float *d = A.at(p.off);
    for (int co = 0; co < M; ++co)
        for (int ck = 0; ck < p.nchunk; ++ck)
            for (int u = 0; u < 4; ++u)
                for (int ky = 0; ky < 3; ++ky)
                    for (int kc = 0; kc < KC; ++kc) {
                        const int ci = ck * KC + kc;
                        double v = 0;
                        if (ci < C)
                            for (int kx = 0; kx < 3; ++kx) v += G[u][kx] * (double)get(co, ci, ky * 3 + kx);
                        d[((size_t)co * p.nchunk + ck) * 12 * KC + (u * 3 + ky) * KC + kc] = (float)v;
                    }
    return p;
}

// Runs f(r0, r1) over [0, n) split into contiguous ranges on up to 16
// host threads (the Winograd weight transforms, one output channel row per
// index: rows never share packed floats).  A range whose thread cannot be
// started runs on the calling thread (no exception leaves the C ABI).
template <class F>
void parallel_rows(int n, F f)
{
    const int nt = std::max(1, std::min({16, n, (int)std::thread::hardware_concurrency()}));
    auto lo = [&](int t) { return (int)((long)n * t / nt); };
    std::vector<std::thread> th;
    int t = 1;
    try {
        for (; t < nt; ++t) th.emplace_back(f, lo(t), lo(t + 1));
    } catch (const std::system_error &) {
        f(lo(t), lo(nt));  // the ranges no thread took
    }
    f(0, lo(1));
    for (std::thread &x : th) x.join();
}

// 3x3 weights for lama_conv3x3w4 / w4n / w4q, transformed by
// U_u = sum over kx of G[u][kx] * w[ky][kx] with
// G = (1/4, 0, 0; -1/6, -1/6, -1/6; -1/6, 1/6, -1/6; 1/24, 1/12, 1/6;
// 1/24, -1/12, 1/6; 0, 0, 1) -- the Winograd F(4,3) weight transform for the
// points 0, 1, -1, 2, -2, infinity, evaluated in f64 and rounded once to f32
// -- in the order the kernels' waves load them as MFMA operands: per block of
// 64 output channels (rows past M zero) and chunk of 4 input channels,
// [wave (wm, wu)][step s = ky * 3 + q][lane (g, j)][c] holds U_u for output
// channel 32 wm + j, input channel 2g + c of the chunk and position
// u = 3 wu + q (with LAMA_W4_WX4, steps 2p and 2p + 1 of a wave interleaved
// as [p][lane][step 2p + h][c], step 8 after them as [lane][c]).  A chunk is 64 x 72 floats (T * KC); the block stride is 64
// rows of wrow = nchunk * 72.
// The F(4,3) layout's shape (p.off unset).  The same floats are written on
// the device by lama_pack_wino (kind 4).
Packed wino4_shape(int M, int C)
{
    constexpr int KC = LAMA_WINO_KC, WK = 72;
    static_assert(KC == 4, "two channels per lane half");
    Packed p;
    p.M = M;
    p.C = C;
    p.KC = KC;
    p.T = 64 * WK / KC;  // chunk stride T * KC = one 64-row block's chunk
    p.nchunk = ((C + KC - 1) / KC + 1) & ~1;  // even: the kernel runs its K loop in chunk pairs
    p.wrow = p.nchunk * WK;
    return p;
}

// floats of a Winograd pack: 64-row blocks (rows past M zero)
size_t wino_floats(const Packed &p) { return (size_t)((p.M + 63) / 64) * 64 * p.wrow; }

template <class Get>
Packed pack_wino4(Arena &A, int M, int C, const Get &get)
{
    static const double G[6][3] = {{0.25, 0, 0},           {-1.0 / 6, -1.0 / 6, -1.0 / 6}, {-1.0 / 6, 1.0 / 6, -1.0 / 6},
                                   {1.0 / 24, 1.0 / 12, 1.0 / 6}, {1.0 / 24, -1.0 / 12, 1.0 / 6}, {0, 0, 1}};
    constexpr int KC = LAMA_WINO_KC, WK = 72;
    Packed p = wino4_shape(M, C);
    p.off = A.add(wino_floats(p));  // zero: rows past M, channels past C
    float *d = A.at(p.off);
    parallel_rows(M, [&](int r0, int r1) {
        for (int co = r0; co < r1; ++co) {
            const int mb = co / 64, wm = co % 64 / 32, j = co % 32;
            for (int ci = 0; ci < C; ++ci) {
                double g[9];
                for (int k = 0; k < 9; ++k) g[k] = (double)get(co, ci, k);
                const int ck = ci / KC, lg = ci % KC / 2, c = ci % 2, lane = lg * 32 + j;
                float *blk = d + ((size_t)mb * p.nchunk + ck) * 64 * WK;
                for (int u = 0; u < 6; ++u)
                    for (int ky = 0; ky < 3; ++ky) {
                        const double v = G[u][0] * g[ky * 3] + G[u][1] * g[ky * 3 + 1] + G[u][2] * g[ky * 3 + 2];
                        const int wave = wm * 2 + u / 3, st = ky * 3 + u % 3;
                        // LAMA_W4_WX4: steps 2q, 2q + 1 interleaved per lane (one 16-byte
                        // load), step 8 after them
                        const size_t at = LAMA_W4_WX4 ? (size_t)wave * 9 * 128 +
                                                            (st < 8 ? (st / 2) * 256 + lane * 4 + (st % 2) * 2
                                                                    : 1024 + lane * 2)
                                                      : ((size_t)(wave * 9 + st) * 64 + lane) * 2;
                        blk[at + c] = (float)v;
                    }
            }
        }
    });
    return p;
}

// 3x3 weights for lama_conv3x3w42 (Winograd F(2x4, 3x3)): U(vy, u) =
// sum over (ky, kx) of Gy[vy][ky] Gx[u][kx] w[ky][kx], Gx the F(4,3) transform
// of pack_wino4 and Gy = (1, 0, 0; 1/2, 1/2, 1/2; 1/2, -1/2, 1/2; 0, 0, 1) the
// F(2,3) one, evaluated in f64 and rounded once to f32, in the order the
// kernel's waves load them: per block of 64 output channels (rows past M
// zero) and chunk of KC = LAMA_W42_KC input channels (H = KC / 2 per lane
// half), [wave (wm, vy)][group h][lane (g, j)][k] holds U(vy, u) for output
// channel 32 wm + j and input channel H g + c of the chunk, with
// H u + c = 4 h + k.  A chunk is 64 x 24 KC floats; the block stride is 64
// rows of wrow = nchunk * 24 KC.
// The F(2x4, 3x3) layout's shape (p.off unset).  The same floats are written
// on the device by lama_pack_wino (kind 42).
Packed wino42_shape(int M, int C)
{
    constexpr int KC = LAMA_W42_KC, WK = 24 * KC;
    static_assert(KC == 4 || KC == 8, "two or four channels per lane half");
    Packed p;
    p.M = M;
    p.C = C;
    p.KC = KC;
    p.T = 64 * WK / KC;  // chunk stride T * KC = one 64-row block's chunk
    p.nchunk = ((C + KC - 1) / KC + 1) & ~1;  // even: the kernel runs its K loop in chunk pairs
    p.wrow = p.nchunk * WK;
    return p;
}

template <class Get>
Packed pack_wino42(Arena &A, int M, int C, const Get &get)
{
    static const double Gx[6][3] = {{0.25, 0, 0},           {-1.0 / 6, -1.0 / 6, -1.0 / 6}, {-1.0 / 6, 1.0 / 6, -1.0 / 6},
                                    {1.0 / 24, 1.0 / 12, 1.0 / 6}, {1.0 / 24, -1.0 / 12, 1.0 / 6}, {0, 0, 1}};
    static const double Gy[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    constexpr int KC = LAMA_W42_KC, H = KC / 2, WK = 24 * KC, WW = 6 * H;
    Packed p = wino42_shape(M, C);
    p.off = A.add(wino_floats(p));  // zero: rows past M, channels past C
    float *d = A.at(p.off);
    parallel_rows(M, [&](int r0, int r1) {
        for (int co = r0; co < r1; ++co) {
            const int mb = co / 64, wm = co % 64 / 32, j = co % 32;
            for (int ci = 0; ci < C; ++ci) {
                double g[3][3], t[4][3];
                for (int k = 0; k < 9; ++k) g[k / 3][k % 3] = (double)get(co, ci, k);
                for (int vy = 0; vy < 4; ++vy)  // G_y g
                    for (int kx = 0; kx < 3; ++kx)
                        t[vy][kx] = Gy[vy][0] * g[0][kx] + Gy[vy][1] * g[1][kx] + Gy[vy][2] * g[2][kx];
                const int ck = ci / KC, lg = ci % KC / H, c = ci % KC % H;
                float *blk = d + ((size_t)mb * p.nchunk + ck) * 64 * WK;
                for (int vy = 0; vy < 4; ++vy)
                    for (int u = 0; u < 6; ++u) {  // (G_y g) G_x^T
                        const double v = Gx[u][0] * t[vy][0] + Gx[u][1] * t[vy][1] + Gx[u][2] * t[vy][2];
                        const int idx = H * u + c, wave = wm * 4 + vy, lane = lg * 32 + j;
                        blk[(size_t)wave * WW * 64 + (idx / 4) * 256 + lane * 4 + idx % 4] = (float)v;
                    }
            }
        }
    });
    return p;
}

// cpu.rs:58-62: s = w / sqrt(var + 1e-5), t = b - mean * s, in f32.
void fold_into(const std::vector<float> &w, const std::vector<float> &b, const std::vector<float> &mean,
               const std::vector<float> &var, float *scale, float *shift)
{
    for (size_t i = 0; i < w.size(); ++i) {
        const float s = w[i] / std::sqrt(var[i] + 1e-5f);
        scale[i] = s;
        const float ms = mean[i] * s;
        shift[i] = b[i] - ms;
    }
}

bool fold_bns(Arena &A, const WeightSrc &S, const std::vector<std::pair<std::string, int>> &parts, size_t &off,
              std::string &err)
{
    int n = 0;
    for (auto &p : parts) n += p.second;
    off = A.add(2 * (size_t)n);
    int at = 0;
    for (auto &p : parts) {
        std::vector<float> w, b, m, v;
        const int64_t c = p.second;
        if (!S.get(p.first + ".weight", {c}, w, err) || !S.get(p.first + ".bias", {c}, b, err) ||
            !S.get(p.first + ".running_mean", {c}, m, err) || !S.get(p.first + ".running_var", {c}, v, err))
            return false;
        fold_into(w, b, m, v, A.at(off) + at, A.at(off) + n + at);
        at += p.second;
    }
    return true;
}

bool is_pow2(int n) { return n > 0 && (n & (n - 1)) == 0; }

// Plane stride of the bottleneck activations and of the stacked spectrum:
// the plane length rounded up to a multiple of 4 floats, so that every plane
// of a 256-byte aligned buffer is 16-byte aligned and the float4 kernels run
// on planes of any length (75 x 75 = 5625, 75 x 38 = 2850 at 600 x 600).
// The padding floats are never read as data: the pointwise kernels' last
// float4 run of a plane feeds only output columns past the plane, which are
// not stored, and the transforms and 3x3 convolutions index rows.
size_t pad4(size_t n) { return (n + 3) & ~(size_t)3; }

}  // namespace

void Engine::release_scratch_owner()
{
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch.find(device_);
    if (it != g_scratch.end() && it->second.owner == id_) it->second.owner = 0;
}

Engine::~Engine()
{
    if (!hip_) return;
    if (id_) release_scratch_owner();
    for (auto &kv : plans_) free_plan(kv.second);
    for (auto &kv : spec_plans_)
        if (kv.second.arena) hip_->hipFree(kv.second.arena);
    if (warena_) hip_->hipFree(warena_);
    if (ev_done_) hip_->hipEventDestroy(ev_done_);
    if (stamp_buf_) hip_->hipFree(stamp_buf_);
    for (auto &p : pending_) {
        hip_->hipEventDestroy(p.a);
        hip_->hipEventDestroy(p.b);
    }
    for (auto e : event_pool_) hip_->hipEventDestroy(e);
    for (auto e : ev_)
        if (e) hip_->hipEventDestroy(e);
    if (g2l_) hip_->hipStreamDestroy(g2l_);
    if (side_) hip_->hipStreamDestroy(side_);
    if (stream_) hip_->hipStreamDestroy(stream_);
    if (module_) hip_->hipModuleUnload(module_);
}

bool Engine::check(hipError_t e, const char *what, std::string &err)
{
    if (e == hipSuccess) return true;
    err = hip_error(*hip_, e, what);
    return false;
}

extern "C" const unsigned char lama_hsaco_start[];
extern "C" const unsigned char lama_hsaco_end[];
extern "C" const unsigned char lama_scratch_hsaco_start[];

namespace {
using Clock = std::chrono::steady_clock;
double since(Clock::time_point a) { return std::chrono::duration<double>(Clock::now() - a).count(); }
}  // namespace

bool Engine::open(std::string &err)
{
    const auto t_open = Clock::now();
    hip_ = hip_api(err);
    if (!hip_) return false;
    if (!check(hip_->hipInit(0), "hipInit", err)) return false;
    int count = 0;
    if (!check(hip_->hipGetDeviceCount(&count), "hipGetDeviceCount", err)) return false;
    if (count < 1) {
        err = "no HIP device visible";
        return false;
    }
    const char *dev = getenv("LAMA_HIP_DEVICE");
    device_ = dev ? atoi(dev) : 0;
    if (device_ < 0 || device_ >= count) {
        err = "LAMA_HIP_DEVICE=" + std::to_string(device_) + " but " + std::to_string(count) + " device(s) visible";
        return false;
    }
    if (!check(hip_->hipSetDevice(device_), "hipSetDevice", err)) return false;
    hipDeviceProp_t prop;
    if (!check(hip_->hipGetDevicePropertiesR0600(&prop, device_), "hipGetDeviceProperties", err)) return false;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        err = std::string("device ") + prop.name + " is " + prop.gcnArchName +
              "; this backend carries gfx950 (MI355X) code only";
        return false;
    }
    const double t_runtime = since(t_open);
    const auto t_mod = Clock::now();
    if (!check(hip_->hipModuleLoadData(&module_, lama_hsaco_start), "hipModuleLoadData", err)) return false;
    const double t_kernels = since(t_mod);
    id_ = ++g_engine_ids;
    for (int f = 0; f < F_COUNT; ++f)
        if (!get_fn(fn_[f], kKernelName[f], err)) return false;
    for (int f = 0; f < 4; ++f)
        if (!get_fn(fn_split_[f], kSplitName[f], err)) return false;
    for (int s = 0; s < 2; ++s)
        for (int f = 0; f < 4; ++f)
            if (!get_fn(fn_split_ct_[s][f], kSplitCtName[s][f], err))
                return false;
    for (int f = 0; f < 2; ++f)
        if (!get_fn(fn_pw_any_[f], kPwAnyName[f], err) ||
            !get_fn(fn_pw_v2_[f], kPwV2Name[f], err))
            return false;
    if (!get_fn(fn_wino_, "lama_conv3x3w", err) ||
        !get_fn(fn_wino4_[0], "lama_conv3x3w4", err) ||
        !get_fn(fn_wino4_[1], "lama_conv3x3w4n", err) ||
        !get_fn(fn_wino4_[2], "lama_conv3x3w4q", err) || !get_fn(fn_wino42_, "lama_conv3x3w42", err) ||

        !get_fn(fn_tail_u8_, "lama_tail_u8", err) ||
        !get_fn(fn_finalize_ks_[0], "lama_finalize10", err) ||
        !get_fn(fn_finalize_ks_[1], "lama_finalize20", err) ||
        !get_fn(fn_finalize_g2_[0], "lama_finalize_g2", err) ||
        !get_fn(fn_finalize_g2_[1], "lama_finalize10_g2", err) ||
        !get_fn(fn_finalize_g2_[2], "lama_finalize20_g2", err) ||
        !get_fn(fn_head_r_, "lama_conv7x7r", err) || !get_fn(fn_pw_kh_[0], "lama_conv1x1_kh", err) ||
        !get_fn(fn_pw_kh_[1], "lama_conv1x1_res_kh", err) || !get_fn(fn_edge_q_[0], "lama_conv3x3s2_q", err) ||
        !get_fn(fn_edge_q_[1], "lama_convt_q", err) ||
        !get_fn(fn_convt_rows_[0], "lama_convt_rows", err) ||
        !get_fn(fn_convt_rows_[1], "lama_convt_rows_q", err) || !get_fn(fn_pack_, "lama_pack_wino", err))
        return false;
    fn_build_in_ = fn_[F_INPUT];
    if (const char *wv = getenv("LAMA_FFC_WINO")) {
        const int v = atoi(wv);
        wino_ = v == 0 ? 0 : v == 4 ? 4 : v == 42 ? 42 : 2;
        w42_packed_ = false;  // a forced algorithm runs on every plane
    }
    if (const char *t = getenv("LAMA_W42")) w42_packed_ = w42_packed_ && atoi(t) != 0;
    if (const char *t = getenv("LAMA_HOST_PACK")) dev_pack_ = atoi(t) == 0;
    if (const char *t = getenv("LAMA_W4_TILE")) w4_force_ = atoi(t);
    if (const char *t = getenv("LAMA_KSPLIT")) ksplit_force_ = atoi(t);
    if (const char *t = getenv("LAMA_PW_KSPLIT")) pw_ksplit_force_ = atoi(t);
    if (const char *t = getenv("LAMA_FIN_GROUPS")) fin_groups_force_ = atoi(t);
    if (const char *t = getenv("LAMA_EDGE_TILE")) edge_force_ = atoi(t);
    if (const char *t = getenv("LAMA_PW_TILE")) pw_force_ = atoi(t);
    if (const char *t = getenv("LAMA_W4_LDSPAD")) w4_ldspad_force_ = atoi(t);
    if (const char *t = getenv("LAMA_CONVT_ROWS")) convt_rows_ = atoi(t) != 0;
    if (const char *t = getenv("LAMA_HEAD_R")) head_r_ = atoi(t) != 0;

    for (int s = 0; s < 4; ++s)
        for (int f = 0; f < 2; ++f)
            if (!get_fn(fn_fft_ct_[s][f], kFftCtName[s][f], err))
                return false;
    {
        int lds = 0;
        if (hip_->hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device_) == hipSuccess && lds > 0)
            max_lds_ = (size_t)lds;
        int khz = 0;  // the rate of the s_memrealtime clock the stamps read
        if (hip_->hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device_) == hipSuccess && khz > 0)
            clock_khz_ = khz;
    }
    if (!check(hip_->hipStreamCreate(&stream_), "hipStreamCreate", err) ||
        !check(hip_->hipStreamCreate(&side_), "hipStreamCreate", err) ||
        !check(hip_->hipStreamCreate(&g2l_), "hipStreamCreate", err))
        return false;
    // The cross-stream events only order work between this device's
    // streams: no system-scope fence (a host-visible cache write-back at each
    // record costs microseconds on the critical path).
#ifndef LAMA_EV_FLAGS
#define LAMA_EV_FLAGS (hipEventDisableTiming | hipEventDisableSystemFence)
#endif
    for (auto &e : ev_)
        if (!check(hip_->hipEventCreateWithFlags(&e, LAMA_EV_FLAGS), "hipEventCreate", err)) return false;
    if (!check(hip_->hipEventCreateWithFlags(&ev_done_, hipEventDisableTiming), "hipEventCreate", err)) return false;
    // the reference engine's debug flags (cuda.rs:127-150, 1574): set = present
    flag_profile_ = getenv("LAMA_PROFILE") != nullptr;
    flag_profile_sync_ = getenv("LAMA_PROFILE_SYNC") != nullptr;
    flag_profile_ops_ = getenv("LAMA_PROFILE_OPS") != nullptr;
    flag_profile_sub_ = getenv("LAMA_PROFILE_SUB") != nullptr;
    if (const char *d = getenv("LAMA_DUMP_STEP")) {
        char *end = nullptr;
        const long v = strtol(d, &end, 10);
        dump_step_ = (end != d && *end == 0 && v >= 0 && v < kSteps) ? (int)v : -1;  // parse().ok()
    }
    if (flag_profile_ops_ || flag_profile_sub_) prof_mask_ = (1u << F_COUNT) - 1;
    if (flag_profile_)
        fprintf(stderr, "gpu open: %.3fs (runtime and device %.3fs, kernels %.3fs)\n", since(t_open), t_runtime,
                t_kernels);
    return true;
}

bool Engine::load_weights(const uint8_t *blob, size_t len, const lama_tensor_info *t, size_t n, std::string &err)
{
    const auto t_load = Clock::now();
    WeightSrc S{blob, len, {}};
    for (size_t i = 0; i < n; ++i) S.idx[t[i].name] = &t[i];
    Arena A;
    std::vector<float> w, w2;
    // model.1: 7x7 4 -> 64 (model.rs:142-144)
    if (!S.get("model.1.ffc.convl2l.weight", {64, 4, 7, 7}, w, err)) return false;
    head_ = pack(A, 64, 4, 49, 4, [&](int co, int ci, int t) { return w[((size_t)co * 4 + ci) * 49 + t]; });
    if (!fold_bns(A, S, {{"model.1.bn_l", 64}}, head_bn_, err)) return false;
    // model.2 / model.3: 3x3 s2, local only
    const int dc[2][2] = {{64, 128}, {128, 256}};
    for (int d = 0; d < 2; ++d) {
        const int cin = dc[d][0], cout = dc[d][1];
        const std::string p = "model." + std::to_string(d + 2);
        if (!S.get(p + ".ffc.convl2l.weight", {cout, cin, 3, 3}, w, err)) return false;
        down_[d] = pack(A, cout, cin, 9, LAMA_S2_KC, [&](int co, int ci, int t) { return w[((size_t)co * cin + ci) * 9 + t]; });
        if (!fold_bns(A, S, {{p + ".bn_l", cout}}, down_bn_[d], err)) return false;
    }
    // model.4: 256 -> 128 local + 384 global, stacked along M
    if (!S.get("model.4.ffc.convl2l.weight", {128, 256, 3, 3}, w, err) ||
        !S.get("model.4.ffc.convl2g.weight", {384, 256, 3, 3}, w2, err))
        return false;
    down_[2] = pack(A, 512, 256, 9, LAMA_S2_KC, [&](int co, int ci, int t) {
        return co < 128 ? w[((size_t)co * 256 + ci) * 9 + t] : w2[((size_t)(co - 128) * 256 + ci) * 9 + t];
    });
    if (!fold_bns(A, S, {{"model.4.bn_l", 128}, {"model.4.bn_g", 384}}, down_bn_[2], err)) return false;
    // The Winograd packs of the FFC 3x3 convolutions (F(4,3), and F(2x4, 3x3)
    // for the large planes: 692 of the 749 MB of packed weights) are made on
    // the device from the raw weights (149 MB), laid out after the host-packed
    // part of the arena (offsets relative to that part's end until the upload).
    struct DevJob {
        Packed *p;
        const lama_tensor_info *s0, *s1;
        int kind;
    };
    std::vector<DevJob> dev;
    size_t dev_n = 0;  // floats of the device-packed part
    auto dev_job = [&](Packed &p, const Packed &shape, int kind, const lama_tensor_info *s0,
                       const lama_tensor_info *s1) {
        p = shape;
        p.off = (dev_n + 63) / 64 * 64;
        dev_n = p.off + wino_floats(p);
        dev.push_back({&p, s0, s1, kind});
    };
    const bool dev_wino = dev_pack_ && (wino_ == 4 || wino_ == 42);
    // model.5..22: 36 FFC_BN_ACT (model.rs:157-165), ratio 0.75: 128 local / 384 global
    for (int i = 5; i <= 22; ++i)
        for (int s = 1; s <= 2; ++s) {
            FfcW &F = ffc_[(i - 5) * 2 + (s - 1)];
            const std::string pb = "model." + std::to_string(i) + ".conv" + std::to_string(s);
            const std::string pf = pb + ".ffc";
            std::vector<float> l2l, g2l, l2g, c1, c2, fu;
            const lama_tensor_info *tl2l = S.find(pf + ".convl2l.weight", {128, 128, 3, 3}, err);
            const lama_tensor_info *tg2l = tl2l ? S.find(pf + ".convg2l.weight", {128, 384, 3, 3}, err) : nullptr;
            const lama_tensor_info *tl2g = tg2l ? S.find(pf + ".convl2g.weight", {384, 128, 3, 3}, err) : nullptr;
            if (!tl2g || (!dev_wino && (!S.get(pf + ".convl2l.weight", {128, 128, 3, 3}, l2l, err) ||
                                        !S.get(pf + ".convg2l.weight", {128, 384, 3, 3}, g2l, err) ||
                                        !S.get(pf + ".convl2g.weight", {384, 128, 3, 3}, l2g, err))) ||
                !S.get(pf + ".convg2g.conv1.0.weight", {192, 384, 1, 1}, c1, err) ||
                !S.get(pf + ".convg2g.fu.conv_layer.weight", {384, 384, 1, 1}, fu, err) ||
                !S.get(pf + ".convg2g.conv2.weight", {384, 192, 1, 1}, c2, err))
                return false;
            if (dev_wino) {
                // the F(2x4) packs beside the default F(4,3) ones, for the large planes
                if (w42_packed_) {
                    dev_job(F.local42, wino42_shape(128, 512), 42, tl2l, tg2l);
                    dev_job(F.l2g42, wino42_shape(384, 128), 42, tl2g, nullptr);
                }
                dev_job(F.local, wino_ == 42 ? wino42_shape(128, 512) : wino4_shape(128, 512), wino_, tl2l, tg2l);
                dev_job(F.l2g, wino_ == 42 ? wino42_shape(384, 128) : wino4_shape(384, 128), wino_, tl2g, nullptr);
            } else {
                auto local = [&](int co, int ci, int t) {
                    return ci < 128 ? l2l[((size_t)co * 128 + ci) * 9 + t]
                                    : g2l[((size_t)co * 384 + ci - 128) * 9 + t];
                };
                auto l2gw = [&](int co, int ci, int t) { return l2g[((size_t)co * 128 + ci) * 9 + t]; };
                if (w42_packed_) {
                    F.local42 = pack_wino42(A, 128, 512, local);
                    F.l2g42 = pack_wino42(A, 384, 128, l2gw);
                }
                F.local = wino_ == 42  ? pack_wino42(A, 128, 512, local)
                          : wino_ == 4 ? pack_wino4(A, 128, 512, local)
                          : wino_      ? pack_wino(A, 128, 512, local)
                                       : pack(A, 128, 512, 9, 8, local);
                F.l2g = wino_ == 42  ? pack_wino42(A, 384, 128, l2gw)
                        : wino_ == 4 ? pack_wino4(A, 384, 128, l2gw)
                        : wino_      ? pack_wino(A, 384, 128, l2gw)
                                     : pack(A, 384, 128, 9, 8, l2gw);
            }
            // rows of C channels in order: each launch sets the chunk count of
            // its kernel (pw_kc)
            F.conv2 = pack(A, 384, 192, 1, LAMA_PW_KC, [&](int co, int ci, int) { return c2[(size_t)co * 192 + ci]; });
            F.conv1 = pack(A, 192, 384, 1, LAMA_PW_KC, [&](int co, int ci, int) { return c1[(size_t)co * 384 + ci]; });
            F.fu = pack(A, 384, 384, 1, LAMA_PW_KC, [&](int co, int ci, int) { return fu[(size_t)co * 384 + ci]; });
            if (!fold_bns(A, S, {{pf + ".convg2g.conv1.1", 192}}, F.bn1, err) ||
                !fold_bns(A, S, {{pf + ".convg2g.fu.bn", 384}}, F.fu_bn, err) ||
                !fold_bns(A, S, {{pb + ".bn_l", 128}}, F.bn_l, err) || !fold_bns(A, S, {{pb + ".bn_g", 384}}, F.bn_g, err))
                return false;
        }
    // model.24/27/30: ConvTranspose2d k3 s2 p1 op1 + BN (model.rs:172-201)
    const int ups[3][3] = {{24, 512, 256}, {27, 256, 128}, {30, 128, 64}};
    for (int u = 0; u < 3; ++u) {
        UpW &U = up_[u];
        U.cin = ups[u][1];
        U.cout = ups[u][2];
        const std::string p = "model." + std::to_string(ups[u][0]);
        std::vector<float> bias;
        if (!S.get(p + ".weight", {U.cin, U.cout, 3, 3}, w, err) || !S.get(p + ".bias", {U.cout}, bias, err))
            return false;
        // sub-pixel phase taps (convt_tap): one pack of all nine, or one per phase
        if (convt_rows_) {
            for (int py = 0; py < 2; ++py) U.row[py] = pack_convt_rows(A, U.cout, U.cin, py, w.data());
        } else {
            for (int ph = 0; ph < 4; ++ph) U.ph[ph] = pack_convt_phase(A, U.cout, U.cin, ph, w.data());
        }
        U.bias = A.add(U.cout);
        std::copy(bias.begin(), bias.end(), A.at(U.bias));
        if (!fold_bns(A, S, {{"model." + std::to_string(ups[u][0] + 1), U.cout}}, U.bn, err)) return false;
    }
    // model.34: 7x7 64 -> 3 with bias
    std::vector<float> tb;
    if (!S.get("model.34.weight", {3, 64, 7, 7}, w, err) || !S.get("model.34.bias", {3}, tb, err)) return false;
    tail_w_ = A.add(w.size());
    std::copy(w.begin(), w.end(), A.at(tail_w_));
    tail_b_ = A.add(3);
    std::copy(tb.begin(), tb.end(), A.at(tail_b_));

    // one upload (cuda.rs:330-369 does one HtoD of the raw file), into a new
    // arena: the engine's state changes only once it has succeeded, so a
    // failed load leaves the previous weights and their plans usable
    const size_t dev_base = (A.size() + 63) / 64 * 64, total = dev.empty() ? A.size() : dev_base + dev_n;
    for (DevJob &j : dev) j.p->off += dev_base;
    // The device-packed part: zeroed (rows past M, channels past C), the raw
    // matrices copied once each into a temporary buffer, one lama_pack_wino
    // launch over all jobs, then the temporaries freed.
    auto pack_on_device = [&](float *w) {
        if (dev.empty()) return true;
        std::map<const lama_tensor_info *, size_t> raw_off;
        size_t raw_n = 0;
        for (const DevJob &j : dev)
            for (const lama_tensor_info *t : {j.s0, j.s1})
                if (t && !raw_off.count(t)) {
                    raw_off[t] = raw_n;
                    raw_n += (t->nbytes / 4 + 63) / 64 * 64;
                }
        float *raw = nullptr;
        WinoPackJob *djobs = nullptr;
        auto done = [&](bool ok) {
            if (raw) hip_->hipFree(raw);
            if (djobs) hip_->hipFree(djobs);
            return ok;
        };
        if (!check(hip_->hipMemset(w + dev_base, 0, dev_n * 4), "hipMemset(weights)", err) ||
            !check(hip_->hipMalloc((void **)&raw, raw_n * 4), "hipMalloc(raw weights)", err))
            return done(false);
        for (const auto &kv : raw_off)
            if (!check(hip_->hipMemcpy(raw + kv.second, blob + kv.first->offset, kv.first->nbytes,
                                       hipMemcpyHostToDevice),
                       "hipMemcpy(raw weights)", err))
                return done(false);
        std::vector<WinoPackJob> jobs(dev.size());
        long most = 0;
        for (size_t i = 0; i < dev.size(); ++i) {
            const DevJob &d = dev[i];
            WinoPackJob &J = jobs[i];
            J = WinoPackJob{};
            J.src0 = raw + raw_off[d.s0];
            J.src1 = d.s1 ? raw + raw_off[d.s1] : nullptr;
            J.dst = w + d.p->off;
            J.M = d.p->M;
            J.C = d.p->C;
            J.C0 = (int)d.s0->shape[1];  // input channels from src0; the rest from src1
            J.nchunk = d.p->nchunk;
            J.kind = d.kind;
            if ((J.C0 < J.C) != (d.s1 != nullptr) || d.s0->shape[0] != J.M ||
                (d.s1 && (d.s1->shape[0] != J.M || d.s1->shape[1] != J.C - J.C0))) {
                err = "internal: inconsistent weight pack job";
                return done(false);
            }
            most = std::max(most, (long)J.M * J.C);
        }
        if (!check(hip_->hipMalloc((void **)&djobs, jobs.size() * sizeof(WinoPackJob)), "hipMalloc(pack jobs)",
                   err) ||
            !check(hip_->hipMemcpy(djobs, jobs.data(), jobs.size() * sizeof(WinoPackJob), hipMemcpyHostToDevice),
                   "hipMemcpy(pack jobs)", err))
            return done(false);
        void *params[1] = {&djobs};
        const unsigned gx = (unsigned)std::min<long>(256, (most + 255) / 256);
        if (!check(hip_->hipModuleLaunchKernel(fn_pack_, gx, (unsigned)jobs.size(), 1, 256, 1, 1, 0, stream_, params,
                                               nullptr),
                   "lama_pack_wino", err) ||
            !check(hip_->hipStreamSynchronize(stream_), "lama_pack_wino", err))
            return done(false);
        return done(true);
    };
    const double t_host = since(t_load);
    const auto t_up = Clock::now();
    float *fresh = nullptr;
    if (!check(hip_->hipMalloc((void **)&fresh, total * 4), "hipMalloc(weights)", err)) return false;
    if (!A.upload(hip_, fresh, err)) {
        hip_->hipFree(fresh);
        return false;
    }
    const double t_upload = since(t_up);
    const auto t_dev = Clock::now();
    if (!pack_on_device(fresh)) {
        hip_->hipFree(fresh);
        return false;
    }
    const double t_device = since(t_dev);
    // plans hold pointers into the old arena; no pass may still read it
    if (!check(hip_->hipDeviceSynchronize(), "hipDeviceSynchronize", err)) {
        hip_->hipFree(fresh);
        return false;
    }
    for (auto &kv : plans_) free_plan(kv.second);
    plans_.clear();
    for (auto &kv : spec_plans_)
        if (kv.second.arena) hip_->hipFree(kv.second.arena);
    spec_plans_.clear();
    na_plan_ = Plan{};  // its descriptors point into the old weights
    release_scratch_owner();
    if (warena_) hip_->hipFree(warena_);
    warena_ = fresh;
    warena_bytes_ = total * 4;
    if (flag_profile_)
        fprintf(stderr,
                "gpu weights: %.3fs, %.1f MB resident (host packing %.3fs, arena allocation and upload of %.1f MB %.3fs, "
                "raw 3x3 upload and Winograd packing on the device %.3fs)\n",
                since(t_load), total * 4 / 1e6, t_host, A.size() * 4 / 1e6, t_upload, t_device);
    have_weights_ = true;
    return true;
}

bool Engine::fft_len(int n, FftLen &L, std::vector<float> &tw, std::string &err)
{
    std::memset(&L, 0, sizeof L);
    L.n = n;
    L.sign_fwd = is_pow2(n) ? -1 : 1;
    int m = n;
    auto push = [&](int r) {
        if (L.nstages >= 16) return false;
        L.radix[L.nstages++] = r;
        m /= r;
        return true;
    };
    while (m % 8 == 0)
        if (!push(8)) break;
    while (m % 4 == 0)
        if (!push(4)) break;
    while (m % 2 == 0)
        if (!push(2)) break;
    for (int p = 3; m > 1 && p <= m; p += 2)
        while (m % p == 0)
            if (!push(p)) break;
    if (m != 1) {
        err = "FFT length " + std::to_string(n) + " needs too many passes";
        return false;
    }
    tw.resize(2 * (size_t)n);
    for (int k = 0; k < n; ++k) {
        const double a = -2.0 * M_PI * (double)k / (double)n;
        tw[2 * k] = (float)std::cos(a);
        tw[2 * k + 1] = (float)std::sin(a);
    }
    return true;
}

// Single-block mode keeps a whole plane (two ping-pong buffers + both
// twiddle tables) in one block's LDS; it is used while that fits in 64 KB.
// Larger planes (or LAMA_FFT_SPLIT=1) use the row/column launches, each
// block holding at most LAMA_FFT_SPLIT_LDS bytes of ping-pong buffers.
// The kernel of a conv launch: the 1x1 families use float4 activation loads
// only when every plane is 16-byte aligned and a multiple of 4 floats long.
hipFunction_t Engine::conv_fn(int family, const ConvProblem *probs, size_t n, int wino) const
{
    if (wino < 0) wino = wino_;
    // the head as one chunk and one M block: the kernel with register-resident weights
    if (family == F_CONV7 && head_r_ && n == 1 && probs[0].s0.nchunk == 1 && probs[0].mblocks == 1) return fn_head_r_;
    if ((family == F_CONV3 || family == F_CONV3G) && wino == 42) return fn_wino42_;
    if ((family == F_CONV3 || family == F_CONV3G) && wino == 4) return fn_wino4_[w4_variant(probs[0].OH, probs[0].OW)];
    if ((family == F_CONV3 || family == F_CONV3G) && wino) return fn_wino_;
    if (family == F_CONVT && convt_rows_) return fn_convt_rows_[tile_variant(family, probs[0].OH, probs[0].OW)];
    if ((family == F_CONV3S2 || family == F_CONVT) && tile_variant(family, probs[0].OH, probs[0].OW) == 1)
        return fn_edge_q_[family == F_CONVT];
    if (family != F_CONV1 && family != F_CONV1R) return fn_[family];
    // the widest activation loads every plane of the launch allows: float4
    // runs need 16-byte aligned planes a multiple of 4 floats apart (the last
    // run of a plane may then read up to 3 floats of its padding)
    bool v4 = true, v2 = true;
    for (size_t i = 0; i < n; ++i) {
        const ConvSeg &s = probs[i].s0;
        const size_t N = (size_t)s.IH * s.IW;
        if (s.cs % 4 != 0 || (uintptr_t)s.src % 16 != 0) v4 = false;
        if (N % 2 != 0 || s.cs % 2 != 0 || N < 4 || (uintptr_t)s.src % 8 != 0) v2 = false;
    }
    const int vw = v4 ? 4 : v2 ? 2 : 1;
    if (vw == 4 && tile_variant(family, probs[0].OH, probs[0].OW, probs[0].M, probs[0].s0.cs) == 0)
        return fn_pw_kh_[family == F_CONV1R];
    return vw == 4 ? fn_[family] : vw == 2 ? fn_pw_v2_[family == F_CONV1R] : fn_pw_any_[family == F_CONV1R];
}

// F(4,3) blocks of 32 Winograd tiles: 2 rows x 64 pixels (lama_conv3x3w4),
// 4 x 32 (w4n) or 8 x 16 (w4q).  The shape that covers the plane with the
// fewest blocks, 2 x 64 on a tie; LAMA_W4_TILE=64, 32 or 16 (read at open)
// forces one.  Measured with the current kernels (passes/s, 64 / 32-pixel
// blocks, each as many blocks): 512x512 281.2 / 277.8-278.0, 1024x1024
// 79.7-80.1 / 77.6-77.7, 2048x2048 20.63-20.71 / 20.43-20.54; 600x600 (76 /
// 57 / 50 blocks of 64 / 32 / 16 pixels) 148.8 / - / 166.4.  (With the
// LDS-staged weights and 64 x 64 pointwise tiles 2 x 64 had been the
// slowest: 512x512 228.7 vs 253.6.)
int Engine::w4_variant(int OH, int OW) const
{
    if (w4_force_ == 64) return 0;
    if (w4_force_ == 32) return 1;
    if (w4_force_ == 16) return 2;
    auto blocks = [&](int v) {
        const int tr = 2 << v, tc = 128 / tr;
        return (long)((OW + tc - 1) / tc) * ((OH + tr - 1) / tr);
    };
    // fewest blocks; on a tie 2 x 64 before 4 x 32 before 8 x 16
    int best = 1;
    if (blocks(2) < blocks(best)) best = 2;
    if (blocks(0) <= blocks(best)) best = 0;
    return best;
}

// Tile variant of a conv family at an OH x OW output (for the transposed
// convolution, the phase grid): the F(4,3) block shape, or for the
// stride-2 and transposed convolutions 4 x 16 tiles (1) where they cover the
// plane with fewer tiles than 2 x 32 (0), which is where the width leaves
// much of a 32-pixel row empty (75: 3 x 32 columns for 75, 5 x 16 for 80).
// LAMA_EDGE_TILE=32 or 16 (read at open) forces one.
int Engine::tile_variant(int family, int OH, int OW, int M, long cs) const
{
    if (family == F_CONV3 || family == F_CONV3G) return w4_variant(OH, OW);
    // pointwise over N = OH * OW pixels into M channels, input planes cs
    // floats apart (0: N): 0 = the K-half kernels, for float4-aligned planes
    // (cs % 4 == 0) whose 64 x 64 tiles would give at most two workgroups per
    // CU (512x512: 277.8-278.1 vs 274.8 passes/s with conv1 and the FU conv
    // in them, 256x256 429-436 vs 426; at 1024x1024 and 2048x2048, with three
    // or more workgroups per CU, 64 x 64 tiles were 1-2% faster); 1 = 64 x 64
    // tiles
    if (family == F_CONV1 || family == F_CONV1R) {
        const long n = (long)OH * OW, tiles = (n + 63) / 64 * ((M + 63) / 64);
        const bool kh = pw_force_ ? pw_force_ == 32 : tiles <= 2 * LAMA_CUS;
        return LAMA_PW_KH && (cs ? cs : n) % 4 == 0 && kh ? 0 : 1;
    }
    if (family != F_CONV3S2 && family != F_CONVT) return 0;
    if (edge_force_ == 32) return 0;
    if (edge_force_ == 16) return 1;
    const long t32 = (long)((OW + 31) / 32) * ((OH + 1) / 2), t16 = (long)((OW + 15) / 16) * ((OH + 3) / 4);
    return t16 < t32 ? 1 : 0;
}

// Dynamic LDS added to each F(4,3) workgroup (bytes), to hold the GEMMs at
// two workgroups per CU.  The kernels need 33.5 KB and 132-138 registers, so
// three fit on a CU.  Padding was faster where the FFC's A and B launches
// have between two and four workgroups per CU (600 x 600: 800 workgroups)
// while the SpectralTransform's 1x1 convolutions ran with per-element loads
// on the unaligned 75 x 75 planes (159.8 padded vs 157.9 passes/s); with the
// planes at 16-byte aligned strides and float4 loads, three GEMM workgroups
// per CU are faster there (175.2-175.3 vs 161.5-171.9), so it is off unless
// LAMA_W4_LDSPAD=1 (read at open) forces it on.
unsigned Engine::w4_lds_pad(int h8, int w8, int ks) const
{
    (void)h8;
    (void)w8;
    (void)ks;
    return wino_ == 4 && w4_ldspad_force_ == 1 ? 24576u : 0u;
}

// The FFC GEMMs' K split: at small planes the F(4,3) launches have few
// workgroups (16 per block of 4 rows x 32 pixels for A and B together, 128 at
// 256 x 256), each walking the whole K, and most CUs idle; splitting K into s
// slices (raw partials summed by finalize, and by conv2's epilogue for l2g)
// gives s times the workgroups with 1/s of the K loop.  The largest s of
// 1, 2, 4 that keeps A and B within two workgroups per CU.
int Engine::ksplit_for(int h, int w) const
{
    const int wm = wino_for(h / 8, w / 8);
    if (wm != 4 && wm != 42) return 1;
    if (ksplit_force_ == 1 || ksplit_force_ == 2 || ksplit_force_ == 4) return ksplit_force_;
    int tr, tc;
    tile_shape(F_CONV3, tr, tc, wm, w4_variant(h / 8, w / 8));
    const int tiles = ((w / 8 + tc - 1) / tc) * ((h / 8 + tr - 1) / tr);
    // every slice an even number of chunks: the l2l and l2g ranges (128
    // channels) and each of the g2l ranges (384 / LAMA_G2L_RANGES)
    const int kc = wm == 42 ? LAMA_W42_KC : LAMA_WINO_KC;
    auto even = [&](int s) { return (128 / kc) % (2 * s) == 0 && (384 / LAMA_G2L_RANGES / kc) % (2 * s) == 0; };
    int s = 1;
    while (s < LAMA_KSPLIT_MAX && 16 * tiles * (2 * s) <= 2 * LAMA_CUS && even(2 * s)) s *= 2;
    return s;
}

// The FFC 3x3 algorithm of an h8 x w8 bottleneck plane: LAMA_FFC_WINO's,
// except that the default F(4,3) hands the plane to F(2x4, 3x3) where the
// l2l + l2g launch has at least two of its workgroups (64 channels x 4 rows
// x 64 pixels) per CU and its 64-pixel columns overhang the plane by at most
// an eighth of its width: 1024 x 1024 inputs and up.  Measured (passes/s,
// F(4,3) / F(2x4)): 2048x2048 21.3-21.6 / 22.3-22.5, 1024x1024 80.9-81.2 /
// 84.1-84.6, 512x512 286.7 / 249.6 (128 workgroups); LAMA_W42=0 (read at
// open) keeps F(4,3) everywhere.
int Engine::wino_for(int h8, int w8) const
{
    if (wino_ != 4 || !w42_packed_) return wino_;
    const long blocks = (long)((h8 + 3) / 4) * ((w8 + 63) / 64) * (512 / 64);
    const int overhang = (w8 + 63) / 64 * 64 - w8;
    return blocks >= 2 * LAMA_CUS && 8 * overhang <= w8 ? 42 : 4;
}

// Groups of 4 elements per finalize thread (1 or 2): two where one group per
// thread would give fewer blocks than CUs or between 2.5 and 4 per CU.
// Measured: at 32 x 32 (128 blocks with one group) two groups gave 448.8-450.4
// vs 431.3-437.1 passes/s; at 75 x 75
// 768 blocks ran slower beside the concurrent kernels than 384 (157.4 vs
// 158.9 passes/s); at 64 x 64 512 blocks ran faster than 256 (260.2 vs
// 258.5); at 128 x 128 and 256 x 256 planes (8 and 32 blocks per CU) one
// group was as fast or 0.3% faster.
int Engine::fin_groups(size_t plane) const
{
    if (fin_groups_force_ == 1 || fin_groups_force_ == 2) return fin_groups_force_;
    const size_t blocks = 128 * ((plane + 4 * LAMA_NT - 1) / (4 * LAMA_NT));
    return blocks < (size_t)LAMA_CUS || (2 * blocks > 5 * (size_t)LAMA_CUS && blocks <= 4 * (size_t)LAMA_CUS) ? 2 : 1;
}

// The K split of the SpectralTransform's two pointwise convolutions that
// feed a transform (conv1: 384 -> 192 over the x_g planes; the FourierUnit
// conv: 384 -> 384 over the spectrum): at small planes their 64 x 64 tiles
// leave most CUs idle while each wave walks K = 384, so the launch is split
// into s K slices of raw partials that the single-block transform sums (with
// the BN + ReLU) while loading them.  The largest s of 1, 2, 4 that keeps the
// launch within LAMA_PW_KSPLIT_WG workgroups, one per CU; 1 with split-mode
// transforms.  Measured (passes/s, split / unsplit): 256x256 (s = 4) 411.2 /
// 384.7; 512x512 with s = 2 (two workgroups per CU) 241.8 / 253.1, so 512x512
// stays unsplit.  LAMA_PW_KSPLIT=1, 2 or 4 (read at open) forces s.
#ifndef LAMA_PW_KSPLIT_WG
#define LAMA_PW_KSPLIT_WG LAMA_CUS
#endif
void Engine::pw_ksplit_for(int h, int w, const FftGeom &fg, int &k1, int &ku) const
{
    k1 = ku = 1;
    if (fg.split) return;
    const long p8 = (long)(h / 8) * (w / 8), ps = (long)(h / 8) * ((w / 8) / 2 + 1);
    auto pick = [&](long nb) {
        if (pw_ksplit_force_ == 1 || pw_ksplit_force_ == 2 || pw_ksplit_force_ == 4) return pw_ksplit_force_;
        int s = 1;
        while (s < LAMA_PW_KSPLIT_MAX && nb * 2 * s <= LAMA_PW_KSPLIT_WG) s *= 2;
        return s;
    };
    auto blocks = [&](long n, int m) {  // workgroups of the launch's tile variant (padded planes)
        const long tc = tile_variant(F_CONV1, 1, (int)n, m, (long)pad4(n)) == 0 ? 32 : 64;
        return (n + tc - 1) / tc * ((m + 63) / 64);
    };
    k1 = pick(blocks(p8, 192));
    ku = pick(blocks(ps, 384));
}

bool Engine::fft_geom(int C, int H, int W, FftGeom &g, std::string &err) const
{
    const int Wh = W / 2 + 1, HP = (H + 1) / 2;
    const size_t f2 = 8;  // bytes per complex value
    g = FftGeom{};
    g.lds = (2 * (size_t)lama_fft_nb(H, W) + H + W) * f2;
    const char *env = getenv("LAMA_FFT_SPLIT");
    const bool force = env && atoi(env) == 1;
    // the single-block kernels fetch at most 8 plane values per thread
    const bool fits = std::max((size_t)HP * W, (size_t)H * Wh) <= 8 * (size_t)LAMA_FFT_NT;
    if (!force && fits && g.lds <= std::min<size_t>(max_lds_, 64 * 1024)) {
        g.grid_rows = g.grid_cols = (unsigned)C;  // one block per plane
        // square 64, 32 or 75 planes have kernels with the shape compiled in
        // (LAMA_FFT_GENERIC=1 keeps the runtime-shaped ones, for tests)
        const char *gen = getenv("LAMA_FFT_GENERIC");
        const char *shfl = getenv("LAMA_FFT64_SHFL");
        if (H == W && !(gen && atoi(gen) == 1))
            for (int s = 0; s < 3; ++s)
                if (H == kFftCtSide[s]) {
                    g.ct = (s == 0 && shfl && atoi(shfl) == 1) ? 4 : s + 1;
                    if (kFftCtInPlace[s]) g.lds = ((size_t)lama_fft_nb(H, W) + H + W) * f2;
                }
        return true;
    }
    // complex values the two ping-pong buffers may hold next to the twiddles
    const size_t cap = max_lds_ / f2, buf = LAMA_FFT_SPLIT_LDS / f2;
    const size_t avail_r = cap > (size_t)W ? std::min(buf, cap - W) : 0;
    const size_t avail_c = cap > (size_t)H ? std::min(buf, cap - H) : 0;
    g.split = true;
    g.rows_per_block = (int)std::max<size_t>(1, std::min<size_t>(HP, avail_r / (2 * (size_t)W)));
    g.cols_per_block = (int)std::max<size_t>(1, std::min<size_t>(Wh, avail_c / (2 * (size_t)H)));
    g.lds_rows = (2 * (size_t)g.rows_per_block * W + W) * f2;
    g.lds_cols = (2 * (size_t)g.cols_per_block * H + H) * f2;
    if (g.lds_rows > max_lds_ || g.lds_cols > max_lds_) {
        err = "FFT plane " + std::to_string(W) + "x" + std::to_string(H) + " needs more LDS per block than the device has";
        return false;
    }
    g.grid_rows = (unsigned)(C * ((HP + g.rows_per_block - 1) / g.rows_per_block));
    g.grid_cols = (unsigned)(C * ((Wh + g.cols_per_block - 1) / g.cols_per_block));
    g.tmp_bytes = (size_t)C * H * Wh * f2;
    // square 256 or 128 planes have split kernels with the shape compiled in,
    // whose blocks hold LAMA_FFT_SPLIT_LDS / (16 N) row pairs or columns
    // (LAMA_FFT_GENERIC=1 keeps the runtime-shaped ones, for tests)
    const char *gen = getenv("LAMA_FFT_GENERIC");
    const int per_block = (int)(buf / (2 * (size_t)H));
    if (H == W && (H == 256 || H == 128) && !(gen && atoi(gen) == 1) && g.rows_per_block == per_block &&
        g.cols_per_block == per_block)
        g.ct_split = H;
    // the 256 x 256 column launches: four-step blocks of LAMA_FFT_C4 columns
    // (16 threads each) plus one Nyquist-column block per channel
    if (g.ct_split == 256) {
        g.grid_cols = (unsigned)(C * (128 / LAMA_FFT_C4 + 1));
        g.block_cols = 16 * LAMA_FFT_C4;
        g.lds_cols = (std::max<size_t>(256 * LAMA_FFT_C4, 2 * (size_t)per_block * 256) + 256) * f2;
    }
    return true;
}

// The launches of one rfft2 (inverse = false) or irfft2 over the descriptor
// `arg`: one in single-block mode, row + column launches in split mode (the
// inverse runs columns first).  bytes_a / bytes_b: algorithmic bytes of the
// input and output sides, for the profile.
void Engine::push_fft(Plan &p, bool inverse, const FftGeom &g, void *arg, int stream, double bytes_a, double bytes_b)
{
    Launch L{};
    L.family = inverse ? F_IRFFT : F_RFFT;
    L.block = LAMA_FFT_NT;
    L.stream = stream;
    L.wait_ev = L.record_ev = -1;
    L.arg = arg;
    L.nparams = 1;
    L.step_end = -1;
    if (!g.split) {
        L.fn = g.ct ? fn_fft_ct_[g.ct - 1][inverse ? 1 : 0] : fn_[L.family];
        L.grid = g.grid_rows;
        L.shmem = (unsigned)g.lds;
        L.bytes = bytes_a + bytes_b;
        p.launches.push_back(L);
        return;
    }
    for (int k = 0; k < 2; ++k) {
        const bool rows = inverse ? k == 1 : k == 0;
        L.fn = g.ct_split ? fn_split_ct_[g.ct_split == 256 ? 0 : 1][inverse ? 2 + k : k] : fn_split_[inverse ? 2 + k : k];
        L.grid = rows ? g.grid_rows : g.grid_cols;
        L.block = !rows && g.block_cols ? g.block_cols : LAMA_FFT_NT;
        L.shmem = (unsigned)(rows ? g.lds_rows : g.lds_cols);
        L.bytes = k == 0 ? bytes_a : bytes_b;
        p.launches.push_back(L);
    }
}

// Input shapes the plan supports: multiples of 8, and at most 2^27 pixels --
// the convolution kernels address one K chunk (at most 8 channels of a
// full-resolution plane) with 32-bit byte offsets, 32 * h * w < 2^32.
static bool shape_ok(int h, int w, std::string &err)
{
    if (h < 8 || w < 8 || h % 8 || w % 8) {
        err = "input " + std::to_string(w) + "x" + std::to_string(h) + " is not a multiple of 8 (the caller pads)";
        return false;
    }
    if ((size_t)h * w > ((size_t)1 << 27)) {
        err = "input " + std::to_string(w) + "x" + std::to_string(h) + " exceeds 2^27 pixels, the largest this engine plans";
        return false;
    }
    return true;
}

Plan *Engine::plan_for(int h, int w, std::string &err)
{
    if (!have_weights_) {
        err = "no weights loaded";
        return nullptr;
    }
    if (!shape_ok(h, w, err)) return nullptr;
    auto key = std::make_pair(h, w);
    auto it = plans_.find(key);
    if (it != plans_.end()) return &it->second;
    Plan p;
    p.H = h;
    p.W = w;
    if (!build_plan(p, nullptr, err) || !upload_plan(p, nullptr, err)) {
        free_plan(p);
        return nullptr;
    }
    return &(plans_[key] = std::move(p));
}

// Copies what build_plan staged on the host (descriptors, twiddles) into the
// plan's arena: synchronously when s is null, else enqueued on s.
bool Engine::upload_plan(const Plan &p, hipStream_t s, std::string &err)
{
    char *base = (char *)p.arena;
    const std::pair<size_t, std::pair<const void *, size_t>> parts[3] = {
        {p.desc_off, {p.desc_host.data(), p.desc_host.size()}},
        {p.twr_off, {p.twr_host.data(), p.twr_host.size() * 4}},
        {p.twc_off, {p.twc_host.data(), p.twc_host.size() * 4}}};
    for (const auto &q : parts) {
        const hipError_t e = s ? hip_->hipMemcpyAsync(base + q.first, q.second.first, q.second.second,
                                                      hipMemcpyHostToDevice, s)
                               : hip_->hipMemcpy(base + q.first, q.second.first, q.second.second, hipMemcpyHostToDevice);
        if (!check(e, "hipMemcpy(plan descriptors)", err)) return false;
    }
    return true;
}

// Byte offsets of every buffer of the per-shape activation arena (each
// 256-byte aligned) and its total size.
size_t Engine::arena_layout(int H, int W, const FftGeom &fg, size_t ntwr, size_t ntwc, int ksplit, int pk1, int pku,
                            ArenaLayout &L)
{
    const size_t P = (size_t)H * W, P2 = (size_t)(H / 2) * (W / 2), P4 = (size_t)(H / 4) * (W / 4);
    // bottleneck and spectrum planes at their padded strides
    const size_t P8 = pad4((size_t)(H / 8) * (W / 8)), PS = pad4((size_t)(H / 8) * ((W / 8) / 2 + 1));
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off = (off + bytes + 255) / 256 * 256;
        return o;
    };
    L.in = take(4 * P * 4);
    L.a1 = take(64 * P * 4);
    L.a2 = take(128 * P2 * 4);
    L.a3 = take(256 * P4 * 4);
    L.x = take(512 * P8 * 4);
    L.y = take(512 * P8 * 4);
    L.f = take((size_t)pk1 * 192 * P8 * 4);  // conv1's output (its K partials when split)
    L.g = take(192 * P8 * 4);
    L.s = take(384 * PS * 4);
    L.s2 = take((size_t)pku * 384 * PS * 4);  // the FourierUnit conv's output (partials when split)
    L.out = take(3 * P * 4);
    // the l2g partials (ksplit of them), double-buffered by FFC parity
    L.gc = take(2 * (size_t)ksplit * 384 * P8 * 4);
    // the FFC local GEMM's K-range partials: l2l (ksplit of them), then the g2l
    // ranges twice (by FFC parity: B(k+1) may run while finalize(k) still
    // reads B(k)'s)
    L.lq = take((size_t)ksplit * (1 + 2 * LAMA_G2L_RANGES) * 128 * P8 * 4);
    L.tmp = take(fg.split ? fg.tmp_bytes : 0);
    L.twr = take(ntwr * 4);
    L.twc = take(ntwc * 4);
    L.rgb8 = take(3 * P);
    L.mask8 = take(P);
    L.out8 = take(3 * P);
    const size_t n_conv = 4 + 36 * 9 + 4 * 3;      // problems
    const size_t n_fft = 2 + 2 * 36;                      // FFT descriptors (per FFC with a pointwise K split)
    const size_t n_puts = 4 + 36 * 6 + 3 + 3 + 4 + n_fft;  // descriptor uploads, each 256-byte aligned
    L.desc = take(n_conv * sizeof(ConvProblem) + n_fft * sizeof(FftArgs) + 2 * sizeof(TailArgs) + sizeof(InputArgs) +
                  n_puts * 256 + 4096);
    return off;
}

bool Engine::plan_bytes(int h, int w, uint64_t &arena, uint64_t &weights, std::string &err)
{
    if (!shape_ok(h, w, err)) return false;
    auto it = plans_.find({h, w});
    weights = warena_bytes_;
    if (it != plans_.end()) {
        arena = it->second.arena_bytes;
        return true;
    }
    FftLen fr, fc;
    std::vector<float> twr, twc;
    FftGeom fg;
    if (!fft_len(w / 8, fr, twr, err) || !fft_len(h / 8, fc, twc, err) || !fft_geom(192, h / 8, w / 8, fg, err))
        return false;
    ArenaLayout lay;
    int pk1, pku;
    pw_ksplit_for(h, w, fg, pk1, pku);
    arena = arena_layout(h, w, fg, twr.size(), twc.size(), ksplit_for(h, w), pk1, pku, lay);
    return true;
}

// Lays out the activation arena of p's shape and records its launch list.
// `arena` null: the engine allocates the arena; else the plan uses that
// memory (at least p.arena_bytes).  The descriptors and twiddles are staged
// in p.desc_host / twr_host / twc_host for upload_plan.
bool Engine::build_plan(Plan &p, void *arena, std::string &err)
{
    const int H = p.H, W = p.W, H2 = H / 2, W2 = W / 2, H4 = H / 4, W4 = W / 4, H8 = H / 8, W8 = W / 8;
    const int Wh = W8 / 2 + 1;
    const size_t P = (size_t)H * W, P2 = (size_t)H2 * W2, P4 = (size_t)H4 * W4, P8 = (size_t)H8 * W8;
    const size_t PS = (size_t)H8 * Wh;
    // plane strides of the bottleneck activations and the spectrum (pad4)
    const size_t P8s = pad4(P8), PSs = pad4(PS);

    FftLen frow, fcol;
    std::vector<float> twr, twc;
    if (!fft_len(W8, frow, twr, err) || !fft_len(H8, fcol, twc, err)) return false;
    FftGeom fg;
    if (!fft_geom(192, H8, W8, fg, err)) return false;

    ArenaLayout lay;
    const int ks = ksplit_for(H, W);
    const int wm = wino_for(H8, W8);  // the FFC 3x3 algorithm of this plane
    const unsigned w4_shmem = wm == 4 ? w4_lds_pad(H8, W8, ks) : 0u;
    int pk1, pku;  // K split of the SpectralTransform conv1 and of the FourierUnit conv
    pw_ksplit_for(H, W, fg, pk1, pku);
    p.arena_bytes = arena_layout(H, W, fg, twr.size(), twc.size(), ks, pk1, pku, lay);
    const size_t o_in = lay.in, o_a1 = lay.a1, o_a2 = lay.a2, o_a3 = lay.a3, o_x = lay.x, o_y = lay.y, o_f = lay.f,
                 o_g = lay.g, o_s = lay.s, o_s2 = lay.s2, o_out = lay.out, o_gc = lay.gc, o_lq = lay.lq, o_tmp = lay.tmp,
                 o_twr = lay.twr, o_twc = lay.twc, o_desc = lay.desc;
    if (arena) {
        p.arena = arena;
        p.own_arena = false;
    } else {
        if (!check(hip_->hipMalloc(&p.arena, p.arena_bytes), "hipMalloc(activations)", err)) return false;
        p.own_arena = true;
    }
    char *base = (char *)p.arena;
    auto F = [&](size_t o) { return (float *)(base + o); };
    float *in = F(o_in), *a1 = F(o_a1), *a2 = F(o_a2), *a3 = F(o_a3), *X = F(o_x), *Y = F(o_y), *Fb = F(o_f),
          *G = F(o_g), *Sb = F(o_s), *S2 = F(o_s2), *out = F(o_out), *GC = F(o_gc), *LQ = F(o_lq);
    p.in = in;
    p.out = out;
    p.rgb8 = (uint8_t *)(base + lay.rgb8);
    p.mask8 = (uint8_t *)(base + lay.mask8);
    p.out8 = (uint8_t *)(base + lay.out8);
    frow.tw = F(o_twr);
    fcol.tw = F(o_twc);

    // descriptors, staged on the host and uploaded once
    std::vector<char> desc;
    auto put = [&](const void *src, size_t bytes) {
        size_t o = (desc.size() + 255) / 256 * 256;
        desc.resize(o + bytes);
        std::memcpy(desc.data() + o, src, bytes);
        return (void *)(base + o_desc + o);
    };
    auto seg = [&](const float *src, const Packed &pk, int C, int IH, int IW, size_t cs = 0) {
        ConvSeg s{};
        s.src = src;
        s.wt = wp(pk.off);
        s.C = C;
        s.IH = IH;
        s.IW = IW;
        s.nchunk = pk.nchunk;
        s.wrow = pk.wrow;
        s.cs = (int)(cs ? cs : (size_t)IH * IW);
        return s;
    };
    bool bad_problem = false;
    auto problem = [&](int family, const ConvSeg &s0, int M, int OH, int OW, size_t bn, int bn_n, float *o,
                       size_t ocs, int outW, const float *res) {
        ConvProblem q{};
        q.s0 = s0;
        q.M = M;
        q.OH = OH;
        q.OW = OW;
        int tr, tc;
        tile_shape(family, tr, tc, wm, tile_variant(family, OH, OW, M, s0.cs));
        q.tiles_x = (OW + tc - 1) / tc;
        q.tiles_y = (OH + tr - 1) / tr;
        // output channels per block: 64, or the F(2x4) kernel's LAMA_W42_CH
        const int mw = (family == F_CONV3 || family == F_CONV3G) && wm == 42 ? LAMA_W42_CH : 64;
        q.mblocks = (M + mw - 1) / mw;
        q.nblocks = q.tiles_x * q.tiles_y * q.mblocks;
        if (family == F_CONV1 || family == F_CONV1R) {
            // the chunk count of the kernel's chunk size over the packed row
            const int kc = pw_kc(tile_variant(family, OH, OW, M, s0.cs));
            q.s0.nchunk = (q.s0.C + kc - 1) / kc;
            if (q.s0.nchunk * kc > q.s0.wrow) bad_problem = true;
        }
        q.scale = wp(bn);
        q.shift = wp(bn + bn_n);
        q.relu = 1;
        q.res = res;
        q.out = o;
        q.out_cstride = (long)ocs;
        q.outW = outW;
        q.oy_mul = q.ox_mul = 1;
        return q;
    };
    auto conv_launch = [&](int family, std::vector<ConvProblem> probs, int step, double flops, double bytes,
                           int stream = S_MAIN, int wait_ev = -1, int record_ev = -1) {
        Launch L{};
        if (probs.size() == 1) pw_xcd_pad(family, probs[0]);
        L.fn = conv_fn(family, probs.data(), probs.size(), wm);
        L.family = family;
        L.stream = stream;
        L.wait_ev = wait_ev;
        L.record_ev = record_ev;
        unsigned nb = 0;
        for (auto &q : probs) {
            nb += (unsigned)q.nblocks;
            const bool pw = family == F_CONV1 || family == F_CONV1R;
            // the float4 kernel's tile width is the one the problem was tiled for
            if (pw && (tile_variant(family, q.OH, q.OW, q.M, q.s0.cs) == 0) != (L.fn == fn_pw_kh_[family == F_CONV1R]))
                bad_problem = true;
            // every input plane stride set, and at least the plane
            if (q.s0.cs < q.s0.IH * q.s0.IW || (q.s1.nchunk > 0 && q.s1.cs < q.s1.IH * q.s1.IW)) bad_problem = true;
            const int tx = pw && q.ksplit <= 1 && q.nblocks == pw_xcd_blocks(q) ? (q.tiles_x + 7) / 8 * 8 : q.tiles_x;
            if (q.nblocks != std::max(1, q.ksplit) * tx * q.tiles_y * q.mblocks ||
                (q.ksplit > 1 && L.fn != fn_wino4_[0] && L.fn != fn_wino4_[1] && L.fn != fn_wino4_[2] && L.fn != fn_wino42_ &&
                 family != F_CONV1))
                bad_problem = true;
        }
        // the head kernels walk their tiles: three (register weights) or two
        // (weights in LDS) resident workgroups per CU
        L.grid = family == F_CONV7 ? std::min(nb, (L.fn == fn_head_r_ ? (unsigned)LAMA_HEAD_WGS : 2u) * LAMA_CUS) : nb;
        L.shmem = (family == F_CONV3 || family == F_CONV3G) && wm == 4 ? w4_shmem : 0;
        L.block = L.fn == fn_wino42_ ? 8 * LAMA_W42_CH : 0;  // the F(2x4) kernel's 4 waves per 32 channels
        L.arg = put(probs.data(), probs.size() * sizeof(ConvProblem));
        L.ps = prob_starts(probs.data(), probs.size());
        if (probs.size() > LAMA_MAX_PROBS) bad_problem = true;
        L.nparams = 2;
        L.step_end = step;
        L.flops = flops;
        L.bytes = bytes;
        p.launches.push_back(L);
    };
    const double f4 = 4.0;  // bytes per float

    // step 1: model.1 (ReflectionPad2d(3) folded into the 7x7's reflect indexing)
    conv_launch(F_CONV7, {problem(F_CONV7, seg(in, head_, 4, H, W), 64, H, W, head_bn_, 64, a1, P, W, nullptr)}, 1,
                2.0 * 4 * 64 * 49 * P, f4 * (4 * P + 64 * P + 64 * 4 * 49));
    // steps 2-4: the stride-2 downsamplers (model.4 emits local and global)
    conv_launch(F_CONV3S2, {problem(F_CONV3S2, seg(a1, down_[0], 64, H, W), 128, H2, W2, down_bn_[0], 128, a2, P2, W2, nullptr)},
                2, 2.0 * 64 * 128 * 9 * P2, f4 * (64 * P + 128 * P2 + 128 * 64 * 9));
    conv_launch(F_CONV3S2, {problem(F_CONV3S2, seg(a2, down_[1], 128, H2, W2), 256, H4, W4, down_bn_[1], 256, a3, P4, W4, nullptr)},
                3, 2.0 * 128 * 256 * 9 * P4, f4 * (128 * P2 + 256 * P4 + 256 * 128 * 9));
    conv_launch(F_CONV3S2, {problem(F_CONV3S2, seg(a3, down_[2], 256, H4, W4), 512, H8, W8, down_bn_[2], 512, X, P8s, W8, nullptr)},
                4, 2.0 * 256 * 512 * 9 * P8, f4 * (256 * P4 + 512 * P8 + 512 * 256 * 9), S_MAIN, -1, EV_FORK);

    // FFT descriptors (the same buffers serve all 36 spectral transforms)
    FftArgs fa{};
    fa.row = frow;
    fa.col = fcol;
    fa.C = 192;
    fa.H = H8;
    fa.W = W8;
    fa.Wh = Wh;
    fa.scale = (float)(1.0 / std::sqrt((double)H8 * W8));
    fa.rows_per_block = fg.rows_per_block;
    fa.cols_per_block = fg.cols_per_block;
    fa.tmp = fg.split ? (float *)(base + o_tmp) : nullptr;
    fa.rs = (long)P8s;
    fa.ss = (long)PSs;
    fa.in = Fb;
    fa.out = Sb;
    fa.in_np = fa.feat_np = 1;
    void *d_rfft = put(&fa, sizeof fa);
    fa.in = S2;
    fa.out = G;
    fa.feat = Fb;
    void *d_irfft = put(&fa, sizeof fa);
    // with a pointwise K split the transforms reduce the partials and apply
    // the producer's BN + ReLU: one descriptor pair per FFC (its BN)
    std::vector<void *> d_rfft_k(36, d_rfft), d_irfft_k(36, d_irfft);
    if (pk1 > 1 || pku > 1)
        for (int k = 0; k < 36; ++k) {
            const FfcW &Fw = ffc_[k];
            FftArgs fk = fa;
            fk.in = Fb;
            fk.out = Sb;
            fk.feat = nullptr;
            fk.in_np = pk1;
            fk.in_pstride = (long)192 * P8s;
            fk.in_scale = wp(Fw.bn1);
            fk.in_shift = wp(Fw.bn1 + 192);
            fk.feat_np = 1;
            d_rfft_k[k] = put(&fk, sizeof fk);
            fk.in = S2;
            fk.out = G;
            fk.in_np = pku;
            fk.in_pstride = (long)384 * PSs;
            fk.in_scale = wp(Fw.fu_bn);
            fk.in_shift = wp(Fw.fu_bn + 384);
            fk.feat = Fb;
            fk.feat_np = pk1;
            fk.feat_pstride = (long)192 * P8s;
            fk.feat_scale = wp(Fw.bn1);
            fk.feat_shift = wp(Fw.bn1 + 192);
            d_irfft_k[k] = put(&fk, sizeof fk);
        }

    // steps 5-22: 18 resblocks = 36 FFCs, ping-ponging X -> Y -> X (+ residual).
    // FFC k's 3x3 convolutions run on the main stream as two grouped launches:
    //   A(k): l2l (input x_l) and l2g (raw, into GC[k % 2]);
    //   B(k): g2l in four K ranges (input x_g);
    // then the local finalize.  The side stream runs the SpectralTransform
    // chain and conv2, whose epilogue adds GC[k % 2] before BN_g.  A(k+1)
    // needs only x_l(k+1), the main stream's own finalize output, so it is
    // issued right after finalize(k) and overlaps conv2(k); only B(k+1) waits
    // for the side stream (x_g(k+1) from conv2(k)), and conv2(k) waits for
    // A(k), which finished long before.
    auto ffc_src = [&](int k) { return k % 2 == 0 ? X : Y; };
    auto ffc_dst = [&](int k) { return k % 2 == 0 ? Y : X; };
    auto ffc_res = [&](int k) -> const float * { return k % 2 == 0 ? nullptr : X; };
    auto gc_buf = [&](int k) { return GC + (size_t)(k % 2) * ks * 384 * P8s; };
    auto raw = [](ConvProblem q) {
        q.scale = q.shift = nullptr;
        q.relu = 0;
        return q;
    };
    // LQ plane of local partial q of FFC k: the ks l2l slices at 0 .. ks-1, then
    // the 4 ks g2l slices of FFC parity k % 2
    auto lq_plane = [&](int k, int q) {
        return LQ + (size_t)(q < ks ? q : q + (k % 2) * LAMA_G2L_RANGES * ks) * 128 * P8s;
    };
    // a problem split into s K slices of the packed chunks (F(4,3) kernels)
    auto kslices = [&](ConvProblem q, int s, long out_kstride) {
        if (s > 1) {
            q.ksplit = s;
            q.kchunks = q.s0.nchunk / s;
            q.out_kstride = out_kstride;
            q.nblocks *= s;
            if (q.kchunks * s != q.s0.nchunk || q.kchunks % 2) bad_problem = true;
        }
        return q;
    };
    // Local GEMM part q of FFC k, a raw partial into LQ plane q: part 0 is l2l
    // (input channels 0..127, 16 chunks of 8), parts 1-4 are g2l over input
    // channels 128 + 96 (q-1) .. +95 (12 chunks each), so the g2l launch is 512
    // equal workgroups -- one per slot of two per CU.
    auto part = [&](int k, int q) {
        const FfcW &Fw = ffc_[k];
        constexpr int RC = 384 / LAMA_G2L_RANGES;  // channels per g2l K range
        static_assert(RC % 8 == 0 && RC % (2 * LAMA_WINO_KC) == 0 && RC % (2 * LAMA_W42_KC) == 0,
                      "whole K chunks (Winograd: chunk pairs) per range");
        const int c0 = q == 0 ? 0 : 128 + RC * (q - 1), nch = q == 0 ? 128 : RC;
        const Packed &pk = wm == 42 && wino_ != 42 ? Fw.local42 : Fw.local;
        ConvSeg sq = seg(ffc_src(k) + (size_t)c0 * P8s, pk, nch, H8, W8, P8s);
        sq.wt = wp(pk.off) + (size_t)(c0 / pk.KC) * pk.T * pk.KC;  // chunk c0/KC of the packed rows
        sq.nchunk = nch / pk.KC;
        return raw(problem(F_CONV3, sq, 128, H8, W8, 0, 0, lq_plane(k, q), P8s, W8, nullptr));
    };
    auto launch_a = [&](int k) {
        const FfcW &Fw = ffc_[k];
        std::vector<ConvProblem> probs{
            kslices(part(k, 0), ks, (long)128 * P8s),
            kslices(raw(problem(F_CONV3, seg(ffc_src(k), wm == 42 && wino_ != 42 ? Fw.l2g42 : Fw.l2g, 128, H8, W8, P8s),
                                384, H8, W8, 0, 0, gc_buf(k), P8s,
                                W8, nullptr)),
                    ks, (long)384 * P8s)};
        // 16-byte input loads where the plane width allows (B: LAMA_W4_VEC_B)
        for (ConvProblem &q : probs) q.vec_in = (wm == 4 || wm == 42) && W8 % 4 == 0;
        conv_launch(F_CONV3, probs, -1, 2.0 * P8 * (128.0 * 128 * 9 + 384.0 * 128 * 9),
                    f4 * (128 * P8 + 128 * P8 + 384 * P8 + 128 * 128 * 9 + 384 * 128 * 9), S_MAIN, -1,
                    k % 2 ? EV_A1 : EV_A0);
    };
    // B(k) on its own stream overlaps A(k+1); LAMA_B_STREAM=0 keeps it in the
    // main stream's order (the two are bit-identical)
    const bool b_stream = !(getenv("LAMA_B_STREAM") && atoi(getenv("LAMA_B_STREAM")) == 0);
    auto launch_b = [&](int k) {
        std::vector<ConvProblem> probs;
        if (ks > 1) {
            // split: the g2l ranges as the K slices of one problem (F(4,3) kernels)
            const FfcW &Fw = ffc_[k];
            const Packed &pk = wm == 42 && wino_ != 42 ? Fw.local42 : Fw.local;
            ConvSeg sq = seg(ffc_src(k) + (size_t)128 * P8s, pk, 384, H8, W8, P8s);
            sq.wt = wp(pk.off) + (size_t)(128 / pk.KC) * pk.T * pk.KC;
            sq.nchunk = 384 / pk.KC;
            probs.push_back(kslices(raw(problem(F_CONV3, sq, 128, H8, W8, 0, 0, lq_plane(k, ks), P8s, W8, nullptr)),
                                    LAMA_G2L_RANGES * ks, (long)128 * P8s));
        } else {
            for (int q = 1; q <= LAMA_G2L_RANGES; ++q) probs.push_back(part(k, q));
        }
        // own stream: waits for x_g(k) (conv2(k-1), or model.4 for k = 0) and
        // records EV_B for finalize(k); else in the main stream's order
        const int xg = k == 0 ? EV_FORK : ((k - 1) % 2 ? EV_S1 : EV_S0);
        if (LAMA_W4_VEC_B)
            for (ConvProblem &q : probs) q.vec_in = (wm == 4 || wm == 42) && W8 % 4 == 0;
        conv_launch(F_CONV3G, probs, -1, 2.0 * P8 * (128.0 * 384 * 9),
                    f4 * (384 * P8 + LAMA_G2L_RANGES * 128 * P8 + 128 * 384 * 9),
                    b_stream ? S_G2L : S_MAIN, b_stream || k > 0 ? xg : -1, b_stream ? (k % 2 ? EV_B1 : EV_B0) : -1);
    };
    auto launch_finalize = [&](int k) {
        const FfcW &Fw = ffc_[k];
        FinalizeArgs fa2{};
        const int np = LAMA_FIN_PARTS * ks;  // l2l slices, then the g2l slices, in K order
        for (int q = 0; q < np; ++q) fa2.part[q] = lq_plane(k, q);
        fa2.nparts = np;
        fa2.C = 128;
        fa2.plane = (long)P8s;  // the padding floats too: whole float4 groups
        fa2.scale = wp(Fw.bn_l);
        fa2.shift = wp(Fw.bn_l + 128);
        fa2.res = ffc_res(k);
        fa2.out = ffc_dst(k);
        Launch L{};
        const int g = fin_groups(P8s);
        const int ki = ks == 1 ? 0 : ks == 2 ? 1 : 2;
        L.fn = g == 2 ? fn_finalize_g2_[ki] : ki == 0 ? fn_[F_FINAL] : fn_finalize_ks_[ki - 1];
        L.family = F_FINAL;
        L.stream = S_MAIN;
        L.wait_ev = b_stream ? (k % 2 ? EV_B1 : EV_B0) : -1;
        L.record_ev = -1;
        L.grid = (unsigned)(128 * ((P8s + 4 * LAMA_NT * g - 1) / (4 * LAMA_NT * g)));
        L.arg = put(&fa2, sizeof fa2);
        L.nparams = 1;
        L.step_end = -1;
        L.bytes = f4 * 128 * P8 * (np + 1 + (fa2.res ? 1 : 0));
        p.launches.push_back(L);
    };
    // a pointwise problem split into s K slices of its chunks: raw partials
    // s planes apart, reduced (with BN + ReLU) by the consuming transform
    auto pw_kslices = [&](ConvProblem q, int s, long out_kstride) {
        if (s > 1) {
            q = raw(q);
            q.ksplit = s;
            q.kchunks = q.s0.nchunk / s;
            q.out_kstride = out_kstride;
            q.nblocks *= s;
            if (q.kchunks * s != q.s0.nchunk) bad_problem = true;
        }
        return q;
    };
    auto launch_spectral = [&](int k) {
        const FfcW &Fw = ffc_[k];
        // SpectralTransform conv1: f = ReLU(BN(W1 x_g)) over flat planes
        conv_launch(F_CONV1,
                    {pw_kslices(problem(F_CONV1, seg(ffc_src(k) + 128 * P8s, Fw.conv1, 384, 1, (int)P8, P8s), 192, 1,
                                        (int)P8, Fw.bn1, 192, Fb, P8s, (int)P8, nullptr),
                                pk1, (long)192 * P8s)},
                    -1, 2.0 * 384 * 192 * P8, f4 * (384 * P8 + pk1 * 192 * P8 + 192 * 384), S_SIDE,
                    k == 0 ? EV_FORK : -1);
        push_fft(p, false, fg, d_rfft_k[k], S_SIDE, f4 * pk1 * 192 * P8, 8.0 * 192 * PS);
        // FourierUnit conv over the stacked spectrum + BN + ReLU
        conv_launch(F_CONV1,
                    {pw_kslices(problem(F_CONV1, seg(Sb, Fw.fu, 384, 1, (int)PS, PSs), 384, 1, (int)PS, Fw.fu_bn, 384,
                                        S2, PSs, (int)PS, nullptr),
                                pku, (long)384 * PSs)},
                    -1, 2.0 * 384 * 384 * PS, f4 * ((1 + pku) * 384 * PS + 384 * 384), S_SIDE);
        push_fft(p, true, fg, d_irfft_k[k], S_SIDE, 8.0 * pku * 192 * PS, (1 + pk1) * f4 * 192 * P8);  // + the fused feat read
    };
    auto launch_conv2 = [&](int k) {
        const FfcW &Fw = ffc_[k];
        const float *res = ffc_res(k);
        // global: BN_g(l2g(x_l) + conv2(f + ifft)) (+ residual)
        ConvProblem q2 = problem(F_CONV1R, seg(G, Fw.conv2, 192, 1, (int)P8, P8s), 384, 1, (int)P8, Fw.bn_g, 384,
                                 ffc_dst(k) + 128 * P8s, P8s, (int)P8, res ? res + 128 * P8s : nullptr);
        q2.addend = gc_buf(k);
        q2.naddend = ks;  // the l2g K slices
        q2.addend_kstride = (long)384 * P8s;
        conv_launch(F_CONV1R, {q2}, k % 2 == 1 ? 5 + k / 2 : -1, 2.0 * 192 * 384 * P8,
                    f4 * (192 * P8 + 384 * P8 * (res ? 3 : 2) + 384 * 192), S_SIDE, k % 2 ? EV_A1 : EV_A0,
                    k % 2 ? EV_S1 : EV_S0);
    };
    launch_a(0);
    for (int k = 0; k < 36; ++k) {
        launch_spectral(k);
        launch_b(k);
        launch_finalize(k);
        if (k + 1 < 36) launch_a(k + 1);
        launch_conv2(k);
    }
    // step 23 (concat) is the same buffer as step 22; steps 24-26 the upsamplers
    const float *usrc[3] = {X, a3, a2};
    float *udst[3] = {a3, a2, a1};
    const int uh[3] = {H8, H4, H2}, uw[3] = {W8, W4, W2};
    for (int u = 0; u < 3; ++u) {
        const UpW &U = up_[u];
        std::vector<ConvProblem> ph;
        for (int k = 0; k < (convt_rows_ ? 2 : 4); ++k) {
            const size_t oplane = (size_t)(2 * uh[u]) * (2 * uw[u]);
            ConvProblem q = problem(F_CONVT,
                                    seg(usrc[u], convt_rows_ ? U.row[k] : U.ph[k], U.cin, uh[u], uw[u], u == 0 ? P8s : 0),
                                    U.cout,
                                    uh[u], uw[u], U.bn, U.cout, udst[u], oplane, 2 * uw[u], nullptr);
            q.bias = wp(U.bias);
            q.oy_mul = q.ox_mul = 2;
            q.oy_off = k >> 1;
            q.ox_off = k & 1;
            ph.push_back(q);
        }
        const double pin = (double)uh[u] * uw[u];
        conv_launch(F_CONVT, ph, 24 + u, 2.0 * U.cin * U.cout * 9 * pin,
                    f4 * (U.cin * pin + U.cout * 4 * pin + U.cin * U.cout * 9), S_MAIN, u == 0 ? EV_S1 : -1);
    }
    // step 28: model.34 + sigmoid (ReflectionPad2d(3) folded into the indexing)
    TailArgs ta{};
    ta.src = a1;
    ta.wt = wp(tail_w_);
    ta.bias = wp(tail_b_);
    ta.out = out;
    ta.Cin = 64;
    ta.H = H;
    ta.W = W;
    {
        Launch L{};
        L.fn = fn_[F_TAIL];
        L.family = F_TAIL;
        L.stream = S_MAIN;
        L.wait_ev = L.record_ev = -1;
        L.grid = (unsigned)(((W + LAMA_TAIL_COLS - 1) / LAMA_TAIL_COLS) * ((H + LAMA_TAIL_ROWS - 1) / LAMA_TAIL_ROWS));
        L.arg = put(&ta, sizeof ta);
        L.nparams = 1;
        L.step_end = 28;
        L.flops = 2.0 * 64 * 3 * 49 * P;
        L.bytes = f4 * (64 * P + 3 * P);
        p.launches.push_back(L);
        // the inpaint pass: the same tail with the 8-bit composite of the
        // caller's h x w crop fused in (h, w are the launch's int parameters)
        ta.rgb = p.rgb8;
        ta.mask = p.mask8;
        ta.out_u8 = p.out8;
        L.fn = fn_tail_u8_;
        L.arg = put(&ta, sizeof ta);
        L.nparams = 3;
        L.bytes += 7.0 * P;
        p.tail_u8 = L;
        // ... and build_input (main.rs:175-196) before the head
        InputArgs ia{};
        ia.rgb = p.rgb8;
        ia.mask = p.mask8;
        ia.out = in;
        ia.H = H;
        ia.W = W;
        Launch B{};
        B.fn = fn_build_in_;
        B.family = F_INPUT;
        B.stream = S_MAIN;
        B.wait_ev = B.record_ev = -1;
        B.grid = (unsigned)((P + LAMA_NT - 1) / LAMA_NT);
        B.arg = put(&ia, sizeof ia);
        B.nparams = 3;
        B.step_end = -1;
        B.bytes = 4.0 * P + f4 * 4 * P;
        p.build_in = B;
    }
    if (bad_problem) {
        err = "internal: inconsistent launch descriptor";
        return false;
    }
    if (desc.size() > p.arena_bytes - o_desc) {
        err = "internal: descriptor region overflow";
        return false;
    }
    // dump sources per step (nullptr: derived on the host)
    p.step_src.assign(kSteps, {nullptr, 0, 0, 0});
    p.step_src[1] = {a1, 64, P, P};
    p.step_src[2] = {a2, 128, P2, P2};
    p.step_src[3] = {a3, 256, P4, P4};
    for (int s = 4; s <= 23; ++s) p.step_src[s] = {X, 512, P8, P8s};
    p.step_src[24] = {a3, 256, P4, P4};
    p.step_src[25] = {a2, 128, P2, P2};
    p.step_src[26] = {a1, 64, P, P};
    p.step_src[28] = {out, 3, P, P};

    p.desc_host = std::move(desc);
    p.desc_off = o_desc;
    p.twr_host = std::move(twr);
    p.twr_off = o_twr;
    p.twc_host = std::move(twc);
    p.twc_off = o_twc;
    return true;
}

static bool is_conv_family(int f)
{
    return f == F_CONV7 || f == F_CONV3S2 || f == F_CONV3 || f == F_CONV1 || f == F_CONVT || f == F_CONV1R ||
           f == F_CONV3G;
}

bool Engine::launch(const Launch &L, hipStream_t s, std::string &err, hipEvent_t record)
{
    void *arg = L.arg;
    ProbStarts ps = L.ps;
    const bool prof = (prof_mask_ >> L.family) & 1u;
    // conv kernels: the table, the three problem starts as scalars, and the
    // kernel-clock stamp array (profiled launches only); the other kernels
    // read the leading parameters they declare
    unsigned long long *stamp = nullptr;
    Pending pe{};
    pe.stamp_off = -1;
    if (((prof && is_conv_family(L.family)) || timeline_) && !capturing_) {
        const size_t need = 2 * (size_t)L.grid;
        if (!stamp_buf_) {
            stamp_cap_ = (size_t)4 << 20;  // 32 MiB of u64 entries
            if (!check(hip_->hipMalloc((void **)&stamp_buf_, stamp_cap_ * 8), "hipMalloc(stamps)", err) ||
                !check(hip_->hipMemset(stamp_buf_, 0, stamp_cap_ * 8), "hipMemset(stamps)", err)) {
                stamp_buf_ = nullptr;
                return false;
            }
        }
        if (stamp_used_ + need <= stamp_cap_) {
            stamp = stamp_buf_ + stamp_used_;
            pe.stamp_off = (long)stamp_used_;
            pe.grid = L.grid;
            if (timeline_) tl_.push_back({L.family, L.stream, (long)stamp_used_, L.grid});
            stamp_used_ += need;
        }
        if (!prof) pe.stamp_off = -1;
    }
    void *params[5] = {&arg, &ps.s[0], &ps.s[1], &ps.s[2], &stamp};
    if (prof) {
        for (hipEvent_t *e : {&pe.a, &pe.b}) {
            if (!event_pool_.empty()) {
                *e = event_pool_.back();
                event_pool_.pop_back();
            } else if (!check(hip_->hipEventCreateWithFlags(e, hipEventDisableSystemFence), "hipEventCreate", err)) {
                // timing only: no host-visible cache write-back at each record
                return false;
            }
        }
        pe.family = L.family;
        pe.flops = L.flops;
        pe.bytes = L.bytes;
    }
    const unsigned block = L.block ? L.block : LAMA_NT;
    if (prof) {
        // the events ride in the dispatch packet itself (no marker packets on
        // the stream), so timing a kernel does not stall the queue around it.
        // A launch issued after a cross-stream wait is timed from the wait's
        // barrier packet (it then reads long by the time spent waiting,
        // whether the events ride in the packet or are separate markers), so
        // kernel time is read from launches that wait on nothing.
        if (!check(hip_->hipExtModuleLaunchKernel(L.fn, L.grid * block, 1, 1, block, 1, 1, L.shmem, s, params, nullptr,
                                                  pe.a, pe.b, 0),
                   kFamilyName[L.family], err))
            return false;
        pending_.push_back(pe);
        return true;
    }
    if (record) {
        // the cross-stream event is recorded by this kernel's dispatch packet
        return check(hip_->hipExtModuleLaunchKernel(L.fn, L.grid * block, 1, 1, block, 1, 1, L.shmem, s, params,
                                                    nullptr, nullptr, record, 0),
                     kFamilyName[L.family], err);
    }
    return check(hip_->hipModuleLaunchKernel(L.fn, L.grid, 1, 1, block, 1, 1, L.shmem, s, params, nullptr),
                 kFamilyName[L.family], err);
}

static void host_reflect_pad(const float *src, int c, int h, int w, int pad, float *dst)
{
    const int oh = h + 2 * pad, ow = w + 2 * pad;
    for (int ch = 0; ch < c; ++ch)
        for (int y = 0; y < oh; ++y) {
            const size_t sy = lama_reflect_index(y - pad, (size_t)h);
            for (int x = 0; x < ow; ++x)
                dst[((size_t)ch * oh + y) * ow + x] =
                    src[((size_t)ch * h + sy) * w + lama_reflect_index(x - pad, (size_t)w)];
        }
}

// Local and global activation shapes after plan step `step` (the reference's
// LAMA_PROFILE / LAMA_DUMP_STEP lines, cuda.rs:1647-1686); c = 0: absent.
static void step_shapes(int step, int h, int w, int l[3], int g[3])
{
    const int h8 = h / 8, w8 = w / 8;
    g[0] = g[1] = g[2] = 0;
    auto set = [](int *v, int c, int y, int x) {
        v[0] = c;
        v[1] = y;
        v[2] = x;
    };
    switch (step) {
    case 0: set(l, 4, h + 6, w + 6); break;
    case 1: set(l, 64, h, w); break;
    case 2: set(l, 128, h / 2, w / 2); break;
    case 3: set(l, 256, h / 4, w / 4); break;
    case 23: set(l, 512, h8, w8); break;
    case 24: set(l, 256, h / 4, w / 4); break;
    case 25: set(l, 128, h / 2, w / 2); break;
    case 26: set(l, 64, h, w); break;
    case 27: set(l, 64, h + 6, w + 6); break;
    case 28: set(l, 3, h, w); break;
    default:
        set(l, 128, h8, w8);
        set(g, 384, h8, w8);
    }
}

static std::string global_desc(const int g[3])
{
    if (!g[0]) return "None";
    return "Some((" + std::to_string(g[0]) + ", " + std::to_string(g[1]) + ", " + std::to_string(g[2]) + "))";
}

bool Engine::run(Plan &p, hipStream_t s, float *const *steps, std::string &err, int u8_h, int u8_w)
{
    // LAMA_STREAMS=1 puts the side-stream work on the main stream (profiling)
    static const bool single = getenv("LAMA_STREAMS") && atoi(getenv("LAMA_STREAMS")) == 1;
    hipStream_t st[S_COUNT] = {s, single ? s : side_, single ? s : g2l_};
    // LAMA_PROFILE: one line per plan step (cuda.rs:1663-1686), the host time
    // since the previous step -- submission only, unless LAMA_PROFILE_SYNC
    // drains every stream at each step's end, which makes it submit + device
    const bool per_step = flag_profile_ && !capturing_;
    auto t_step = std::chrono::steady_clock::now();
    int next_step = 0;
    auto step_done = [&](int stp) -> bool {
        if (!per_step) return true;
        for (; next_step <= stp; ++next_step) {
            if (flag_profile_sync_)
                for (hipStream_t q : st)
                    if (!check(hip_->hipStreamSynchronize(q), "hipStreamSynchronize", err)) return false;
            const auto now = std::chrono::steady_clock::now();
            const double dt = next_step == stp ? std::chrono::duration<double>(now - t_step).count() : 0.0;
            if (next_step == stp) t_step = now;
            int l[3], g[3];
            step_shapes(next_step, p.H, p.W, l, g);
            fprintf(stderr, "gpu step %2d: %6.3fs local %dx%dx%d global %s\n", next_step, dt, l[0], l[1], l[2],
                    global_desc(g).c_str());
        }
        return true;
    };
    if (u8_h > 0) {
        Launch B = p.build_in;
        B.ps.s[0] = u8_h;
        B.ps.s[1] = u8_w;
        if (!launch(B, st[S_MAIN], err)) return false;
    }
    if (!step_done(0)) return false;
    for (const Launch &L0 : p.launches) {
        const Launch *Lp = &L0;
        Launch T;
        if (u8_h > 0 && L0.family == F_TAIL) {
            T = p.tail_u8;
            T.ps.s[0] = u8_h;
            T.ps.s[1] = u8_w;
            Lp = &T;
        }
        const Launch &L = *Lp;
        hipStream_t ls = st[L.stream];
        if (L.wait_ev >= 0 && !check(hip_->hipStreamWaitEvent(ls, ev_[L.wait_ev], 0), "hipStreamWaitEvent", err))
            return false;
        // cross-stream events ride in the dispatch packet, unless the launch is
        // being profiled (its packet then carries the timing events) or the
        // stream is being captured (a graph edge needs an explicit record)
        const bool explicit_rec = capturing_ || ((prof_mask_ >> L.family) & 1u);
        if (!launch(L, ls, err, L.record_ev >= 0 && !explicit_rec ? ev_[L.record_ev] : nullptr)) return false;
        if (L.record_ev >= 0 && explicit_rec &&
            !check(hip_->hipEventRecord(ev_[L.record_ev], ls), "hipEventRecord", err))
            return false;
        if (L.step_end >= 0 && !step_done(L.step_end == 22 ? 23 : L.step_end == 26 ? 27 : L.step_end)) return false;
        if (!steps || L.step_end < 0) continue;
        int done[2] = {L.step_end, L.step_end == 22 ? 23 : -1};
        for (int stp : done) {
            if (stp < 0) continue;
            const bool want = steps[stp] || (stp == 26 && steps[27]);
            if (!want) continue;
            const Plan::StepSrc &src = p.step_src[stp];
            std::vector<float> tmp, padded;
            float *dst = steps[stp];
            if (!dst) {
                tmp.resize(src.planes * src.plane);
                dst = tmp.data();
            }
            // a step is complete when every stream has drained
            for (hipStream_t q : st)
                if (!check(hip_->hipStreamSynchronize(q), "hipStreamSynchronize", err)) return false;
            // planes at a padded stride come down whole and are packed here
            float *land = dst;
            if (src.stride != src.plane) {
                padded.resize(src.planes * src.stride);
                land = padded.data();
            }
            if (!check(hip_->hipMemcpyAsync(land, src.src, src.planes * src.stride * 4, hipMemcpyDeviceToHost, s),
                       "hipMemcpy(dump)", err) ||
                !check(hip_->hipStreamSynchronize(s), "hipStreamSynchronize", err))
                return false;
            if (land != dst)
                for (size_t c = 0; c < src.planes; ++c)
                    std::memcpy(dst + c * src.plane, land + c * src.stride, src.plane * 4);
            if (stp == 26 && steps[27]) host_reflect_pad(dst, 64, p.H, p.W, 3, steps[27]);
        }
    }
    return true;
}

void Engine::free_plan(Plan &p)
{
    if (p.graph) hip_->hipGraphExecDestroy(p.graph);
    p.graph = nullptr;
    if (p.arena && p.own_arena) hip_->hipFree(p.arena);
    p.arena = nullptr;
}

// The plan's launch list as one HIP graph: captured from the engine's three
// streams on the first forward at a shape (the side streams join the capture
// through the fork event and rejoin through the events the main stream waits
// for), then replayed with one hipGraphLaunch.  The graph holds kernel nodes
// and event edges only.  Used where use_graph says; profiling, the timeline
// and step dumps always take the per-launch path.
bool Engine::replay(Plan &p, hipStream_t s, std::string &err)
{
    if (!p.graph) {
        // A capture or instantiation the runtime refuses leaves the plan on
        // the per-launch path (the same launches, issued one by one).
        hipGraph_t g = nullptr;
        if (hip_->hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) != hipSuccess) {
            hip_->hipGetLastError();
            p.graph_failed = true;
            return run(p, s, nullptr, err);
        }
        std::string rerr;
        capturing_ = true;
        const bool ok = run(p, stream_, nullptr, rerr);
        capturing_ = false;
        const hipError_t e = hip_->hipStreamEndCapture(stream_, &g);
        if (!ok) {
            if (g) hip_->hipGraphDestroy(g);
            err = rerr;
            return false;
        }
        const hipError_t ei = e == hipSuccess ? hip_->hipGraphInstantiate(&p.graph, g, nullptr, nullptr, 0) : e;
        if (g) hip_->hipGraphDestroy(g);
        if (ei != hipSuccess) {
            hip_->hipGetLastError();
            p.graph = nullptr;
            p.graph_failed = true;
            return run(p, s, nullptr, err);
        }
    }
    return check(hip_->hipGraphLaunch(p.graph, s), "hipGraphLaunch", err);
}

bool Engine::use_graph(const Plan &p) const
{
    // LAMA_GRAPH=1 / 0 forces the replayed graph on / off.  By default it is
    // used for inputs of at most 256 x 256, where issuing the pass's launches
    // one by one takes the host nearly as long as the device takes to run
    // them (256x256: 1.93-2.13 ms of enqueue against a 2.2 ms pass; one graph
    // launch enqueues in 0.93 ms), so a slower host would make the pass
    // host-bound.  Above that the device time dominates and the per-launch
    // streams measured slightly faster (512x512: 282.2 vs 280.2 passes/s).
    // Profiled and timeline passes always take the per-launch path.
    if (prof_mask_ != 0 || timeline_ || p.graph_failed) return false;
    if (const char *g = getenv("LAMA_GRAPH")) return atoi(g) == 1;
    return (long)p.H * p.W <= 256L * 256;
}

// cuda.rs:1647-1662: /tmp/gpu_step_<n>.f32 (little-endian f32, as
// to_le_bytes) and the "gpu dumped step" line; a failed write is ignored, as
// there.
static void write_step_dump(int n, const std::vector<float> &d, int h, int w)
{
    const std::string path = "/tmp/gpu_step_" + std::to_string(n) + ".f32";
    if (FILE *f = fopen(path.c_str(), "wb")) {
        fwrite(d.data(), 4, d.size(), f);
        fclose(f);
    }
    int l[3], g[3];
    step_shapes(n, h, w, l, g);
    fprintf(stderr, "gpu dumped step %d: local %dx%dx%d global %s\n", n, l[0], l[1], l[2], global_desc(g).c_str());
}

bool Engine::forward_host(const float *in, int h, int w, float *out, float *const *steps, std::string &err)
{
    using clk = std::chrono::steady_clock;
    auto secs = [](clk::time_point a) { return std::chrono::duration<double>(clk::now() - a).count(); };
    const auto t_run = clk::now();
    Plan *p = plan_for(h, w, err);
    if (!p) return false;
    // LAMA_DUMP_STEP=<n> (cuda.rs:1572-1574, 1647-1662): the activation after
    // plan step n, local planes then global, to /tmp/gpu_step_<n>.f32
    std::vector<float> dump;
    float *dsteps[kSteps] = {};
    if (dump_step_ >= 0 && !steps) {
        dump.resize(step_numel(dump_step_, h, w));
        dsteps[dump_step_] = dump.data();
        steps = dsteps;
    }
    if (steps && steps[0]) host_reflect_pad(in, 4, h, w, 3, steps[0]);
    auto t = clk::now();
    if (!check(hip_->hipMemcpyAsync(p->in, in, 4ul * h * w * 4, hipMemcpyHostToDevice, stream_), "hipMemcpy(input)", err))
        return false;
    if (flag_profile_) {
        if (!check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err)) return false;
        fprintf(stderr, "gpu input upload: %.3fs\n", secs(t));
    }
    t = clk::now();
    if (!(steps || flag_profile_ || !use_graph(*p) ? run(*p, stream_, steps, err) : replay(*p, stream_, err))) return false;
    if (flag_profile_) {
        if (!check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err)) return false;
        fprintf(stderr, "gpu step loop: %.3fs\n", secs(t));
    }
    t = clk::now();
    if (!check(hip_->hipMemcpyAsync(out, p->out, 3ul * h * w * 4, hipMemcpyDeviceToHost, stream_), "hipMemcpy(output)", err) ||
        !check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err))
        return false;
    if (flag_profile_) {
        fprintf(stderr, "gpu output download: %.3fs (%zu floats)\n", secs(t), (size_t)3 * h * w);
        fprintf(stderr, "gpu run total: %.3fs\n", secs(t_run));
    }
    if (!dump.empty()) write_step_dump(dump_step_, dump, h, w);
    return true;
}


bool Engine::forward_device(const float *d_in, int h, int w, float *d_out, hipStream_t s, std::string &err)
{
    Plan *p = plan_for(h, w, err);
    if (!p) return false;
    if (!s) s = stream_;
    if (!check(hip_->hipMemcpyAsync(p->in, d_in, 4ul * h * w * 4, hipMemcpyDeviceToDevice, s), "hipMemcpy(input)", err))
        return false;
    if (!(use_graph(*p) ? replay(*p, s, err) : run(*p, s, nullptr, err))) return false;
    if (!check(hip_->hipMemcpyAsync(d_out, p->out, 3ul * h * w * 4, hipMemcpyDeviceToDevice, s), "hipMemcpy(output)", err))
        return false;
    return mark_done(s, err);
}

// forward_device on the device's scratch array instead of an allocated arena.
// Host work only (plan layout, descriptor staging) plus copies and launches on
// `s`: no device allocation, no event or graph creation (profiling and the
// launch timeline are off for these passes).  The descriptors are re-uploaded
// (on `s`) whenever another context or another shape used the array last.
// A stream under capture is refused: a captured pass would replay against
// whatever descriptors the shared array holds at replay time, which another
// context or shape may have replaced, with the captured grid sizes.
// The no-allocation entry point's array, set up by its first call on a
// device, once per device per process, with that device current: its code
// object is loaded and the array's address on this device looked up
// (hipModuleGetGlobal, the module-loaded form of hipGetSymbolAddress); every
// later use goes through that address.  A failed set-up (for instance no room
// on a nearly full device) fails that call, and the next call tries again.
bool Engine::scratch_setup(std::string &err)
{
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    DeviceScratch &d = g_scratch[device_];
    if (!d.ptr) {
        hipModule_t m = nullptr;
        hipDeviceptr_t p = nullptr;
        size_t n = 0;
        std::string serr;
        if (!check(hip_->hipSetDevice(device_), "hipSetDevice", serr) ||
            !check(hip_->hipModuleLoadData(&m, lama_scratch_hsaco_start), "hipModuleLoadData(scratch)", serr)) {
            m = nullptr;
        } else if (!check(hip_->hipModuleGetGlobal(&p, &n, m, "lama_scratch"), "hipModuleGetGlobal(lama_scratch)",
                          serr)) {
            p = nullptr;
        } else if (!p || n < LAMA_SCRATCH_BYTES) {
            serr = "lama_scratch: " + std::to_string(n) + " bytes, expected " + std::to_string(LAMA_SCRATCH_BYTES);
            p = nullptr;
        }
        if (!p) {
            if (m) hip_->hipModuleUnload(m);
            hip_->hipGetLastError();  // reported here, not by a later call
            err = "the no-allocation scratch array could not be set up: " + serr;
            return false;
        }
        d.mod = m;
        d.ptr = p;
        d.bytes = n;
    }
    scratch_ = d.ptr;
    return true;
}

bool Engine::forward_device_noalloc(const float *d_in, int h, int w, float *d_out, hipStream_t s, std::string &err)
{
    if (!have_weights_) {
        err = "no weights loaded";
        return false;
    }
    if (!shape_ok(h, w, err)) return false;
    if (!s) s = stream_;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (!check(hip_->hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing", err)) return false;
    if (cap != hipStreamCaptureStatusNone) {
        err = "forward_device_noalloc cannot be captured into a graph: its launch descriptors live in the "
              "device's shared scratch array, which any later call may overwrite";
        return false;
    }
    if (!scratch_ && !scratch_setup(err)) return false;
    const bool fresh = !(na_plan_.arena && na_plan_.H == h && na_plan_.W == w);
    if (fresh) {
        uint64_t need = 0, wb = 0;
        if (!plan_bytes(h, w, need, wb, err)) return false;
        if (need > LAMA_SCRATCH_BYTES) {
            err = "input " + std::to_string(w) + "x" + std::to_string(h) + " needs " + std::to_string(need >> 20) +
                  " MiB of device memory; the no-allocation entry point's array holds " +
                  std::to_string(LAMA_SCRATCH_BYTES >> 20) + " MiB (up to 512x512)";
            return false;
        }
        Plan p;
        p.H = h;
        p.W = w;
        if (!build_plan(p, scratch_, err)) return false;
        na_plan_ = std::move(p);
    }
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        DeviceScratch &d = g_scratch[device_];
        if (fresh || d.owner != id_ || d.h != h || d.w != w) {
            if (!upload_plan(na_plan_, s, err)) {
                d.owner = 0;
                return false;
            }
            d.owner = id_;
            d.h = h;
            d.w = w;
        }
    }
    // profiling and the timeline would allocate (events, the stamp buffer)
    const uint32_t prof = prof_mask_;
    const bool tl = timeline_;
    prof_mask_ = 0;
    timeline_ = false;
    const bool ok =
        check(hip_->hipMemcpyAsync(na_plan_.in, d_in, 4ul * h * w * 4, hipMemcpyDeviceToDevice, s), "hipMemcpy(input)",
              err) &&
        run(na_plan_, s, nullptr, err) &&
        check(hip_->hipMemcpyAsync(d_out, na_plan_.out, 3ul * h * w * 4, hipMemcpyDeviceToDevice, s),
              "hipMemcpy(output)", err);
    prof_mask_ = prof;
    timeline_ = tl;
    return ok && mark_done(s, err);
}

// A pass enqueued on a caller's stream: synchronize() must also wait for it.
bool Engine::mark_done(hipStream_t s, std::string &err)
{
    if (s == stream_) return true;
    if (!check(hip_->hipEventRecord(ev_done_, s), "hipEventRecord", err)) return false;
    done_pending_ = true;
    return true;
}

bool Engine::synchronize(std::string &err)
{
    if (done_pending_) {
        if (!check(hip_->hipEventSynchronize(ev_done_), "hipEventSynchronize", err)) return false;
        done_pending_ = false;
    }
    return check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err);
}

// The image sizes the inpaint entry points take, and their padded shape
// (main.rs:241-242: up to the next multiple of 8).
static bool inpaint_shape(int h, int w, int &H, int &W, std::string &err)
{
    if (h < 1 || w < 1) {
        err = "image " + std::to_string(w) + "x" + std::to_string(h) + " is empty";
        return false;
    }
    H = h + (8 - h % 8) % 8;
    W = w + (8 - w % 8) % 8;
    return true;
}

bool Engine::inpaint_host(const uint8_t *rgb, const uint8_t *mask, int h, int w, uint8_t *out, float *net_out,
                          std::string &err)
{
    int H, W;
    if (!inpaint_shape(h, w, H, W, err)) return false;
    Plan *p = plan_for(H, W, err);
    if (!p) return false;
    const size_t px = (size_t)h * w;
    if (!check(hip_->hipMemcpyAsync(p->rgb8, rgb, 3 * px, hipMemcpyHostToDevice, stream_), "hipMemcpy(image)", err) ||
        !check(hip_->hipMemcpyAsync(p->mask8, mask, px, hipMemcpyHostToDevice, stream_), "hipMemcpy(mask)", err))
        return false;
    // LAMA_DUMP_STEP, as in forward_host; step 0 (the padded input) is the
    // device-built input, reflect-padded on the host
    std::vector<float> dump;
    float *dsteps[kSteps] = {};
    if (dump_step_ > 0) {
        dump.resize(step_numel(dump_step_, H, W));
        dsteps[dump_step_] = dump.data();
    }
    if (!run(*p, stream_, dump_step_ > 0 ? dsteps : nullptr, err, h, w)) return false;
    if (dump_step_ == 0) {
        std::vector<float> x((size_t)4 * H * W);
        dump.resize(step_numel(0, H, W));
        if (!check(hip_->hipMemcpyAsync(x.data(), p->in, x.size() * 4, hipMemcpyDeviceToHost, stream_), "hipMemcpy(dump)",
                   err) ||
            !check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err))
            return false;
        host_reflect_pad(x.data(), 4, H, W, 3, dump.data());
    }
    if (!check(hip_->hipMemcpyAsync(out, p->out8, 3 * px, hipMemcpyDeviceToHost, stream_), "hipMemcpy(output)", err))
        return false;
    if (net_out && !check(hip_->hipMemcpyAsync(net_out, p->out, 3ul * H * W * 4, hipMemcpyDeviceToHost, stream_),
                          "hipMemcpy(output)", err))
        return false;
    if (!check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err)) return false;
    if (!dump.empty()) write_step_dump(dump_step_, dump, H, W);
    return true;
}

bool Engine::inpaint_device(const uint8_t *d_rgb, const uint8_t *d_mask, int h, int w, uint8_t *d_out, hipStream_t s,
                            std::string &err)
{
    int H, W;
    if (!inpaint_shape(h, w, H, W, err)) return false;
    Plan *p = plan_for(H, W, err);
    if (!p) return false;
    if (!s) s = stream_;
    const size_t px = (size_t)h * w;
    if (!check(hip_->hipMemcpyAsync(p->rgb8, d_rgb, 3 * px, hipMemcpyDeviceToDevice, s), "hipMemcpy(image)", err) ||
        !check(hip_->hipMemcpyAsync(p->mask8, d_mask, px, hipMemcpyDeviceToDevice, s), "hipMemcpy(mask)", err))
        return false;
    if (!run(*p, s, nullptr, err, h, w)) return false;
    if (!check(hip_->hipMemcpyAsync(d_out, p->out8, 3 * px, hipMemcpyDeviceToDevice, s), "hipMemcpy(output)", err))
        return false;
    return mark_done(s, err);
}

// The per-shape plan of the SpectralTransform entry point: the five
// launches (seven with split FFTs) of each FFC's SpectralTransform on one
// stream, over one set of buffers.
SpecPlan *Engine::spec_plan_for(int h, int w, std::string &err)
{
    if (!have_weights_) {
        err = "no weights loaded";
        return nullptr;
    }
    if (h < 1 || w < 1 || (size_t)h * w > ((size_t)1 << 24)) {
        err = "SpectralTransform plane " + std::to_string(w) + "x" + std::to_string(h) + " is empty or above 2^24 pixels";
        return nullptr;
    }
    auto key = std::make_pair(h, w);
    auto it = spec_plans_.find(key);
    if (it != spec_plans_.end()) return &it->second;
    const int Wh = w / 2 + 1;
    const size_t P = (size_t)h * w, PS = (size_t)h * Wh;
    FftLen frow, fcol;
    std::vector<float> twr, twc;
    FftGeom fg;
    if (!fft_len(w, frow, twr, err) || !fft_len(h, fcol, twc, err) || !fft_geom(192, h, w, fg, err)) return nullptr;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off = (off + bytes + 255) / 256 * 256;
        return o;
    };
    const size_t o_x = take(384 * P * 4), o_f = take(192 * P * 4), o_s = take(384 * PS * 4), o_s2 = take(384 * PS * 4),
                 o_g = take(192 * P * 4), o_out = take(384 * P * 4), o_tmp = take(fg.split ? fg.tmp_bytes : 0),
                 o_twr = take(twr.size() * 4), o_twc = take(twc.size() * 4);
    const size_t o_desc = take(36 * 3 * 256 + 2 * 256 + 36 * 3 * sizeof(ConvProblem) + 2 * sizeof(FftArgs) + 4096);
    SpecPlan sp;
    sp.H = h;
    sp.W = w;
    sp.arena_bytes = off;
    if (!check(hip_->hipMalloc(&sp.arena, off), "hipMalloc(SpectralTransform)", err)) return nullptr;
    char *base = (char *)sp.arena;
    auto F = [&](size_t o) { return (float *)(base + o); };
    sp.x = F(o_x);
    sp.f = F(o_f);
    sp.s = F(o_s);
    sp.s2 = F(o_s2);
    sp.g = F(o_g);
    sp.out = F(o_out);
    std::vector<char> desc;
    auto put = [&](const void *src, size_t bytes) {
        size_t o = (desc.size() + 255) / 256 * 256;
        desc.resize(o + bytes);
        std::memcpy(desc.data() + o, src, bytes);
        return (void *)(base + o_desc + o);
    };
    FftArgs fa{};
    fa.row = frow;
    fa.col = fcol;
    fa.row.tw = F(o_twr);
    fa.col.tw = F(o_twc);
    fa.C = 192;
    fa.H = h;
    fa.W = w;
    fa.Wh = Wh;
    fa.scale = (float)(1.0 / std::sqrt((double)h * w));
    fa.rows_per_block = fg.rows_per_block;
    fa.cols_per_block = fg.cols_per_block;
    fa.tmp = fg.split ? F(o_tmp) : nullptr;
    fa.rs = (long)P;  // the isolated transform's planes are unpadded
    fa.ss = (long)PS;
    fa.in = sp.f;
    fa.out = sp.s;
    void *d_rfft = put(&fa, sizeof fa);
    fa.in = sp.s2;
    fa.out = sp.g;
    fa.feat = sp.f;
    void *d_irfft = put(&fa, sizeof fa);
    // a pointwise problem over a flat plane of N pixels: out[M][N] = W src[C][N]
    auto pw = [&](const float *src, const Packed &pk, int C, int M, int N, size_t bn, float *o, bool bn_relu) {
        ConvProblem q{};
        q.s0.src = src;
        q.s0.wt = wp(pk.off);
        q.s0.C = C;
        q.s0.IH = 1;
        q.s0.IW = N;
        q.s0.nchunk = pk.nchunk;
        q.s0.wrow = pk.wrow;
        q.s0.cs = N;
        q.M = M;
        q.OH = 1;
        q.OW = N;
        int tr, tc;
        const int v = tile_variant(F_CONV1, 1, N, M);
        tile_shape(F_CONV1, tr, tc, 0, v);
        q.s0.nchunk = (C + pw_kc(v) - 1) / pw_kc(v);
        q.tiles_x = (N + tc - 1) / tc;
        q.tiles_y = 1;
        q.mblocks = (M + 63) / 64;
        q.nblocks = q.tiles_x * q.mblocks;
        q.scale = bn_relu ? wp(bn) : nullptr;
        q.shift = bn_relu ? wp(bn + M) : nullptr;
        q.relu = bn_relu ? 1 : 0;
        q.out = o;
        q.out_cstride = (long)N;
        q.outW = N;
        q.oy_mul = q.ox_mul = 1;
        return q;
    };
    auto conv = [&](std::vector<Launch> &out, ConvProblem q, double flops, double bytes) {
        Launch L{};
        pw_xcd_pad(F_CONV1, q);
        L.fn = conv_fn(F_CONV1, &q, 1);
        L.family = F_CONV1;
        L.stream = S_MAIN;
        L.wait_ev = L.record_ev = L.step_end = -1;
        L.grid = (unsigned)q.nblocks;
        L.arg = put(&q, sizeof q);
        L.ps = prob_starts(&q, 1);
        L.nparams = 2;
        L.flops = flops;
        L.bytes = bytes;
        out.push_back(L);
    };
    for (int k = 0; k < 36; ++k) {
        const FfcW &Fw = ffc_[k];
        std::vector<Launch> &v = sp.launches[k];
        conv(v, pw(sp.x, Fw.conv1, 384, 192, (int)P, Fw.bn1, sp.f, true), 2.0 * 384 * 192 * P,
             4.0 * (384 * P + 192 * P + 192 * 384));
        Plan tmp;
        push_fft(tmp, false, fg, d_rfft, S_MAIN, 4.0 * 192 * P, 8.0 * 192 * PS);
        conv(tmp.launches, pw(sp.s, Fw.fu, 384, 384, (int)PS, Fw.fu_bn, sp.s2, true), 2.0 * 384 * 384 * PS,
             4.0 * (2 * 384 * PS + 384 * 384));
        push_fft(tmp, true, fg, d_irfft, S_MAIN, 8.0 * 192 * PS, 8.0 * 192 * P);
        conv(tmp.launches, pw(sp.g, Fw.conv2, 192, 384, (int)P, 0, sp.out, false), 2.0 * 192 * 384 * P,
             4.0 * (192 * P + 384 * P + 384 * 192));
        v.insert(v.end(), tmp.launches.begin(), tmp.launches.end());
    }
    if (desc.size() > off - o_desc) {
        hip_->hipFree(sp.arena);
        err = "internal: descriptor region overflow";
        return nullptr;
    }
    if (!check(hip_->hipMemcpy(base + o_desc, desc.data(), desc.size(), hipMemcpyHostToDevice), "hipMemcpy(descriptors)", err) ||
        !check(hip_->hipMemcpy(base + o_twr, twr.data(), twr.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(twiddles)", err) ||
        !check(hip_->hipMemcpy(base + o_twc, twc.data(), twc.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(twiddles)", err)) {
        hip_->hipFree(sp.arena);
        return nullptr;
    }
    return &(spec_plans_[key] = std::move(sp));
}

bool Engine::spectral_device(int k, const float *d_x, int h, int w, float *d_out, hipStream_t s, std::string &err)
{
    if (k < 0 || k >= 36) {
        err = "SpectralTransform index " + std::to_string(k) + " is outside 0..35";
        return false;
    }
    SpecPlan *sp = spec_plan_for(h, w, err);
    if (!sp) return false;
    if (!s) s = stream_;
    const size_t P = (size_t)h * w;
    if (!check(hip_->hipMemcpyAsync(sp->x, d_x, 384 * P * 4, hipMemcpyDeviceToDevice, s), "hipMemcpy(input)", err))
        return false;
    for (const Launch &L : sp->launches[k])
        if (!launch(L, s, err)) return false;
    if (!check(hip_->hipMemcpyAsync(d_out, sp->out, 384 * P * 4, hipMemcpyDeviceToDevice, s), "hipMemcpy(output)", err))
        return false;
    return mark_done(s, err);
}

bool Engine::spectral_host(int k, const float *x, int h, int w, float *out, float *const *stages, std::string &err)
{
    if (k < 0 || k >= 36) {
        err = "SpectralTransform index " + std::to_string(k) + " is outside 0..35";
        return false;
    }
    SpecPlan *sp = spec_plan_for(h, w, err);
    if (!sp) return false;
    const size_t P = (size_t)h * w, PS = (size_t)h * (w / 2 + 1);
    if (!check(hip_->hipMemcpyAsync(sp->x, x, 384 * P * 4, hipMemcpyHostToDevice, stream_), "hipMemcpy(input)", err))
        return false;
    for (const Launch &L : sp->launches[k])
        if (!launch(L, stream_, err)) return false;
    if (!check(hip_->hipMemcpyAsync(out, sp->out, 384 * P * 4, hipMemcpyDeviceToHost, stream_), "hipMemcpy(output)", err))
        return false;
    const std::pair<const float *, size_t> src[4] = {{sp->f, 192 * P}, {sp->s, 384 * PS}, {sp->s2, 384 * PS}, {sp->g, 192 * P}};
    for (int i = 0; stages && i < 4; ++i)
        if (stages[i] && !check(hip_->hipMemcpyAsync(stages[i], src[i].first, src[i].second * 4, hipMemcpyDeviceToHost,
                                                     stream_),
                                "hipMemcpy(stage)", err))
            return false;
    return check(hip_->hipStreamSynchronize(stream_), "hipStreamSynchronize", err);
}

int Engine::launch_count(int h, int w)
{
    auto it = plans_.find({h, w});
    return it == plans_.end() ? -1 : (int)it->second.launches.size();
}

bool Engine::get_fn(hipFunction_t &fn, const char *name, std::string &err)
{
    if (!check(hip_->hipModuleGetFunction(&fn, module_, name), name, err)) return false;
    fn_names_[fn] = name;
    return true;
}

const char *Engine::kernel_name(int h, int w, int family) const
{
    auto it = plans_.find({h, w});
    if (it == plans_.end()) return nullptr;
    for (const Launch &L : it->second.launches)
        if (L.family == family) {
            auto n = fn_names_.find(L.fn);
            return n == fn_names_.end() ? nullptr : n->second;
        }
    return nullptr;
}

void Engine::collect_events()
{
    for (auto &pe : pending_) {
        float ms = 0.f;
        if (hip_->hipEventSynchronize(pe.b) == hipSuccess && hip_->hipEventElapsedTime(&ms, pe.a, pe.b) == hipSuccess) {
            prof_launches_[pe.family] += 1;
            prof_ms_[pe.family] += ms;
            prof_flops_[pe.family] += pe.flops;
            prof_bytes_[pe.family] += pe.bytes;
        }
        event_pool_.push_back(pe.a);
        event_pool_.push_back(pe.b);
    }
    // kernel-clock durations: the last workgroup end minus the first start
    if (stamp_used_ && clock_khz_ > 0) {
        std::vector<unsigned long long> st(stamp_used_);
        if (hip_->hipMemcpy(st.data(), stamp_buf_, stamp_used_ * 8, hipMemcpyDeviceToHost) == hipSuccess) {
            for (auto &pe : pending_) {
                if (pe.stamp_off < 0) continue;
                unsigned long long t0 = ~0ull, t1 = 0;
                for (unsigned b = 0; b < pe.grid; ++b) {
                    const unsigned long long a = st[pe.stamp_off + 2 * b], e = st[pe.stamp_off + 2 * b + 1];
                    if (!a) continue;  // a workgroup that wrote nothing
                    t0 = std::min(t0, a);
                    t1 = std::max(t1, e);
                }
                if (t1 <= t0) continue;
                prof_clock_n_[pe.family] += 1;
                prof_clock_ms_[pe.family] += (double)(t1 - t0) / clock_khz_;
            }
        }
        if (tl_.empty()) {  // the timeline reads the same array later
            hip_->hipMemset(stamp_buf_, 0, stamp_used_ * 8);
            stamp_used_ = 0;
        }
    }
    pending_.clear();
}

bool Engine::set_timeline(bool on, std::string &err)
{
    collect_events();
    tl_.clear();
    if (stamp_buf_ && stamp_used_ &&
        !check(hip_->hipMemset(stamp_buf_, 0, stamp_used_ * 8), "hipMemset(stamps)", err))
        return false;
    stamp_used_ = 0;
    timeline_ = on;
    return true;
}

int Engine::timeline_read(lama_launch_time *out, int max, std::string &err)
{
    if (!check(hip_->hipDeviceSynchronize(), "hipDeviceSynchronize", err)) return -1;
    if (tl_.empty() || !stamp_used_ || clock_khz_ <= 0) return 0;
    std::vector<unsigned long long> st(stamp_used_);
    if (!check(hip_->hipMemcpy(st.data(), stamp_buf_, stamp_used_ * 8, hipMemcpyDeviceToHost), "hipMemcpy(stamps)", err))
        return -1;
    unsigned long long base = ~0ull;
    std::vector<std::pair<unsigned long long, unsigned long long>> w(tl_.size(), {~0ull, 0ull});
    for (size_t i = 0; i < tl_.size(); ++i) {
        for (unsigned b = 0; b < tl_[i].grid; ++b) {
            const unsigned long long a = st[tl_[i].stamp_off + 2 * b], e = st[tl_[i].stamp_off + 2 * b + 1];
            if (!a) continue;
            w[i].first = std::min(w[i].first, a);
            w[i].second = std::max(w[i].second, e);
        }
        base = std::min(base, w[i].first);
    }
    int n = 0;
    for (size_t i = 0; i < tl_.size() && n < max; ++i, ++n) {
        out[n].family = tl_[i].family;
        out[n].stream = tl_[i].stream;
        const bool ok = w[i].second >= w[i].first && w[i].first != ~0ull;
        out[n].start_us = ok ? (double)(w[i].first - base) * 1e3 / clock_khz_ : -1;
        out[n].end_us = ok ? (double)(w[i].second - base) * 1e3 / clock_khz_ : -1;
    }
    return n;
}

bool Engine::profile_read_clock(int i, uint64_t &launches, double &ms)
{
    if (i < 0 || i >= F_COUNT) return false;
    collect_events();
    launches = prof_clock_n_[i];
    ms = prof_clock_ms_[i];
    return true;
}

void Engine::profile_reset()
{
    collect_events();
    for (int f = 0; f < F_COUNT; ++f) {
        prof_launches_[f] = prof_clock_n_[f] = 0;
        prof_ms_[f] = prof_flops_[f] = prof_bytes_[f] = prof_clock_ms_[f] = 0;
    }
}

bool Engine::profile_read(int i, std::string &name, uint64_t &launches, double &ms, double &flops, double &bytes)
{
    if (i < 0 || i >= F_COUNT) return false;
    collect_events();
    name = kFamilyName[i];
    launches = prof_launches_[i];
    ms = prof_ms_[i];
    flops = prof_flops_[i];
    bytes = prof_bytes_[i];
    return true;
}

void Engine::print_stats()
{
    collect_events();
    const bool any = flag_profile_ops_ || flag_profile_sub_ || flag_profile_;
    if (flag_profile_ops_ || !any) {
        double total = 0;
        for (int f = 0; f < F_COUNT; ++f) {
            if (!prof_launches_[f]) continue;
            total += prof_ms_[f] / 1e3;
            fprintf(stderr, "op %-14s %5llu calls %7.3fs  (%lld us avg, 1 launches/call)\n", kFamilyName[f],
                    (unsigned long long)prof_launches_[f], prof_ms_[f] / 1e3,
                    (long long)(prof_ms_[f] * 1e3 / (double)prof_launches_[f]));
        }
        fprintf(stderr, "op total %.3fs\n", total);
    }
    if (flag_profile_sub_)
        for (int f = 0; f < F_COUNT; ++f) {
            if (!prof_launches_[f]) continue;
            const double t = prof_ms_[f] / 1e3;
            fprintf(stderr, "sub %-9s %4llu calls %7.3fs  (%lld us avg)  %.1f MFLOP  %.0f GFLOP/s  %.0f MB moved\n",
                    kFamilyName[f], (unsigned long long)prof_launches_[f], t,
                    (long long)(t * 1e6 / (double)prof_launches_[f]), prof_flops_[f] / 1e6,
                    prof_flops_[f] / 1e9 / std::max(t, 1e-9), prof_bytes_[f] / 1e6);
        }
    if (flag_profile_) {
        size_t arena = 0;
        for (auto &kv : plans_) arena += kv.second.arena_bytes;
        fprintf(stderr, "gpu totals: %zu planned shape(s), %zu MB of activation arenas, %zu MB of resident weights\n",
                plans_.size(), arena >> 20, warena_bytes_ >> 20);
    }
}

// ---------------------------------------------------------------- single ops

namespace {
// Device allocations of one test op, released on scope exit.
struct Scratch {
    const HipApi *h;
    std::vector<void *> ptrs;
    ~Scratch()
    {
        for (void *p : ptrs) h->hipFree(p);
    }
};
}  // namespace

#define UPLOAD(var, hostptr, nfloats)                                                                 \
    float *var = nullptr;                                                                             \
    if (!check(hip_->hipMalloc((void **)&var, std::max<size_t>(1, (nfloats)) * 4), "hipMalloc", err)) \
        return false;                                                                                 \
    sc.ptrs.push_back(var);                                                                           \
    if ((hostptr) && !check(hip_->hipMemcpy(var, (hostptr), (nfloats) * 4, hipMemcpyHostToDevice), "hipMemcpy", err)) \
        return false;

bool Engine::op_conv2d(const float *x, int cin, int h, int w, const float *wt, const float *bias, int cout, int k,
                       int stride, const float *scale, const float *shift, int relu, float *out, std::string &err)
{
    int family;
    if (k == 1 && stride == 1)
        family = F_CONV1;
    else if (k == 3 && stride == 1)
        family = F_CONV3;
    else if (k == 3 && stride == 2)
        family = F_CONV3S2;
    else if (k == 7 && stride == 1)
        family = F_CONV7;
    else {
        err = "op_conv2d: unsupported k/stride";
        return false;
    }
    const int pad = k / 2;
    const int oh = (h + 2 * pad - k) / stride + 1, ow = (w + 2 * pad - k) / stride + 1;
    const int wino = family == F_CONV3 ? wino_ : 0;
    const int KC = family == F_CONV1 ? pw_kc(tile_variant(F_CONV1, 1, h * w, cout)) : family == F_CONV7 ? 4 : wino == 42 ? LAMA_W42_KC : wino ? LAMA_WINO_KC : family == F_CONV3S2 ? LAMA_S2_KC : 8;
    if ((size_t)4 * KC * h * w >= ((size_t)1 << 32)) {  // 32-bit staging offsets within a K chunk
        err = "op_conv2d: plane too large";
        return false;
    }
    Arena A;
    const int T = k * k;
    auto getw = [&](int co, int ci, int t) { return wt[((size_t)co * cin + ci) * T + t]; };
    Packed pk = wino == 42 ? pack_wino42(A, cout, cin, getw)
                : wino == 4 ? pack_wino4(A, cout, cin, getw)
                : wino    ? pack_wino(A, cout, cin, getw)
                          : pack(A, cout, cin, T, KC, getw);
    size_t bn = A.add(2 * (size_t)cout);
    for (int i = 0; i < cout; ++i) {
        A.at(bn)[i] = scale ? scale[i] : 1.f;
        A.at(bn)[cout + i] = scale ? shift[i] : 0.f;
    }
    size_t bo = A.add(cout);
    if (bias) std::copy(bias, bias + cout, A.at(bo));
    Scratch sc{hip_, {}};
    UPLOAD(dx, x, (size_t)cin * h * w);
    UPLOAD(dw, nullptr, A.size());
    if (!A.upload(hip_, dw, err)) return false;
    UPLOAD(dout, nullptr, (size_t)cout * oh * ow);
    ConvProblem q{};
    q.s0.src = dx;
    q.s0.wt = dw + pk.off;
    q.s0.C = cin;
    q.s0.IH = family == F_CONV1 ? 1 : h;
    q.s0.IW = family == F_CONV1 ? h * w : w;
    q.s0.nchunk = pk.nchunk;
    q.s0.wrow = pk.wrow;
    q.s0.cs = h * w;
    q.M = cout;
    q.OH = family == F_CONV1 ? 1 : oh;
    q.OW = family == F_CONV1 ? oh * ow : ow;
    int tr, tc;
    tile_shape(family, tr, tc, wino, tile_variant(family, q.OH, q.OW, q.M, q.s0.cs));
    q.tiles_x = (q.OW + tc - 1) / tc;
    q.tiles_y = (q.OH + tr - 1) / tr;
    const int mw = wino == 42 ? LAMA_W42_CH : 64;  // output channels per block
    q.mblocks = (cout + mw - 1) / mw;
    q.nblocks = q.tiles_x * q.tiles_y * q.mblocks;
    q.bias = bias ? dw + bo : nullptr;
    q.scale = scale ? dw + bn : nullptr;
    q.shift = scale ? dw + bn + cout : nullptr;
    q.relu = relu;
    q.out = dout;
    q.out_cstride = (long)oh * ow;
    q.outW = q.OW;
    q.oy_mul = q.ox_mul = 1;
    q.vec_in = (wino == 4 || wino == 42) && family == F_CONV3 && w % 4 == 0;  // both Winograd load paths, by width
    pw_xcd_pad(family, q);
    UPLOAD(dq, nullptr, (sizeof q + 3) / 4);
    if (!check(hip_->hipMemcpy(dq, &q, sizeof q, hipMemcpyHostToDevice), "hipMemcpy", err)) return false;
    Launch L{};
    L.fn = conv_fn(family, &q, 1);
    L.family = family;
    L.grid = (unsigned)q.nblocks;
    L.block = L.fn == fn_wino42_ ? 8 * LAMA_W42_CH : 0;
    L.arg = dq;
    L.ps = prob_starts(&q, 1);
    L.nparams = 2;
    if (!launch(L, stream_, err) || !check(hip_->hipStreamSynchronize(stream_), "kernel", err)) return false;
    return check(hip_->hipMemcpy(out, dout, (size_t)cout * oh * ow * 4, hipMemcpyDeviceToHost), "hipMemcpy", err);
}

bool Engine::op_convt(const float *x, int cin, int h, int w, const float *wt, const float *bias, int cout,
                      const float *scale, const float *shift, int relu, float *out, std::string &err)
{
    Arena A;
    const int np = convt_rows_ ? 2 : 4;  // problems: the two row phases, or the four phases
    Packed ph[4];
    for (int k = 0; k < np; ++k)
        ph[k] = convt_rows_ ? pack_convt_rows(A, cout, cin, k, wt) : pack_convt_phase(A, cout, cin, k, wt);
    size_t bn = A.add(2 * (size_t)cout), bo = A.add(cout);
    for (int i = 0; i < cout; ++i) {
        A.at(bn)[i] = scale ? scale[i] : 1.f;
        A.at(bn)[cout + i] = scale ? shift[i] : 0.f;
        A.at(bo)[i] = bias ? bias[i] : 0.f;
    }
    Scratch sc{hip_, {}};
    UPLOAD(dx, x, (size_t)cin * h * w);
    UPLOAD(dw, nullptr, A.size());
    if (!A.upload(hip_, dw, err)) return false;
    UPLOAD(dout, nullptr, (size_t)cout * 4 * h * w);
    ConvProblem q[4]{};
    unsigned nb = 0;
    for (int k = 0; k < np; ++k) {
        ConvProblem &c = q[k];
        std::memset(&c, 0, sizeof c);
        c.s0.src = dx;
        c.s0.wt = dw + ph[k].off;
        c.s0.C = cin;
        c.s0.IH = h;
        c.s0.IW = w;
        c.s0.nchunk = ph[k].nchunk;
        c.s0.wrow = ph[k].wrow;
        c.s0.cs = h * w;
        c.M = cout;
        c.OH = h;
        c.OW = w;
        int tr, tc;
        tile_shape(F_CONVT, tr, tc, 0, tile_variant(F_CONVT, h, w));
        c.tiles_x = (w + tc - 1) / tc;
        c.tiles_y = (h + tr - 1) / tr;
        c.mblocks = (cout + 63) / 64;
        c.nblocks = c.tiles_x * c.tiles_y * c.mblocks;
        nb += c.nblocks;
        c.bias = dw + bo;
        c.scale = dw + bn;
        c.shift = dw + bn + cout;
        c.relu = relu;
        c.out = dout;
        c.out_cstride = 4l * h * w;
        c.outW = 2 * w;
        c.oy_mul = c.ox_mul = 2;
        c.oy_off = k >> 1;
        c.ox_off = k & 1;
    }
    UPLOAD(dq, nullptr, (sizeof q + 3) / 4);
    if (!check(hip_->hipMemcpy(dq, q, sizeof q, hipMemcpyHostToDevice), "hipMemcpy", err)) return false;
    Launch L{};
    L.fn = conv_fn(F_CONVT, q, np);
    L.family = F_CONVT;
    L.grid = nb;
    L.arg = dq;
    L.ps = prob_starts(q, np);
    L.nparams = 2;
    if (!launch(L, stream_, err) || !check(hip_->hipStreamSynchronize(stream_), "kernel", err)) return false;
    return check(hip_->hipMemcpy(out, dout, (size_t)cout * 4 * h * w * 4, hipMemcpyDeviceToHost), "hipMemcpy", err);
}

bool Engine::op_fft(bool inverse, const float *in, const float *feat, int c, int h, int w, float *out, std::string &err)
{
    FftLen fr, fc;
    std::vector<float> twr, twc;
    if (!fft_len(w, fr, twr, err) || !fft_len(h, fc, twc, err)) return false;
    FftGeom g;
    if (!fft_geom(c, h, w, g, err)) return false;
    const int Wh = w / 2 + 1;
    const size_t nin = inverse ? 2ul * c * h * Wh : (size_t)c * h * w;
    const size_t nout = inverse ? (size_t)c * h * w : 2ul * c * h * Wh;
    std::vector<float> zeros;
    if (inverse && !feat) {
        zeros.assign((size_t)c * h * w, 0.f);
        feat = zeros.data();
    }
    Scratch sc{hip_, {}};
    UPLOAD(din, in, nin);
    UPLOAD(dout, nullptr, nout);
    UPLOAD(dtr, twr.data(), twr.size());
    UPLOAD(dtc, twc.data(), twc.size());
    UPLOAD(dfeat, inverse ? feat : nullptr, inverse ? (size_t)c * h * w : 1);
    UPLOAD(dtmp, nullptr, g.split ? g.tmp_bytes / 4 : 1);
    FftArgs a{};
    a.row = fr;
    a.col = fc;
    a.row.tw = dtr;
    a.col.tw = dtc;
    a.C = c;
    a.H = h;
    a.W = w;
    a.Wh = Wh;
    a.in = din;
    a.out = dout;
    a.feat = inverse ? dfeat : nullptr;
    a.scale = (float)(1.0 / std::sqrt((double)h * w));
    a.rows_per_block = g.rows_per_block;
    a.cols_per_block = g.cols_per_block;
    a.tmp = g.split ? dtmp : nullptr;
    a.rs = (long)h * w;
    a.ss = (long)h * Wh;
    UPLOAD(da, nullptr, (sizeof a + 3) / 4);
    if (!check(hip_->hipMemcpy(da, &a, sizeof a, hipMemcpyHostToDevice), "hipMemcpy", err)) return false;
    Plan tmp;
    push_fft(tmp, inverse, g, da, S_MAIN, 0, 0);
    for (const Launch &L : tmp.launches)
        if (!launch(L, stream_, err)) return false;
    if (!check(hip_->hipStreamSynchronize(stream_), "kernel", err)) return false;
    return check(hip_->hipMemcpy(out, dout, nout * 4, hipMemcpyDeviceToHost), "hipMemcpy", err);
}

bool Engine::op_tail(const float *x, int cin, int h, int w, const float *wt, const float *bias, float *out,
                     std::string &err)
{
    if (cin < 1 || cin > 64) {
        err = "op_tail: the tail kernel stages at most 64 input channels of weights";
        return false;
    }
    Scratch sc{hip_, {}};
    UPLOAD(dx, x, (size_t)cin * h * w);
    UPLOAD(dw, wt, (size_t)3 * cin * 49);
    UPLOAD(db, bias, 3);
    UPLOAD(dout, nullptr, (size_t)3 * h * w);
    TailArgs a{};
    a.src = dx;
    a.wt = dw;
    a.bias = db;
    a.out = dout;
    a.Cin = cin;
    a.H = h;
    a.W = w;
    UPLOAD(da, nullptr, (sizeof a + 3) / 4);
    if (!check(hip_->hipMemcpy(da, &a, sizeof a, hipMemcpyHostToDevice), "hipMemcpy", err)) return false;
    Launch L{};
    L.fn = fn_[F_TAIL];
    L.family = F_TAIL;
    L.grid = (unsigned)(((w + LAMA_TAIL_COLS - 1) / LAMA_TAIL_COLS) * ((h + LAMA_TAIL_ROWS - 1) / LAMA_TAIL_ROWS));
    L.arg = da;
    L.nparams = 1;
    if (!launch(L, stream_, err) || !check(hip_->hipStreamSynchronize(stream_), "kernel", err)) return false;
    return check(hip_->hipMemcpy(out, dout, (size_t)3 * h * w * 4, hipMemcpyDeviceToHost), "hipMemcpy", err);
}

}  // namespace lama
