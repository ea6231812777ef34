// The HIP engine behind lama_hip.h: weights resident on the device, one
// preplanned buffer set and launch list per input shape.
#pragma once
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "hip_api.h"
#include "kernels/common.h"
#include "lama_host.h"
#include "lama_hip.h"

namespace lama {

// F_CONV3G: the FFC's g2l launches, the same kernel as F_CONV3 (l2l + l2g);
// a family of its own so that profiling keeps the two launches apart.
// F_INPUT: the device build_input of the inpaint entry points.
enum Family { F_CONV7, F_CONV3S2, F_CONV3, F_CONV1, F_CONVT, F_RFFT, F_IRFFT, F_TAIL, F_FINAL, F_CONV1R, F_CONV3G, F_INPUT, F_COUNT };
extern const char *const kFamilyName[F_COUNT];

// Number of plan steps of the reference (model.rs:135-207) and the size in
// floats of the activation after each (cpu.rs:536-546 dump layout).
constexpr int kSteps = 29;
size_t step_numel(int step, int h, int w);

// Convolution weights packed for the MFMA kernels: [M][nchunk][taps][KC].
struct Packed {
    size_t off = 0;  // float offset in the weight arena
    int M = 0, C = 0, T = 0, KC = 0, nchunk = 0, wrow = 0;
};

// Streams of a forward: the main one (the caller's) and a side stream that
// carries the SpectralTransform chain of every FFC concurrently with the
// FFC's spatial GEMM.  Cross-stream order is kept with the engine's events.
// S_G2L carries the FFC's g2l launch B(k), so that B(k+1) overlaps A(k+1): they read
// different inputs (x_g from the side stream, x_l from the main stream's finalize).
// LAMA_B_STREAM=0 runs B on the main stream instead.
enum { S_MAIN = 0, S_SIDE = 1, S_G2L = 2, S_COUNT = 3 };
// EV_FORK: model.4 done (the side stream's first input); EV_A0/1: FFC k's
// l2l + l2g launch done (its GC partial), by parity of k; EV_S0/1: FFC k's
// conv2 done (its global output half), by parity of k.
// EV_B0/1: FFC k's g2l launch done (on S_G2L), by parity of k.
enum { EV_FORK = 0, EV_A0 = 1, EV_A1 = 2, EV_S0 = 3, EV_S1 = 4, EV_B0 = 5, EV_B1 = 6, EV_COUNT = 7 };

struct Launch {
    hipFunction_t fn;
    int family;
    int stream;     // S_MAIN or S_SIDE
    int wait_ev;    // event the stream waits for before the launch, or -1
    int record_ev;  // event recorded on the stream after the launch, or -1
    unsigned grid;
    unsigned block;  // threads per block (0 = LAMA_NT)
    unsigned shmem;
    void *arg;   // device pointer to this launch's descriptor(s)
    ProbStarts ps;  // conv kernels: problem count and first workgroups (second parameter)
    int nparams;
    int step_end;  // plan step completed by this launch, or -1
    double flops, bytes;
};

// How the rfft2/irfft2 of one [C][H][W] batch of planes are launched.
struct FftGeom {
    bool split = false;
    size_t lds = 0;                 // single-block mode: bytes per block
    int rows_per_block = 0, cols_per_block = 0;
    size_t lds_rows = 0, lds_cols = 0;
    unsigned grid_rows = 0, grid_cols = 0;
    size_t tmp_bytes = 0;           // interleaved complex [C][H][W/2+1]
    int ct = 0;                     // single-block square plane with compile-time kernels: 1 + index in kFftCtSide, else 0
    int ct_split = 0;               // split square plane with compile-time kernels (128 or 256), else 0
    unsigned block_cols = 0;        // threads per column-launch block when not LAMA_FFT_NT
};

struct ArenaLayout {
    size_t in, a1, a2, a3, x, y, f, g, s, s2, out, gc, lq, tmp, twr, twc, rgb8, mask8, out8, desc;
};

struct Plan {
    int H = 0, W = 0;
    void *arena = nullptr;
    size_t arena_bytes = 0;
    bool own_arena = true;  // false: the arena is memory the engine did not allocate
    float *in = nullptr, *out = nullptr;
    // 8-bit staging of the inpaint entry points (image, mask, composite), each
    // sized for H x W; a call uses its h x w prefix
    uint8_t *rgb8 = nullptr, *mask8 = nullptr, *out8 = nullptr;
    // per step: the device activation (nullptr: host-derived), its planes of
    // `plane` floats `stride` floats apart
    struct StepSrc {
        const float *src;
        size_t planes, plane, stride;
    };
    std::vector<StepSrc> step_src;
    std::vector<Launch> launches;
    Launch build_in{}, tail_u8{};  // device build_input, and the tail with the composite fused
    // what build_plan uploads into the arena (kept for a re-upload)
    std::vector<char> desc_host;
    std::vector<float> twr_host, twc_host;
    size_t desc_off = 0, twr_off = 0, twc_off = 0;
    hipGraphExec_t graph = nullptr;  // the launch list captured once, replayed per forward
    bool graph_failed = false;       // the runtime refused the capture: per-launch path
};

// The isolated SpectralTransform of each FFC (conv1 -> rfft2 -> FU conv ->
// irfft2 -> conv2) over [384][h][w] planes, for the SpectralTransform entry
// point: one arena per plane shape, the launches of all 36 FFCs.
struct SpecPlan {
    int H = 0, W = 0;
    void *arena = nullptr;
    size_t arena_bytes = 0;
    float *x = nullptr, *f = nullptr, *s = nullptr, *s2 = nullptr, *g = nullptr, *out = nullptr;
    std::vector<Launch> launches[36];
};

class Engine {
public:
    ~Engine();
    bool open(std::string &err);
    bool load_weights(const uint8_t *blob, size_t len, const lama_tensor_info *t, size_t n, std::string &err);
    bool forward_host(const float *in, int h, int w, float *out, float *const *steps, std::string &err);
    bool forward_device(const float *d_in, int h, int w, float *d_out, hipStream_t s, std::string &err);
    // The whole-image flow of main.rs:241-307 on the device: pad to a multiple
    // of 8, build_input, forward, 8-bit composite.  rgb HWC [h][w][3], mask
    // [h][w], out HWC [h][w][3]; net_out (host, optional) receives the
    // [3][H][W] sigmoid plane of the padded shape.
    bool inpaint_host(const uint8_t *rgb, const uint8_t *mask, int h, int w, uint8_t *out, float *net_out,
                      std::string &err);
    bool inpaint_device(const uint8_t *d_rgb, const uint8_t *d_mask, int h, int w, uint8_t *d_out, hipStream_t s,
                        std::string &err);
    // The SpectralTransform of FFC k (0..35) alone over x [384][h][w]:
    // out [384][h][w] = conv2(f + irfft2(FU(rfft2(f)))), f = ReLU(BN1(conv1 x)).
    // stages (host, optional, entries may be NULL): [0] f [192][h][w],
    // [1] spectrum [384][h][w/2+1], [2] FU conv after BN + ReLU [384][h][w/2+1],
    // [3] f + irfft2 [192][h][w].
    bool spectral_host(int k, const float *x, int h, int w, float *out, float *const *stages, std::string &err);
    bool spectral_device(int k, const float *d_x, int h, int w, float *d_out, hipStream_t s, std::string &err);
    // Waits for the engine stream and for the last pass enqueued on a caller's stream.
    bool synchronize(std::string &err);
    // forward_device with no device allocation: the activation arena and the
    // launch descriptors live in the device's lama_scratch array (one per device
    // per process, shared by every context on it; see lama_hip.h).
    bool forward_device_noalloc(const float *d_in, int h, int w, float *d_out, hipStream_t s, std::string &err);

    // profiling (families whose bit is set get per-launch events)
    void set_profile(uint32_t mask) { prof_mask_ = mask; }
    void profile_reset();
    bool profile_read(int i, std::string &name, uint64_t &launches, double &ms, double &flops, double &bytes);
    // The summaries of cuda.rs:1738-1806 to stderr, from the per-family
    // event timings: "op" lines (LAMA_PROFILE_OPS), "sub" lines
    // (LAMA_PROFILE_SUB), the "gpu totals" line (LAMA_PROFILE); with none of
    // the flags set, the "op" lines.
    void print_stats();
    // Family i's profiled conv launches timed by their kernel-clock stamps
    // (first workgroup start to last workgroup end; the conv families only).
    bool profile_read_clock(int i, uint64_t &launches, double &ms);
    // Timeline: while on, every launch (any family) stores its workgroups'
    // kernel-clock stamps, without events; timeline_read waits for the device
    // and returns, per launch in issue order, its family, stream and
    // first-start / last-end in microseconds from the first record's start.
    bool set_timeline(bool on, std::string &err);
    int timeline_read(lama_launch_time *out, int max, std::string &err);
    int launch_count(int h, int w);
    // The kernel of the first launch of `family` in the plan at h x w (null
    // without that plan or launch).
    const char *kernel_name(int h, int w, int family) const;
    // Device bytes of one forward at h x w: the activation arena of that shape
    // (exact, from its layout) and the resident weights (0 before loading).
    bool plan_bytes(int h, int w, uint64_t &arena, uint64_t &weights, std::string &err);

    // single kernel families (parity tests)
    bool op_conv2d(const float *x, int cin, int h, int w, const float *wt, const float *bias, int cout, int k,
                   int stride, const float *scale, const float *shift, int relu, float *out, std::string &err);
    bool op_convt(const float *x, int cin, int h, int w, const float *wt, const float *bias, int cout,
                  const float *scale, const float *shift, int relu, float *out, std::string &err);
    bool op_fft(bool inverse, const float *in, const float *feat, int c, int h, int w, float *out, std::string &err);
    bool op_tail(const float *x, int cin, int h, int w, const float *wt, const float *bias, float *out,
                 std::string &err);

    const HipApi *hip() const { return hip_; }
    hipStream_t stream() const { return stream_; }
    bool check(hipError_t e, const char *what, std::string &err);
    bool get_fn(hipFunction_t &fn, const char *name, std::string &err);  // and records its name

private:
    struct FfcW {
        Packed local, l2g, conv2, conv1, fu;
        Packed local42, l2g42;  // F(2x4, 3x3) packs for the large planes (when w42_packed_)
        size_t bn1, fu_bn, bn_l, bn_g;  // folded: scale at off, shift at off + n
    };
    struct UpW {
        Packed ph[4];
        Packed row[2];  // the taps of row phases 0 and 1 (lama_convt_rows)
        size_t bias = 0, bn = 0;
        int cin = 0, cout = 0;
    };

    Plan *plan_for(int h, int w, std::string &err);
    bool build_plan(Plan &p, void *arena, std::string &err);
    bool upload_plan(const Plan &p, hipStream_t s, std::string &err);
    bool mark_done(hipStream_t s, std::string &err);
    // u8_h > 0: the inpaint pass of an u8_h x u8_w image (build_input first,
    // the tail with the composite fused in)
    bool run(Plan &p, hipStream_t s, float *const *steps, std::string &err, int u8_h = 0, int u8_w = 0);
    SpecPlan *spec_plan_for(int h, int w, std::string &err);
    bool step_hooks(Plan &p, const float *in, std::string &err);
    bool replay(Plan &p, hipStream_t s, std::string &err);
    static size_t arena_layout(int H, int W, const FftGeom &fg, size_t ntwr, size_t ntwc, int ksplit, int pk1, int pku,
                               ArenaLayout &L);
    bool use_graph(const Plan &p) const;
    void free_plan(Plan &p);
    bool launch(const Launch &L, hipStream_t s, std::string &err, hipEvent_t record = nullptr);
    bool fft_len(int n, FftLen &L, std::vector<float> &tw, std::string &err);
    bool fft_geom(int C, int H, int W, FftGeom &g, std::string &err) const;
    void push_fft(Plan &p, bool inverse, const FftGeom &g, void *arg, int stream, double bytes_a, double bytes_b);
    void collect_events();

    const HipApi *hip_ = nullptr;
    int device_ = 0;
    hipModule_t module_ = nullptr;
    std::map<hipFunction_t, const char *> fn_names_;  // every loaded kernel's name
    hipFunction_t fn_[F_COUNT] = {};
    // split-mode FFT kernels: rfft2 rows, rfft2 cols, irfft2 cols, irfft2 rows
    hipFunction_t fn_split_[4] = {};
    hipFunction_t fn_pw_any_[2] = {};  // 1x1 kernels for planes that are not float4-aligned
    hipFunction_t fn_pw_v2_[2] = {};   // 1x1 kernels for float2-aligned planes of even length
    hipFunction_t fn_fft_ct_[4][2] = {};  // [64x64, 32x32, 75x75, 64x64 shuffle rows][rfft2, irfft2]
    hipFunction_t fn_split_ct_[2][4] = {};  // [256x256, 128x128][as fn_split_]
    // FFC 3x3 convolutions as Winograd F(2,3) along x (lama_conv3x3w), or
    // with LAMA_FFC_WINO=0 as the direct implicit GEMM (lama_conv3x3); chosen
    // at open, since the weights are packed for one or the other
    // LAMA_FFC_WINO: 0 direct; 2 F(2,3) (lama_conv3x3w); 4 (default) F(4,3)
    // in blocks of 2 x 64, 4 x 32 or 8 x 16 output pixels (lama_conv3x3w4,
    // w4n, w4q), chosen per plane shape; 42 F(2x4, 3x3) in blocks of 4 x 64
    // (lama_conv3x3w42)
    int wino_ = 4;
    // the default mode also packs F(2x4, 3x3) weights and takes that kernel
    // on large planes (wino_for); LAMA_W42=0 (read at open) keeps F(4,3)
    bool w42_packed_ = true;
    // the Winograd weight transforms of the FFC 3x3 convolutions run on the
    // device (lama_pack_wino) from the raw weights; LAMA_HOST_PACK=1 (read at
    // open) packs them on the host instead (the same floats)
    bool dev_pack_ = true;
    hipFunction_t fn_pack_ = nullptr;
    int w4_force_ = 0;  // LAMA_W4_TILE: 64, 32 or 16 forces the F(4,3) block width
    int w4_variant(int OH, int OW) const;  // index into fn_wino4_
    int tile_variant(int family, int OH, int OW, int M = 0, long cs = 0) const;
    unsigned w4_lds_pad(int h8, int w8, int ks) const;
    int ksplit_force_ = 0;  // LAMA_KSPLIT: 1, 2 or 4 forces the K split of the FFC GEMMs
    int w4_ldspad_force_ = -1;  // LAMA_W4_LDSPAD: 0 or 1 forces the F(4,3) LDS padding off or on
    int edge_force_ = 0;  // LAMA_EDGE_TILE: 32 or 16 forces the stride-2 / transposed conv tile width
    int pw_force_ = 0;    // LAMA_PW_TILE: 32 (K-half) or 64 forces the float4 pointwise tile width
    bool convt_rows_ = true;  // LAMA_CONVT_ROWS=0: the transposed convs as four phase problems (lama_convt)
    int fin_groups_force_ = 0;  // LAMA_FIN_GROUPS: 1 or 2 forces the finalize kernel's groups per thread
    int pw_ksplit_force_ = 0;  // LAMA_PW_KSPLIT: 1, 2 or 4 forces the K split of conv1 and the FourierUnit conv
    // K split of the SpectralTransform conv1 (k1) and FourierUnit conv (ku)
    int fin_groups(size_t plane) const;
    void pw_ksplit_for(int h, int w, const FftGeom &fg, int &k1, int &ku) const;
    // K split of the FFC GEMMs at input h x w (1 unless the F(4,3) kernels
    // would leave CUs idle)
    int ksplit_for(int h, int w) const;
    hipFunction_t fn_wino_ = nullptr, fn_wino4_[3] = {};
    hipFunction_t fn_wino42_ = nullptr;  // lama_conv3x3w42 (LAMA_FFC_WINO=42)
    // wino < 0: the engine's LAMA_FFC_WINO mode
    hipFunction_t conv_fn(int family, const ConvProblem *probs, size_t n, int wino = -1) const;
    int wino_for(int h8, int w8) const;
    size_t max_lds_ = 64 * 1024;  // bytes of LDS one block may use on this device
    hipStream_t stream_ = nullptr, side_ = nullptr, g2l_ = nullptr;
    hipEvent_t ev_[EV_COUNT] = {};
    hipEvent_t ev_done_ = nullptr;  // the end of the last pass enqueued on a caller's stream
    bool done_pending_ = false;
    // the reference's debug flags (cuda.rs:127-150), read at open
    bool flag_profile_ = false, flag_profile_sync_ = false, flag_profile_ops_ = false, flag_profile_sub_ = false;
    int dump_step_ = -1;  // LAMA_DUMP_STEP
    bool capturing_ = false;  // run() is recording a graph

    // weights
    bool have_weights_ = false;
    float *warena_ = nullptr;
    Packed head_, down_[3];
    size_t head_bn_ = 0, down_bn_[3] = {0, 0, 0};
    FfcW ffc_[36];
    UpW up_[3];
    size_t tail_w_ = 0, tail_b_ = 0;
    size_t warena_bytes_ = 0;
    const float *wp(size_t off) const { return warena_ + off; }

    std::map<std::pair<int, int>, Plan> plans_;
    // the no-allocation entry point: its plan (arena = this device's scratch
    // array), the array's address, and this engine's identity in the
    // process-wide record of which context's descriptors the array holds
    Plan na_plan_;
    void *scratch_ = nullptr;  // set by the entry point's first call (scratch_setup)
    uint64_t id_ = 0;
    bool scratch_setup(std::string &err);
    void release_scratch_owner();
    std::map<std::pair<int, int>, SpecPlan> spec_plans_;
    hipFunction_t fn_build_in_ = nullptr, fn_tail_u8_ = nullptr;
    hipFunction_t fn_finalize_ks_[2] = {};  // lama_finalize10, lama_finalize20 (K split 2, 4)
    hipFunction_t fn_finalize_g2_[3] = {};  // the same three with two element groups per thread
    hipFunction_t fn_edge_q_[2] = {};       // lama_conv3x3s2_q, lama_convt_q (4 x 16 tiles)
    hipFunction_t fn_head_r_ = nullptr;     // lama_conv7x7r (the 4 -> 64 head, weights in registers)
    hipFunction_t fn_pw_kh_[2] = {};        // lama_conv1x1_kh, lama_conv1x1_res_kh (64 x 32 K-half tiles)
    bool head_r_ = true;                    // LAMA_HEAD_R=0: the head through lama_conv7x7 (weights in LDS)
    hipFunction_t fn_convt_rows_[2] = {};   // lama_convt_rows (2 x 32 positions), lama_convt_rows_q (4 x 16)

    // profiling
    uint32_t prof_mask_ = 0;
    struct Pending {
        hipEvent_t a, b;
        int family;
        double flops, bytes;
        long stamp_off;  // first entry of the launch's kernel-clock stamps, or -1
        unsigned grid;
    };
    // kernel-clock stamps of profiled conv launches: [2 * workgroup] entries
    // per launch (start, end), zero where unwritten; allocated on first use
    unsigned long long *stamp_buf_ = nullptr;
    size_t stamp_cap_ = 0, stamp_used_ = 0;
    double clock_khz_ = 0;  // device wall-clock rate
    uint64_t prof_clock_n_[F_COUNT] = {};
    bool timeline_ = false;
    struct TlRec {
        int family, stream;
        long stamp_off;
        unsigned grid;
    };
    std::vector<TlRec> tl_;
    double prof_clock_ms_[F_COUNT] = {};
    std::vector<Pending> pending_;
    std::vector<hipEvent_t> event_pool_;
    uint64_t prof_launches_[F_COUNT] = {};
    double prof_ms_[F_COUNT] = {}, prof_flops_[F_COUNT] = {}, prof_bytes_[F_COUNT] = {};
};

}  // namespace lama
