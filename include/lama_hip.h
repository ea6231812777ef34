/*
 * lama_hip.h -- the drop-in C ABI of the MI355X backend (liblama_hip.so).
 *
 * It replaces the reference's CUDA engine, `lama-rs/src/cuda.rs`, at the one
 * boundary its caller uses: `cuda::run(store, model, input, h, w) ->
 * Result<Vec<f32>, String>` (cuda.rs:1542-1548, called from main.rs:330-346),
 * plus the device bring-up, the memory query of `mem.rs` and the stats hooks.
 * Below it, the library dlopens `libamdhip64` (LAMA_HIP_LIB overrides the
 * path, like LA_CUDA_LIB) and loads its own gfx950 code object with
 * hipModuleLoadData; no HIP or torch types cross this interface.
 *
 * Conventions: activations are planar f32 [c][h][w]; `h`, `w` are multiples
 * of 8 (the caller pads, main.rs:241-242), any size >= 8.  Every call returns
 * 0 on success or nonzero with a UTF-8 message in `err` (when non-NULL), the
 * analogue of `Err(String)`; a failed call leaves the process able to run
 * another engine.  Single host thread, not re-entrant (cuda.rs keeps its
 * state thread-local too).
 */
#ifndef LAMA_HIP_H
#define LAMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "lama_host.h" /* lama_tensor_info */

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lama_hip_ctx lama_hip_ctx;

/* Replaces Cuda::open / ctx() (cuda.rs:222-275): load the HIP runtime, pick
 * the device (LAMA_HIP_DEVICE, default 0), load the kernel module, create the
 * engine stream. */
int lama_hip_open(lama_hip_ctx **out, char *err, size_t errlen);
void lama_hip_close(lama_hip_ctx *ctx);

/* The plan this engine implements, as the reference's model::describe
 * (model.rs:260-274) prints it: "29 steps, 40 FFC_BN_ACT calls, 18
 * resblocks", the Big-LaMa generator of model::build (model.rs:117-257).
 * cuda::run takes the Model it runs; this engine's plan is fixed, so the
 * caller compares describe(model) with this string and reports a plan
 * mismatch instead of running another network's weights through it. */
const char *lama_hip_plan_signature(void);

/* Replaces the weight side of load_steps (cuda.rs:330-387 blob_arena,
 * 595-693 Staging, 695-734 load_conv, 737-830 BN fold, 903-962 load_steps):
 * `blob` is the whole safetensors file and `table` its tensor index with
 * absolute offsets (WeightStore, weights.rs:80-139).  Every derived tensor
 * (folded BNs, MFMA-packed convolution weights, sub-pixel phase weights) is
 * built once and uploaded in one copy; it stays resident for later calls. */
int lama_hip_load_weights(lama_hip_ctx *ctx, const void *blob, size_t blob_len,
                          const lama_tensor_info *table, size_t n, char *err, size_t errlen);

/* Replaces cuda::run (cuda.rs:1542-1691): one forward pass.  `input` is the
 * host [4][h][w] tensor of build_input (main.rs:175-196); `output` receives
 * the host [3][h][w] sigmoid output.  Synchronous. */
int lama_hip_forward(lama_hip_ctx *ctx, const float *input, int h, int w, float *output,
                     char *err, size_t errlen);

/* The same pass on device-resident buffers, enqueued on `stream` (a
 * hipStream_t; NULL = the engine's own stream).  Asynchronous. */
int lama_hip_forward_device(lama_hip_ctx *ctx, const float *d_input, int h, int w,
                            float *d_output, void *stream, char *err, size_t errlen);

/* lama_hip_forward_device that allocates nothing.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid it).  A stream under graph capture is
 * refused with an error: a captured pass would replay against whatever
 * descriptors the shared array holds at replay time.
 * The pass's activations, partial sums, FFT scratch and launch descriptors
 * live in a device array of LAMA_SCRATCH_BYTES = 192 MiB (`lama_scratch`, a
 * code object of its own that this entry point's first call on a device
 * loads, once per device per process: that call is the one that loads it,
 * so make it before any phase that must not allocate; the process then holds
 * the array on that device until it ends.  Processes that never call this
 * entry point do not hold it.  If the load fails, that call returns the
 * error and the next call tries again).  Shapes whose arena
 * exceeds it are rejected with an error: up to 512 x 512 fits (177 MiB).
 * The call makes no hipMalloc, hipFree, event or graph creation (and no
 * per-family profiling or launch timeline); the caller passes device input and output as for
 * lama_hip_forward_device.  Every context on a GPU shares that GPU's array,
 * which keeps the last call's contents; no kernel of the pass reads what the
 * pass has not written, and the launch descriptors are re-uploaded on
 * `stream` whenever another context or shape used the array last.  Calls
 * that overlap on one GPU (different streams, threads or contexts) race on
 * the array: the caller orders them.  Asynchronous on `stream` (NULL = the
 * engine's own); lama_hip_synchronize waits for it. */
int lama_hip_forward_device_noalloc(lama_hip_ctx *ctx, const float *d_input, int h, int w,
                                    float *d_output, void *stream, char *err, size_t errlen);

/* The whole-image flow around cuda::run, on the device: the pad to a multiple
 * of 8 (main.rs:241-242), build_input (main.rs:175-196), the forward, and the
 * 8-bit composite of main.rs:272-307 fused into the output convolution's
 * epilogue -- hole pixels (mask > 0) take trunc(clamp(v,0,1)*255 + 0.5), all
 * others the source bytes.  `rgb` is HWC [h][w][3], `mask` [h][w] (the red
 * channel of the mask PNG, image.rs), `out_rgb` HWC [h][w][3]; any h, w >= 1.
 * `net_out` (may be NULL) receives the [3][H][W] sigmoid plane of the padded
 * shape, H = h rounded up to a multiple of 8 (likewise W).  The --tile and
 * --sections flows (main.rs:422-437, 538-552) paste a window's composite.
 * Synchronous. */
int lama_hip_inpaint(lama_hip_ctx *ctx, const uint8_t *rgb, const uint8_t *mask, int h, int w,
                     uint8_t *out_rgb, float *net_out, char *err, size_t errlen);

/* lama_hip_inpaint on device-resident buffers, enqueued on `stream` (NULL =
 * the engine's own).  Asynchronous; lama_hip_synchronize waits for it. */
int lama_hip_inpaint_device(lama_hip_ctx *ctx, const uint8_t *d_rgb, const uint8_t *d_mask, int h, int w,
                            uint8_t *d_out_rgb, void *stream, char *err, size_t errlen);

/* One FFC's SpectralTransform alone (Spectral::forward, cpu.rs:239-265, and
 * FourierUnit::forward, cpu.rs:270-308; GPU spectral_forward, cuda.rs:1460-1539):
 * out [384][h][w] = conv2(f + irfft2(ReLU(BN(FU(rfft2(f)))))), with
 * f = ReLU(BN1(conv1(x))), x [384][h][w], for FFC `ffc` in 0..35 of the loaded
 * weights (model.{5+ffc/2}.conv{1+ffc%2}).  `stages` (may be NULL, as may any
 * entry) receives the LAMA_DUMP_SPECTRAL stages (cpu.rs:242-257): [0] f
 * [192][h][w]; [1] the stacked spectrum [384][h][w/2+1]; [2] the FU conv after
 * BN + ReLU [384][h][w/2+1]; [3] f + irfft2 [192][h][w].  Synchronous. */
int lama_hip_spectral(lama_hip_ctx *ctx, int ffc, const float *x, int h, int w, float *out,
                      float *const *stages, char *err, size_t errlen);
/* The same on device buffers, enqueued on `stream` (NULL = the engine's). */
int lama_hip_spectral_device(lama_hip_ctx *ctx, int ffc, const float *d_x, int h, int w, float *d_out,
                             void *stream, char *err, size_t errlen);

/* LAMA_DUMP_STEP (cuda.rs:1572-1574, 1647-1662): a forward that also copies
 * the activation after plan step i (local planes then global planes, the
 * layout of cpu.rs:536-546) into steps[i] when steps[i] is non-NULL,
 * for i in [0, 29).  Synchronous. */
int lama_hip_forward_steps(lama_hip_ctx *ctx, const float *input, int h, int w, float *output,
                           float *const *steps, char *err, size_t errlen);

/* Replaces mem.rs:93-99 device_memory(): free/total bytes and device name
 * of the device lama_hip_open would use.  Works without an open context. */
int lama_hip_vram(uint64_t *free_bytes, uint64_t *total_bytes, char *name, size_t namelen,
                  char *err, size_t errlen);

/* Per-kernel timing, the analogue of LAMA_PROFILE_OPS / print_op_stats
 * (cuda.rs:1703-1782): while enabled, every launch of a kernel family whose
 * bit is set in `mask` is bracketed by events on the stream it runs on.
 * Families: 0 conv7x7, 1 conv3x3s2, 2 conv3x3 (FFC l2l + l2g), 3 conv1x1,
 * 4 convt, 5 rfft2, 6 irfft2, 7 tail, 8 finalize (FFC local branch
 * epilogue), 9 conv1x1res (SpectralTransform conv2 with the l2g addend),
 * 10 conv3x3g2l (FFC g2l), 11 build_input (the inpaint entry points' device
 * build_input).  A launch issued after a wait on another stream
 * is timed from that wait, so its time includes the wait. */
int lama_hip_profile(lama_hip_ctx *ctx, uint32_t mask);
void lama_hip_profile_reset(lama_hip_ctx *ctx);
/* Family i's accumulated launches, device milliseconds (waits for the
 * recorded events), and algorithmic FLOPs and HBM bytes (sums over launches).
 * Returns 1 for a valid i, 0 past the end. */
int lama_hip_profile_read(lama_hip_ctx *ctx, int i, char *name, size_t namelen, uint64_t *launches,
                          double *ms, double *flops, double *bytes);
/* Family i's profiled launches timed on the device clock instead of by
 * events: each workgroup of a profiled convolution launch records its start
 * and end (s_memrealtime); a launch lasts from its first workgroup start to
 * its last workgroup end, the window a kernel trace reports, without the
 * dispatch latency the event interval includes.  Conv families only (0-4, 9,
 * 10); returns 1 for a valid i, 0 past the end. */
int lama_hip_profile_read_clock(lama_hip_ctx *ctx, int i, uint64_t *launches, double *ms);
/* A launch's place on the device clock (lama_hip_timeline_read). */
typedef struct lama_launch_time {
    int32_t family;   /* kernel family, as lama_hip_profile numbers them */
    int32_t stream;   /* 0 the pass's stream, 1 the SpectralTransform stream, 2 the g2l stream */
    double start_us;  /* first workgroup start, from the first recorded launch's start (-1: none) */
    double end_us;    /* last workgroup end */
} lama_launch_time;
/* Timeline of launches without a tracer (whose interception changes how the
 * three streams overlap): while enabled, every launch's workgroups store
 * kernel-clock stamps (no events, no synchronisation).  enable != 0 starts a
 * new recording, 0 stops.  lama_hip_timeline_read waits for the device and
 * returns up to `max` launches in issue order (the count, or -1 on error). */
int lama_hip_timeline(lama_hip_ctx *ctx, int enable);
int lama_hip_timeline_read(lama_hip_ctx *ctx, lama_launch_time *out, int max);
/* print_op_stats / print_sub_stats / print_stats (cuda.rs:1738-1806): the
 * per-family event timings to stderr as "op" lines (LAMA_PROFILE_OPS), "sub"
 * lines (LAMA_PROFILE_SUB) and a "gpu totals" line (LAMA_PROFILE); the "op"
 * lines when none of the three is set.  LAMA_PROFILE_OPS and LAMA_PROFILE_SUB
 * turn the per-family timing on for every family when the context opens
 * (events in the dispatch packets, no synchronisation).  The engine also
 * honours, in lama_hip_forward: LAMA_DUMP_STEP=<n> (the activation after plan
 * step n to /tmp/gpu_step_<n>.f32, little-endian f32, local planes then
 * global), LAMA_PROFILE (per-step lines and upload / step loop / download
 * times on stderr, cuda.rs:1560-1686) and LAMA_PROFILE_SYNC (each step's line
 * after draining every stream: submit + device time). */
void lama_hip_print_stats(lama_hip_ctx *ctx);
/* Device memory one forward at h x w needs, for the --gpu capacity guard
 * (the role of mem.rs:26-36 estimated_bytes, exact for this engine): the
 * activation arena of that shape, from its layout, and the resident weights
 * (0 before lama_hip_load_weights).  h, w multiples of 8. */
int lama_hip_plan_bytes(lama_hip_ctx *ctx, int h, int w, uint64_t *arena_bytes, uint64_t *weight_bytes,
                        char *err, size_t errlen);
/* Launches per forward at h x w (after a plan exists for that shape). */
int lama_hip_launch_count(lama_hip_ctx *ctx, int h, int w);
/* The kernel symbol of the first launch of family `family` (numbered as in
 * lama_hip_profile) in the plan at h x w, e.g. which F(4,3) block shape the
 * FFC GEMMs take at that plane size.  No reference counterpart: it names the
 * kernel a trace of the pass shows.  0 on success; 1 without that plan or
 * launch, or a name longer than namelen - 1. */
int lama_hip_kernel_name(lama_hip_ctx *ctx, int h, int w, int family, char *name, size_t namelen);

/* Device buffers for callers that keep their data resident (the role of
 * lightgpu's upload/download, cuda.rs:390-444). */
int lama_hip_malloc(lama_hip_ctx *ctx, size_t bytes, void **ptr, char *err, size_t errlen);
int lama_hip_free(lama_hip_ctx *ctx, void *ptr);
int lama_hip_memcpy(lama_hip_ctx *ctx, void *dst, const void *src, size_t bytes, int kind,
                    char *err, size_t errlen); /* kind: 1 HtoD, 2 DtoH, 3 DtoD */
/* Waits for the engine's own stream and for the last pass (forward,
 * inpaint or SpectralTransform) that was enqueued on a caller's stream.  A
 * context keeps one activation arena per shape: passes of one context on
 * different caller streams must be ordered by the caller. */
int lama_hip_synchronize(lama_hip_ctx *ctx, char *err, size_t errlen);

/* Single kernel families on host buffers, for parity tests against the
 * oracle.  These have no counterpart in the reference; each runs one family
 * on freshly uploaded data and returns the result synchronously.
 *  conv2d: k in {1,3,7}; reflect padding k/2; stride 1 or 2 (k = 3 only);
 *          weights [cout][cin][k][k]; optional bias, BN scale/shift, relu.
 *  conv_transpose: k3 s2 p1 op1, weights [cin][cout][3][3] + bias, optional
 *          BN scale/shift, relu; output [cout][2h][2w].
 *  rfft2:  [c][h][w] -> stacked [2c][h][w/2+1] (ortho).
 *  irfft2: stacked [2c][h][w/2+1] -> [c][h][w] (ortho), plus feat if given.
 *  tail:   7x7 reflect-padded conv [cin] -> 3 with bias, then sigmoid. */
int lama_hip_op_conv2d(lama_hip_ctx *ctx, const float *x, int cin, int h, int w, const float *wt,
                       const float *bias, int cout, int k, int stride, const float *scale,
                       const float *shift, int relu, float *out, char *err, size_t errlen);
int lama_hip_op_conv_transpose(lama_hip_ctx *ctx, const float *x, int cin, int h, int w,
                               const float *wt, const float *bias, int cout, const float *scale,
                               const float *shift, int relu, float *out, char *err, size_t errlen);
int lama_hip_op_rfft2(lama_hip_ctx *ctx, const float *x, int c, int h, int w, float *out,
                      char *err, size_t errlen);
int lama_hip_op_irfft2(lama_hip_ctx *ctx, const float *spec, const float *feat, int c, int h, int w,
                       float *out, char *err, size_t errlen);
int lama_hip_op_tail(lama_hip_ctx *ctx, const float *x, int cin, int h, int w, const float *wt,
                     const float *bias, float *out, char *err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif
