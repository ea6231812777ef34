/*
 * lama_host.h -- C ABI of the host side (liblama_host.so): the parts of the
 * reference's `main.rs`, `image.rs` and `weights.rs` that sit around the
 * forward pass, restated in C++ because no Rust toolchain is available, plus
 * the deterministic synthetic-fixture writer.
 *
 * All functions return 0 on success and nonzero on failure with a UTF-8
 * message in `err` (when `err` is non-NULL), mirroring `Result<_, String>`.
 * Images are HWC u8 RGB, masks HW u8, network tensors planar f32 [c][h][w].
 */
#ifndef LAMA_HOST_H
#define LAMA_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- weights (replaces lama-rs/src/weights.rs:80-139 WeightStore) ---- */

/* One tensor of the container; `offset` is absolute in the file so a copy of
 * the whole file addresses it at base+offset (weights.rs:36-37). */
typedef struct lama_tensor_info {
    const char *name;
    int32_t ndim;
    int64_t shape[4];
    uint64_t offset;
    uint64_t nbytes;
} lama_tensor_info;

typedef struct lama_store lama_store;

/* WeightStore::open (weights.rs:80-106): mmap (map=1) or read the file,
 * parse the header, reject any non-F32 tensor and an empty container. */
int lama_store_open(const char *path, int map, lama_store **out, char *err, size_t errlen);
void lama_store_close(lama_store *s);
/* The whole file (WeightStore::bytes, weights.rs:122-124). */
const void *lama_store_bytes(const lama_store *s, size_t *len);
/* Tensors in container order (WeightIndex.order). */
size_t lama_store_count(const lama_store *s);
const lama_tensor_info *lama_store_table(const lama_store *s);
/* WeightStore::total_bytes (weights.rs:126-133). */
uint64_t lama_store_total_bytes(const lama_store *s);

/* ---- synthetic fixtures (the writer of lama-rs/safetensors_light.py:21-65) ---- */

/* Writes the 989-tensor Big-LaMa F32 safetensors file in state-dict order,
 * 8-byte-aligned payloads, weights drawn from one seeded stream:
 * convs He-normal std sqrt(2/(shape[1]*kh*kw)); BN gamma U(0.8,1.2),
 * beta N(0,0.05), running_mean N(0,0.1), running_var U(0.5,1.5),
 * num_batches_tracked 0; conv-transpose and output biases N(0,0.05). */
int lama_synth_weights(const char *path, uint64_t seed, char *err, size_t errlen);
/* i.i.d. U{0..255} RGB, separable Gaussian blur sigma 4 (radius 12, reflect
 * borders, f64), rounded half up and clamped. */
void lama_synth_image(uint8_t *rgb, int h, int w, uint64_t seed);
/* One axis-aligned rect_w x rect_h hole (255) at a seeded position; writes the
 * chosen corner to x0/y0. */
void lama_synth_mask_rect(uint8_t *mask, int h, int w, int rect_w, int rect_h, uint64_t seed,
                          int *x0, int *y0);
/* 4-8 random-walk brush strokes, 20-40 px wide, extended one segment at a
 * time (round robin) until at least `coverage` of the pixels are holes.
 * Returns the achieved coverage. */
double lama_synth_mask_strokes(uint8_t *mask, int h, int w, double coverage, uint64_t seed);

/* ---- image helpers (main.rs:175-196, 272-307; image.rs:159-169) ---- */

size_t lama_reflect_index(long i, size_t n);
/* main.rs:175-196: [4][h+pad_h][w+pad_w] network input. */
void lama_build_input(const uint8_t *rgb, const uint8_t *mask, int h, int w, int pad_h, int pad_w,
                      float *out);
/* main.rs:272-307: whole-image composite of [3][h+pad_h][w+pad_w] output. */
void lama_composite(const uint8_t *rgb, const uint8_t *mask, int h, int w, int pad_h, int pad_w,
                    const float *net, uint8_t *out);

/* ---- window geometry (main.rs:585-799) ---- */

typedef struct lama_tile {
    int64_t x0, y0, side, bbox_w, bbox_h;
} lama_tile;

typedef struct lama_section {
    int64_t x0, y0, x1, y1;
} lama_section;

/* main.rs:722-725 */
int64_t lama_window_origin(int64_t c, int64_t side, int64_t extent);
/* main.rs:740-777: returns 0 and fills *t, or 1 when the mask is empty. */
int lama_tile_rect(const uint8_t *mask, int w, int h, lama_tile *t);
/* main.rs:664-717: BFS depth; unmasked pixels get UINT32_MAX. */
void lama_mask_depth(const uint8_t *mask, int w, int h, uint32_t *depth);
/* main.rs:597-659: writes up to `cap` sections in pass order, returns the
 * total count (0 for an empty mask). */
size_t lama_section_rects(const uint8_t *mask, int w, int h, lama_section *out, size_t cap);

/* ---- PNG (image.rs:38-155) ---- */

/* Decode any 8/16-bit gray/GA/RGB/RGBA/indexed PNG to RGB8 (16-bit keeps the
 * high byte).  *rgb is malloc'd; free with lama_free.  path "-" = stdin. */
int lama_png_read_rgb(const char *path, uint8_t **rgb, int *w, int *h, char *err, size_t errlen);
/* image.rs:123-130: the red channel. */
int lama_png_read_gray(const char *path, uint8_t **gray, int *w, int *h, char *err, size_t errlen);
/* RGB8 PNG encoder; path "-" = stdout. */
int lama_png_write_rgb(const char *path, const uint8_t *rgb, int w, int h, char *err, size_t errlen);
void lama_free(void *p);

/* ---- memory guard (mem.rs:26-36) ---- */
uint64_t lama_estimated_bytes(uint64_t px);

#ifdef __cplusplus
}
#endif
#endif
