// Image side of the host: PNG codec on zlib (lama-rs/src/image.rs:38-155),
// the reflect index (image.rs:159-169), the network input builder
// (main.rs:175-196), the 8-bit composite (main.rs:272-307) and the memory
// estimate (mem.rs:26-36).
#include "lama_host.h"

#include <zlib.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <system_error>
#include <thread>
#include <vector>

namespace {
void set_err(char *err, size_t len, const std::string &m)
{
    if (err && len) snprintf(err, len, "%s", m.c_str());
}

uint32_t be32(const uint8_t *p) { return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | p[3]; }

// One zlib stream (RFC 1950) of `n` bytes, deflated at `level` in bands of
// 1 MiB on up to 16 threads: each band is a raw deflate stream ending on a
// byte boundary (a sync flush; the last band finishes the stream), so the
// bands concatenate into one valid deflate stream, behind the zlib header
// and ahead of the Adler-32 of the whole input (combined from the bands').
// A band whose thread cannot be started is deflated on the calling thread.
bool zlib_bands(const uint8_t *in, size_t n, int level, std::vector<uint8_t> &out)
{
    const size_t BAND = (size_t)1 << 20;
    const size_t nb = std::max<size_t>(1, (n + BAND - 1) / BAND);
    std::vector<std::vector<uint8_t>> z(nb);
    std::vector<uLong> ad(nb);
    std::vector<char> ok(nb, 0);
    auto band = [&](size_t b) {
        const size_t off = b * BAND, len = std::min(BAND, n - std::min(n, off));
        z_stream zs{};
        if (deflateInit2(&zs, level, Z_DEFLATED, -15, 8, Z_DEFAULT_STRATEGY) != Z_OK) return;
        z[b].resize(deflateBound(&zs, len) + 16);  // + a sync flush's empty stored block
        zs.next_in = const_cast<Bytef *>(in + off);
        zs.avail_in = (uInt)len;
        zs.next_out = z[b].data();
        zs.avail_out = (uInt)z[b].size();
        const bool last = b + 1 == nb;
        const int r = deflate(&zs, last ? Z_FINISH : Z_SYNC_FLUSH);
        ok[b] = (last ? r == Z_STREAM_END : r == Z_OK) && zs.avail_in == 0 && zs.avail_out > 0;
        z[b].resize(z[b].size() - zs.avail_out);
        deflateEnd(&zs);
        ad[b] = adler32(1L, in + off, (uInt)len);
    };
    const size_t nt = std::min<size_t>({16, nb, std::max(1u, std::thread::hardware_concurrency())});
    std::vector<std::thread> th;
    auto run = [&](size_t t) {
        for (size_t b = t; b < nb; b += nt) band(b);
    };
    size_t t = 1;
    try {
        for (; t < nt; ++t) th.emplace_back(run, t);
    } catch (const std::system_error &) {
        for (size_t u = t; u < nt; ++u) run(u);  // the shares no thread took
    }
    run(0);
    for (std::thread &x : th) x.join();
    uLong adler = 1L;
    out = {0x78, 0x01};  // deflate, 32 KiB window, no dictionary, check bits
    for (size_t b = 0; b < nb; ++b) {
        if (!ok[b]) return false;
        out.insert(out.end(), z[b].begin(), z[b].end());
        const size_t len = std::min(BAND, n - std::min(n, b * BAND));
        adler = b ? adler32_combine(adler, ad[b], (z_off_t)len) : ad[b];
    }
    for (int k = 3; k >= 0; --k) out.push_back((uint8_t)(adler >> (8 * k)));
    return true;
}

bool slurp(const char *path, std::vector<uint8_t> &out, std::string &err)
{
    FILE *f = strcmp(path, "-") == 0 ? stdin : fopen(path, "rb");
    if (!f) {
        err = std::string(path) + ": " + strerror(errno);
        return false;
    }
    // a regular file in one read; a pipe in 64 KiB pieces
    if (f != stdin && fseek(f, 0, SEEK_END) == 0) {
        const long size = ftell(f);
        if (size > 0 && fseek(f, 0, SEEK_SET) == 0) {
            out.resize((size_t)size);
            out.resize(fread(out.data(), 1, out.size(), f));
        }
    }
    uint8_t buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.insert(out.end(), buf, buf + n);
    if (f != stdin) fclose(f);
    return true;
}

uint8_t paeth(int a, int b, int c)
{
    int p = a + b - c, pa = abs(p - a), pb = abs(p - b), pc = abs(p - c);
    if (pa <= pb && pa <= pc) return (uint8_t)a;
    return (uint8_t)(pb <= pc ? b : c);
}

// Undo the per-scanline filters of one (sub)image: a = the byte bpp to the
// left, b = the byte above, c = above-left (0 outside the image).
bool unfilter(uint8_t *data, size_t rows, size_t stride, size_t bpp, std::vector<uint8_t> &out)
{
    out.resize(rows * stride);
    const std::vector<uint8_t> zero(stride, 0);
    for (size_t y = 0; y < rows; ++y) {
        const uint8_t ft = data[y * (stride + 1)];
        const uint8_t *src = data + y * (stride + 1) + 1;
        uint8_t *dst = out.data() + y * stride;
        const uint8_t *up = y ? dst - stride : zero.data();
        const size_t lead = std::min(bpp, stride);
        switch (ft) {
        case 0: memcpy(dst, src, stride); break;
        case 1:
            memcpy(dst, src, lead);
            for (size_t i = bpp; i < stride; ++i) dst[i] = (uint8_t)(src[i] + dst[i - bpp]);
            break;
        case 2:
            for (size_t i = 0; i < stride; ++i) dst[i] = (uint8_t)(src[i] + up[i]);
            break;
        case 3:
            for (size_t i = 0; i < lead; ++i) dst[i] = (uint8_t)(src[i] + up[i] / 2);
            for (size_t i = bpp; i < stride; ++i) dst[i] = (uint8_t)(src[i] + (dst[i - bpp] + up[i]) / 2);
            break;
        case 4:
            for (size_t i = 0; i < lead; ++i) dst[i] = (uint8_t)(src[i] + paeth(0, up[i], 0));
            for (size_t i = bpp; i < stride; ++i)
                dst[i] = (uint8_t)(src[i] + paeth(dst[i - bpp], up[i], up[i - bpp]));
            break;
        default: return false;
        }
    }
    return true;
}
}  // namespace

extern "C" size_t lama_reflect_index(long i, size_t n)
{
    if (n == 1) return 0;
    long period = 2 * ((long)n - 1);
    long m = i % period;
    if (m < 0) m += period;
    if (m >= (long)n) m = period - m;
    return (size_t)m;
}

extern "C" void lama_build_input(const uint8_t *rgb, const uint8_t *mask, int h, int w, int pad_h,
                                 int pad_w, float *out)
{
    const int oh = h + pad_h, ow = w + pad_w;
    const size_t plane = (size_t)oh * ow;
    for (int y = 0; y < oh; ++y) {
        size_t sy = lama_reflect_index(y, (size_t)h);
        for (int x = 0; x < ow; ++x) {
            size_t sx = lama_reflect_index(x, (size_t)w);
            float m = (float)mask[sy * w + sx] / 255.0f;
            m = m > 0.0f ? 1.0f : 0.0f;
            size_t o = (size_t)y * ow + x;
            for (int c = 0; c < 3; ++c) {
                float v = (float)rgb[(sy * w + sx) * 3 + c] / 255.0f;
                out[c * plane + o] = v * (1.0f - m);
            }
            out[3 * plane + o] = m;
        }
    }
}

extern "C" void lama_composite(const uint8_t *rgb, const uint8_t *mask, int h, int w, int pad_h,
                               int pad_w, const float *net, uint8_t *out)
{
    const int ow = w + pad_w;
    const size_t plane = (size_t)(h + pad_h) * ow;
    for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x) {
            size_t pi = (size_t)y * ow + x, o = ((size_t)y * w + x) * 3;
            if (!(mask[(size_t)y * w + x] > 0)) {
                out[o] = rgb[o];
                out[o + 1] = rgb[o + 1];
                out[o + 2] = rgb[o + 2];
                continue;
            }
            for (int c = 0; c < 3; ++c) {
                float v = net[c * plane + pi];
                v = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
                v = v * 255.0f;
                out[o + c] = (uint8_t)(v + 0.5f);
            }
        }
}

extern "C" uint64_t lama_estimated_bytes(uint64_t px)
{
    // mem.rs:26-36: 1170 B/px + 343 MiB, saturating (GTX 1080 calibration).
    const uint64_t per = 1170, fixed = 343ull << 20;
    uint64_t a = px > UINT64_MAX / per ? UINT64_MAX : px * per;
    return a > UINT64_MAX - fixed ? UINT64_MAX : a + fixed;
}

extern "C" void lama_free(void *p) { free(p); }

extern "C" int lama_png_read_rgb(const char *path, uint8_t **rgb, int *w_out, int *h_out, char *err,
                                 size_t errlen)
{
    std::vector<uint8_t> f;
    std::string e;
    if (!slurp(path, f, e)) {
        set_err(err, errlen, e);
        return 1;
    }
    const std::string src = strcmp(path, "-") == 0 ? "stdin" : path;
    static const uint8_t sig[8] = {0x89, 'P', 'N', 'G', '\r', '\n', 0x1a, '\n'};
    if (f.size() < 8 || memcmp(f.data(), sig, 8) != 0) {
        set_err(err, errlen, src + ": not a PNG file");
        return 1;
    }
    uint32_t width = 0, height = 0;
    int depth = 0, color = -1, interlace = 0;
    std::vector<uint8_t> idat, palette;
    for (size_t p = 8; p + 12 <= f.size();) {
        uint32_t len = be32(&f[p]);
        if (p + 12 + (size_t)len > f.size()) break;
        const uint8_t *type = &f[p + 4], *d = &f[p + 8];
        if (!memcmp(type, "IHDR", 4) && len >= 13) {
            width = be32(d);
            height = be32(d + 4);
            depth = d[8];
            color = d[9];
            interlace = d[12];
        } else if (!memcmp(type, "PLTE", 4)) {
            palette.assign(d, d + len);
        } else if (!memcmp(type, "IDAT", 4)) {
            idat.insert(idat.end(), d, d + len);
        } else if (!memcmp(type, "IEND", 4)) {
            break;
        }
        p += 12 + (size_t)len;
    }
    int channels = color == 0 ? 1 : color == 2 ? 3 : color == 3 ? 1 : color == 4 ? 2 : color == 6 ? 4 : 0;
    if (!width || !height || !channels) {
        set_err(err, errlen, src + ": unsupported or missing PNG header");
        return 1;
    }
    // image.rs:52-56: only 8- and 16-bit samples are accepted
    if (depth != 8 && depth != 16) {
        set_err(err, errlen, "unsupported PNG bit depth " + std::to_string(depth));
        return 1;
    }
    const size_t sbytes = depth / 8, bpp = channels * sbytes;
    // inflate, into a buffer of the expected size (grown if the data runs on)
    std::vector<uint8_t> raw(((size_t)width * bpp + 1) * height + (interlace ? height + 64 : 0));
    z_stream zs;
    memset(&zs, 0, sizeof zs);
    if (inflateInit(&zs) != Z_OK) {
        set_err(err, errlen, src + ": zlib init failed");
        return 1;
    }
    zs.next_in = idat.data();
    zs.avail_in = (uInt)idat.size();
    size_t got = 0;
    int zr;
    do {
        if (got == raw.size()) raw.resize(raw.size() + (1 << 16));
        zs.next_out = raw.data() + got;
        zs.avail_out = (uInt)std::min<size_t>(raw.size() - got, 1u << 30);
        const uInt before = zs.avail_out;
        zr = inflate(&zs, Z_NO_FLUSH);
        got += before - zs.avail_out;
    } while (zr == Z_OK);
    inflateEnd(&zs);
    raw.resize(got);
    if (zr != Z_STREAM_END) {
        set_err(err, errlen, src + ": corrupt image data");
        return 1;
    }
    // Full-resolution samples, row-major, `bpp` bytes per pixel.
    std::vector<uint8_t> pix((size_t)width * height * bpp);
    if (!interlace) {
        size_t stride = (size_t)width * bpp;
        if (raw.size() < (stride + 1) * height) {
            set_err(err, errlen, src + ": truncated image data");
            return 1;
        }
        std::vector<uint8_t> out;
        if (!unfilter(raw.data(), height, stride, bpp, out)) {
            set_err(err, errlen, src + ": bad filter type");
            return 1;
        }
        pix.swap(out);
    } else {  // Adam7
        static const int xs[7] = {0, 4, 0, 2, 0, 1, 0}, ys[7] = {0, 0, 4, 0, 2, 0, 1};
        static const int dx[7] = {8, 8, 4, 4, 2, 2, 1}, dy[7] = {8, 8, 8, 4, 4, 2, 2};
        size_t off = 0;
        for (int pass = 0; pass < 7; ++pass) {
            size_t pw = width > (uint32_t)xs[pass] ? (width - xs[pass] + dx[pass] - 1) / dx[pass] : 0;
            size_t ph = height > (uint32_t)ys[pass] ? (height - ys[pass] + dy[pass] - 1) / dy[pass] : 0;
            if (!pw || !ph) continue;
            size_t stride = pw * bpp;
            if (raw.size() < off + (stride + 1) * ph) {
                set_err(err, errlen, src + ": truncated image data");
                return 1;
            }
            std::vector<uint8_t> out;
            if (!unfilter(raw.data() + off, ph, stride, bpp, out)) {
                set_err(err, errlen, src + ": bad filter type");
                return 1;
            }
            for (size_t y = 0; y < ph; ++y)
                for (size_t x = 0; x < pw; ++x)
                    memcpy(&pix[((ys[pass] + y * dy[pass]) * width + xs[pass] + x * dx[pass]) * bpp],
                           &out[y * stride + x * bpp], bpp);
            off += (stride + 1) * ph;
        }
    }
    uint8_t *img = (uint8_t *)malloc((size_t)width * height * 3);
    if (!img) {
        set_err(err, errlen, src + ": out of memory");
        return 1;
    }
    if (color == 2 && depth == 8) {  // RGB8: the samples are the image
        memcpy(img, pix.data(), (size_t)width * height * 3);
        *rgb = img;
        *w_out = (int)width;
        *h_out = (int)height;
        return 0;
    }
    const size_t entries = palette.size() / 3;
    for (size_t i = 0; i < (size_t)width * height; ++i) {
        // image.rs:64-74: the high byte of 16-bit samples
        auto s = [&](int c) { return pix[(i * channels + c) * sbytes]; };
        uint8_t r, g, b;
        switch (color) {
        case 2:
        case 6: r = s(0), g = s(1), b = s(2); break;
        case 0:
        case 4: r = g = b = s(0); break;
        default: {  // indexed: clamp to the last entry (image.rs:103-111)
            size_t k = s(0);
            if (entries) k = k < entries - 1 ? k : entries - 1;
            size_t o = k * 3;
            if (o + 2 < palette.size()) {
                r = palette[o], g = palette[o + 1], b = palette[o + 2];
            } else {
                r = g = b = 0;
            }
        }
        }
        img[i * 3] = r;
        img[i * 3 + 1] = g;
        img[i * 3 + 2] = b;
    }
    *rgb = img;
    *w_out = (int)width;
    *h_out = (int)height;
    return 0;
}

extern "C" int lama_png_read_gray(const char *path, uint8_t **gray, int *w, int *h, char *err,
                                  size_t errlen)
{
    uint8_t *rgb = nullptr;
    if (lama_png_read_rgb(path, &rgb, w, h, err, errlen)) return 1;
    size_t n = (size_t)(*w) * (*h);
    uint8_t *g = (uint8_t *)malloc(n ? n : 1);
    for (size_t i = 0; i < n; ++i) g[i] = rgb[i * 3];  // red channel
    free(rgb);
    *gray = g;
    return 0;
}

// Every scanline with the Up filter (the byte above subtracted; row 0 keeps
// its bytes), deflated at zlib level 1 in parallel bands (zlib_bands).  On a
// 2048 x 2048 photograph-like image the filter and level alone are 2.3x
// faster than unfiltered rows at level 6, and the file 40% smaller.
extern "C" int lama_png_write_rgb(const char *path, const uint8_t *rgb, int w, int h, char *err,
                                  size_t errlen)
{
    const size_t stride = (size_t)w * 3;
    std::vector<uint8_t> raw((stride + 1) * h);
    for (int y = 0; y < h; ++y) {
        uint8_t *r = &raw[y * (stride + 1)];
        const uint8_t *cur = rgb + y * stride;
        r[0] = 2;
        if (y == 0) {
            memcpy(r + 1, cur, stride);
        } else {
            const uint8_t *up = cur - stride;
            for (size_t i = 0; i < stride; ++i) r[1 + i] = (uint8_t)(cur[i] - up[i]);
        }
    }
    std::vector<uint8_t> z;
    if (!zlib_bands(raw.data(), raw.size(), 1, z)) {
        set_err(err, errlen, std::string(path) + ": compression failed");
        return 1;
    }
    std::vector<uint8_t> png = {0x89, 'P', 'N', 'G', '\r', '\n', 0x1a, '\n'};
    auto chunk = [&](const char *type, const uint8_t *d, size_t n) {
        uint8_t l[4] = {(uint8_t)(n >> 24), (uint8_t)(n >> 16), (uint8_t)(n >> 8), (uint8_t)n};
        png.insert(png.end(), l, l + 4);
        size_t start = png.size();
        png.insert(png.end(), type, type + 4);
        if (n) png.insert(png.end(), d, d + n);
        uLong crc = crc32(0L, &png[start], (uInt)(n + 4));
        uint8_t c[4] = {(uint8_t)(crc >> 24), (uint8_t)(crc >> 16), (uint8_t)(crc >> 8), (uint8_t)crc};
        png.insert(png.end(), c, c + 4);
    };
    uint8_t ihdr[13] = {(uint8_t)(w >> 24), (uint8_t)(w >> 16), (uint8_t)(w >> 8), (uint8_t)w,
                        (uint8_t)(h >> 24), (uint8_t)(h >> 16), (uint8_t)(h >> 8), (uint8_t)h,
                        8, 2, 0, 0, 0};
    chunk("IHDR", ihdr, 13);
    chunk("IDAT", z.data(), z.size());
    chunk("IEND", nullptr, 0);
    bool to_stdout = strcmp(path, "-") == 0;
    FILE *f = to_stdout ? stdout : fopen(path, "wb");
    if (!f) {
        set_err(err, errlen, std::string(path) + ": " + strerror(errno));
        return 1;
    }
    bool ok = fwrite(png.data(), 1, png.size(), f) == png.size();
    ok = (to_stdout ? fflush(f) == 0 : fclose(f) == 0) && ok;
    if (!ok) {
        set_err(err, errlen, std::string(to_stdout ? "stdout" : path) + ": write failed");
        return 1;
    }
    return 0;
}
