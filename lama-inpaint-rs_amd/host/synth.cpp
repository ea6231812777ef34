// Deterministic synthetic fixtures: the Big-LaMa weight container, blurred
// noise images and hole masks.  Self-contained PRNG (SplitMix64 seeding a
// xoshiro256**) and Box-Muller in f64, so the bits depend on nothing but the
// seed.  The container layout follows the reference's writer
// (lama-rs/safetensors_light.py:21-65): little-endian u64 header length, JSON
// header padded with spaces to an 8-byte boundary, payloads each aligned to 8
// bytes, offsets relative to the payload section.  Tensor names, shapes and
// order are the generator's state_dict (lama-rs/export_weights.py:37-43 writes
// every tensor as F32, including num_batches_tracked).
#include "lama_host.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

struct Rng {
    uint64_t s[4];
    explicit Rng(uint64_t seed)
    {
        uint64_t x = seed;
        for (auto &v : s) {
            x += 0x9E3779B97F4A7C15ull;
            uint64_t z = x;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            v = z ^ (z >> 31);
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next()
    {
        uint64_t r = rotl(s[1] * 5, 7) * 9;
        uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    // uniform in [0, 1) with 53 random bits
    double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    double uniform(double a, double b) { return a + (b - a) * uniform(); }
    // Box-Muller, one value per call (the pair's sine half is discarded so the
    // stream position never depends on call history)
    double normal()
    {
        double u1 = uniform();
        double u2 = uniform();
        if (u1 < 1e-300) u1 = 1e-300;
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2);
    }
    uint64_t below(uint64_t n) { return n ? next() % n : 0; }
};

struct Tensor {
    std::string name;
    std::vector<int64_t> shape;
    std::vector<float> data;
};

int64_t numel(const std::vector<int64_t> &s)
{
    int64_t n = 1;
    for (auto d : s) n *= d;
    return n;
}

void he_normal(Rng &r, Tensor &t)
{
    // PyTorch fan_in convention: dim1 * receptive field (for a transposed conv
    // weight [cin][cout][kh][kw] that is cout*kh*kw).
    int64_t fan_in = t.shape[1];
    for (size_t i = 2; i < t.shape.size(); ++i) fan_in *= t.shape[i];
    double std = std::sqrt(2.0 / (double)fan_in);
    for (auto &v : t.data) v = (float)(r.normal() * std);
}

struct Builder {
    Rng rng;
    std::vector<Tensor> out;
    explicit Builder(uint64_t seed) : rng(seed) {}

    void conv(const std::string &name, std::vector<int64_t> shape)
    {
        Tensor t{name, shape, std::vector<float>((size_t)numel(shape))};
        he_normal(rng, t);
        out.push_back(std::move(t));
    }
    void bias(const std::string &name, int64_t n)
    {
        Tensor t{name, {n}, std::vector<float>((size_t)n)};
        for (auto &v : t.data) v = (float)(rng.normal() * 0.05);
        out.push_back(std::move(t));
    }
    void bn(const std::string &p, int64_t n)
    {
        Tensor w{p + ".weight", {n}, std::vector<float>((size_t)n)};
        for (auto &v : w.data) v = (float)rng.uniform(0.8, 1.2);
        Tensor b{p + ".bias", {n}, std::vector<float>((size_t)n)};
        for (auto &v : b.data) v = (float)(rng.normal() * 0.05);
        Tensor m{p + ".running_mean", {n}, std::vector<float>((size_t)n)};
        for (auto &v : m.data) v = (float)(rng.normal() * 0.1);
        Tensor var{p + ".running_var", {n}, std::vector<float>((size_t)n)};
        for (auto &v : var.data) v = (float)rng.uniform(0.5, 1.5);
        Tensor nbt{p + ".num_batches_tracked", {}, std::vector<float>(1, 0.0f)};
        out.push_back(std::move(w));
        out.push_back(std::move(b));
        out.push_back(std::move(m));
        out.push_back(std::move(var));
        out.push_back(std::move(nbt));
    }
    // One FFC_BN_ACT: `ffc` is the ".ffc" prefix, `part` the BN prefix.
    void ffc(const std::string &ffc, const std::string &part, int64_t in_l, int64_t in_g,
             int64_t out_l, int64_t out_g, int64_t k)
    {
        if (in_l && out_l) conv(ffc + ".convl2l.weight", {out_l, in_l, k, k});
        if (in_l && out_g) conv(ffc + ".convl2g.weight", {out_g, in_l, k, k});
        if (in_g && out_l) conv(ffc + ".convg2l.weight", {out_l, in_g, k, k});
        if (in_g && out_g) {
            int64_t half = out_g / 2;
            conv(ffc + ".convg2g.conv1.0.weight", {half, in_g, 1, 1});
            bn(ffc + ".convg2g.conv1.1", half);
            conv(ffc + ".convg2g.fu.conv_layer.weight", {2 * half, 2 * half, 1, 1});
            bn(ffc + ".convg2g.fu.bn", 2 * half);
            conv(ffc + ".convg2g.conv2.weight", {out_g, half, 1, 1});
        }
        if (out_l) bn(part + ".bn_l", out_l);
        if (out_g) bn(part + ".bn_g", out_g);
    }
};

std::vector<Tensor> big_lama(uint64_t seed)
{
    Builder b(seed);
    b.ffc("model.1.ffc", "model.1", 4, 0, 64, 0, 7);
    b.ffc("model.2.ffc", "model.2", 64, 0, 128, 0, 3);
    b.ffc("model.3.ffc", "model.3", 128, 0, 256, 0, 3);
    b.ffc("model.4.ffc", "model.4", 256, 0, 128, 384, 3);
    for (int i = 5; i <= 22; ++i)
        for (int c = 1; c <= 2; ++c) {
            std::string p = "model." + std::to_string(i) + ".conv" + std::to_string(c);
            b.ffc(p + ".ffc", p, 128, 384, 128, 384, 3);
        }
    const int up[3] = {24, 27, 30};
    const int64_t cin[3] = {512, 256, 128}, cout[3] = {256, 128, 64};
    for (int u = 0; u < 3; ++u) {
        std::string p = "model." + std::to_string(up[u]);
        b.conv(p + ".weight", {cin[u], cout[u], 3, 3});
        b.bias(p + ".bias", cout[u]);
        b.bn("model." + std::to_string(up[u] + 1), cout[u]);
    }
    b.conv("model.34.weight", {3, 64, 7, 7});
    b.bias("model.34.bias", 3);
    return std::move(b.out);
}

void set_err(char *err, size_t len, const std::string &m)
{
    if (err && len) snprintf(err, len, "%s", m.c_str());
}

}  // namespace

extern "C" int lama_synth_weights(const char *path, uint64_t seed, char *err, size_t errlen)
{
    std::vector<Tensor> ts = big_lama(seed);
    std::string header = "{";
    uint64_t off = 0;
    std::vector<uint64_t> starts;
    for (size_t i = 0; i < ts.size(); ++i) {
        off = (off + 7) / 8 * 8;
        starts.push_back(off);
        uint64_t nb = ts[i].data.size() * 4;
        header += (i ? "," : "") + std::string("\"") + ts[i].name + "\":{\"dtype\":\"F32\",\"shape\":[";
        for (size_t d = 0; d < ts[i].shape.size(); ++d)
            header += (d ? "," : "") + std::to_string(ts[i].shape[d]);
        header += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + nb) + "]}";
        off += nb;
    }
    header += "}";
    while ((8 + header.size()) % 8) header += ' ';
    FILE *f = fopen(path, "wb");
    if (!f) {
        set_err(err, errlen, std::string(path) + ": cannot create");
        return 1;
    }
    uint64_t hl = header.size();
    uint8_t le[8];
    for (int i = 0; i < 8; ++i) le[i] = (uint8_t)(hl >> (8 * i));
    bool ok = fwrite(le, 1, 8, f) == 8 && fwrite(header.data(), 1, hl, f) == hl;
    uint64_t pos = 0;
    static const uint8_t zeros[8] = {0};
    for (size_t i = 0; ok && i < ts.size(); ++i) {
        if (starts[i] > pos) ok = fwrite(zeros, 1, starts[i] - pos, f) == starts[i] - pos;
        size_t nb = ts[i].data.size() * 4;
        ok = ok && fwrite(ts[i].data.data(), 1, nb, f) == nb;
        pos = starts[i] + nb;
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) {
        set_err(err, errlen, std::string(path) + ": write failed");
        return 1;
    }
    return 0;
}

extern "C" void lama_synth_image(uint8_t *rgb, int h, int w, uint64_t seed)
{
    Rng r(seed);
    std::vector<double> a((size_t)h * w * 3), b((size_t)h * w * 3);
    for (auto &v : a) v = (double)r.below(256);
    const double sigma = 4.0;
    const int rad = 12;
    double k[2 * rad + 1], ks = 0;
    for (int i = -rad; i <= rad; ++i) ks += (k[i + rad] = std::exp(-0.5 * i * i / (sigma * sigma)));
    for (auto &v : k) v /= ks;
    // rows
    for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x)
            for (int c = 0; c < 3; ++c) {
                double s = 0;
                for (int i = -rad; i <= rad; ++i) {
                    size_t sx = lama_reflect_index(x + i, (size_t)w);
                    s += k[i + rad] * a[((size_t)y * w + sx) * 3 + c];
                }
                b[((size_t)y * w + x) * 3 + c] = s;
            }
    // columns
    for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x)
            for (int c = 0; c < 3; ++c) {
                double s = 0;
                for (int i = -rad; i <= rad; ++i) {
                    size_t sy = lama_reflect_index(y + i, (size_t)h);
                    s += k[i + rad] * b[(sy * w + x) * 3 + c];
                }
                double v = std::floor(s + 0.5);
                rgb[((size_t)y * w + x) * 3 + c] = (uint8_t)(v < 0 ? 0 : (v > 255 ? 255 : v));
            }
}

extern "C" void lama_synth_mask_rect(uint8_t *mask, int h, int w, int rect_w, int rect_h,
                                     uint64_t seed, int *x0, int *y0)
{
    Rng r(seed);
    std::memset(mask, 0, (size_t)h * w);
    if (rect_w > w) rect_w = w;
    if (rect_h > h) rect_h = h;
    int x = (int)r.below((uint64_t)(w - rect_w + 1));
    int y = (int)r.below((uint64_t)(h - rect_h + 1));
    for (int yy = y; yy < y + rect_h; ++yy) std::memset(mask + (size_t)yy * w + x, 255, (size_t)rect_w);
    if (x0) *x0 = x;
    if (y0) *y0 = y;
}

extern "C" double lama_synth_mask_strokes(uint8_t *mask, int h, int w, double coverage,
                                          uint64_t seed)
{
    Rng r(seed);
    std::memset(mask, 0, (size_t)h * w);
    struct Stroke {
        double x, y, ang, width;
    };
    int n = 4 + (int)r.below(5);
    std::vector<Stroke> st((size_t)n);
    for (auto &s : st) {
        s.x = r.uniform(0, w);
        s.y = r.uniform(0, h);
        s.ang = r.uniform(0, 2 * M_PI);
        s.width = r.uniform(20, 40);
    }
    size_t holes = 0, total = (size_t)h * w;
    auto dab = [&](double cx, double cy, double rad) {
        int ylo = (int)std::floor(cy - rad), yhi = (int)std::ceil(cy + rad);
        int xlo = (int)std::floor(cx - rad), xhi = (int)std::ceil(cx + rad);
        for (int y = ylo < 0 ? 0 : ylo; y <= yhi && y < h; ++y)
            for (int x = xlo < 0 ? 0 : xlo; x <= xhi && x < w; ++x) {
                double dx = x + 0.5 - cx, dy = y + 0.5 - cy;
                if (dx * dx + dy * dy <= rad * rad) {
                    uint8_t &m = mask[(size_t)y * w + x];
                    if (!m) {
                        m = 255;
                        ++holes;
                    }
                }
            }
    };
    // extend strokes round robin, one segment each, until the coverage target
    for (int seg = 0; seg < 100000 && (double)holes < coverage * (double)total; ++seg) {
        Stroke &s = st[(size_t)seg % st.size()];
        s.ang += r.uniform(-0.8, 0.8);
        double len = r.uniform(20, 60);
        double nx = s.x + std::cos(s.ang) * len, ny = s.y + std::sin(s.ang) * len;
        // reflect the walk back inside the frame
        if (nx < 0 || nx >= w) {
            s.ang = M_PI - s.ang;
            nx = nx < 0 ? -nx : 2.0 * w - nx - 1;
        }
        if (ny < 0 || ny >= h) {
            s.ang = -s.ang;
            ny = ny < 0 ? -ny : 2.0 * h - ny - 1;
        }
        int steps = (int)std::ceil(len / 2.0);
        for (int i = 0; i <= steps; ++i) {
            double t = (double)i / steps;
            dab(s.x + (nx - s.x) * t, s.y + (ny - s.y) * t, s.width / 2);
        }
        s.x = nx;
        s.y = ny;
    }
    return (double)holes / (double)total;
}
