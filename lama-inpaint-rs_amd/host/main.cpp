// lama-inpaint: the command line of the reference (lama-rs/src/main.rs) over
// the MI355X engine.  Same flags, same flows and the same output contract:
//   whole image   main.rs:213-313   pad to a multiple of 8, one forward, composite
//   --tile        main.rs:378-443   one square window around the mask
//   --sections    main.rs:465-566   one 512 window per 256-block section, rim inward
// The network runs through liblama_hip.so (include/lama_hip.h); image I/O,
// input building, compositing and the window geometry come from
// liblama_host.so (include/lama_host.h).  There is no CPU engine in this
// build: --cpu is refused, and a GPU failure is an error rather than a
// fallback (main.rs:330-360 falls back to its CPU engine).
#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <chrono>
#include <string>
#include <system_error>
#include <thread>
#include <vector>

#include <limits.h>
#include <unistd.h>

#include "lama_hip.h"
#include "lama_host.h"

namespace {

constexpr int PAD_MOD = 8;    // main.rs:568
constexpr int TILE_MIN = 512;  // main.rs:570

const char *USAGE =
    "usage: lama-inpaint --image IN.png --mask MASK.png --output OUT.png\n"
    "                    [--weights big-lama.safetensors]\n"
    "                    [--cpu | --gpu]\n"
    "                    [--tile | --sections]\n"
    "\n"
    "Runs the big-lama FFC ResNet generator over IN.png on an MI355X, inpainting the\n"
    "pixels the mask marks (any non-black pixel is a hole), and writes OUT.png at the\n"
    "input size.  Use - for either input (but not both) to read a PNG from stdin, or\n"
    "for the output to write PNG data to stdout.  Diagnostics always go to stderr.\n"
    "This build has no CPU engine: --cpu is refused.\n"
    "Images at or below 512px on the short side are run whole even with --tile.\n"
    "\n"
    "--tile runs the network on a square window around the mask instead of the whole\n"
    "image: the window is twice the mask bounding box, at least 512x512, centred on\n"
    "the mask and clamped inside the image.  Only the masked pixels are taken from\n"
    "the network, so the output is identical to cropping the window out by hand,\n"
    "running this binary on it and pasting the hole back.\n"
    "\n"
    "--sections fills a mask larger than 256x256 in discrete 256x256 sections, one\n"
    "512x512 window per section, from the edge of the hole inward.  Each pass masks\n"
    "only its own section and writes back only its own section.\n"
    "Sections and --tile are mutually exclusive.";

struct Args {
    std::string image, mask, output, weights;
    bool force_cpu = false, force_gpu = false, tile = false, sections = false;
};

struct Rgb {
    int w = 0, h = 0;
    std::vector<uint8_t> d;  // HWC
};
struct Gray {
    int w = 0, h = 0;
    std::vector<uint8_t> d;
};

struct Fail {
    std::string msg;
};

using Clock = std::chrono::steady_clock;
double since(Clock::time_point t) { return std::chrono::duration<double>(Clock::now() - t).count(); }

void log(const std::string &m) { std::fprintf(stderr, "%s\n", m.c_str()); }

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    std::vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

bool exists(const std::string &p) { return access(p.c_str(), F_OK) == 0; }

// main.rs:131-168: beside the executable, then models/, then up the tree,
// then the current directory.
std::string default_weights(const std::string &rel)
{
    char exe[PATH_MAX];
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    if (n > 0) {
        exe[n] = 0;
        std::string dir(exe);
        dir = dir.substr(0, dir.rfind('/'));
        if (exists(dir + "/" + rel)) return dir + "/" + rel;
        if (exists(dir + "/models/" + rel)) return dir + "/models/" + rel;
        std::string base = dir;
        for (int i = 0; i < 6 && !base.empty(); ++i) {
            if (exists(base + "/" + rel)) return base + "/" + rel;
            if (exists(base + "/models/" + rel)) return base + "/models/" + rel;
            const size_t s = base.rfind('/');
            if (s == std::string::npos) break;
            base = base.substr(0, s);
        }
    }
    return rel;
}

// main.rs:60-112
Args parse_args(int argc, char **argv)
{
    Args a;
    bool have_image = false, have_mask = false, have_output = false, have_weights = false;
    for (int i = 1; i < argc; ++i) {
        const std::string s = argv[i];
        auto val = [&](const char *name) -> std::string {
            if (i + 1 >= argc) throw Fail{std::string(name) + " needs a value"};
            return argv[++i];
        };
        if (s == "--image") {
            a.image = val("--image");
            have_image = true;
        } else if (s == "--mask") {
            a.mask = val("--mask");
            have_mask = true;
        } else if (s == "--output") {
            a.output = val("--output");
            have_output = true;
        } else if (s == "--weights") {
            a.weights = val("--weights");
            have_weights = true;
        } else if (s == "--cpu") {
            a.force_cpu = true;
        } else if (s == "--gpu") {
            a.force_gpu = true;
        } else if (s == "--tile") {
            a.tile = true;
        } else if (s == "--sections") {
            a.sections = true;
        } else if (s == "-h" || s == "--help") {
            std::printf("%s\n", USAGE);
            std::exit(0);
        } else {
            throw Fail{"unknown argument " + s};
        }
    }
    if (!have_image) throw Fail{"--image is required"};
    if (!have_mask) throw Fail{"--mask is required"};
    if (!have_output) throw Fail{"--output is required"};
    if (a.image == "-" && a.mask == "-")
        throw Fail{"--image and --mask cannot both be '-' (stdin has only one stream)"};
    if (a.tile && a.sections) throw Fail{"--tile and --sections are mutually exclusive"};
    if (!have_weights) a.weights = default_weights("big-lama.safetensors");
    return a;
}

Rgb read_rgb(const std::string &path)
{
    Rgb r;
    uint8_t *p = nullptr;
    char err[512];
    if (lama_png_read_rgb(path.c_str(), &p, &r.w, &r.h, err, sizeof err)) throw Fail{err};
    r.d.assign(p, p + (size_t)r.w * r.h * 3);
    lama_free(p);
    return r;
}

Gray read_gray(const std::string &path)
{
    Gray g;
    uint8_t *p = nullptr;
    char err[512];
    if (lama_png_read_gray(path.c_str(), &p, &g.w, &g.h, err, sizeof err)) throw Fail{err};
    g.d.assign(p, p + (size_t)g.w * g.h);
    lama_free(p);
    return g;
}

void write_rgb(const std::string &path, const Rgb &img)
{
    char err[512];
    if (lama_png_write_rgb(path.c_str(), img.d.data(), img.w, img.h, err, sizeof err)) throw Fail{err};
}

// mem.rs:74-81
std::string mib(uint64_t bytes)
{
    const uint64_t GIB = 1ull << 30;
    if (bytes >= GIB) return fmt("%.1f GB", (double)bytes / (double)GIB);
    return fmt("%.0f MB", (double)bytes / (double)(1 << 20));
}

// The engine, opened on first use with the weights resident for every pass
// (cuda.rs keeps its state process-wide the same way).
struct Engine {
    lama_hip_ctx *ctx = nullptr;
    lama_store *store = nullptr;
    bool loaded = false;
    char err[4096];

    void open()
    {
        if (!ctx && lama_hip_open(&ctx, err, sizeof err)) throw Fail{err};
    }
    void load()
    {
        open();
        if (loaded) return;
        size_t len = 0;
        const void *blob = lama_store_bytes(store, &len);
        if (lama_hip_load_weights(ctx, blob, len, lama_store_table(store), lama_store_count(store), err, sizeof err))
            throw Fail{err};
        loaded = true;
    }
    ~Engine()
    {
        if (ctx) lama_hip_close(ctx);
    }
};

// mem.rs:38-72 for this engine: the exact bytes of one h x w forward (its
// activation arena plus the resident weights) against 90% of what is free.
void check_capacity(Engine &eng, int h, int w, const char *hint)
{
    uint64_t free_b = 0, total_b = 0;
    char name[256] = "the GPU", err[512];
    if (lama_hip_vram(&free_b, &total_b, name, sizeof name, err, sizeof err)) return;  // nothing can answer
    eng.open();
    uint64_t arena = 0, weights = 0;
    if (lama_hip_plan_bytes(eng.ctx, h, w, &arena, &weights, eng.err, sizeof eng.err)) throw Fail{eng.err};
    if (!eng.loaded) weights = lama_store_total_bytes(eng.store);
    const uint64_t need = arena + weights;
    if (need <= free_b - free_b / 10) return;
    throw Fail{fmt("an inference over %dx%d needs about %s of device memory, but only %s is free of %s on \"%s\".  %s",
                   w, h, mib(need).c_str(), mib(free_b).c_str(), mib(total_b).c_str(), name, hint)};
}

// main.rs:318-361, without a CPU engine to fall back to.  The pass runs as
// lama_hip_inpaint: build_input (main.rs:175-196, with the pad to a multiple
// of 8), the forward and the 8-bit composite (main.rs:272-307) all on the
// device; the result is the h x w composite of this image and mask.
Rgb infer(Engine &eng, const Rgb &img, const Gray &mask, const Args &args)
{
    if (args.force_cpu)
        throw Fail{"--cpu was requested, but this is the MI355X build (no CPU engine is compiled in).\n"
                   "Run without --cpu."};
    try {
        eng.load();
        Rgb out;
        out.w = img.w;
        out.h = img.h;
        out.d.resize((size_t)img.w * img.h * 3);
        if (lama_hip_inpaint(eng.ctx, img.d.data(), mask.d.data(), img.h, img.w, out.d.data(), nullptr, eng.err,
                             sizeof eng.err))
            throw Fail{eng.err};
        if (getenv("LAMA_PROFILE_OPS") || getenv("LAMA_PROFILE_SUB") || getenv("LAMA_PROFILE"))
            lama_hip_print_stats(eng.ctx);
        return out;
    } catch (const Fail &f) {
        if (args.force_gpu) throw Fail{"gpu inference failed: " + f.msg};
        throw Fail{"gpu unavailable (" + f.msg + ") and this build has no CPU engine to fall back to"};
    }
}

// main.rs:779-799
Rgb crop_rgb(const Rgb &img, const lama_tile &t)
{
    Rgb o;
    o.w = o.h = (int)t.side;
    o.d.resize((size_t)t.side * t.side * 3);
    for (int64_t y = 0; y < t.side; ++y)
        std::memcpy(&o.d[(size_t)y * t.side * 3], &img.d[((size_t)(t.y0 + y) * img.w + t.x0) * 3], (size_t)t.side * 3);
    return o;
}

Gray crop_gray(const Gray &img, const lama_tile &t)
{
    Gray o;
    o.w = o.h = (int)t.side;
    o.d.resize((size_t)t.side * t.side);
    for (int64_t y = 0; y < t.side; ++y)
        std::memcpy(&o.d[(size_t)y * t.side], &img.d[(size_t)(t.y0 + y) * img.w + t.x0], (size_t)t.side);
    return o;
}

void run_tiled(Engine &eng, const Rgb &src, const Gray &mask, const Args &args)
{
    const auto t_start = Clock::now();
    lama_tile t;
    if (lama_tile_rect(mask.d.data(), mask.w, mask.h, &t)) {
        log("--tile: mask is empty; copying the input to the output");
        write_rgb(args.output, src);
        return;
    }
    log(fmt("tile: %ldx%ld window at (%ld,%ld) covering a %ldx%ld mask", (long)t.side, (long)t.side, (long)t.x0,
            (long)t.y0, (long)t.bbox_w, (long)t.bbox_h));
    const Rgb sub = crop_rgb(src, t);
    const Gray sub_mask = crop_gray(mask, t);
    const int side = (int)t.side, pad = (PAD_MOD - side % PAD_MOD) % PAD_MOD;
    if (args.force_gpu)
        check_capacity(eng, side + pad, side + pad,
                       "Use --sections, which fills the mask in 512x512 passes, or run without --tile.");
    const auto t0 = Clock::now();
    const Rgb comp = infer(eng, sub, sub_mask, args);
    log(fmt("inference %dx%d in %.2fs", side, side, since(t0)));
    // paste the window's hole pixels (main.rs:422-437)
    Rgb img = src;
    for (int y = 0; y < side; ++y)
        for (int x = 0; x < side; ++x) {
            if (sub_mask.d[(size_t)y * side + x] == 0) continue;
            const size_t o = ((size_t)(t.y0 + y) * src.w + t.x0 + x) * 3, q = ((size_t)y * side + x) * 3;
            for (int c = 0; c < 3; ++c) img.d[o + c] = comp.d[q + c];
        }
    write_rgb(args.output, img);
    log("wrote " + args.output);
    log(fmt("total %.2fs", since(t_start)));
}

void run_sections(Engine &eng, const Rgb &src, const Gray &mask, const Args &args)
{
    const auto t_start = Clock::now();
    const int width = src.w, height = src.h;
    const size_t n = lama_section_rects(mask.d.data(), width, height, nullptr, 0);
    if (n == 0) {
        log("--sections: mask is empty; copying the input to the output");
        write_rgb(args.output, src);
        return;
    }
    std::vector<lama_section> sections(n);
    lama_section_rects(mask.d.data(), width, height, sections.data(), n);
    const int side = std::max(1, std::min(TILE_MIN, std::min(width, height)));
    log(fmt("sections: %zu passes, %dx%d window each, rim inward", n, side, side));
    Rgb working = src;
    for (size_t i = 0; i < n; ++i) {
        const lama_section &s = sections[i];
        const int64_t cx = (s.x0 + s.x1) / 2, cy = (s.y0 + s.y1) / 2;
        lama_tile win;
        win.x0 = lama_window_origin(cx, side, width);
        win.y0 = lama_window_origin(cy, side, height);
        win.side = side;
        win.bbox_w = s.x1 - s.x0;
        win.bbox_h = s.y1 - s.y0;
        const Rgb sub = crop_rgb(working, win);
        // this pass's holes: its own section's pixels only (main.rs:505-520)
        Gray sub_mask = crop_gray(mask, win);
        for (int y = 0; y < side; ++y)
            for (int x = 0; x < side; ++x) {
                const int64_t gx = win.x0 + x, gy = win.y0 + y;
                if (!(gx >= s.x0 && gx < s.x1 && gy >= s.y0 && gy < s.y1)) sub_mask.d[(size_t)y * side + x] = 0;
            }
        const auto t0 = Clock::now();
        const Rgb comp = infer(eng, sub, sub_mask, args);
        log(fmt("  pass %zu/%zu: %dx%d window at (%ld,%ld), %.2fs", i + 1, n, side, side, (long)win.x0, (long)win.y0,
                since(t0)));
        // write back this section's mask pixels only (main.rs:538-552)
        for (int64_t gy = s.y0; gy < s.y1; ++gy)
            for (int64_t gx = s.x0; gx < s.x1; ++gx) {
                if (mask.d[(size_t)gy * width + gx] == 0) continue;
                const size_t q = ((size_t)(gy - win.y0) * side + (gx - win.x0)) * 3;
                const size_t o = ((size_t)gy * width + gx) * 3;
                for (int c = 0; c < 3; ++c) working.d[o + c] = comp.d[q + c];
            }
        if (const char *dir = getenv("LAMA_DUMP_SECTIONS")) {
            char p[4096];
            std::snprintf(p, sizeof p, "%s/pass-%02zu.png", dir, i + 1);
            char err[512];
            lama_png_write_rgb(p, working.d.data(), working.w, working.h, err, sizeof err);
        }
    }
    write_rgb(args.output, working);
    log("wrote " + args.output);
    log(fmt("total %.2fs", since(t_start)));
}

void run(const Args &args)
{
    const auto t_start = Clock::now();
    // the two files decode on two threads (the image's error is reported
    // first, as when they are read in turn)
    Rgb src;
    Gray mask;
    std::string mask_err;
    auto load_mask = [&] {
        try {
            mask = read_gray(args.mask);
        } catch (const Fail &f) {
            mask_err = f.msg;
        } catch (const std::exception &x) {
            mask_err = args.mask + ": " + x.what();
        }
    };
    std::thread tm;
    try {
        tm = std::thread(load_mask);
    } catch (const std::system_error &) {
        load_mask();
    }
    std::string img_err;
    try {
        src = read_rgb(args.image);
    } catch (const Fail &f) {
        img_err = f.msg;
    } catch (const std::exception &x) {
        img_err = args.image + ": " + x.what();
    }
    if (tm.joinable()) tm.join();
    if (!img_err.empty()) throw Fail{img_err};
    if (!mask_err.empty()) throw Fail{mask_err};
    if (mask.w != src.w || mask.h != src.h)
        throw Fail{fmt("mask is %dx%d but image is %dx%d", mask.w, mask.h, src.w, src.h)};
    const int width = src.w, height = src.h;
    log(fmt("loaded %dx%d image + mask in %.2fs", width, height, since(t_start)));

    Engine eng;
    char err[1024];
    if (lama_store_open(args.weights.c_str(), args.force_cpu ? 0 : 1, &eng.store, err, sizeof err)) throw Fail{err};
    struct StoreGuard {
        lama_store *s;
        ~StoreGuard() { lama_store_close(s); }
    } guard{eng.store};
    log(fmt("weights: %zu tensors, %.1f MB", lama_store_count(eng.store),
            (double)lama_store_total_bytes(eng.store) / (1024.0 * 1024.0)));
    log("plan: big-lama FFC ResNet generator, 29 steps (18 resblocks, 36 FFCs) on an MI355X");

    const int pad_h = (PAD_MOD - height % PAD_MOD) % PAD_MOD, pad_w = (PAD_MOD - width % PAD_MOD) % PAD_MOD;
    if (args.sections) {
        if (std::min(width, height) <= TILE_MIN)
            log(fmt("--sections: %dx%d is at or below %dpx on its short side; running the whole image", width, height,
                    TILE_MIN));
        else
            return run_sections(eng, src, mask, args);
    }
    if (args.tile) return run_tiled(eng, src, mask, args);

    if (args.force_gpu)
        check_capacity(eng, height + pad_h, width + pad_w,
                       "Use --tile to run on a window around the mask, or --sections for a large mask.");
    const auto t0 = Clock::now();
    const Rgb img = infer(eng, src, mask, args);
    log(fmt("inference %dx%d in %.2fs", width, height, since(t0)));
    write_rgb(args.output, img);
    log("wrote " + args.output);
    log(fmt("total %.2fs", since(t_start)));
}

}  // namespace

int main(int argc, char **argv)
{
    Args args;
    try {
        args = parse_args(argc, argv);
    } catch (const Fail &f) {
        std::fprintf(stderr, "error: %s\n\n%s\n", f.msg.c_str(), USAGE);
        return 2;
    }
    try {
        run(args);
    } catch (const Fail &f) {
        std::fprintf(stderr, "error: %s\n", f.msg.c_str());
        return 1;
    }
    return 0;
}
