// Window geometry of `--tile` and `--sections`: lama-rs/src/main.rs:585-799.
// Integer work only; results must be identical to the reference's, so the
// rules (and their tie-breaks) are kept as they are there.
#include "lama_host.h"

#include <algorithm>
#include <cstdint>
#include <deque>
#include <vector>

namespace {
const int64_t PAD_MOD = 8;        // main.rs:569
const int64_t TILE_MIN = 512;     // main.rs:571
const int64_t SECTION_BLOCK = 256;  // main.rs:574
}  // namespace

// main.rs:722-725: centre a `side` window on `c`, clamped to [0, extent-side].
extern "C" int64_t lama_window_origin(int64_t c, int64_t side, int64_t extent)
{
    int64_t max0 = extent > side ? extent - side : 0;
    int64_t v = c - side / 2;
    return v < 0 ? 0 : (v > max0 ? max0 : v);
}

// main.rs:740-777
extern "C" int lama_tile_rect(const uint8_t *mask, int w, int h, lama_tile *t)
{
    int64_t min_x = w, min_y = h, max_x = 0, max_y = 0;
    for (int64_t y = 0; y < h; ++y)
        for (int64_t x = 0; x < w; ++x)
            if (mask[y * w + x] > 0) {
                min_x = std::min(min_x, x);
                min_y = std::min(min_y, y);
                max_x = std::max(max_x, x);
                max_y = std::max(max_y, y);
            }
    if (min_x > max_x || min_y > max_y) return 1;
    int64_t bbox_w = max_x - min_x + 1, bbox_h = max_y - min_y + 1;
    int64_t want = std::max(TILE_MIN, 2 * std::max(bbox_w, bbox_h));
    int64_t cap = std::min<int64_t>(w, h) / PAD_MOD * PAD_MOD;
    int64_t side = cap >= PAD_MOD ? std::min((want + PAD_MOD - 1) / PAD_MOD * PAD_MOD, cap)
                                  : std::min<int64_t>(w, h);
    side = std::max<int64_t>(side, 1);
    int64_t cx = min_x + bbox_w / 2, cy = min_y + bbox_h / 2;
    t->x0 = lama_window_origin(cx, side, w);
    t->y0 = lama_window_origin(cy, side, h);
    t->side = side;
    t->bbox_w = bbox_w;
    t->bbox_h = bbox_h;
    return 0;
}

// main.rs:664-717: multi-source BFS from the rim (masked pixels touching a
// non-mask pixel or the image edge), 4-neighbourhood, FIFO order.
extern "C" void lama_mask_depth(const uint8_t *mask, int w, int h, uint32_t *depth)
{
    const size_t n = (size_t)w * h;
    std::fill(depth, depth + n, UINT32_MAX);
    std::deque<size_t> q;
    for (int64_t y = 0; y < h; ++y)
        for (int64_t x = 0; x < w; ++x) {
            size_t i = (size_t)(y * w + x);
            if (mask[i] == 0) continue;
            bool rim = x == 0 || y == 0 || x + 1 == w || y + 1 == h || mask[i - 1] == 0 ||
                       mask[i + 1] == 0 || mask[i - w] == 0 || mask[i + w] == 0;
            if (rim) {
                depth[i] = 0;
                q.push_back(i);
            }
        }
    while (!q.empty()) {
        size_t i = q.front();
        q.pop_front();
        uint32_t d = depth[i];
        size_t x = i % (size_t)w, y = i / (size_t)w;
        size_t nb[4];
        int k = 0;
        if (x > 0) nb[k++] = i - 1;
        if (x + 1 < (size_t)w) nb[k++] = i + 1;
        if (y > 0) nb[k++] = i - w;
        if (y + 1 < (size_t)h) nb[k++] = i + w;
        for (int j = 0; j < k; ++j)
            if (mask[nb[j]] > 0 && depth[nb[j]] == UINT32_MAX) {
                depth[nb[j]] = d == UINT32_MAX ? d : d + 1;  // saturating_add
                q.push_back(nb[j]);
            }
    }
}

// main.rs:597-659
extern "C" size_t lama_section_rects(const uint8_t *mask, int w, int h, lama_section *out, size_t cap)
{
    int64_t min_x = w, min_y = h, max_x = 0, max_y = 0;
    size_t count = 0;
    for (int64_t y = 0; y < h; ++y)
        for (int64_t x = 0; x < w; ++x)
            if (mask[y * w + x] > 0) {
                min_x = std::min(min_x, x);
                min_y = std::min(min_y, y);
                max_x = std::max(max_x, x);
                max_y = std::max(max_y, y);
                ++count;
            }
    if (count == 0) return 0;
    std::vector<std::pair<uint32_t, lama_section>> cells;
    if (max_x - min_x + 1 <= SECTION_BLOCK && max_y - min_y + 1 <= SECTION_BLOCK) {
        cells.push_back({0, lama_section{min_x, min_y, max_x + 1, max_y + 1}});
    } else {
        std::vector<uint32_t> depth((size_t)w * h);
        lama_mask_depth(mask, w, h, depth.data());
        int64_t y0 = min_y;
        for (;;) {
            int64_t x0 = min_x;
            for (;;) {
                int64_t x1 = std::min(x0 + SECTION_BLOCK, max_x + 1);
                int64_t y1 = std::min(y0 + SECTION_BLOCK, max_y + 1);
                uint32_t shallowest = UINT32_MAX;
                for (int64_t y = y0; y < y1; ++y)
                    for (int64_t x = x0; x < x1; ++x)
                        if (mask[y * w + x] > 0) shallowest = std::min(shallowest, depth[(size_t)(y * w + x)]);
                if (shallowest != UINT32_MAX) cells.push_back({shallowest, lama_section{x0, y0, x1, y1}});
                if (x1 >= max_x + 1) break;
                x0 += SECTION_BLOCK;
            }
            if (y0 + SECTION_BLOCK >= max_y + 1) break;
            y0 += SECTION_BLOCK;
        }
        // sort by (depth, y0, x0); stable like Rust's sort_by
        std::stable_sort(cells.begin(), cells.end(), [](const auto &a, const auto &b) {
            if (a.first != b.first) return a.first < b.first;
            if (a.second.y0 != b.second.y0) return a.second.y0 < b.second.y0;
            return a.second.x0 < b.second.x0;
        });
    }
    for (size_t i = 0; i < cells.size() && i < cap; ++i) out[i] = cells[i].second;
    return cells.size();
}
