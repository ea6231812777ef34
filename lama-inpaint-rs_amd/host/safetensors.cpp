// The weight container reader: WeightStore of lama-rs/src/weights.rs:80-139.
// A `.safetensors` file is a little-endian u64 header length, that many bytes
// of JSON {"name": {"dtype", "shape", "data_offsets": [begin, end]}, ...,
// "__metadata__": {...}}, then the payloads; offsets are relative to the
// payload section and are turned into absolute file offsets here so that a
// verbatim copy of the file addresses each tensor at base + offset.
#include <cstdint>
#include "lama_host.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

struct lama_store {
    const uint8_t *bytes = nullptr;
    size_t len = 0;
    bool mapped = false;
    std::vector<std::string> names;
    std::vector<lama_tensor_info> table;
};

namespace {

void set_err(char *err, size_t len, const std::string &m)
{
    if (err && len) snprintf(err, len, "%s", m.c_str());
}

// Minimal JSON walker for the safetensors header: objects, arrays, strings,
// integers; anything else is skipped as a scalar token.
struct Json {
    const char *p, *end;
    std::string error;
    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool expect(char c)
    {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        error = std::string("expected '") + c + "'";
        return false;
    }
    bool string(std::string &out)
    {
        ws();
        if (p >= end || *p != '"') {
            error = "expected string";
            return false;
        }
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            if (*p == '\\' && p + 1 < end) {
                ++p;
                char c = *p;
                out += c == 'n' ? '\n' : c == 't' ? '\t' : c;
            } else {
                out += *p;
            }
            ++p;
        }
        if (p >= end) {
            error = "unterminated string";
            return false;
        }
        ++p;
        return true;
    }
    // A JSON integer, parsed within [p, end): the header is not
    // NUL-terminated, so nothing may read past `end`; values that do not fit
    // in int64 are an error.
    bool integer(int64_t &v)
    {
        ws();
        bool neg = false;
        if (p < end && (*p == '-' || *p == '+')) {
            neg = *p == '-';
            ++p;
        }
        if (p >= end || *p < '0' || *p > '9') {
            error = "expected integer";
            return false;
        }
        uint64_t u = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            const unsigned d = (unsigned)(*p - '0');
            if (u > (UINT64_MAX - d) / 10 || u * 10 + d > (uint64_t)INT64_MAX + (neg ? 1u : 0u)) {
                error = "integer out of range";
                return false;
            }
            u = u * 10 + d;
            ++p;
        }
        v = neg ? (int64_t)(0 - u) : (int64_t)u;
        return true;
    }
    bool skip()  // skip any value
    {
        ws();
        if (p >= end) return false;
        if (*p == '"') {
            std::string s;
            return string(s);
        }
        if (*p == '{' || *p == '[') {
            char open = *p, close = open == '{' ? '}' : ']';
            ++p;
            ws();
            if (p < end && *p == close) {
                ++p;
                return true;
            }
            for (;;) {
                if (open == '{') {
                    std::string k;
                    if (!string(k) || !expect(':')) return false;
                }
                if (!skip()) return false;
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                return expect(close);
            }
        }
        while (p < end && *p != ',' && *p != '}' && *p != ']') ++p;
        return true;
    }
    bool int_array(std::vector<int64_t> &out)
    {
        out.clear();
        if (!expect('[')) return false;
        ws();
        if (p < end && *p == ']') {
            ++p;
            return true;
        }
        for (;;) {
            int64_t v;
            if (!integer(v)) return false;
            out.push_back(v);
            ws();
            if (p < end && *p == ',') {
                ++p;
                continue;
            }
            return expect(']');
        }
    }
};

}  // namespace

extern "C" int lama_store_open(const char *path, int map, lama_store **out, char *err, size_t errlen)
{
    *out = nullptr;
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_err(err, errlen, std::string(path) + ": " + strerror(errno));
        return 1;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
        close(fd);
        set_err(err, errlen, std::string(path) + ": not a safetensors file (too short)");
        return 1;
    }
    auto *s = new lama_store;
    s->len = (size_t)st.st_size;
    if (map) {
        void *m = mmap(nullptr, s->len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            delete s;
            set_err(err, errlen, std::string(path) + ": mmap failed");
            return 1;
        }
        s->bytes = (const uint8_t *)m;
        s->mapped = true;
    } else {
        uint8_t *buf = (uint8_t *)malloc(s->len);
        size_t got = 0;
        while (buf && got < s->len) {
            ssize_t r = read(fd, buf + got, s->len - got);
            if (r <= 0) break;
            got += (size_t)r;
        }
        if (!buf || got != s->len) {
            free(buf);
            close(fd);
            delete s;
            set_err(err, errlen, std::string(path) + ": read failed");
            return 1;
        }
        s->bytes = buf;
    }
    close(fd);

    uint64_t hl = 0;
    for (int i = 0; i < 8; ++i) hl |= (uint64_t)s->bytes[i] << (8 * i);
    if (hl > s->len - 8) {
        lama_store_close(s);
        set_err(err, errlen, std::string(path) + ": header length exceeds the file");
        return 1;
    }
    uint64_t data0 = 8 + hl;
    Json j{(const char *)s->bytes + 8, (const char *)s->bytes + 8 + hl, {}};
    std::string fail;
    struct Raw {
        std::string name, dtype;
        std::vector<int64_t> shape, offs;
    };
    std::vector<Raw> raws;
    if (!j.expect('{')) fail = j.error;
    j.ws();
    bool empty_obj = j.p < j.end && *j.p == '}';
    if (empty_obj) ++j.p;
    while (fail.empty() && !empty_obj) {
        Raw r;
        if (!j.string(r.name) || !j.expect(':')) {
            fail = j.error;
            break;
        }
        if (r.name == "__metadata__") {
            if (!j.skip()) fail = "bad __metadata__";
        } else {
            if (!j.expect('{')) {
                fail = j.error;
                break;
            }
            for (;;) {
                std::string key;
                if (!j.string(key) || !j.expect(':')) {
                    fail = j.error;
                    break;
                }
                bool ok = key == "dtype"          ? j.string(r.dtype)
                          : key == "shape"        ? j.int_array(r.shape)
                          : key == "data_offsets" ? j.int_array(r.offs)
                                                  : j.skip();
                if (!ok) {
                    fail = j.error.empty() ? "bad field " + key : j.error;
                    break;
                }
                j.ws();
                if (j.p < j.end && *j.p == ',') {
                    ++j.p;
                    continue;
                }
                if (!j.expect('}')) fail = j.error;
                break;
            }
            if (fail.empty()) raws.push_back(r);
        }
        if (!fail.empty()) break;
        j.ws();
        if (j.p < j.end && *j.p == ',') {
            ++j.p;
            continue;
        }
        if (!j.expect('}')) fail = j.error;
        break;
    }
    if (!fail.empty()) {
        lama_store_close(s);
        set_err(err, errlen, std::string(path) + ": bad safetensors header: " + fail);
        return 1;
    }
    // container order = payload order (the state_dict order the writer used)
    std::vector<size_t> idx(raws.size());
    for (size_t i = 0; i < idx.size(); ++i) idx[i] = i;
    std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) {
        return raws[a].offs.size() == 2 && raws[b].offs.size() == 2 && raws[a].offs[0] < raws[b].offs[0];
    });
    for (size_t k : idx) {
        Raw &r = raws[k];
        // weights.rs:102-110: every tensor must be F32
        if (r.dtype != "F32") {
            lama_store_close(s);
            set_err(err, errlen, "tensor " + r.name + " is " + r.dtype + ", not F32 - is this a big-lama checkpoint?");
            return 1;
        }
        if (r.offs.size() != 2 || r.offs[0] < 0 || r.offs[1] < r.offs[0] || r.shape.size() > 4 ||
            data0 + (uint64_t)r.offs[1] > s->len) {
            lama_store_close(s);
            set_err(err, errlen, "tensor " + r.name + ": data_offsets outside the file");
            return 1;
        }
        // dimensions are non-negative and their product (in bytes) fits the payload
        uint64_t n = 1;
        bool shape_ok = true;
        for (auto d : r.shape) {
            if (d < 0 || (d > 0 && n > (UINT64_MAX / 4) / (uint64_t)d)) {
                shape_ok = false;
                break;
            }
            n *= (uint64_t)d;
        }
        if (!shape_ok) {
            lama_store_close(s);
            set_err(err, errlen, "tensor " + r.name + ": invalid shape");
            return 1;
        }
        if (n * 4 != (uint64_t)(r.offs[1] - r.offs[0])) {
            lama_store_close(s);
            set_err(err, errlen, "tensor " + r.name + ": size does not match its shape");
            return 1;
        }
        s->names.push_back(r.name);
        lama_tensor_info ti{};
        ti.ndim = (int32_t)r.shape.size();
        for (size_t d = 0; d < r.shape.size(); ++d) ti.shape[d] = r.shape[d];
        ti.offset = data0 + (uint64_t)r.offs[0];
        ti.nbytes = (uint64_t)(r.offs[1] - r.offs[0]);
        s->table.push_back(ti);
    }
    for (size_t i = 0; i < s->table.size(); ++i) s->table[i].name = s->names[i].c_str();
    if (s->table.empty()) {
        lama_store_close(s);
        set_err(err, errlen, std::string("no tensors found in ") + path);
        return 1;
    }
    *out = s;
    return 0;
}

extern "C" void lama_store_close(lama_store *s)
{
    if (!s) return;
    if (s->mapped)
        munmap((void *)s->bytes, s->len);
    else
        free((void *)s->bytes);
    delete s;
}

extern "C" const void *lama_store_bytes(const lama_store *s, size_t *len)
{
    if (len) *len = s->len;
    return s->bytes;
}

extern "C" size_t lama_store_count(const lama_store *s) { return s->table.size(); }

extern "C" const lama_tensor_info *lama_store_table(const lama_store *s) { return s->table.data(); }

extern "C" uint64_t lama_store_total_bytes(const lama_store *s)
{
    uint64_t t = 0;
    for (auto &ti : s->table) t += ti.nbytes;
    return t;
}
