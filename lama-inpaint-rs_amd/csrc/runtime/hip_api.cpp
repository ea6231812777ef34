#include "hip_api.h"

#include <dlfcn.h>
#include <link.h>

#include <cstdlib>
#include <cstring>
#include <mutex>

namespace lama {

namespace {

// Path of a libamdhip64 already mapped into this process (another component
// brought its own runtime): two HIP runtimes in one process must not coexist.
int find_loaded(struct dl_phdr_info *info, size_t, void *data)
{
    if (info->dlpi_name && strstr(info->dlpi_name, "libamdhip64.so")) {
        *static_cast<std::string *>(data) = info->dlpi_name;
        return 1;
    }
    return 0;
}

HipApi g_api;
std::string g_err;
bool g_tried = false;
std::mutex g_mu;

bool load(HipApi &h, std::string &err)
{
    std::string loaded;
    dl_iterate_phdr(find_loaded, &loaded);
    const char *env = getenv("LAMA_HIP_LIB");
    std::string tried;
    auto attempt = [&](const std::string &p) {
        if (h.handle || p.empty()) return;
        h.handle = dlopen(p.c_str(), RTLD_NOW | RTLD_GLOBAL);
        if (h.handle)
            h.path = p;
        else
            tried += "\n  " + p + ": " + dlerror();
    };
    if (env && *env) {
        attempt(env);  // an explicit choice is the only candidate
    } else {
        attempt(loaded);
        attempt("libamdhip64.so.7");
        attempt("/opt/rocm/lib/libamdhip64.so.7");
        attempt("libamdhip64.so");
    }
    if (!h.handle) {
        err = "cannot load the HIP runtime (set LAMA_HIP_LIB to libamdhip64.so):" + tried;
        return false;
    }
#define LAMA_HIP_FN(name)                                                              \
    h.name = reinterpret_cast<decltype(h.name)>(dlsym(h.handle, #name));               \
    if (!h.name) {                                                                     \
        err = std::string("HIP runtime ") + h.path + " lacks " #name;                 \
        return false;                                                                  \
    }
#define LAMA_HIP_FN_T(name, type) LAMA_HIP_FN(name)
#include "hip_fns.inc"
#undef LAMA_HIP_FN_T
#undef LAMA_HIP_FN
    return true;
}

}  // namespace

const HipApi *hip_api(std::string &err)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_tried) {
        g_tried = true;
        if (!load(g_api, g_err)) g_api.handle = nullptr;
    }
    if (!g_api.handle) {
        err = g_err;
        return nullptr;
    }
    return &g_api;
}

std::string hip_error(const HipApi &h, hipError_t e, const char *what)
{
    const char *n = h.hipGetErrorName ? h.hipGetErrorName(e) : "?";
    return std::string(what) + ": " + (n ? n : "?") + " (" + std::to_string((int)e) + ")";
}

}  // namespace lama
