// A stand-in HIP runtime for CPU tests of liblama_hip.so's host logic, loaded
// through LAMA_HIP_LIB: one "gfx950" device whose memory is the host heap.
// Kernel launches are counted per kernel name and not run, so every result is
// garbage, but the engine's own work -- opening, packing and uploading the
// weights, planning each shape, issuing its launches and events, and its
// error paths -- runs as on a GPU.  Checks the engine cannot see:
//   * a memcpy, memset or launch argument that points into freed memory, and a
//     double free, count as violations (fakehip_violations);
//   * FAKEHIP_FAIL_MALLOC_ABOVE=<bytes> makes every hipMalloc of at least that
//     size fail with hipErrorOutOfMemory while it is set;
//   * FAKEHIP_CAPTURING=1 makes every stream report an active stream capture.
// Test infrastructure only (tests/test_fake_hip.py); no product code links it.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

namespace {

std::mutex g_mu;
std::map<uintptr_t, size_t> g_live, g_freed;  // device allocations (base -> bytes)
std::map<std::string, long> g_launches;       // kernel name -> launches
long g_violations = 0, g_mallocs = 0, g_frees = 0;

struct Fn {
    std::string name;
};

bool in_range(const std::map<uintptr_t, size_t> &m, const void *p)
{
    const uintptr_t a = (uintptr_t)p;
    auto it = m.upper_bound(a);
    if (it == m.begin()) return false;
    --it;
    return a >= it->first && a < it->first + it->second;
}

// a pointer into freed device memory (and into no live allocation)
void check_ptr(const void *p, const char *what)
{
    if (p && in_range(g_freed, p) && !in_range(g_live, p)) {
        ++g_violations;
        fprintf(stderr, "fakehip: %s uses freed device memory %p\n", what, p);
    }
}

size_t fail_above()
{
    const char *e = getenv("FAKEHIP_FAIL_MALLOC_ABOVE");
    return e ? (size_t)strtoull(e, nullptr, 10) : 0;
}

}  // namespace

extern "C" {

long fakehip_violations() { return g_violations; }
long fakehip_mallocs() { return g_mallocs; }
long g_modules = 0;
long fakehip_modules() { return g_modules; }
long fakehip_frees() { return g_frees; }
long fakehip_live_bytes()
{
    std::lock_guard<std::mutex> lk(g_mu);
    long n = 0;
    for (auto &kv : g_live) n += (long)kv.second;
    return n;
}
long fakehip_launches(const char *name)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (!name) {
        long n = 0;
        for (auto &kv : g_launches) n += kv.second;
        return n;
    }
    auto it = g_launches.find(name);
    return it == g_launches.end() ? 0 : it->second;
}
void fakehip_reset_launches()
{
    std::lock_guard<std::mutex> lk(g_mu);
    g_launches.clear();
}

hipError_t hipInit(unsigned int) { return hipSuccess; }
hipError_t hipGetDeviceCount(int *n)
{
    *n = 1;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipDeviceGetName(char *name, int len, int)
{
    snprintf(name, (size_t)len, "fake MI355X");
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t attr, int)
{
    *v = attr == hipDeviceAttributeMaxSharedMemoryPerBlock ? 160 * 1024
         : attr == hipDeviceAttributeWallClockRate         ? 100000
         : attr == hipDeviceAttributeMultiprocessorCount   ? 256
                                                           : 0;
    return hipSuccess;
}
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_t *p, int)
{
    memset(p, 0, sizeof *p);
    snprintf(p->name, sizeof p->name, "fake MI355X");
    snprintf(p->gcnArchName, sizeof p->gcnArchName, "gfx950:sramecc+:xnack-");
    p->totalGlobalMem = (size_t)288 << 30;
    p->multiProcessorCount = 256;
    p->sharedMemPerBlock = 160 * 1024;
    return hipSuccess;
}
hipError_t hipMemGetInfo(size_t *f, size_t *t)
{
    *t = (size_t)288 << 30;
    *f = *t - (size_t)fakehip_live_bytes();
    return hipSuccess;
}
hipError_t hipModuleLoadData(hipModule_t *m, const void *image)
{
    ++g_modules;
    *m = (hipModule_t)image;  // any non-null handle
    return image ? hipSuccess : hipErrorInvalidImage;
}
hipError_t hipModuleUnload(hipModule_t) { return hipSuccess; }
hipError_t hipModuleGetFunction(hipFunction_t *f, hipModule_t, const char *name)
{
    *f = (hipFunction_t) new Fn{name};
    return hipSuccess;
}
hipError_t hipModuleGetGlobal(hipDeviceptr_t *p, size_t *bytes, hipModule_t, const char *name)
{
    if (strcmp(name, "lama_scratch") != 0) return hipErrorNotFound;
    static void *scratch = nullptr;
    const size_t n = (size_t)192 << 20;
    if (!scratch) scratch = calloc(1, n);
    std::lock_guard<std::mutex> lk(g_mu);
    g_live[(uintptr_t)scratch] = n;
    *p = scratch;
    *bytes = n;
    return hipSuccess;
}
// FAKEHIP_TRACE=<file>: one line per launch, "<kernel> <grid x>", appended
static void trace(hipFunction_t f, unsigned gx)
{
    static const char *path = getenv("FAKEHIP_TRACE");
    if (!path) return;
    if (FILE *fp = fopen(path, "a")) {
        fprintf(fp, "%s %u\n", ((Fn *)f)->name.c_str(), gx);
        fclose(fp);
    }
}
static void launched(hipFunction_t f, void **params)
{
    std::lock_guard<std::mutex> lk(g_mu);
    ++g_launches[((Fn *)f)->name];
    // every kernel of the engine takes its descriptor (or problem table)
    // pointer as the first argument
    if (params && params[0]) check_ptr(*(void **)params[0], ((Fn *)f)->name.c_str());
}
hipError_t hipModuleLaunchKernel(hipFunction_t f, unsigned gx, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned,
                                 hipStream_t, void **params, void **)
{
    trace(f, gx);
    launched(f, params);
    return hipSuccess;
}
hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t gx, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, size_t,
                                    hipStream_t, void **params, void **, hipEvent_t, hipEvent_t, uint32_t)
{
    trace(f, gx);
    launched(f, params);
    return hipSuccess;
}
hipError_t hipMalloc(void **p, size_t n)
{
    const size_t lim = fail_above();
    if (lim && n >= lim) return hipErrorOutOfMemory;
    *p = calloc(1, n ? n : 1);
    if (!*p) return hipErrorOutOfMemory;
    std::lock_guard<std::mutex> lk(g_mu);
    ++g_mallocs;
    g_live[(uintptr_t)*p] = n ? n : 1;
    g_freed.erase((uintptr_t)*p);
    return hipSuccess;
}
hipError_t hipFree(void *p)
{
    if (!p) return hipSuccess;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_live.find((uintptr_t)p);
    if (it == g_live.end()) {
        ++g_violations;
        fprintf(stderr, "fakehip: hipFree of %p, not a live allocation\n", p);
        return hipErrorInvalidValue;
    }
    g_freed[it->first] = it->second;
    g_live.erase(it);
    ++g_frees;
    free(p);
    return hipSuccess;
}
// Only the device side(s) of a copy are checked: the fake device memory is
// host heap, so a host buffer may later occupy the range of a freed device
// allocation.
static hipError_t copy(void *d, const void *s, size_t n, hipMemcpyKind k)
{
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (k != hipMemcpyDeviceToHost) check_ptr(d, "memcpy destination");
        if (k != hipMemcpyHostToDevice) check_ptr(s, "memcpy source");
    }
    memmove(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind k) { return copy(d, s, n, k); }
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind k, hipStream_t) { return copy(d, s, n, k); }
hipError_t hipMemset(void *d, int v, size_t n)
{
    {
        std::lock_guard<std::mutex> lk(g_mu);
        check_ptr(d, "memset");
    }
    memset(d, v, n);
    return hipSuccess;
}
hipError_t hipStreamCreate(hipStream_t *s)
{
    *s = (hipStream_t) new int(0);
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s)
{
    delete (int *)s;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t *e)
{
    *e = (hipEvent_t) new int(0);
    return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) { return hipEventCreate(e); }
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
hipError_t hipEventDestroy(hipEvent_t e)
{
    delete (int *)e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t)
{
    *ms = 0.001f;
    return hipSuccess;
}
const char *hipGetErrorName(hipError_t e)
{
    return e == hipErrorOutOfMemory ? "hipErrorOutOfMemory" : e == hipSuccess ? "hipSuccess" : "hipError";
}
hipError_t hipGetLastError() { return hipSuccess; }
hipError_t hipRuntimeGetVersion(int *v)
{
    *v = 70200000;
    return hipSuccess;
}
hipError_t hipStreamBeginCapture(hipStream_t, hipStreamCaptureMode) { return hipErrorNotSupported; }
// FAKEHIP_CAPTURING=1: every stream reports an active capture
hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus *st)
{
    const char *e = getenv("FAKEHIP_CAPTURING");
    *st = e && atoi(e) == 1 ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t, hipGraph_t *) { return hipErrorNotSupported; }
hipError_t hipGraphInstantiate(hipGraphExec_t *, hipGraph_t, hipGraphNode_t *, char *, size_t)
{
    return hipErrorNotSupported;
}
hipError_t hipGraphLaunch(hipGraphExec_t, hipStream_t) { return hipErrorNotSupported; }
hipError_t hipGraphExecDestroy(hipGraphExec_t) { return hipErrorNotSupported; }
hipError_t hipGraphDestroy(hipGraph_t) { return hipErrorNotSupported; }

}  // extern "C"
