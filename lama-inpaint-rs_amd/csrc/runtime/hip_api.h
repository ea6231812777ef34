// The HIP runtime, reached only through dlopen (the way the reference reaches
// libcuda.so.1 through lightgpu::ffi).  The HIP headers are used for types
// alone; nothing links against libamdhip64.
#pragma once
#include <hip/hip_runtime_api.h>

// AMD extension launch (hip_ext.h, which needs the device-side headers): the
// start/stop events are recorded by the dispatch packet itself.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams, void **extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent, uint32_t flags);

#include <string>

namespace lama {

// hipMalloc is overloaded in C++; the C entry point's type:
using HipMallocFn = hipError_t (*)(void **, size_t);

struct HipApi {
    void *handle = nullptr;
    std::string path;
#define LAMA_HIP_FN(name) decltype(&::name) name = nullptr;
#define LAMA_HIP_FN_T(name, type) type name = nullptr;
#include "hip_fns.inc"
#undef LAMA_HIP_FN_T
#undef LAMA_HIP_FN
};

// Loads (once per process) the runtime named by LAMA_HIP_LIB, else the copy
// already mapped into the process, else libamdhip64.so.7 / libamdhip64.so.
// Returns nullptr with a message on failure.
const HipApi *hip_api(std::string &err);

// "<what>: <hipGetErrorName> (<code>)", the shape of cuda.rs:294-296.
std::string hip_error(const HipApi &h, hipError_t e, const char *what);

}  // namespace lama
