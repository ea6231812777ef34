// The device array of lama_hip_forward_device_noalloc, in a code object of
// its own (lama_scratch.hsaco, embedded in liblama_hip.so): a forward whose
// activations, partial sums, FFT scratch and launch descriptors live here
// instead of in memory the engine allocates.  The engine loads this code
// object once per device per process, when the first context opens on that
// device, and looks the array up by name (hipModuleGetGlobal, the
// module-loaded form of hipGetSymbolAddress).  That lookup needs an exported
// symbol, so the array has external linkage rather than `static`; no kernel
// refers to it by name -- the kernels receive addresses inside it through
// their descriptors, as they receive the engine's own arena.
#include <hip/hip_runtime.h>

#include "kernels/common.h"

__device__ __align__(256) unsigned char lama_scratch[LAMA_SCRATCH_BYTES];
