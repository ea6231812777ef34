// The single gfx950 code object of the backend: every kernel family is
// compiled into one module that the engine loads with hipModuleLoadData.
#include "kernels/conv.hip"
#include "kernels/wino.hip"
#include "kernels/wino4.hip"
#include "kernels/fft.hip"
#include "kernels/tail.hip"
#include "kernels/eltwise.hip"
#include "kernels/pack.hip"
