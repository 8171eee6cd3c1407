// k_scratch.hip — the fixed device scratch of the no-allocation entry points
// (rt_*_noalloc) and the fill kernel that clears its counters.
//
// Callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops) get the K-split partial sums, the activation records
// and the arrival counters of a launch from this array instead of the
// context's on-demand workspace.  It lives in the code object: every device
// that loads the module holds its own copy, at its own address, until the
// process ends.  The host takes that address from the loaded module once per
// context (hipModuleGetGlobal) and passes it to kernels as an ordinary
// pointer.  All calls on one device share the array: calls that overlap on
// one device race.
#include "rt_device.h"
#include "rt_shared.h"

extern "C" {
__device__ __align__(256) uint8_t scratch[RT_SCRATCH_BYTES];
}

// out[i] = v for i < n (a kernel, not a memset: safe inside captured graphs)
extern "C" __global__ void __launch_bounds__(256) k_fill_u32(uint32_t* out, uint32_t v, uint32_t n) {
    for (uint32_t i = blockIdx.x * wg_threads() + threadIdx.x; i < n; i += gridDim.x * wg_threads())
        out[i] = v;
}
