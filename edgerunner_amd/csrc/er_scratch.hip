// er_scratch.hip -- the device scratch array of the allocation-free entry
// points (er_hip_encode_q6k_weights_packed_top1_noalloc).
//
// Every load of this code object (one per er_hip_ctx, on the context's
// device) holds its own copy, for as long as the code object stays loaded.
// The host library finds its device address once, at context creation, with
// hipModuleGetGlobal (the code object is loaded with hipModuleLoadData, so
// the module's symbol query is the way to it), and passes only that address
// to kernels.  External linkage keeps the symbol in the code object's symbol
// table, where the module query looks it up; nothing outside this code
// object can name it.  (The linkage block makes this a definition; a bare
// `extern "C"` declaration would leave the code object without the array.)
#include "er_scratch.h"

#include <stdint.h>

extern "C" {
__device__ __attribute__((aligned(256))) uint8_t er_scratch[ER_SCRATCH_BYTES];
}
