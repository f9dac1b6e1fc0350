// kernels_1b.hip -- the persistent kernel specialised for the Llama-3.2-1B
// shape (hidden 2048, 16 layers, 32/8 heads of 64, SwiGLU 8192, vocabulary
// 128256, tied head): the same device code as the generic kernel, compiled
// with the model's dimensions as constants.
#include <hip/hip_runtime.h>

#define DG_NS dg1b
#define DG_SHAPE_LLAMA32_1B 1
#include "persistent.h"
