// kernels_8b.hip -- the persistent kernel specialised for the Llama-3-8B
// shape (hidden 4096, 32 layers, 32/8 heads of 128, SwiGLU 14336, vocabulary
// 128256, untied head): the same device code as the generic kernel, compiled
// with the model's dimensions as constants.
#include <hip/hip_runtime.h>

#define DG_NS dg8b
#define DG_SHAPE_LLAMA3_8B 1
#include "persistent.h"
