// kernels_135m.hip -- the persistent kernel specialised for the
// SmolLM2-135M shape (hidden 576, 30 layers, 9/3 heads of 64, SwiGLU 1536,
// vocabulary 49152, tied head): the same device code as the generic kernel,
// compiled with the model's dimensions as constants.
#include <hip/hip_runtime.h>

#define DG_NS dg135
#define DG_SHAPE_SMOLLM2_135M 1
#include "persistent.h"
