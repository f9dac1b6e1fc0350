// kernels_360m.hip -- the persistent kernel specialised for the
// SmolLM2-360M shape (hidden 960, 32 layers, 15/5 heads of 64, SwiGLU 2560,
// vocabulary 49152, tied head): the same device code as the generic kernel,
// compiled with the model's dimensions as constants.
#include <hip/hip_runtime.h>

#define DG_NS dg360
#define DG_SHAPE_SMOLLM2_360M 1
#include "persistent.h"
