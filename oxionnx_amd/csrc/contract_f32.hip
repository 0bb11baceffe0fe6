// MFMA contraction kernels, f32.
#define OHIP_OP Op::F32
#define OHIP_OUT float
#define OHIP_SUFFIX f32
#include "contract.inc"
