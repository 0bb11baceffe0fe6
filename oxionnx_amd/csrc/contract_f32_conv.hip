// MFMA contraction kernels, f32, implicit im2col.
#define OHIP_OP Op::F32
#define OHIP_OUT float
#define OHIP_SUFFIX f32
#define OHIP_PART 2
#include "contract.inc"
