// MFMA contraction kernels, f32, dense operands.
#define OHIP_OP Op::F32
#define OHIP_OUT float
#define OHIP_SUFFIX f32
#define OHIP_PART 1
#include "contract.inc"
