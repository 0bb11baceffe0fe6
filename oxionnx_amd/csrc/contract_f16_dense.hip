// MFMA contraction kernels, f16, dense operands.
#define OHIP_OP Op::F16
#define OHIP_OUT _Float16
#define OHIP_SUFFIX f16
#define OHIP_PART 1
#include "contract.inc"
