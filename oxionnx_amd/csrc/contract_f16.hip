// MFMA contraction kernels, f16.
#define OHIP_OP Op::F16
#define OHIP_OUT _Float16
#define OHIP_SUFFIX f16
#include "contract.inc"
