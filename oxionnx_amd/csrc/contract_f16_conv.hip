// MFMA contraction kernels, f16, implicit im2col.
#define OHIP_OP Op::F16
#define OHIP_OUT _Float16
#define OHIP_SUFFIX f16
#define OHIP_PART 2
#include "contract.inc"
