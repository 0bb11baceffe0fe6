// MFMA contraction kernels, i8, implicit im2col.
#define OHIP_OP Op::I8
#define OHIP_OUT void
#define OHIP_SUFFIX i8
#define OHIP_PART 2
#define OHIP_QUANT 1
#include "contract.inc"
