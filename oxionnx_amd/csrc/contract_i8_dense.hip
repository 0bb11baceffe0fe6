// MFMA contraction kernels, i8, dense operands.
#define OHIP_OP Op::I8
#define OHIP_OUT void
#define OHIP_SUFFIX i8
#define OHIP_PART 1
#define OHIP_QUANT 1
#include "contract.inc"
