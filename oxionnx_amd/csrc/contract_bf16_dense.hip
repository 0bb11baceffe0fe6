// MFMA contraction kernels, bf16, dense operands.
#define OHIP_OP Op::BF16
#define OHIP_OUT __bf16
#define OHIP_SUFFIX bf16
#define OHIP_PART 1
#include "contract.inc"
