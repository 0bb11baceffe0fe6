// MFMA contraction kernels, bf16, implicit im2col.
#define OHIP_OP Op::BF16
#define OHIP_OUT __bf16
#define OHIP_SUFFIX bf16
#define OHIP_PART 2
#include "contract.inc"
