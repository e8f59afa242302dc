// The head-size-128 wide and long tiles of attn_fwd.hip (the 32k and 131k global layers) as a build unit of their
// own, compiled under the backend's iterative-ILP machine scheduler (build.py): about 1% faster at 32k, while the
// same option costs 6.6% at head size 512, and the option applies to a whole file.
#define KA_FWD_UNIT 1
#include "attn_fwd.hip"
