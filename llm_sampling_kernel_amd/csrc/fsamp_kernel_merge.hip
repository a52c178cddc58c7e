// fsamp_kernel_merge.hip -- the MERGE instantiations of the sampler kernel (the workgroup
// hand-off and merge for split rows with k > 128), compiled apart from the common ones so
// that the two build in parallel.  The kernel table lives in fsamp_kernel.hip.
#define FSAMP_KERNEL_MERGE_TU
#include "fsamp_kernel.hip"
