#include <hip/hip_runtime.h>
__global__ void k(unsigned* o){ o[threadIdx.x] = __builtin_amdgcn_ubfe(o[threadIdx.x],0u,3u); }
