#include <hip/hip_runtime.h>
__global__ void k(const unsigned* m, const int* t, int* out) {
  int i = threadIdx.x;
  unsigned b = __builtin_amdgcn_ubfe(m[i], 0u, static_cast<unsigned>(t[i]) & 31u);
  const int h = b ? __builtin_clz(b) : -1;
  out[i] = 31 - h;
  int x = t[i + 64];
  out[i + 64] = x < 0 ? 0 : (x > 16 ? 16 : x);
}
