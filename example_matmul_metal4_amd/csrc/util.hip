// Small utility kernels: a 16-bit fill (used instead of hipMemsetAsync so callers may
// capture it in a HIP graph).
#include "device.hpp"

extern "C" __global__ void __launch_bounds__(256) mtk_fill_u16(const mtk_fill_args a) {
  uint16_t *p = (uint16_t *)a.p;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = (uint16_t)a.v;
}
