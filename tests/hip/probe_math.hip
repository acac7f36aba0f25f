// Test hook, not product code: evaluates the MLP kernels' per-sample math helpers (ffn_device.h) elementwise
// so that a GPU test can bound each one's error against float64 references.  Built by the package's build
// step into tests/hip/libffn_probe_math.so; only the tests load it.
#include <hip/hip_runtime.h>
#include "../../ffnerf-experimental_amd/csrc/ffn_device.h"

using namespace ffn;

enum ProbeFn { P_EXP = 0, P_SOFTPLUS = 1, P_SOFTPLUS_PRIME = 2, P_SIGMOID_SOFT = 3, P_CHARBONNIER_PRIME = 4, P_RCP = 5 };

__global__ void k_probe_math(int fn, const float* __restrict__ x, float* __restrict__ y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  float r;
  switch (fn) {
    case P_EXP: r = fast_exp(v); break;
    case P_SOFTPLUS: r = softplus(v); break;
    case P_SOFTPLUS_PRIME: r = softplus_prime_from_pre(v); break;
    case P_SIGMOID_SOFT: r = sigmoid_soft(v); break;
    case P_CHARBONNIER_PRIME: r = charbonnier_prime(v); break;
    default: r = fast_rcp(v); break;
  }
  y[i] = r;
}

// x, y: device arrays of n floats.  Returns 0, or 1 for an unknown function or a launch error.
extern "C" int ffn_probe_math(int fn, const float* x, float* y, int n) {
  if (fn < 0 || fn > P_RCP || n < 0) return 1;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_probe_math, dim3((n + 255) / 256), dim3(256), 0, 0, fn, x, y, n);
  if (hipGetLastError() != hipSuccess) return 1;
  return hipDeviceSynchronize() == hipSuccess ? 0 : 1;
}
