// Code object loaded by tests/native/registry_smoke.cpp through the module
// registry (built with `hipcc --genco --offload-arch=gfx950`).
#include <hip/hip_runtime.h>

extern "C" __global__ void kc_registry_probe_affine(const float* in, float* out, int n, float scale, float shift) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) {
        out[i] = in[i] * scale + shift;
    }
}
