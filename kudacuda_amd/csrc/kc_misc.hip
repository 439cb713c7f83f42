// Small ops the reference's C ABI exports besides the decode path: fp32
// vector add (pointer/stream/graph plumbing check, reference
// kernels/vector_add.cu:11-37), fp32 row RMSNorm (reference
// kernels/common/rmsnorm.cuh:11-65) and the dense fp16 fused RMSNorm+QKV
// foundation op (reference kernels/common/rmsnorm_qkv_reference.cuh:12-66,
// weight [3h, h], bias [3h], output [rows, 3h]).  None is on the decode hot
// path; each is a plain wave64 kernel.
#include "kc_device.h"
#include "kc_kernels.h"

namespace kc {
namespace {

__global__ __launch_bounds__(256) void vector_add_kernel(const float* a, const float* b, float* out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        out[i] = a[i] + b[i];
    }
}

// One block per row; thread t accumulates elements t, t+256, ...; the block
// total is a wave butterfly per wave followed by the 4 wave sums in order.
__global__ __launch_bounds__(256) void rmsnorm_f32_kernel(const float* x, const float* w, float* y, int64_t hidden,
                                                          float eps) {
    __shared__ float s_w[4];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * hidden;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < hidden; i += 256) {
        ss = fmaf(xr[i], xr[i], ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) {
        s_w[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    const float total = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
    const float r = inv_rms(total, static_cast<float>(hidden), eps);
    for (int64_t i = threadIdx.x; i < hidden; i += 256) {
        y[row * hidden + i] = (xr[i] * r) * w[i];
    }
}

// grid (ceil(3h / 4), rows): one wave per output feature; every wave
// recomputes the row's inverse RMS (lane-strided sum, butterfly).
__global__ __launch_bounds__(256) void dense_rmsnorm_qkv_f16_kernel(const uint16_t* x, const uint16_t* gamma,
                                                                        const uint16_t* w, const uint16_t* bias,
                                                                        uint16_t* out, int64_t hidden, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t feature = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t row = blockIdx.y;
    const int64_t features = 3 * hidden;
    if (feature >= features) {
        return;
    }
    const uint16_t* xr = x + row * hidden;
    float ss = 0.0f;
    for (int64_t i = lane; i < hidden; i += 64) {
        const float v = f16_to_f32(xr[i]);
        ss = fmaf(v, v, ss);
    }
    const float r = inv_rms(wave_sum(ss), static_cast<float>(hidden), eps);
    const uint16_t* wr = w + feature * hidden;
    float acc = 0.0f;
    for (int64_t i = lane; i < hidden; i += 64) {
        const float xn = (f16_to_f32(xr[i]) * r) * f16_to_f32(gamma[i]);
        acc = fmaf(xn, f16_to_f32(wr[i]), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        if (bias != nullptr) {
            acc = acc + f16_to_f32(bias[feature]);
        }
        out[row * features + feature] = f32_to_f16(acc);
    }
}

}  // namespace

hipError_t launch_vector_add(const float* a, const float* b, float* out, int64_t n, hipStream_t stream) {
    if (n <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(vector_add_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, a, b,
                       out, n);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_f32(const float* x, const float* w, float* y, int64_t rows, int64_t hidden, float eps,
                              hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, x, w, y, hidden,
                       eps);
    return hipGetLastError();
}

hipError_t launch_dense_rmsnorm_qkv_f16(const uint16_t* x, const uint16_t* gamma, const uint16_t* w,
                                        const uint16_t* bias, uint16_t* out, int64_t rows, int64_t hidden, float eps,
                                        hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((3 * hidden + 3) / 4), static_cast<unsigned>(rows));
    hipLaunchKernelGGL(dense_rmsnorm_qkv_f16_kernel, grid, dim3(256), 0, stream, x, gamma, w, bias, out, hidden,
                       eps);
    return hipGetLastError();
}

}  // namespace kc
