// Smoke test of the module registry (include/kudacuda_registry.h), in the
// style of the reference's C++ smokes (tests/*.cu): prints one line and exits
// 0 on success.
//
//   registry_smoke <code object>   load, resolve, launch through a descriptor,
//                                  check, then the frozen, duplicate, missing-
//                                  file and non-AMDGPU-file guards
//   registry_smoke --no-device     on a host without a GPU: every call must
//                                  report the missing device
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/kudacuda_registry.h"

namespace {

int fail(const char* what, const std::string& detail) {
    std::fprintf(stderr, "registry smoke FAILED: %s: %s\n", what, detail.c_str());
    return 1;
}

int no_device() {
    kudacuda::KudaCudaModuleRegistry registry(0);
    std::string error;
    if (registry.load("probe", "missing.hsaco", &error) != 1 || error != "HIP device is unavailable") {
        return fail("load without a device", error);
    }
    if (registry.freeze(&error) != 1 || error != "HIP device is unavailable" || registry.frozen()) {
        return fail("freeze without a device", error);
    }
    hipFunction_t fn = nullptr;
    if (registry.resolve("probe", "kc_registry_probe_affine", &fn, &error) != 1 ||
        error != "module is not loaded: probe") {
        return fail("resolve without a module", error);
    }
    if (registry.resolve("probe", "x", nullptr, &error) != 1 || error != "function output pointer is null") {
        return fail("resolve into null", error);
    }
    std::printf("registry smoke ok (no device)\n");
    return 0;
}

int with_device(const char* path, const char* self_path) {
    kudacuda::KudaCudaModuleRegistry registry(0);
    std::string error;
    if (registry.load("probe", path, &error) != 0) {
        return fail("load", error);
    }
    if (registry.load("probe", path, &error) != 1 || error != "module already loaded: probe") {
        return fail("duplicate load", error);
    }
    if (registry.load("other", "/nonexistent/none.hsaco", &error) != 1 ||
        error != "code object is not readable: /nonexistent/none.hsaco") {
        return fail("load of a missing file", error);
    }
    // this program itself: an ELF file, but an x86-64 one
    if (registry.load("host", self_path, &error) != 1 ||
        error != std::string("not an AMDGPU code object (hipcc --genco): ") + self_path) {
        return fail("load of a host executable", error);
    }
    hipFunction_t fn = nullptr;
    if (registry.resolve("probe", "kc_registry_probe_affine", &fn, &error) != 0 || fn == nullptr) {
        return fail("resolve", error);
    }
    if (registry.resolve("probe", "no_such_kernel", &fn, &error) != 1 ||
        error.rfind("hipModuleGetFunction failed: ", 0) != 0) {
        return fail("resolve of a missing symbol", error);
    }
    if (registry.resolve("nope", "kc_registry_probe_affine", &fn, &error) != 1 ||
        error != "module is not loaded: nope") {
        return fail("resolve in an unknown module", error);
    }
    hipFunction_t again = nullptr;
    if (registry.resolve("probe", "kc_registry_probe_affine", &again, &error) != 0 || again != fn) {
        return fail("resolve again (the table's handle)", error);
    }

    const int n = 1000;
    const kudacuda::KudaCudaKernelDescriptor desc = {
        "probe_affine", "kc_registry_probe_affine", (n + 255) / 256, 1, 1, 256, 1, 1, 0};
    std::vector<float> host(n);
    for (int i = 0; i < n; ++i) {
        host[i] = static_cast<float>(i) * 0.25f - 7.0f;
    }
    float* d_in = nullptr;
    float* d_out = nullptr;
    if (hipMalloc(&d_in, n * sizeof(float)) != hipSuccess || hipMalloc(&d_out, n * sizeof(float)) != hipSuccess) {
        return fail("hipMalloc", "");
    }
    (void)hipMemcpy(d_in, host.data(), n * sizeof(float), hipMemcpyHostToDevice);
    int count = n;
    float scale = 2.0f;
    float shift = 1.5f;
    void* args[] = {&d_in, &d_out, &count, &scale, &shift};
    hipError_t status = hipModuleLaunchKernel(fn, desc.grid_x, desc.grid_y, desc.grid_z, desc.block_x, desc.block_y,
                                              desc.block_z, desc.shared_memory_bytes, nullptr, args, nullptr);
    if (status != hipSuccess) {
        return fail("hipModuleLaunchKernel", hipGetErrorString(status));
    }
    std::vector<float> got(n);
    status = hipMemcpy(got.data(), d_out, n * sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(d_in);
    (void)hipFree(d_out);
    if (status != hipSuccess) {
        return fail("hipMemcpy", hipGetErrorString(status));
    }
    for (int i = 0; i < n; ++i) {
        const float want = host[i] * 2.0f + 1.5f;
        if (got[i] != want) {
            return fail("kernel output", std::to_string(i) + ": " + std::to_string(got[i]));
        }
    }

    if (registry.freeze(&error) != 0 || !registry.frozen()) {
        return fail("freeze", error);
    }
    if (registry.load("late", path, &error) != 1 || error != "module registry is frozen") {
        return fail("load after freeze", error);
    }
    if (registry.resolve("probe", "kc_registry_probe_affine", &fn, &error) != 1 ||
        error != "module registry is frozen") {
        return fail("resolve after freeze", error);
    }
    std::printf("registry smoke ok (%d outputs via %s)\n", n, desc.name);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc == 2 && std::strcmp(argv[1], "--no-device") == 0) {
        return no_device();
    }
    if (argc != 2) {
        std::fprintf(stderr, "usage: registry_smoke <code object> | --no-device\n");
        return 2;
    }
    return with_device(argv[1], argv[0]);
}
