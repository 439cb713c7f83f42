// C++ module registry of libkudacuda for gfx950: load HIP code objects by
// name, resolve kernels, then freeze.  Same class, members and error texts
// as the reference's CUDA driver-API registry
// (include/kudacuda_registry.h:10-41, runtime/kudacuda_registry.cu:33-115),
// on the HIP module API: hipModule_t / hipFunction_t in place of
// CUmodule / CUfunction, code objects (.hsaco, `hipcc --genco`) in place of
// cubin/PTX files.  Launch a resolved kernel with hipModuleLaunchKernel,
// using a KudaCudaKernelDescriptor for the grid, block and LDS size.
//
// Not thread-safe (like the reference): one registry per thread, or external
// locking.  Frozen registries refuse load and resolve; resolved functions stay
// valid until the registry is destroyed (which unloads its modules).
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_map>

namespace kudacuda {

// include/kudacuda_registry.h:10-20
struct KudaCudaKernelDescriptor {
    const char* name;
    const char* symbol;
    unsigned int grid_x;
    unsigned int grid_y;
    unsigned int grid_z;
    unsigned int block_x;
    unsigned int block_y;
    unsigned int block_z;
    unsigned int shared_memory_bytes;
};

// include/kudacuda_registry.h:22-41
class KudaCudaModuleRegistry {
public:
    // Initialises HIP and makes `device_id` current; on failure every later
    // call reports "HIP device is unavailable".
    explicit KudaCudaModuleRegistry(int device_id);
    ~KudaCudaModuleRegistry();

    KudaCudaModuleRegistry(const KudaCudaModuleRegistry&) = delete;
    KudaCudaModuleRegistry& operator=(const KudaCudaModuleRegistry&) = delete;

    // 0 on success, 1 with *error set (when error is not null) otherwise.
    int load(const std::string& name, const std::string& path, std::string* error);
    int resolve(const std::string& module_name, const std::string& symbol, hipFunction_t* function,
                std::string* error);
    int freeze(std::string* error);
    bool frozen() const { return frozen_; }

private:
    int device_id_ = 0;
    bool device_ready_ = false;
    bool frozen_ = false;
    std::unordered_map<std::string, hipModule_t> modules_;
    std::unordered_map<std::string, hipFunction_t> functions_;
};

}  // namespace kudacuda
