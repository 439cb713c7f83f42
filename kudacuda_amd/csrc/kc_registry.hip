// HIP module registry (include/kudacuda_registry.h); behaviour follows
// runtime/kudacuda_registry.cu:33-115: load refuses a frozen registry, a
// missing device and duplicate names; resolve refuses a frozen registry, a
// null output and unknown modules; freeze needs a device.  Errors name the
// failing HIP call with its error name and string.
#include "../../include/kudacuda_registry.h"

#include <sstream>

namespace kudacuda {
namespace {

int set_hip_error(std::string* error, const char* operation, hipError_t status) {
    if (error != nullptr) {
        std::ostringstream stream;
        stream << operation << " failed: " << hipGetErrorName(status) << " (" << hipGetErrorString(status) << ")";
        *error = stream.str();
    }
    return 1;
}

int set_text_error(std::string* error, const std::string& message) {
    if (error != nullptr) {
        *error = message;
    }
    return 1;
}

}  // namespace

KudaCudaModuleRegistry::KudaCudaModuleRegistry(int device_id) : device_id_(device_id) {
    if (hipInit(0) != hipSuccess) {
        return;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device_id < 0 || device_id >= count) {
        return;
    }
    device_ready_ = hipSetDevice(device_id) == hipSuccess;
}

KudaCudaModuleRegistry::~KudaCudaModuleRegistry() {
    for (const auto& entry : modules_) {
        if (entry.second != nullptr) {
            (void)hipModuleUnload(entry.second);
        }
    }
}

int KudaCudaModuleRegistry::load(const std::string& name, const std::string& path, std::string* error) {
    if (frozen_) {
        return set_text_error(error, "module registry is frozen");
    }
    if (!device_ready_) {
        return set_text_error(error, "HIP device is unavailable");
    }
    if (modules_.find(name) != modules_.end()) {
        return set_text_error(error, "module already loaded: " + name);
    }
    hipError_t status = hipSetDevice(device_id_);
    if (status != hipSuccess) {
        return set_hip_error(error, "hipSetDevice", status);
    }
    hipModule_t module = nullptr;
    status = hipModuleLoad(&module, path.c_str());
    if (status != hipSuccess) {
        return set_hip_error(error, "hipModuleLoad", status);
    }
    modules_.emplace(name, module);
    return 0;
}

int KudaCudaModuleRegistry::resolve(const std::string& module_name, const std::string& symbol,
                                    hipFunction_t* function, std::string* error) {
    if (frozen_) {
        return set_text_error(error, "module registry is frozen");
    }
    if (function == nullptr) {
        return set_text_error(error, "function output pointer is null");
    }
    const auto module = modules_.find(module_name);
    if (module == modules_.end()) {
        return set_text_error(error, "module is not loaded: " + module_name);
    }
    const hipError_t status = hipModuleGetFunction(function, module->second, symbol.c_str());
    if (status != hipSuccess) {
        return set_hip_error(error, "hipModuleGetFunction", status);
    }
    functions_[module_name + "::" + symbol] = *function;
    return 0;
}

int KudaCudaModuleRegistry::freeze(std::string* error) {
    if (!device_ready_) {
        return set_text_error(error, "HIP device is unavailable");
    }
    frozen_ = true;
    return 0;
}

}  // namespace kudacuda
