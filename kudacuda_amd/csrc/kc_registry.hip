// Module registry of include/kudacuda_registry.h on the HIP module API.
//
// Contract (the reference's runtime/kudacuda_registry.cu:33-115 as seen by a
// caller): every operation returns 0, or 1 with the reason in *error when the
// caller passed a string; a frozen registry refuses load and resolve; a
// registry whose device did not come up refuses load and freeze with "HIP
// device is unavailable"; names are unique; a failing HIP call is reported as
// "<call> failed: <error name> (<error string>)".
//
// Beyond that contract this implementation inspects a code object before
// handing it to HIP (an AMDGPU ELF, or a clang offload bundle with an amdgcn
// entry), so a missing file or a file that is not an AMDGPU code object (a
// CUDA cubin or PTX file from the reference's build, say) is refused with
// that reason instead of a bare loader status, and resolving the same symbol
// twice returns the handle already in the table.
#include "../../include/kudacuda_registry.h"

#include <cstdint>
#include <cstring>
#include <fstream>
#include <iterator>
#include <utility>
#include <vector>

namespace kudacuda {
namespace {

// One operation's result: 0, or 1 with the reason copied to the caller's
// string (when it passed one).
class Outcome {
public:
    explicit Outcome(std::string* sink) : sink_(sink) {}
    int refuse(std::string reason) const {
        if (sink_ != nullptr) {
            *sink_ = std::move(reason);
        }
        return 1;
    }
    int hip_failure(const char* call, hipError_t status) const {
        return refuse(std::string(call) + " failed: " + hipGetErrorName(status) + " (" + hipGetErrorString(status) +
                      ")");
    }

private:
    std::string* sink_;
};

constexpr unsigned char kElfMagic[4] = {0x7f, 'E', 'L', 'F'};
constexpr int kElfClass64 = 2;
constexpr uint16_t kElfMachineAmdgpu = 224;  // EM_AMDGPU
constexpr char kBundleMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
constexpr size_t kBundleMagicLen = sizeof(kBundleMagic) - 1;
// `hipcc --genco --offload-compress` writes a compressed offload bundle: this
// magic, then a version, the compression method and sizes, then the
// compressed bundle.  Its entries cannot be read without decompressing, so
// it is handed to hipModuleLoad, which decompresses it and judges the target.
constexpr char kCompressedBundleMagic[] = "CCOB";
constexpr size_t kCompressedBundleMagicLen = sizeof(kCompressedBundleMagic) - 1;

enum class CodeObject { kUnreadable, kForeign, kAmdgpu, kCompressedBundle };

// ELF identification and e_machine of the 20 bytes at `p`.
bool is_amdgpu_elf(const unsigned char* p, size_t n) {
    if (n < 20 || std::memcmp(p, kElfMagic, sizeof(kElfMagic)) != 0 || p[4] != kElfClass64) {
        return false;
    }
    // e_machine at offset 18, in the byte order of EI_DATA (1 = little endian)
    const uint16_t machine = p[5] == 1 ? static_cast<uint16_t>(p[18] | (p[19] << 8))
                                       : static_cast<uint16_t>((p[18] << 8) | p[19]);
    return machine == kElfMachineAmdgpu;
}

uint64_t le64(const unsigned char* p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) {
        v = (v << 8) | p[i];
    }
    return v;
}

// A code object as hipModuleLoad takes it: an AMDGPU ELF, a compressed
// offload bundle (passed through, see above), or a clang offload
// bundle (what `hipcc --genco` writes: magic, entry count, then per entry
// offset, size, id length and id, all little-endian uint64) with an
// "amdgcn-amd-amdhsa" entry whose payload is an AMDGPU ELF.
CodeObject inspect_code_object(const std::string& path) {
    std::ifstream file(path, std::ios::binary);
    if (!file.is_open()) {
        return CodeObject::kUnreadable;
    }
    std::vector<unsigned char> bytes((std::istreambuf_iterator<char>(file)), std::istreambuf_iterator<char>());
    if (is_amdgpu_elf(bytes.data(), bytes.size())) {
        return CodeObject::kAmdgpu;
    }
    if (bytes.size() >= kCompressedBundleMagicLen &&
        std::memcmp(bytes.data(), kCompressedBundleMagic, kCompressedBundleMagicLen) == 0) {
        return CodeObject::kCompressedBundle;
    }
    if (bytes.size() < kBundleMagicLen + 8 || std::memcmp(bytes.data(), kBundleMagic, kBundleMagicLen) != 0) {
        return CodeObject::kForeign;
    }
    const uint64_t entries = le64(bytes.data() + kBundleMagicLen);
    size_t at = kBundleMagicLen + 8;
    for (uint64_t e = 0; e < entries && at + 24 <= bytes.size(); ++e) {
        const uint64_t offset = le64(bytes.data() + at);
        const uint64_t size = le64(bytes.data() + at + 8);
        const uint64_t id_len = le64(bytes.data() + at + 16);
        at += 24;
        if (id_len > bytes.size() - at) {
            break;
        }
        const std::string id(reinterpret_cast<const char*>(bytes.data() + at), static_cast<size_t>(id_len));
        at += static_cast<size_t>(id_len);
        if (id.find("amdgcn-amd-amdhsa") != std::string::npos && offset < bytes.size() &&
            size <= bytes.size() - offset && is_amdgpu_elf(bytes.data() + offset, static_cast<size_t>(size))) {
            return CodeObject::kAmdgpu;
        }
    }
    return CodeObject::kForeign;
}

}  // namespace

KudaCudaModuleRegistry::KudaCudaModuleRegistry(int device_id) : device_id_(device_id) {
    int count = 0;
    device_ready_ = hipInit(0) == hipSuccess && hipGetDeviceCount(&count) == hipSuccess && device_id >= 0 &&
                    device_id < count && hipSetDevice(device_id) == hipSuccess;
}

KudaCudaModuleRegistry::~KudaCudaModuleRegistry() {
    functions_.clear();  // handles into the modules below
    for (auto& [name, module] : modules_) {
        if (module != nullptr) {
            (void)hipModuleUnload(module);
        }
    }
}

int KudaCudaModuleRegistry::load(const std::string& name, const std::string& path, std::string* error) {
    const Outcome outcome(error);
    if (frozen_) {
        return outcome.refuse("module registry is frozen");
    }
    if (!device_ready_) {
        return outcome.refuse("HIP device is unavailable");
    }
    if (modules_.count(name) != 0) {
        return outcome.refuse("module already loaded: " + name);
    }
    switch (inspect_code_object(path)) {
        case CodeObject::kUnreadable:
            return outcome.refuse("code object is not readable: " + path);
        case CodeObject::kForeign:
            return outcome.refuse("not an AMDGPU code object (hipcc --genco): " + path);
        case CodeObject::kAmdgpu:
        case CodeObject::kCompressedBundle:
            break;
    }
    if (const hipError_t status = hipSetDevice(device_id_); status != hipSuccess) {
        return outcome.hip_failure("hipSetDevice", status);
    }
    hipModule_t module = nullptr;
    if (const hipError_t status = hipModuleLoad(&module, path.c_str()); status != hipSuccess) {
        return outcome.hip_failure("hipModuleLoad", status);
    }
    modules_.emplace(name, module);
    return 0;
}

int KudaCudaModuleRegistry::resolve(const std::string& module_name, const std::string& symbol,
                                    hipFunction_t* function, std::string* error) {
    const Outcome outcome(error);
    if (frozen_) {
        return outcome.refuse("module registry is frozen");
    }
    if (function == nullptr) {
        return outcome.refuse("function output pointer is null");
    }
    const auto module = modules_.find(module_name);
    if (module == modules_.end()) {
        return outcome.refuse("module is not loaded: " + module_name);
    }
    const std::string key = module_name + "::" + symbol;
    if (const auto known = functions_.find(key); known != functions_.end()) {
        *function = known->second;
        return 0;
    }
    hipFunction_t resolved = nullptr;
    if (const hipError_t status = hipModuleGetFunction(&resolved, module->second, symbol.c_str());
        status != hipSuccess) {
        return outcome.hip_failure("hipModuleGetFunction", status);
    }
    functions_.emplace(key, resolved);
    *function = resolved;
    return 0;
}

int KudaCudaModuleRegistry::freeze(std::string* error) {
    if (!device_ready_) {
        return Outcome(error).refuse("HIP device is unavailable");
    }
    frozen_ = true;
    return 0;
}

}  // namespace kudacuda
