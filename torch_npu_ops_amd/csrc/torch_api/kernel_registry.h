// Compatibility shim for xLLM's triton_npu/kernel_registry.h: the same
// KernelRegistry API, but kernels are built into libxk.so, so there is no
// .npubin to load and no JSON launch config to parse.
//  * register_kernel(name, path) succeeds for every built-in kernel name of
//    the reference's operation table and ignores the path;
//  * get_kernel_stub(name) returns the address of the xk_* C-ABI entry point
//    that runs that kernel's family (include/xk_ops.h);
//  * parse_json_config always fails (workspace sizes come from the
//    xk_*_workspace_bytes functions) and get_kernel_workspace_config reports
//    no workspace, lock or lock value for built-in names;
//  * cleanup is a no-op.
// Like the reference singleton, it is not meant to be mutated from several
// threads at once; lookups only read a static table.
#pragma once

#include <cstdint>
#include <string>

namespace xllm::kernel::npu {

using KernelStubHandle = void*;

class KernelRegistry {
 public:
  static KernelRegistry& get_instance();

  KernelRegistry(const KernelRegistry&) = delete;
  KernelRegistry& operator=(const KernelRegistry&) = delete;

  bool register_kernel(const std::string& kernel_name, const std::string& binary_path);
  KernelStubHandle get_kernel_stub(const std::string& kernel_name) const;
  bool is_kernel_registered(const std::string& kernel_name) const;
  void cleanup();
  bool parse_json_config(const std::string& json_path, std::string& kernel_name,
                         std::string& mix_mode, int64_t& workspace_size,
                         int64_t& lock_init_value, int64_t& lock_num);
  bool get_kernel_workspace_config(const std::string& kernel_name, int64_t& workspace_size,
                                   int64_t& lock_init_value, int64_t& lock_num) const;

 private:
  KernelRegistry() = default;
  ~KernelRegistry() = default;
};

}  // namespace xllm::kernel::npu
