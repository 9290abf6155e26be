// plugin.cpp -- the kernel-plugin exports (r97/rad_plugin_abi.h): what radiance's loader reads when
// it dlopens this library next to its own plugins (the reference's src/adjoint/device/plugin.hip).
//
// The rows themselves register into r97's registry from rows.cpp when the library loads; the
// registry, the stored-weight store, the gradient staging and the scratch ledger are this library's
// own weak definitions, so a process that does not link the reference's executable (a tool that only
// dlopens the plugin) still finds every symbol the rows call, and a process that does gets the
// executable's definitions (the dynamic loader prefers them).
#include "r97/rad_plugin_abi.h"

#ifndef R97_RAD_ABI_VERSION
#define R97_RAD_ABI_VERSION 0u
#endif
#ifndef R97_RAD_PLUGIN_KERNEL
#define R97_RAD_PLUGIN_KERNEL 0
#endif
#ifndef R97_DEVICE_BUILD_TARGET
#define R97_DEVICE_BUILD_TARGET "gfx950"
#endif

namespace {

const R97RadPluginInfo kInfo = {
    R97_RAD_PLUGIN_KERNEL, "r97", "0.1",
    "r97 device adjoints for MI355X: gemm_nt, gemm_nt_q, lora_shrink, lora_expand(_mm), the activation "
    "quantisers; no radiance op rows",
    R97_DEVICE_BUILD_TARGET,
};

}  // namespace

extern "C" uint32_t rad_plugin_abi_version(void) { return R97_RAD_ABI_VERSION; }
extern "C" const R97RadPluginInfo* rad_plugin_info(void) { return &kInfo; }
extern "C" int rad_kernel_schema_count(void) { return 0; }
extern "C" const void* rad_kernel_schema_at(int) { return nullptr; }
extern "C" int rad_kernel_count(void) { return 0; }
extern "C" const void* rad_kernel_at(int) { return nullptr; }
