// r97/rad_plugin_abi.h -- the kernel-plugin table radiance's loader reads from libr97rows.so, the
// exports of the reference's src/adjoint/device/plugin.hip:38-80.
//
// The plugin carries no radiance op rows: its rows register into r97's registry (r97/adjoint.h)
// when the library loads, so both tables are empty and every entry lookup returns null. What the
// loader gets is the plugin's identity and the ABI version it was built against.
//
// Radiance's rad_plugin.h is not in this tree (the reference builds against the un-vendored
// third_party/radiance), so two things it would supply are stated here instead:
//   * the info record's layout follows the field order of the reference's initializer
//     (plugin.hip:31-34): kind, name, version, description, build target;
//   * the constants RAD_ABI_VERSION and RAD_PLUGIN_KERNEL are build parameters, R97_RAD_ABI_VERSION
//     and R97_RAD_PLUGIN_KERNEL (0 unless defined), so a build for a radiance loader sets them from
//     that header; a loader that checks the version refuses a build made without them.
// The reference's RAD_PLUGIN_ABI_LAYOUT_EXPORT (a layout check radiance's header defines) has no
// counterpart for the same reason.
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct R97RadPluginInfo {
    int32_t kind;             // RAD_PLUGIN_KERNEL
    const char* name;         // "r97"
    const char* version;
    const char* description;
    const char* target;       // the GPU architecture the kernels are built for ("gfx950")
} R97RadPluginInfo;

uint32_t rad_plugin_abi_version(void);
const R97RadPluginInfo* rad_plugin_info(void);
// radiance op schemas and kernels this plugin serves: none (counts 0, every entry null)
int rad_kernel_schema_count(void);
const void* rad_kernel_schema_at(int index);
int rad_kernel_count(void);
const void* rad_kernel_at(int index);

#ifdef __cplusplus
}
#endif
