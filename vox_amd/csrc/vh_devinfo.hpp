// vh_devinfo.hpp — the device description that gpu_enumerate hands to the planner (vox::GpuDeviceInfo,
// gpu.hpp:22-30, through voxhip_device_info), made from HIP's device properties. Host code with no HIP calls, so a
// recorded property set converts the same way on a machine without the GPU.
#pragma once
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "voxhip.h"

namespace vh {

struct DevProps {
    std::string name;       // hipDeviceProp_t::name (empty on some ROCm installs)
    std::string arch;       // hipDeviceProp_t::gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    uint64_t total = 0;     // totalGlobalMem
    uint64_t free = 0;      // hipMemGetInfo's free bytes, or total when the device is not the current one
    int integrated = 0, major = 0, minor = 0;
    int runtime = 0;        // hipRuntimeGetVersion
};

// The device's name for gpu_device_name / GpuDeviceInfo::name: the property name with trailing blanks dropped (the
// MI350 series name when it is empty on a gfx950), then the architecture in parentheses.
inline std::string device_label(const std::string &raw, const std::string &arch) {
    std::string name = raw;
    while (!name.empty() && (name.back() == ' ' || name.back() == '\n')) name.pop_back();
    if (name.empty()) name = arch.compare(0, 6, "gfx950") == 0 ? "AMD Instinct MI350 series (MI350X / MI355X)" : "AMD GPU";
    return name + " (" + arch + ")";
}

// GpuDeviceInfo fields as the planner reads them (resources.cpp:376-395, :535-547): a discrete, hardware device
// whose free memory is the budget base; MFMA counts as the cooperative-matrix feature.
inline void device_info_of(int index, const DevProps &p, voxhip_device_info *out) {
    std::memset(out, 0, sizeof *out);
    out->index = index;
    std::snprintf(out->name, sizeof out->name, "%s", device_label(p.name, p.arch).c_str());
    std::snprintf(out->type, sizeof out->type, "%s", p.integrated ? "integrated" : "discrete");
    out->software = 0;
    out->unified_memory = p.integrated ? 1 : 0;
    out->vram_total = p.total;
    out->vram_free = p.free;
    out->max_storage_range = p.total;
    out->subgroup_arith = 1;
    out->coop_matrix = 1;
    out->memory_budget = 1;
    out->api_version = uint32_t(p.major * 100 + p.minor);
    out->vendor_id = 0x1002;
    out->driver_version = uint32_t(p.runtime);
}

}  // namespace vh
