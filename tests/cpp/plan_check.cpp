// plan_check.cpp — the reference's planner (vox::make_plan, resources.cpp:496-586) on what this backend's
// gpu_enumerate (vox_amd/csrc/gpu_hip.cpp, libvox_gpu_hip.so) reports for a recorded MI355X property set. The
// executable defines voxhip_device_count / voxhip_device_info_get over that record, through the runtime's own
// conversion (vh_devinfo.hpp), and exports them (-rdynamic), so the adapter's calls land here and no GPU is needed.
// The Qwen3-TTS footprint is the one backend_qwen3.cpp:675-722 builds, with the 0.6B model's sizes and q8 weights.
//
// argv: name arch total_bytes free_bytes integrated major minor runtime. Exit status 0 = every check passed.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "gpu.hpp"        // reference (GpuDeviceInfo, gpu_enumerate)
#include "resources.hpp"  // reference (make_plan)
#include "vh_devinfo.hpp"

namespace {
vh::DevProps g_props;
bool g_software = false;
int g_fail = 0;

void check(bool ok, const std::string &what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) ++g_fail;
}

// xfmr_layer_params (backend_qwen3.cpp): q, k, v, o and the three FFN matrices of one layer
double layer_params(double H, double heads, double kv, double hd, double I) {
    return H * heads * hd + 2 * H * kv * hd + heads * hd * H + 3 * H * I;
}

vox::ModelFootprint qwen3_0p6b() {
    const double H = 1024, L = 28, heads = 16, kv = 8, hd = 128, I = 3072, V = 3072;  // talker
    const double PL = 5, PV = 2048;                                                   // code predictor (same widths)
    const int groups = 16;
    const double q8 = 34.0 / 32.0;  // int8 weight + f16 scale per 32-block (bytes per weight)
    const uint64_t cap = 512 + 2048 + 16;
    vox::ModelFootprint fp;
    fp.family = "qwen3_tts";
    fp.variant = "0.6B";
    vox::StageDesc tk;
    tk.name = "talker";
    tk.layers = int(L);
    tk.splittable = true;
    tk.layer_bytes = uint64_t(layer_params(H, heads, kv, hd, I) * q8);
    tk.weight_bytes = tk.layer_bytes * uint64_t(L) + uint64_t(H * V * q8);
    tk.bytes_per_frame = double(tk.weight_bytes);
    tk.flops_per_frame = 2 * (L * layer_params(H, heads, kv, hd, I) + H * V);
    tk.session_vram_bytes = uint64_t(L * 2 * kv * hd * 4) * cap;
    tk.session_ram_bytes = tk.session_vram_bytes;
    fp.stages.push_back(tk);
    vox::StageDesc pr;
    pr.name = "predictor";
    pr.weight_bytes = uint64_t((PL * layer_params(H, heads, kv, hd, I) + (groups - 1) * H * PV * 2) * q8);
    pr.bytes_per_frame = double(groups - 1) * PL * layer_params(H, heads, kv, hd, I) * q8;
    pr.flops_per_frame = 2 * double(groups - 1) * (PL * layer_params(H, heads, kv, hd, I) + H * PV);
    pr.session_vram_bytes = uint64_t(PL * 2 * kv * hd * 4) * 40;
    pr.session_ram_bytes = pr.session_vram_bytes;
    fp.stages.push_back(pr);
    vox::StageDesc cd;
    cd.name = "codec";
    cd.weight_bytes = uint64_t(115) << 20;
    cd.bytes_per_frame = double(cd.weight_bytes) / 4.0;
    cd.flops_per_frame = 4e9;
    cd.session_vram_bytes = 24u << 20;
    cd.session_ram_bytes = 24u << 20;
    fp.stages.push_back(cd);
    fp.always_ram_bytes = uint64_t(64) << 20;
    return fp;
}

vox::SystemInfo host() {
    vox::SystemInfo s;
    s.cpu_logical = s.cpu_allowed = 16;
    s.cpu_physical = 8;
    s.ram_total = uint64_t(64) << 30;
    s.ram_available = uint64_t(48) << 30;
    s.os = "linux";
    return s;
}
}  // namespace

extern "C" int voxhip_device_count(void) { return 1; }
extern "C" int voxhip_device_info_get(int index, voxhip_device_info *out) {
    if (index != 0 || !out) return 0;
    vh::device_info_of(index, g_props, out);
    out->software = g_software ? 1 : 0;
    return 1;
}

int main(int argc, char **argv) {
    if (argc != 9) {
        std::fprintf(stderr, "usage: %s name arch total free integrated major minor runtime\n", argv[0]);
        return 2;
    }
    g_props.name = argv[1];
    g_props.arch = argv[2];
    g_props.total = std::strtoull(argv[3], nullptr, 10);
    g_props.free = std::strtoull(argv[4], nullptr, 10);
    g_props.integrated = std::atoi(argv[5]);
    g_props.major = std::atoi(argv[6]);
    g_props.minor = std::atoi(argv[7]);
    g_props.runtime = std::atoi(argv[8]);

    const std::vector<vox::GpuDeviceInfo> gpus = vox::gpu_enumerate();
    check(gpus.size() == 1, "gpu_enumerate reports the one device");
    if (gpus.size() != 1) return 1;
    const vox::GpuDeviceInfo &d = gpus[0];
    std::printf("device: %s, %s, total %llu, free %llu\n", d.name.c_str(), d.type.c_str(), (unsigned long long)d.vram_total,
                (unsigned long long)d.vram_free);
    check(d.type == "discrete" && !d.software && !d.unified_memory, "a discrete hardware device");
    check(d.vram_total == g_props.total && d.vram_free == g_props.free, "VRAM total and free as recorded");
    check(d.name.find("gfx950") != std::string::npos, "the name carries the architecture");

    const vox::ModelFootprint fp = qwen3_0p6b();
    for (const char *dev : {"auto", "gpu"}) {
        vox::ResourceConfig cfg;
        cfg.device = dev;
        const vox::ResourcePlan P = vox::make_plan(cfg, fp, host(), gpus);
        std::printf("device=%s:\n%s\n", dev, P.summary().c_str());
        check(P.uses_gpu() && P.gpu_index == 0 && P.gpu_name == d.name, std::string("device=") + dev + ": the plan takes the GPU");
        for (const char *st : {"talker", "predictor", "codec"})
            check(P.place_of(st) == vox::Place::Gpu && P.gpu_layers_of(st) == -1,
                  std::string("device=") + dev + ": stage " + st + " wholly on the GPU");
        check(P.feasible, std::string("device=") + dev + ": feasible");
    }
    // the same planner keeps the CPU for a software device in auto mode (resources.cpp:545-547), so the check
    // above depends on what the adapter reports
    g_software = true;
    const vox::ResourcePlan S = vox::make_plan(vox::ResourceConfig(), fp, host(), vox::gpu_enumerate());
    check(!S.uses_gpu(), "a software device stays unused in auto mode");
    std::printf("%s\n", g_fail ? "FAILED" : "all passed");
    return g_fail ? 1 : 0;
}
