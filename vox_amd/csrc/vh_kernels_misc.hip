// Launchers of the non-GEMV kernels: q/k post-processing, attention, sampler, quantizers, synthetic data.
#include <cxxabi.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include <mutex>
#include <map>

#include "vh_attn.hpp"
#include "vh_pattn.hpp"
#include "vh_launch.hpp"
#include "vh_sample.hpp"
#include "vh_util.hpp"

namespace vh {

namespace {
std::mutex g_tmu;
hipEvent_t g_tq[16][2];
int g_thead = 0;
std::atomic<int> g_tcount{0};
}  // namespace

void timing_arm(hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lk(g_tmu);
    if (!stop) return;
    if (g_tcount == 16) return;
    const int i = (g_thead + g_tcount) % 16;
    g_tq[i][0] = start;
    g_tq[i][1] = stop;
    ++g_tcount;
}
void timing_clear() {
    std::lock_guard<std::mutex> lk(g_tmu);
    g_tcount = 0;
}
bool timing_take(hipEvent_t *start, hipEvent_t *stop) {
    if (!g_tcount) return false;  // fast path; arming and launching happen on the calling thread
    std::lock_guard<std::mutex> lk(g_tmu);
    if (!g_tcount) return false;
    *start = g_tq[g_thead][0];
    *stop = g_tq[g_thead][1];
    g_thead = (g_thead + 1) % 16;
    --g_tcount;
    return true;
}

// ------------------------------------------------------------------ VOX_PROFILE=gpu
namespace {
struct ProfRec {
    const std::string *label;
    hipEvent_t e0, e1;
};
struct ProfAcc {
    double ns = 0.0;
    uint64_t calls = 0;
};
std::atomic<bool> g_prof{false};
std::mutex g_pmu;
std::string g_stage = "-";
std::vector<ProfRec> g_pending;
std::vector<hipEvent_t> g_pool;
std::map<std::pair<const void *, std::string>, std::string> g_labels;  // (kernel, stage) -> "<stage>/<kernel name>"
std::vector<std::pair<std::string, ProfAcc>> g_acc;                     // first-seen order, sorted at report time
uint64_t g_batches = 0;
std::string g_report;

// "void vh::k_gemv_int<3, 1, 4, 2, 1, 0, true, false>(vh::GemvArgs)" -> "k_gemv_int<3,1,4,2,1,0,true,false>"
std::string kernel_name(const void *kernel, hipStream_t s) {
    const char *m = hipKernelNameRefByPtr(kernel, s);
    if (!m) return "kernel";
    // the host demangler predates _Float16 ("DF16_"); spelled as the half type ("Dh") it demangles the rest
    std::string mm = m;
    for (size_t p; (p = mm.find("DF16_")) != std::string::npos;) mm.replace(p, 5, "Dh");
    int st = 0;
    char *d = abi::__cxa_demangle(mm.c_str(), nullptr, nullptr, &st);
    std::string n = st == 0 && d ? d : m;
    std::free(d);
    int depth = 0;  // cut the parameter list: the first '(' outside template brackets
    for (size_t i = 0; i < n.size(); ++i) {
        if (n[i] == '<') ++depth;
        else if (n[i] == '>') --depth;
        else if (n[i] == '(' && depth == 0) { n.resize(i); break; }
    }
    for (const char *pre : {"void ", "vh::"})
        for (size_t p; (p = n.find(pre)) != std::string::npos;) n.erase(p, std::strlen(pre));
    n.erase(std::remove(n.begin(), n.end(), ' '), n.end());  // one column of the table
    return n;
}
hipEvent_t pool_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}
}  // namespace

bool prof_on() { return g_prof.load(std::memory_order_relaxed); }
void prof_enable() { g_prof = true; }
void prof_stage(const char *stage) {
    if (!prof_on()) return;
    std::lock_guard<std::mutex> lk(g_pmu);
    g_stage = stage && *stage ? stage : "-";
}
void prof_take(const void *kernel, hipStream_t s, hipEvent_t *start, hipEvent_t *stop) {
    std::lock_guard<std::mutex> lk(g_pmu);
    auto key = std::make_pair(kernel, g_stage);
    auto it = g_labels.find(key);
    if (it == g_labels.end()) it = g_labels.emplace(key, g_stage + "/" + kernel_name(kernel, s)).first;
    *start = pool_event();
    *stop = pool_event();
    g_pending.push_back({&it->second, *start, *stop});
}
void prof_collect() {
    if (!prof_on()) return;
    std::lock_guard<std::mutex> lk(g_pmu);
    if (g_pending.empty()) return;
    for (const ProfRec &r : g_pending) {
        float ms = 0.f;
        if (r.e0 && r.e1 && hipEventElapsedTime(&ms, r.e0, r.e1) == hipSuccess) {
            auto it = std::find_if(g_acc.begin(), g_acc.end(), [&](const auto &p) { return p.first == *r.label; });
            if (it == g_acc.end()) {
                g_acc.push_back({*r.label, ProfAcc{}});
                it = g_acc.end() - 1;
            }
            it->second.ns += double(ms) * 1e6;
            it->second.calls += 1;
        }
        for (hipEvent_t e : {r.e0, r.e1})
            if (e) g_pool.push_back(e);
    }
    g_pending.clear();
    g_batches += 1;
}
const char *prof_report(const char *device) {
    std::lock_guard<std::mutex> lk(g_pmu);
    g_report.clear();
    if (!prof_on() || g_acc.empty()) return g_report.c_str();
    auto v = g_acc;
    std::sort(v.begin(), v.end(), [](const auto &a, const auto &b) { return a.second.ns > b.second.ns; });
    double total = 0.0;
    for (const auto &p : v) total += p.second.ns;
    char line[512];
    std::snprintf(line, sizeof line, "[vox gpu profile] %s: GPU busy %.1f ms in %llu submits\n  %-28s %8s %10s %9s %6s\n",
                  device ? device : "", total / 1e6, (unsigned long long)g_batches, "stage/kernel", "calls", "total ms",
                  "avg us", "share");
    g_report += line;
    for (const auto &p : v) {
        std::snprintf(line, sizeof line, "  %-28s %8llu %10.2f %9.1f %5.1f%%\n", p.first.c_str(),
                      (unsigned long long)p.second.calls, p.second.ns / 1e6,
                      p.second.ns / 1e3 / double(std::max<uint64_t>(1, p.second.calls)), 100.0 * p.second.ns / std::max(1.0, total));
        g_report += line;
    }
    return g_report.c_str();
}

hipError_t ensure_smem(const void *kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    static std::mutex mu;
    static std::map<const void *, size_t> done;  // largest size opted in per kernel
    std::lock_guard<std::mutex> lk(mu);
    auto it = done.find(kernel);
    if (it != done.end() && it->second >= bytes) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    if (e == hipSuccess) done[kernel] = bytes;
    return e;
}

hipError_t launch_qk_post(const QkArgs &a, int m, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    const int nh = a.heads + a.kv_heads;
    if (a.hd == 64) return launch(k_qk_post_wide<32>, dim3(unsigned((nh + 7) / 8), m), dim3(256), 0, s, a);
    if (a.hd == 128) return launch(k_qk_post_wide<64>, dim3(unsigned((nh + 3) / 4), m), dim3(256), 0, s, a);
    return launch(k_qk_post, dim3(nh, m), dim3(64), 0, s, a);
}

struct AttnLaunch {
    const _Float16 *kc0, *vc0;
    const float *qkv, *rope_rows;
    int32_t cap0, layer;
    bool lng;  // one row at a position past kAttnSpecKeys
};

template <int HD, int G>
static hipError_t attn_hg(const AttnArgs &a, const AttnLaunch &l, int m, bool fused, hipStream_t s) {
    const size_t smem = sizeof(AttnSmem<HD, G>);
    const dim3 grid(kAttnMaxSplits, a.kv_heads * (a.group / G), m);
    if (fused && m == 1 && l.lng) {
        hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_attn<HD, G, true, true, true>), smem);
        if (e != hipSuccess) return e;
        return launch(k_attn<HD, G, true, true, true>, grid, dim3(256), smem, s, l.kc0, l.vc0, l.qkv, l.rope_rows, l.cap0, l.layer,
                      a);
    }
    if (fused && m == 1) {
        hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_attn<HD, G, true, true>), smem);
        if (e != hipSuccess) return e;
        return launch(k_attn<HD, G, true, true>, grid, dim3(256), smem, s, l.kc0, l.vc0, l.qkv, l.rope_rows, l.cap0, l.layer, a);
    }
    if (fused) {
        hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_attn<HD, G, true>), smem);
        if (e != hipSuccess) return e;
        return launch(k_attn<HD, G, true>, grid, dim3(256), smem, s, l.kc0, l.vc0, l.qkv, l.rope_rows, l.cap0, l.layer, a);
    }
    hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_attn<HD, G, false>), smem);
    if (e != hipSuccess) return e;
    return launch(k_attn<HD, G, false>, grid, dim3(256), smem, s, l.kc0, l.vc0, l.qkv, l.rope_rows, l.cap0, l.layer, a);
}

// Query heads per block: the whole group, or, when a launch has few blocks (few kv heads, few rows), the largest
// divisor of the group that gives at least kAttnMinBlocks blocks (more blocks share the work; each reads its kv
// head's keys, so a split multiplies the key reads by group / G). The attention is latency-bound: at 8 sessions of
// the 1.7B talker (8 kv heads, group 2), one head per block (1024 blocks, twice the key reads) measured 1.586-1.590 ->
// 1.564-1.572 ms per step against two (512 blocks); one-row launches had one head per block already.
constexpr int kAttnMinBlocks = 1024;
static int attn_heads_per_block(int kv_heads, int group, int m) {
    int gb = group;
    while (gb > 1 && int64_t(m) * kv_heads * (group / gb) * kAttnMaxSplits < kAttnMinBlocks) {
        int d = gb - 1;
        while (d > 1 && group % d) --d;
        gb = d;
    }
    return gb;
}

template <int HD>
static hipError_t attn_h(const AttnArgs &a, const AttnLaunch &l, int m, bool fused, hipStream_t s) {
    switch (attn_heads_per_block(a.kv_heads, a.group, m)) {
        case 1: return attn_hg<HD, 1>(a, l, m, fused, s);
        case 2: return attn_hg<HD, 2>(a, l, m, fused, s);
        case 3: return attn_hg<HD, 3>(a, l, m, fused, s);
        case 4: return attn_hg<HD, 4>(a, l, m, fused, s);
        case 5: return attn_hg<HD, 5>(a, l, m, fused, s);
        case 6: return attn_hg<HD, 6>(a, l, m, fused, s);
        case 7: return attn_hg<HD, 7>(a, l, m, fused, s);
        case 8: return attn_hg<HD, 8>(a, l, m, fused, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attention(const AttnArgs &a, const _Float16 *kc0, const _Float16 *vc0, int64_t cap0, const float *qkv,
                            const float *rope_rows, int layer, int hd, int group, int m, bool fused, hipStream_t s,
                            bool long_ctx) {
    if (m <= 0) return hipSuccess;
    if (cap0 <= 0 || cap0 > INT32_MAX) return hipErrorInvalidValue;
    if (group < 1 || group > 8) return hipErrorInvalidValue;
    const AttnLaunch l{kc0, vc0, qkv, rope_rows, int32_t(cap0), int32_t(layer), long_ctx};
    AttnArgs ag = a;
    ag.group = group;
    if (hd == 128) return attn_h<128>(ag, l, m, fused, s);
    if (hd == 64) return attn_h<64>(ag, l, m, fused, s);
    return hipErrorInvalidValue;
}

// Key splits for a prefill attention grid of tiles x heads blocks: when that leaves most CUs idle and the longest
// query tile has at least 4 key tiles (positions from the host's pos0; a captured pass replayed elsewhere keeps its
// count, which changes only the speed), up to kAttnMaxSplits runs per query tile, about 512 blocks in all.
static int pattn_splits(const PrefillAttnArgs &a) {
    const int64_t blocks = int64_t((a.m + 63) / 64) * a.heads;
    if (!a.part.pm || !a.part.pl || !a.part.po || blocks >= 256 || a.pos0 + a.m < 256) return 1;
    return int(std::min<int64_t>(kAttnMaxSplits, std::max<int64_t>(2, 512 / blocks)));
}
template <int HD>
static hipError_t prefill_attn_hd(const PrefillAttnArgs &a0, hipStream_t s) {
    PrefillAttnArgs a = a0;
    a.splits = pattn_splits(a0);
    a.status = status_word();
    const dim3 grid(unsigned((a.m + 63) / 64), unsigned(a.heads), unsigned(a.splits));
    hipError_t e = launch(k_prefill_attn<HD>, grid, dim3(256), 0, s, a);
    if (e != hipSuccess || a.splits == 1) return e;
    return launch(k_pattn_merge<HD>, dim3(unsigned((a.heads * HD + 255) / 256), unsigned(a.m)), dim3(256), 0, s, a);
}
hipError_t launch_prefill_attn(const PrefillAttnArgs &a, int hd, hipStream_t s) {
    if (a.m <= 0) return hipSuccess;
    if (a.kv_heads <= 0 || a.heads % a.kv_heads || a.pos0 < 0 || a.pos0 + a.m > a.cap) return hipErrorInvalidValue;
    if (hd == 64) return prefill_attn_hd<64>(a, s);
    if (hd == 128) return prefill_attn_hd<128>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_attn_rows(const AttnRowsArgs &a, int m, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (a.hd <= 0 || a.hd > 128 || a.hd % 2 || a.kv_heads <= 0 || a.heads % a.kv_heads || !a.q || !a.out || !a.rows)
        return hipErrorInvalidValue;
    return launch(k_attn_rows, dim3(unsigned(a.heads), unsigned(m)), dim3(256), 0, s, a);
}

template <int E>
static hipError_t sample_e(const SampleCfgDev *cfg, const float *logits, int n, int32_t *out, hipStream_t s, int rows) {
    const size_t smem = sample_smem_bytes(n);
    hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_sample<E>), smem);
    if (e != hipSuccess) return e;
    return launch(k_sample<E>, dim3(unsigned(rows)), dim3(kSampleThreads), smem, s, cfg, logits, n, out);
}

hipError_t launch_sample(const SampleCfgDev *cfg, const float *logits, int n, int32_t *out, hipStream_t s, int rows) {
    if (n <= 0 || n > kSampleMaxN || rows <= 0) return hipErrorInvalidValue;
    const int per = (n + kSampleThreads - 1) / kSampleThreads;
    if (per <= 1) return sample_e<1>(cfg, logits, n, out, s, rows);
    if (per <= 2) return sample_e<2>(cfg, logits, n, out, s, rows);
    if (per <= 4) return sample_e<4>(cfg, logits, n, out, s, rows);
    if (per <= 8) return sample_e<8>(cfg, logits, n, out, s, rows);
    static_assert(kSampleMaxN == 16 * kSampleThreads, "the sampler's largest instance holds 16 logits per thread");
    return sample_e<16>(cfg, logits, n, out, s, rows);
}

static dim3 grid1(int64_t n, int bs) { return dim3(unsigned((n + bs - 1) / bs)); }

hipError_t launch_quant_q8(const float *w, int64_t nblocks, int8_t *q, float *scale, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    return launch(k_quant_q8, grid1(nblocks, 256), dim3(256), 0, s, w, nblocks, q, scale);
}
hipError_t launch_quant_q4(const float *w, int64_t nblocks, uint8_t *q, float *scale, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    return launch(k_quant_q4, grid1(nblocks, 128), dim3(128), 0, s, w, nblocks, q, scale);
}
hipError_t launch_quant_act(const float *x, int64_t nblocks, int8_t *xq, float *xs, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    return launch(k_quant_act, grid1(nblocks, 256), dim3(256), 0, s, x, nblocks, xq, xs);
}
hipError_t launch_to_f16(const float *x, int64_t n, void *y, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    return launch(k_to_f16, grid1(n, 256), dim3(256), 0, s, x, n, static_cast<_Float16 *>(y));
}
hipError_t launch_to_bf16(const float *x, int64_t n, void *y, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    return launch(k_to_bf16, grid1(n, 256), dim3(256), 0, s, x, n, static_cast<uint16_t *>(y));
}
hipError_t launch_rmsnorm_rows(const float *x, int64_t ldx, const float *w, int K, float eps, float *out, int64_t ldo,
                               int m, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    return launch(k_rmsnorm_rows, dim3(m), dim3(256), 0, s, x, ldx, w, K, eps, out, ldo);
}
hipError_t launch_rmsnorm_rows_h16(const float *x, int64_t ldx, const float *w, int K, float eps, _Float16 *out16,
                                   int64_t ldo, int64_t lo_off, int m, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (!out16 || ldo < K || lo_off < int64_t(m) * ldo) return hipErrorInvalidValue;
    return launch(k_rmsnorm_rows_h16, dim3(m), dim3(256), 0, s, x, ldx, w, K, eps, out16, ldo, lo_off, status_word());
}
hipError_t launch_q8_to_f16(const int8_t *q, _Float16 *out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n % 8) return hipErrorInvalidValue;
    return launch(k_q8_to_f16, grid1(n / 8, 256), dim3(256), 0, s, q, out, n);
}
hipError_t launch_fill_normal(float *out, int64_t n, uint64_t seed, uint32_t stream, float mean, float std,
                              hipStream_t s) {
    if (n <= 0) return hipSuccess;
    return launch(k_fill_normal, grid1((n + 1) / 2, 256), dim3(256), 0, s, out, n, seed, stream, mean, std);
}
hipError_t launch_fill_cache(void *c, int64_t planes, int64_t cap, int64_t len, int hd, uint64_t seed, uint32_t stream,
                             float mean, float std, hipStream_t s) {
    const int64_t pairs = planes * len * hd / 2;
    if (pairs <= 0) return hipSuccess;
    return launch(k_fill_cache, grid1(pairs, 256), dim3(256), 0, s, static_cast<_Float16 *>(c), planes, cap, len, hd,
                       seed, stream, mean, std);
}

hipError_t launch_absmax(const float *x, int64_t n, uint32_t *out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    return launch(k_absmax, dim3(unsigned(std::min<int64_t>(1024, (n + 255) / 256))), dim3(256), 0, s, x, n, out);
}

hipError_t launch_check_split(uint64_t base, uint64_t pairs, unsigned long long *bad, hipStream_t s) {
    if (pairs == 0) return hipSuccess;
    if (pairs > (uint64_t(1) << 31)) return hipErrorInvalidValue;
    return launch(k_check_split, dim3(unsigned((pairs + 255) / 256)), dim3(256), 0, s, base, pairs, bad);
}

hipError_t launch_hold(double us, hipStream_t s) {
    static int khz = 0;  // the real-time counter's rate
    if (khz <= 0) {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
        if (e != hipSuccess) return e;
        if (khz <= 0) return hipErrorInvalidValue;
    }
    if (!(us > 0.0) || us > 1e5) return hipErrorInvalidValue;
    const uint64_t ticks = uint64_t(us * 1e-3 * double(khz));
    // 512 cycles per sleep at most 2.5 GHz: about 0.2 us, so the cap is 4x the hold at any clock
    const int max_iter = int(std::min(2e7, 4.0 * us / 0.2 + 64.0));
    return launch(k_hold, dim3(1), dim3(64), 0, s, ticks, max_iter);
}
hipError_t launch_copy16(const void *src, void *dst, int64_t bytes, hipStream_t s) {
    const int64_t n = bytes / 16;
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 256 * 16);
    return launch(k_copy16, dim3(unsigned(blocks)), dim3(256), 0, s, static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), n);
}

}  // namespace vh
