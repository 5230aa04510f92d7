// energy.cpp -- the GPU's own energy counter, for the placement adapter's
// calibration loop (rce-placement-adapter/src/lib.rs L48-74 `EnergyMeter`;
// its Linux meter reads RAPL, substrate_meter.rs L60-130).  The counter is
// the device's accumulated energy as ROCm SMI reports it
// (rsmi_dev_energy_count_get: a count and its resolution in microjoules).
// librocm_smi64 is opened at first use with dlopen, so the library has no
// link-time dependency on it and reports "not found" where it is absent.
#include "abi_internal.h"

#include <dlfcn.h>

#include <mutex>

using namespace rce_qmm_abi;

namespace {

typedef int (*rsmi_init_fn)(uint64_t);
typedef int (*rsmi_energy_fn)(uint32_t, uint64_t *, float *, uint64_t *);

struct Smi {
    std::once_flag once;
    rsmi_energy_fn energy = nullptr;
    std::string why;
};
Smi g_smi;

void smi_open() {
    void *h = dlopen("librocm_smi64.so.1", RTLD_NOW | RTLD_LOCAL);
    if (!h) h = dlopen("librocm_smi64.so", RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        g_smi.why = "librocm_smi64 is not available";
        return;
    }
    auto init = reinterpret_cast<rsmi_init_fn>(dlsym(h, "rsmi_init"));
    auto energy = reinterpret_cast<rsmi_energy_fn>(dlsym(h, "rsmi_dev_energy_count_get"));
    if (!init || !energy) {
        g_smi.why = "librocm_smi64 lacks rsmi_init / rsmi_dev_energy_count_get";
        return;
    }
    const int st = init(0);
    if (st != 0) {
        g_smi.why = "rsmi_init failed with status " + std::to_string(st);
        return;
    }
    g_smi.energy = energy;
}

}  // namespace

extern "C" {

// The accumulated energy of GPU `device` (ROCm SMI's index, which is the HIP
// index on a single-GPU node) in microjoules, and the reading's timestamp in
// ns.  RCE_QMM_NOT_FOUND when no counter can be read here.
rce_qmm_status rce_qmm_energy_read(int device, uint64_t *microjoules, uint64_t *timestamp_ns) {
    if (!microjoules) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (device < 0) return fail(RCE_QMM_BAD_SHAPE, "negative device index");
    std::call_once(g_smi.once, smi_open);
    if (!g_smi.energy) return fail(RCE_QMM_NOT_FOUND, g_smi.why);
    uint64_t count = 0, ts = 0;
    float res = 0.0f;
    const int st = g_smi.energy((uint32_t)device, &count, &res, &ts);
    if (st != 0 || !(res > 0.0f))
        return fail(RCE_QMM_NOT_FOUND, "rsmi_dev_energy_count_get: status " + std::to_string(st));
    *microjoules = (uint64_t)((double)count * (double)res);
    if (timestamp_ns) *timestamp_ns = ts;
    return RCE_QMM_OK;
}

}  // extern "C"
