// Error plumbing and version entry points of the C ABI.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "oc_common.h"

namespace oc {

static thread_local char g_msg[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  return set_error(OC_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// Plan knobs: the launch plans are fixed functions of the shape and the device; a
// test (or a tuning script) may pin one choice through oc_set_plan_override.  The
// table is read on every call only while some override is set.
static const char* const kKnobNames[] = {
    "OC_SKINNY_NT",      "OC_SKINNY_S",    "OC_GEMV_NT",         "OC_GEMV_W",     "OC_GEMV_DEEP",
    "OC_GEMV_S",         "OC_GEMV_STREAM", "OC_GEMV_STREAM_KS",  "OC_GEMV_STREAM_D",
    "OC_GEMV_STREAM_BAL", "OC_GEMM_STREAM", "OC_GEMM_MT",        "OC_GEMM_MIN_M", "OC_GEMM_SPLIT",
    "OC_GROUP_NT",       "OC_MOE_RM",      "OC_MOE_W2",          "OC_MOE_GEMM",   "OC_MOE_GEMM_MT",
    "OC_SIGN_W",         "OC_SIGN_GEMM_MIN_M", "OC_HAD_MM_M",    "OC_SIGN_PLAN",  "OC_GEMM_PLAN",
    "OC_GEMM_STREAM_S", "OC_GEMM_STREAM_NTW", "OC_GEMM_STREAM_MZ", "OC_SIGN_STREAM", "OC_SIGN_STREAM_S", "OC_SIGN_STREAM_MZ"};
constexpr int kKnobs = (int)(sizeof(kKnobNames) / sizeof(kKnobNames[0]));
static int g_knob_val[kKnobs];
static bool g_knob_set[kKnobs];
static std::atomic<int> g_knobs_on{0};
static std::atomic<int> g_knob_gen{0};

int knob(const char* name, int dflt) {
  if (g_knobs_on.load(std::memory_order_relaxed) == 0) return dflt;
  for (int i = 0; i < kKnobs; ++i)
    if (g_knob_set[i] && strcmp(kKnobNames[i], name) == 0) return g_knob_val[i];
  return dflt;
}

}  // namespace oc

extern "C" int oc_set_plan_override(const char* name, int value) {
  OC_REQUIRE(name, OC_ERR_INVALID, "null knob name");
  for (int i = 0; i < oc::kKnobs; ++i)
    if (strcmp(oc::kKnobNames[i], name) == 0) {
      oc::g_knob_val[i] = value;
      if (!oc::g_knob_set[i]) {
        oc::g_knob_set[i] = true;
        oc::g_knobs_on.fetch_add(1);
      }
      oc::g_knob_gen.fetch_add(1);
      return 0;
    }
  return oc::set_error(OC_ERR_INVALID, "unknown plan knob %s", name);
}

extern "C" void oc_clear_plan_overrides(void) {
  for (int i = 0; i < oc::kKnobs; ++i) oc::g_knob_set[i] = false;
  oc::g_knobs_on.store(0);
  oc::g_knob_gen.fetch_add(1);
}

extern "C" int oc_plan_generation(void) { return oc::g_knob_gen.load(); }

extern "C" int oc_abi_version(void) { return OC_ABI_VERSION; }

extern "C" const char* oc_last_error(void) { return oc::g_msg; }
