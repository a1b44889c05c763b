// Library-level entry points of the C ABI: version, status strings and the
// tuning configuration read from the environment.
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"

namespace hrm {
namespace {

// Whole-string base-10 integer; false for empty, trailing text or overflow.
bool parse_int(const char* s, long long* out) {
  while (*s == ' ' || *s == '\t') ++s;
  if (!*s) return false;
  char* end = nullptr;
  errno = 0;
  const long long v = strtoll(s, &end, 10);
  if (errno != 0 || end == s) return false;
  while (*end == ' ' || *end == '\t' || *end == '\n') ++end;
  if (*end) return false;
  *out = v;
  return true;
}

Config g_config;
bool g_loaded = false;

// The CU margin: the first of the three names that is set and non-empty.  A
// value that is not a non-negative integer is rejected (the reference raises
// ValueError for it, models/moe_triton_grouped_gemm.py:33-47).
bool read_margin(int* out) {
  for (const char* name : {"HRM_MOE_HIP_CU_MARGIN", "HRM_MOE_TRITON_SM_MARGIN", "XTUNER_SM_MARGIN"}) {
    const char* s = getenv(name);
    if (!s || !*s) continue;
    long long v = 0;
    if (!parse_int(s, &v) || v < 0 || v > (1 << 20)) {
      fprintf(stderr, "hrm_moe: %s must be a non-negative integer, got '%s'; using 0\n", name, s);
      return false;
    }
    *out = (int)v;
    return true;
  }
  *out = 0;
  return true;
}

}  // namespace

int reload_config() {
  Config c;
  bool ok = read_margin(&c.cu_margin);
  if (const char* s = getenv("HRM_MOE_GEMM_CFG"); s && *s) {
    int bm = 0, bn = 0, st = 0, nw = 4, bk = 64;
    const int n = sscanf(s, "%dx%dx%dx%dx%d", &bm, &bn, &st, &nw, &bk);
    if (n >= 3) {
      c.gemm_bm = bm; c.gemm_bn = bn; c.gemm_stages = st; c.gemm_waves = nw; c.gemm_bk = bk;
    } else {
      ok = false;
    }
  }
  if (const char* s = getenv("HRM_MOE_SKINNY"); s && *s) c.skinny = s[0] == '1' ? 1 : (s[0] == '0' ? 0 : -1);
  if (const char* s = getenv("HRM_MOE_WGRAD_STAGES"); s && *s) {
    long long v = 0;
    if (parse_int(s, &v) && (v == 2 || v == 3)) c.wgrad_stages = (int)v;
    else ok = false;
  }
  if (const char* s = getenv("HRM_MOE_GATE_SPLIT_ROWS"); s && *s) {
    long long v = 0;
    if (parse_int(s, &v) && v > 0) c.gate_split_rows = v < 64 ? 64 : v;
    else ok = false;
  }
  if (const char* s = getenv("HRM_MOE_WAVE_ROUTER"); s && *s) c.wave_router = s[0] != '0';
  g_config = c;
  g_loaded = true;
  return ok ? HRM_MOE_OK : HRM_MOE_ERR_INVALID;
}

const Config& config() {
  if (!g_loaded) reload_config();
  return g_config;
}

}  // namespace hrm

extern "C" int hrm_moe_reload_config(void) { return hrm::reload_config(); }

extern "C" int hrm_moe_cu_margin(void) { return hrm::config().cu_margin; }

extern "C" int hrm_moe_abi_version(void) { return HRM_MOE_ABI_VERSION; }

extern "C" const char* hrm_moe_status_string(int status) {
  switch (status) {
    case HRM_MOE_OK: return "ok";
    case HRM_MOE_ERR_INVALID: return "invalid argument (null pointer, negative or inconsistent size)";
    case HRM_MOE_ERR_DTYPE: return "dtype not supported by this entry point";
    case HRM_MOE_ERR_UNSUPPORTED: return "shape outside the kernel limits";
    case HRM_MOE_ERR_WORKSPACE: return "workspace missing or too small";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}
