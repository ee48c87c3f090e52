// Error state of the C ABI (include/fragpack_hip.h).
#include <string.h>

#include "../../include/fragpack_hip.h"
#include "fp_capi_internal.hpp"

namespace fp {
namespace {
thread_local char g_error[512] = "";
}  // namespace

void set_error(const char* msg) {
  strncpy(g_error, msg ? msg : "unknown error", sizeof(g_error) - 1);
  g_error[sizeof(g_error) - 1] = '\0';
}
}  // namespace fp

extern "C" const char* fp_last_error(void) { return fp::g_error; }

extern "C" int fp_abi_version(void) { return 1; }
