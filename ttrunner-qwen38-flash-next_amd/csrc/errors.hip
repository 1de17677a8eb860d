// Thread-local error reporting and version of the qwen4mix C ABI.
#include <stdio.h>
#include <string.h>

#include "qwen4mix_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

int qm_fail(int code, const char* msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg ? msg : "unknown error");
  return code;
}

extern "C" const char* qm_last_error(void) { return g_last_error; }

extern "C" int qm_version(void) { return 1; }
