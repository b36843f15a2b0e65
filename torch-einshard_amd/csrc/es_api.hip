// Library-wide entry points of libeinshard_hip: version, per-thread error and
// kernel-variant reporting.
#include "es_common.h"

namespace es {

namespace {
thread_local std::string g_last_error;
thread_local const char* g_last_kernel = "";
}  // namespace

void set_error(const std::string& message) { g_last_error = message; }

void set_kernel(const char* name) { g_last_kernel = name; }

int fail(int status, const std::string& message) {
  g_last_error = message;
  return status;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(ES_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(err));
  }
  return ES_OK;
}

}  // namespace es

extern "C" {

int es_abi_version(void) { return ES_ABI_VERSION; }

const char* es_version(void) { return "einshard_hip 0.1.0 (gfx950)"; }

const char* es_last_error(void) { return es::g_last_error.c_str(); }

const char* es_last_kernel(void) { return es::g_last_kernel; }

}  // extern "C"
