// abi.cpp — error reporting and version of the C ABI (include/flagsparse_hip.h).
#include <hip/hip_runtime.h>

#include <string>

#include "fs_common.hpp"

namespace fs {

namespace {
thread_local std::string g_last_error;
thread_local const char* g_last_kernel = "";
}

void note_kernel(const char* name) { g_last_kernel = name; }

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return FS_OK;
  // clear the runtime's last-error state too: a failed API call must not be
  // reported again by the caller's next, unrelated launch check
  (void)hipGetLastError();
  return fail(FS_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool valid_types(int val_t, int idx_t, int ptr_t) {
  return val_t >= FS_F32 && val_t <= FS_C128 && (idx_t == FS_I32 || idx_t == FS_I64) &&
         (ptr_t == FS_I32 || ptr_t == FS_I64);
}

}  // namespace fs

extern "C" const char* fs_last_error(void) { return fs::g_last_error.c_str(); }

extern "C" const char* fs_last_kernel(void) { return fs::g_last_kernel; }

extern "C" const char* fs_version(void) { return "flagsparse_hip 0.1.0 (gfx950)"; }
