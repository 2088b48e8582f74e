// Error reporting and shared argument checks for the C ABI.
#include "api.hpp"

#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

static thread_local char g_err[512] = "";

void stk_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int stk_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    stk_set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return STK_EHIP;
  }
  return STK_OK;
}

StkCheck stk_check_kv(int dtype, int hq, int hkv, int n, int b, int d) {
  if (dtype < stk::DT_F32 || dtype > stk::DT_BF16) return {false, "unsupported element dtype"};
  if (hq < 0 || hkv <= 0 || n <= 0 || b <= 0 || d <= 0) return {false, "expected nonempty shapes"};
  if (hq % hkv != 0) return {false, "Hq must be divisible by Hkv"};
  if (d > 1024) return {false, "head dimension above 1024 is not supported"};
  return {true, ""};
}

extern "C" {

STK_API const char* stk_last_error(void) { return g_err; }

STK_API int stk_abi_version(void) { return 1; }

}  // extern "C"
