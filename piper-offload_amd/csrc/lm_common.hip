// lm_common.hip -- ABI version, error reporting, workspace sizing, factor prep.
#include "lm_impl.h"

static thread_local std::string g_err;

int lm_fail_v(int code, const char* fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof buf, fmt, ap);
  g_err = buf;
  return code;
}

extern "C" int lm_version(void) { return LM_ABI_VERSION; }
extern "C" const char* lm_last_error(void) { return g_err.c_str(); }
extern "C" size_t lm_workspace_size(int64_t M, int64_t N, int32_t rank) { return ws_layout(M, N, rank).total; }

int launch_prep(const PrepItem& it, hipStream_t st) {
  int64_t total = prep_units(it);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_prep1, dim3((unsigned)blocks), dim3(256), 0, st, it, total);
  LAUNCH_CHECK();
  return LM_OK;
}

