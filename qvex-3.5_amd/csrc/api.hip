// Library-wide C ABI plumbing: thread-local error text and the ABI version.
#include "qvex_common.h"

#include <string.h>

namespace qvex {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace qvex

extern "C" const char* qvex_last_error(void) { return qvex::g_err; }

extern "C" int qvex_abi_version(void) { return 8; }
