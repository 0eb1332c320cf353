// Error reporting and version of the e2v2 C ABI.
#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {
static thread_local char g_error[1024] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code == 0 ? -1 : code;
}
}  // namespace e2v2

E2V2_API const char* e2v2_last_error(void) { return e2v2::g_error; }
E2V2_API int e2v2_version(void) { return 1; }
