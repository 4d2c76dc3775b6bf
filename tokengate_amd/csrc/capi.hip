// Library-wide C entry points: ABI stamp and the thread-local error string.
#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {
thread_local char g_err[1024] = {0};
}
int set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return 1;
}
void clear_error() { g_err[0] = 0; }
const char *last_error() { return g_err; }
}  // namespace tg

extern "C" int tg_abi_version(void) { return 2; }
extern "C" const char *tg_last_error(void) { return tg::last_error(); }
