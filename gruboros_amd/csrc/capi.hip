// Library-wide entry points: version and per-thread error text.
#include "mg_common.h"

namespace mg {
char* last_error_buf() {
  static thread_local char buf[512] = {0};
  return buf;
}
}  // namespace mg

extern "C" int mg_version(void) { return 206; }  // 0.2.6

extern "C" const char* mg_last_error(void) { return mg::last_error_buf(); }
