// C-ABI bookkeeping shared by every entry point: thread-local error text and
// the ABI version query.
#include "fd_common.h"

namespace fd {

std::string& last_error_slot() {
  static thread_local std::string slot;
  return slot;
}

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error_slot() = buf;
  return code;
}

}  // namespace fd

extern "C" const char* fd_last_error(void) { return fd::last_error_slot().c_str(); }

extern "C" int fd_abi_version(void) { return FD_ABI_VERSION; }
