// C-ABI bookkeeping shared by every entry point: thread-local error text, the
// opt-in launch record and the ABI version query.
#include <cxxabi.h>

#include <atomic>
#include <cstdlib>
#include <utility>

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

namespace {
std::atomic<bool> g_record_launches{false};

std::string& launch_record_slot() {
  static thread_local std::string slot;
  return slot;
}
}  // namespace

bool launch_record_on() { return g_record_launches.load(std::memory_order_relaxed); }

void clear_launch_record() {
  if (launch_record_on()) launch_record_slot().clear();
}

// The kernel's demangled name without its parameter list, e.g.
// "fd::decode_mfma_kernel<__bf16, 32, 0, false, 32, true, 128, 1>".
void record_launch(const void* kernel, hipStream_t stream) {
  const char* mangled = hipKernelNameRefByPtr(kernel, stream);
  std::string name = mangled ? mangled : "?";
  // the host demangler may predate the __bf16 / _Float16 manglings (DF16b,
  // DF16_): spell them as vendor types, which it prints by name
  std::string spelled = name;
  for (const auto& [from, to] : {std::pair<std::string, std::string>{"DF16b", "u6__bf16"}, {"DF16_", "u8_Float16"}})
    for (size_t at = spelled.find(from); at != std::string::npos; at = spelled.find(from, at + to.size()))
      spelled.replace(at, from.size(), to);
  int status = 0;
  char* demangled = abi::__cxa_demangle(spelled.c_str(), nullptr, nullptr, &status);
  if (status == 0 && demangled) {
    name = demangled;
    const size_t paren = name.rfind('(');
    if (paren != std::string::npos) name.resize(paren);
    if (name.compare(0, 5, "void ") == 0) name.erase(0, 5);
  }
  std::free(demangled);
  std::string& slot = launch_record_slot();
  if (!slot.empty()) slot += ';';
  slot += name;
}

}  // namespace fd

extern "C" void fd_record_launches(int on) { fd::g_record_launches.store(on != 0, std::memory_order_relaxed); }

extern "C" const char* fd_last_launch(void) { return fd::launch_record_slot().c_str(); }

extern "C" const char* fd_last_error(void) { return fd::last_error_slot().c_str(); }

extern "C" int fd_abi_version(void) { return FD_ABI_VERSION; }
