// Status plumbing of the C ABI: a thread-local last-error message.
#include "status.hpp"

#include <cstdarg>
#include <cstdio>
#include <string>

namespace gptq {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

}  // namespace gptq

extern "C" const char* gptq_last_error(void) { return gptq::g_last_error.c_str(); }
extern "C" int gptq_abi_version(void) { return 1; }
