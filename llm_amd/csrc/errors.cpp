// The thread's last error (errors.h).
#include "errors.h"

#include <cstdarg>
#include <cstdio>
#include <string>

namespace llmhip {

static thread_local std::string g_err;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

void clear_error() { g_err.clear(); }

const char* last_error() { return g_err.c_str(); }

}  // namespace llmhip

extern "C" const char* llmhip_last_error(void) { return llmhip::last_error(); }
