// The C ABI's status reporting: one thread-local last error per calling thread, set by every
// entry point ("<op>: <message>" on failure, empty on success) and read back through
// astro_moe_last_error.  Host code only.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/astro_moe.h"
#include "status.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

int astro::vreport(int status, const char *op, const char *fmt, va_list ap) {
  char buf[768];
  vsnprintf(buf, sizeof buf, fmt, ap);
  g_last_error = std::string(op) + ": " + buf;
  return status;
}

int astro::report(int status, const char *op, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = vreport(status, op, fmt, ap);
  va_end(ap);
  return r;
}

int astro::report_ok() {
  g_last_error.clear();
  return ASTRO_MOE_OK;
}

extern "C" const char *astro_moe_last_error(void) { return g_last_error.c_str(); }
