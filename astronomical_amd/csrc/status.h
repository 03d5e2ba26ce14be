// The C ABI's status reporting, shared by its source files: the message goes to the
// thread-local last error (astro_moe_last_error) as "<op>: <message>".
#pragma once

#include <cstdarg>

namespace astro {

int report(int status, const char *op, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int vreport(int status, const char *op, const char *fmt, va_list ap);
int report_ok();

}  // namespace astro
