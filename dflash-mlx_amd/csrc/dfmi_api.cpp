// Library-wide C-ABI entry points: version and thread-local error message.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "dfmi_host.h"

namespace dfmi {

static thread_local std::string g_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error.assign(buf);
}

}  // namespace dfmi

extern "C" const char* dfmi_version(void) { return "dfmi 0.1.0 gfx950"; }

extern "C" const char* dfmi_last_error(void) { return dfmi::g_error.c_str(); }
