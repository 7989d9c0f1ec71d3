// C-ABI error state and version query.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace sgl {

static thread_local char g_last_error[1024] = {0};

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

}  // namespace sgl

extern "C" int sgl_abi_version(void) { return SGL_ABI_VERSION; }

extern "C" const char *sgl_last_error(void) { return sgl::g_last_error; }
