// Library-wide C ABI pieces: error message storage and version.
#include <cstdarg>

#include "common.hpp"

namespace atlas {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace atlas

extern "C" const char* atlas_last_error(void) { return atlas::g_last_error; }

extern "C" int atlas_abi_version(void) { return 18; }
