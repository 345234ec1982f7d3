// api.hip — library-wide entry points: error reporting and build identification.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace geo {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

}  // namespace geo

#ifndef GEO_BUILD_FLAGS
#define GEO_BUILD_FLAGS "unknown"
#endif

extern "C" const char* geo_last_error(void) { return geo::g_last_error.c_str(); }

extern "C" const char* geo_build_info(void) {
  return "libgeoembodied_hip: target gfx950 (wave64), clang " __clang_version__
         ", flags: " GEO_BUILD_FLAGS;
}

extern "C" int geo_abi_version(void) { return 2; }
