// Thread-local error message of the C ABI.
#include "status.h"

#include <string.h>

namespace d3 {

namespace {
thread_local char g_message[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, args);
  va_end(args);
  return code;
}

void clear_error() { g_message[0] = '\0'; }

}  // namespace d3

extern "C" int d3_abi_version(void) { return 12; }

extern "C" const char* d3_last_error(void) { return d3::g_message; }
