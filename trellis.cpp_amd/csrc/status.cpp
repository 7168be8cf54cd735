// Error state of the C ABI: a thread-local message per calling thread.
#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace tsp {
namespace {
thread_local char g_msg[1024] = "";
}
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
}
void clear_error() { g_msg[0] = '\0'; }
}  // namespace tsp

extern "C" const char* tsp_last_error(void) { return tsp::g_msg; }
extern "C" int tsp_version(void) { return 100; }
