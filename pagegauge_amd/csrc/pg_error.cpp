// Thread-local error text for the C ABI (pg_last_error).
#include <string>

#include "pg_host.h"

namespace pg {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }
void clear_error() { g_last_error.clear(); }

}  // namespace pg

extern "C" const char* pg_last_error(void) { return pg::g_last_error.c_str(); }

extern "C" int32_t pg_abi_version(void) { return 4; }
