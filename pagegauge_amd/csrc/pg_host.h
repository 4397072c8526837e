// Host-side definitions shared by every source of the library: the decode
// shapes and the error reporting of the C ABI.  Plain C++ (no HIP), so the
// host-only parts (the planner) also build with a host compiler.
#pragma once

#include <stdint.h>

#include <exception>
#include <new>
#include <string>

#include "pagegauge_hip.h"

namespace pg {

constexpr int kHeadDim = 128;
constexpr int kPageSize = 16;
constexpr int kWave = 64;
constexpr int kGqa = 4;  // query heads per KV head handled by the decode kernels

// Records the message of a failing call for pg_last_error().
void set_error(const std::string& message);
void clear_error();

inline int32_t fail(int32_t code, const std::string& message) {
  set_error(message);
  return code;
}

// Runs ``body`` (returning a PG_* code) so that no C++ exception unwinds
// through the C ABI: a host allocation failure (an absurd batch size, say)
// becomes an error code with its message.
template <typename Body>
int32_t guarded(Body&& body) {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    return fail(PG_ERROR_UNSUPPORTED, "out of host memory while planning");
  } catch (const std::exception& e) {
    return fail(PG_ERROR_INVALID_ARGUMENT, e.what());
  }
}

}  // namespace pg
