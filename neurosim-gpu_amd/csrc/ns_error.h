// Thread-local error text of the C ABI (plain C++, shared by the HIP entry
// points and the host-side planners).
#pragma once

#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "neurosim_hip.h"

namespace ns {

char* error_buffer();

inline void clear_error() { error_buffer()[0] = '\0'; }

__attribute__((format(printf, 1, 2))) inline int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return NS_ERR_INVALID;
}

}  // namespace ns
