// The library's one error channel: every C-ABI call that fails stores a
// message that mhsa_last_error() returns (thread-local).
#pragma once

#include <stdint.h>

namespace mhsa {
// Store `msg` as the calling thread's last error and return `code`.
int32_t set_error(int32_t code, const char* msg);
}  // namespace mhsa
