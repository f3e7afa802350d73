// hawk_internal.h — helpers shared by hawk_core.cpp and hawk_team.hip
// (not part of the C-ABI).
#ifndef HAWK_INTERNAL_H
#define HAWK_INTERNAL_H

#include <hip/hip_runtime.h>
#include <string>

namespace hawk_internal {
// Record `text` as this thread's hk_last_error() and return `code`.
int set_error(int code, const std::string& text);
// Record a failed HIP call (name and HIP's own error text) as HK_EHIP.
int set_hip_error(const char* what, hipError_t err);
}  // namespace hawk_internal

#endif
