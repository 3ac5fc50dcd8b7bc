// Status and the thread-local error message shared by every C ABI source file of the library
// (SA_OK / SA_ERR_* from supra_attn.h; sa_last_error() returns the message).
#pragma once

#include <hip/hip_runtime.h>

namespace sa {

// Records the formatted message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns SA_OK.
int ok();
// SA_ERR_HIP with "<what>: <runtime message> (<code>)".
int hip_fail(hipError_t e, const char* what);
// The message buffer itself (sizeof = kErrorBytes), for callers that must keep it across a call.
const char* last_error();
constexpr int kErrorBytes = 512;

}  // namespace sa
