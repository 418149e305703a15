// tsk_runtime.h — error reporting and the per-device workspace of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace tsk {

// record a message for tsk_last_error() and return status
int fail(int status, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);
// TSK_OK if tsk_init() was called
int require_init();
// device scratch of at least `bytes`, owned by the library (one per device and
// slot: slot 0 serves single operators, slot 1 the composite entry points that
// call them); growing it synchronises the device
int workspace(size_t bytes, void **out, int slot = 0);

}  // namespace tsk
