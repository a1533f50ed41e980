// btl_host.hpp -- host helpers shared by the C-ABI sources (btl_api.cpp,
// btl_model_api.cpp).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>

namespace btl {
namespace host {
// Sets the calling thread's btl_last_error() message; returns `code`.
int fail_msg(int code, const char* msg);
// BTL_ERR_HIP with the HIP error string.
int hip_error(hipError_t e, const char* what);
// The current HIP device, probed once (gfx950 only).
int device(int* dev);
// The caller's workspace when ws != NULL (checked against `need`), else the
// library's per-device workspace grown to `need` bytes.
int workspace(int dev, void* ws, size_t ws_bytes, size_t need, void** out, hipStream_t st);
}  // namespace host
}  // namespace btl
