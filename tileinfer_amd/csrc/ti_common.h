// Shared host/device helpers of the gfx950 paged KV-cache library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tileinfer_amd.h"

namespace ti {

// Records a printf-style message as the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks the launch that was just enqueued; returns TI_OK or TI_ELAUNCH with the runtime's text.
int check_launch(const char* what);

// Number of compute units of the current device (cached per device id).
int device_cu_count();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// 4 x 32-bit registers: one 16-byte global access, or the 8 x 16-bit operand of a
// 16x16x32 MFMA.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

}  // namespace ti
