// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/dfmi.h"

namespace dfmi {

// Thread-local error message (dfmi_last_error).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return DFMI_ELAUNCH;
  }
  return DFMI_OK;
}

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Shapes the streaming main loop takes (int4 or 8-bit): M <= 32, whole 256-k steps and
// scale blocks of 8 groups; buffer offsets are 32-bit and the record count a
// signed int, so the packed weights stay under 2 GiB.
inline bool stream_eligible(int64_t M, int64_t K, int64_t N, int gs, int bits = 4) {
  return M <= 32 && K % 256 == 0 && K % (8 * gs) == 0 && K < (1ll << 24) &&
         N * (K / 8 * bits) < (1ll << 31);
}

}  // namespace dfmi

// 8-bit affine qmm launch (dfmi_qmm8.hip), called by dfmi_qmm_affine_ex after
// its argument checks.
int dfmi_qmm8_launch(const void* x, int x_dtype, const uint32_t* w_q, const void* scales,
                     const void* biases, void* y, int64_t M, int64_t K, int64_t N, int gs,
                     void* stream);
