// kore_hip_internal.hpp -- host-side helpers shared by the entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kore_hip.h"

namespace kore {

// Largest element count any entry point accepts: keeps every grid below
// 2^31 blocks and every byte offset far from 64-bit overflow.
constexpr uint64_t kMaxElements = 1ull << 46;

// Status of the launch just enqueued: 0, or the hipError_t it raised.
// hipGetLastError also clears a sticky launch error so it is reported once.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? KORE_HIP_OK : (int)e;
}

// a*b without 64-bit wrap-around; false on overflow.
inline bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
    if (a != 0 && b > UINT64_MAX / a) return false;
    *out = a * b;
    return true;
}

}  // namespace kore
