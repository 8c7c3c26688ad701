// abi.cpp -- host-only entry points of libkore_hip.so: version, status text
// and the RoPE inverse-frequency table.
#include <math.h>

#include "kore_hip.h"

extern "C" int kore_hip_version(void) { return 100; }  // 0.1.0

extern "C" const char* kore_hip_status_string(int status) {
    switch (status) {
        case KORE_HIP_OK: return "ok";
        case KORE_HIP_ERR_NULL_PTR: return "null pointer argument";
        case KORE_HIP_ERR_BAD_DIM: return "invalid dimension";
        case KORE_HIP_ERR_OVERFLOW: return "element count overflows the supported range";
        case KORE_HIP_ERR_ALIAS: return "overlapping buffers";
        case KORE_HIP_ERR_SCRATCH: return "work exceeds the library's fixed scratch array";
        default: return status > 0 ? "HIP runtime error (hipError_t)" : "unknown status";
    }
}

// crates/kore-serve/src/layered/engine.rs:694-700:
//   1.0 / base.powf(2.0 * i as f32 / head_dim as f32)
// Evaluated on the host with the C library's powf (what Rust's f32::powf
// calls on linux-gnu) so the table is the reference's, bit for bit; the
// device only multiplies it by the position.
extern "C" int kore_hip_rope_inv_freq_f32(float* inv_freq_host, uint32_t head_dim, float base) {
    if (head_dim == 0) return KORE_HIP_OK;
    if (!inv_freq_host) return KORE_HIP_ERR_NULL_PTR;
    if (head_dim & 1u) return KORE_HIP_ERR_BAD_DIM;
    const uint32_t half = head_dim / 2;
    for (uint32_t i = 0; i < half; ++i) {
        volatile float e = (2.0f * (float)i) / (float)head_dim;
        inv_freq_host[i] = 1.0f / powf(base, e);
    }
    return KORE_HIP_OK;
}
