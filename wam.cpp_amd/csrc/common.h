// Internal helpers shared by the host code and the HIP kernels of libwamx.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <string>

#include "wamx/wamx.h"

namespace wamx {

// Thread-local last error, surfaced through wamx_last_error().
void set_error(const std::string & msg);
void set_errorf(const char * fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define WAMX_HIP_TRY(expr)                                                          \
    do {                                                                            \
        hipError_t err__ = (expr);                                                  \
        if (err__ != hipSuccess) {                                                  \
            ::wamx::set_errorf("%s:%d: %s failed: %s", __FILE__, __LINE__, #expr,   \
                               hipGetErrorString(err__));                           \
            return WAMX_STATUS_FAILED;                                              \
        }                                                                           \
    } while (0)

#define WAMX_REQUIRE(cond, ...)                                                     \
    do {                                                                            \
        if (!(cond)) {                                                              \
            ::wamx::set_errorf(__VA_ARGS__);                                        \
            return WAMX_STATUS_FAILED;                                              \
        }                                                                           \
    } while (0)

// bf16 <-> f32 on the host: round-to-nearest-even with NaN kept quiet, the
// conversion ggml_fp32_to_bf16 performs.
static inline uint16_t f32_to_bf16_host(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32_host(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

}  // namespace wamx
