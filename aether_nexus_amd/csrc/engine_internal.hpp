// engine_internal.hpp — what the library's other sources (ops.hip) use of an
// aw_engine, whose definition stays private to weaver_engine.hip.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/aether_weaver.h"

namespace aw_engine_internal {

// Bits of the engine's device error word (aw_engine_check_device_errors):
// 1 hot block ref, 2 cold block ref, 4 atom index (weaver_kernels.hpp), 8 token id.
constexpr uint32_t kErrTokenBit = 8u;

int device(const aw_engine* e);        // HIP device ordinal
uint32_t compute_units(const aw_engine* e);
uint32_t* error_word(const aw_engine* e); // device address of the error word
// Records the message as the engine's last error and returns `code`.
int fail(aw_engine* e, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

// Lets the dense-ops kernels that stage more than 64 KiB of LDS use `max_lds`
// bytes (ops.hip); false when the runtime refuses.
bool ops_set_lds_limits(size_t max_lds);

} // namespace aw_engine_internal
