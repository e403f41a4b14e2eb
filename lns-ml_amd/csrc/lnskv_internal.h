// Internal helpers shared by the host and device translation units of liblnskv.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <string>

#include "lnskv.h"

namespace lnskv {

// Records `fmt` as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline size_t dtype_bytes(int32_t dtype) {
  return dtype == LNSKV_DTYPE_F32 ? 4 : dtype == LNSKV_DTYPE_F16 ? 2 : 1;
}

// Checks the geometry of a page descriptor (not its pointers).
int check_geometry(const lnskv_pages* c);
// Checks geometry and that the pools (and Q8A scales) are non-null.
int check_pages(const lnskv_pages* c);
uint16_t f32_to_f16_bits(float f);
float f16_bits_to_f32(uint16_t h);

}  // namespace lnskv
