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

// The process's workspace error word: pinned host memory that a decode or Q4L
// kernel sets to 1 when an arrival count in a workspace header exceeds the
// number of workgroups that share it (a header that was not zero before its
// first use).  Allocated on first use outside stream capture; nullptr while it
// does not exist (a capturing stream, or allocate == false).
uint32_t* ws_error_word(void* stream, bool allocate);
// Reads and clears the word (after a stream synchronization): 1 if set.
int take_ws_error();
float f16_bits_to_f32(uint16_t h);
// Writes val[j] to dst_dev[idx[j]] for j < n (n <= LNSKV_TABLE_PATCH_MAX) with
// one small kernel whose arguments carry the pairs; async on stream.
int table_patch(uint32_t* dst_dev, int n, const uint32_t* idx, const uint32_t* val, void* stream);

}  // namespace lnskv
