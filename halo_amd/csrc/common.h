// Internal helpers of the halo_mi355x library: status codes with a thread-local message.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/halo_mi355x.h"

namespace halo_mi {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// row_bytes for a quant or F32 type; 0 with *code set on error.
uint64_t row_bytes_checked(uint32_t type, uint32_t cols, int* code, const char* op);

}  // namespace halo_mi
