// resident.h — the resident int8 / int4 weight objects shared by resident.cpp (packing and
// the products) and weights_io.cpp (their serialised form).
#pragma once

#include <stddef.h>

#include "ops.h"
#include "rocket_matmul.h"

// One HIP handle per context; one HBM buffer per weight: int8 rows [N][K] as given, or
// int4 nibble-packed [N][K/2] (the I4P layout). M is the row count the weight was packed
// for (the layout does not depend on it).
struct rocket_i8_ctx      { int fd; int nthreads; };
struct rocket_i8_weights  { int M, K, N, group; void *dev; size_t bytes; };
struct rocket_i4_ctx      { int fd; int nthreads; };
struct rocket_i4_weights  { int M, K, N, group; void *dev; size_t bytes; };

namespace rk {
// Copies `bytes` from host or device memory into a new HBM buffer (blocking).
void *upload(int fd, const void *src, size_t bytes, const char *who);
// Frees a resident buffer once nothing queued on the handle can still read it.
void release(int fd, void *dev);
}  // namespace rk
