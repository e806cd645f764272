// origami_internal.h -- helpers shared by the HIP sources of
// liborigami_layout.so (not part of the public C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <string>

#include "origami_layout.h"

namespace origami_internal {

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const std::string& msg);

// ORIGAMI_ERR_HIP with the launch error of the last kernel, or ORIGAMI_OK.
int check_launch(const char* what);

// Row strides of a paged cache, in rows of H * D elements:
// [2, NB, bs, H, D] -> blk_stride = bs, half_stride = NB * bs;
// [NB, 2, bs, H, D] -> blk_stride = 2 * bs, half_stride = bs.
int cache_geometry(int64_t cache_layout, int64_t num_blocks, int64_t block_size,
                   int64_t* blk_stride, int64_t* half_stride);

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

inline unsigned grid_for(int64_t work, int64_t per_block, int64_t cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g);
}

}  // namespace origami_internal

#define ORIGAMI_REQUIRE(cond, msg)                                              \
  do {                                                                          \
    if (!(cond)) return ::origami_internal::fail(ORIGAMI_ERR_INVALID, msg);     \
  } while (0)
