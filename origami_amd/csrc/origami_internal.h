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

// ---------------------------------------------------------------------------
// Device helpers shared by the row kernels
// ---------------------------------------------------------------------------

// The dword at byte offset `byte` (a multiple of 4) of a 4-byte aligned
// buffer of `nbytes` readable bytes; bytes at or past nbytes read as 0.  A
// dword is read only when it holds at least one readable byte, so the read
// never leaves the pages the buffer occupies; its unreadable bytes are masked.
__device__ __forceinline__ uint32_t load_dword_guarded(const uint8_t* base, int64_t byte,
                                                       int64_t nbytes) {
  const int64_t avail = nbytes - byte;
  if (avail <= 0) return 0;
  const uint32_t w = *reinterpret_cast<const uint32_t*>(base + byte);
  return avail >= 4 ? w : (w & ((1u << (8 * avail)) - 1u));
}

// Spreads 16 b-bit symbols packed LSB-first in u[] into 16 bytes
// (byte j of the result, dword j / 4, is symbol j).
template <int BITS>
__device__ __forceinline__ void expand16(const uint32_t* u, uint32_t (&out)[4]) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = u[i];
  } else {
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int bp = j * BITS;
      const int dw = bp >> 5, off = bp & 31;
      uint32_t s = u[dw] >> off;
      if (off + BITS > 32) s |= u[dw + 1] << (32 - off);
      out[j >> 2] |= (s & mask) << (8 * (j & 3));
    }
  }
}

}  // namespace origami_internal

#define ORIGAMI_REQUIRE(cond, msg)                                              \
  do {                                                                          \
    if (!(cond)) return ::origami_internal::fail(ORIGAMI_ERR_INVALID, msg);     \
  } while (0)
