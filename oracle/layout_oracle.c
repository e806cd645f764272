/*
 * layout_oracle.c -- CPU restatement of Origami's canonical KV codec layout.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle that the HIP kernels of
 * origami_amd are checked against.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it, and only as the checker or as
 * the timed CPU baseline; the product path never calls it.
 *
 * Every function is a scalar restatement of the reference algorithm, written
 * for obviousness, not speed.  OpenMP is used only to spread independent
 * chunks / blocks over host cores for the CPU baseline timing; each thread
 * runs the same scalar code.
 *
 * Reference files (nothatDinger/origami):
 *   csrc/origami/bitpack_layout_cuda.cu   (cu)   -- decode, chunk order, index
 *   csrc/origami/bitpack_layout_cuda.cpp  (cpp)  -- validation, zero init
 *   vllm/.../origami/benchmark_utils.py   (bu)   -- paged scatter, tail pad
 *   vllm/.../origami/worker.py            (wk)   -- block gather for save
 *
 * Parity pinning (what checks each function; see tests/test_oracle_pinning.py):
 *   oracle_unpack_symbol      -- brute-force LSB-first bit list, KIVI 2/4-bit
 *                                packers, out-of-range window bytes read as 0
 *   oracle_unpack_canonical   -- bits 8: numpy transpose closed form; all bits:
 *                                bit-list brute force; uncovered bytes are 0
 *   oracle_pack_canonical     -- unique inverse: round trips both ways, KIVI
 *                                packers, zero pad bits, byte counts
 *   oracle_scatter_kv_cache   -- numpy fancy-index assignment (index_copy_)
 *   oracle_gather_kv_cache    -- numpy fancy-index read (index_select)
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OK 0
#define ORACLE_EINVAL -1

static char g_err[512];
static int g_threads = 1;

const char* oracle_last_error(void) { return g_err; }

void oracle_set_threads(int n) { g_threads = n > 0 ? n : 1; }

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static int fail(const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return ORACLE_EINVAL;
}

/* cu:70-89 (unpack_symbol): b == 8 reads the byte; otherwise a 16-bit
 * little-endian window at byte floor(i*b/8), bytes past the chunk read as 0,
 * shifted right by (i*b mod 8) and masked to b bits (LSB-first). */
uint8_t oracle_unpack_symbol(const uint8_t* src, int64_t src_bytes,
                             int64_t i, int bits) {
  if (bits == 8) return src[i];
  int64_t bit_pos = i * (int64_t)bits;
  int64_t k = bit_pos >> 3;
  int r = (int)(bit_pos & 7);
  uint32_t w = 0;
  if (k < src_bytes) w = src[k];
  if (k + 1 < src_bytes) w |= (uint32_t)src[k + 1] << 8;
  return (uint8_t)((w >> r) & ((1u << bits) - 1u));
}

/* cpp:98-109 (read_source_layout): row-major strides from the shape. */
static void row_major_strides(const int64_t* shape, int rank, int64_t* stride) {
  stride[rank - 1] = 1;
  for (int a = rank - 2; a >= 0; --a) stride[a] = stride[a + 1] * shape[a + 1];
}

/* cu:52-68 (source_index): coordinates placed on the token / head / head_dim
 * axes, the layer axis (if any) is coordinate 0. */
static int64_t source_index(const int64_t* stride, const int64_t* axes,
                            int64_t t, int64_t h, int64_t c) {
  return t * stride[axes[0]] + h * stride[axes[1]] + c * stride[axes[2]];
}

static int64_t spec_symbols(const int64_t* s) {
  return (s[1] - s[0]) * (s[3] - s[2]) * (s[5] - s[4]);
}

/* cpp:43-185 and cpp:326-362: the checks the reference extension makes
 * before launching (shape rank 3|4, positive dims, axes present, axis sizes,
 * layer axis size 1, spec ranges, bits 1..8, packed byte counts). */
static int validate(const int64_t* offsets, const int64_t* bits,
                    const int64_t* specs, int64_t n, const int64_t* shape,
                    int rank, const int64_t* axes) {
  if (rank != 3 && rank != 4)
    return fail("Origami source layout supports rank 3 or rank 4");
  for (int a = 0; a < rank; ++a)
    if (shape[a] <= 0) return fail("source_shape dimensions must be positive");
  for (int a = 0; a < 3; ++a)
    if (axes[a] < 0 || axes[a] >= rank)
      return fail("token/head/head_dim axis must be present in source layout");
  if (!(axes[3] == -1 || (axes[3] >= 0 && axes[3] < rank)))
    return fail("layer axis must be -1 or present in source layout");
  if (axes[3] != -1 && shape[axes[3]] != 1)
    return fail("per-layer Origami native layout requires layer axis size 1");
  int64_t T = shape[axes[0]], H = shape[axes[1]], C = shape[axes[2]];
  for (int64_t k = 0; k < n; ++k) {
    const int64_t* s = specs + 6 * k;
    if (!(0 <= s[0] && s[0] < s[1] && s[1] <= H))
      return fail("invalid head range in Origami chunk spec");
    if (!(0 <= s[2] && s[2] < s[3] && s[3] <= C))
      return fail("invalid channel range in Origami chunk spec");
    if (!(0 <= s[4] && s[4] < s[5] && s[5] <= T))
      return fail("invalid token range in Origami chunk spec");
    if (bits[k] < 1 || bits[k] > 8)
      return fail("Origami CUDA bitpack supports only 1..8 bit symbols");
    if (offsets[k + 1] - offsets[k] != (spec_symbols(s) * bits[k] + 7) / 8)
      return fail("Origami CUDA packed chunk byte size mismatch");
  }
  return ORACLE_OK;
}

/* cpp:316-400 + cu:91-128 (unpack_canonical_storage_chunks_cuda and
 * unpack_canonical_kernel): output of prod(shape) bytes, zeroed, then every
 * chunk's local symbol i goes to
 *   h = hs + i / (Cc*Tc), c = cs + (i % (Cc*Tc)) / Tc, t = ts + i % Tc
 * (head-major, channel, token fastest). */
int oracle_unpack_canonical(const uint8_t* flat, const int64_t* offsets,
                            const int64_t* bits, const int64_t* specs,
                            int64_t n, const int64_t* shape, int rank,
                            const int64_t* axes, uint8_t* out,
                            int64_t out_bytes) {
  int rc = validate(offsets, bits, specs, n, shape, rank, axes);
  if (rc) return rc;
  int64_t stride[4];
  row_major_strides(shape, rank, stride);
  int64_t total = 1;
  for (int a = 0; a < rank; ++a) total *= shape[a];
  if (total != out_bytes) return fail("output size must equal prod(source_shape)");
  memset(out, 0, (size_t)out_bytes);
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
  for (int64_t k = 0; k < n; ++k) {
    const int64_t* s = specs + 6 * k;
    const uint8_t* src = flat + offsets[k];
    int64_t src_bytes = offsets[k + 1] - offsets[k];
    int64_t Tc = s[5] - s[4], Cc = s[3] - s[2];
    int64_t per_head = Cc * Tc, cnt = spec_symbols(s);
    for (int64_t i = 0; i < cnt; ++i) {
      int64_t h = s[0] + i / per_head;
      int64_t rem = i % per_head;
      int64_t c = s[2] + rem / Tc;
      int64_t t = s[4] + rem % Tc;
      out[source_index(stride, axes, t, h, c)] =
          oracle_unpack_symbol(src, src_bytes, i, (int)bits[k]);
    }
  }
  return ORACLE_OK;
}

/* Pack: the unique inverse of oracle_unpack_canonical for in-range symbols.
 * The reference ships no packer (native_cpu.py:137-161 raises); its format is
 * fixed by the decoder (cu:70-128) and the byte count check (cpp:357-361):
 * chunk k holds ceil(n_k*b/8) bytes, symbol i occupies bits [i*b, i*b+b)
 * LSB-first, and the pad bits after the last symbol are zero. */
int oracle_pack_canonical(const uint8_t* symbols, int64_t symbol_bytes,
                          const int64_t* offsets, const int64_t* bits,
                          const int64_t* specs, int64_t n, const int64_t* shape,
                          int rank, const int64_t* axes, uint8_t* flat,
                          int64_t flat_bytes) {
  int rc = validate(offsets, bits, specs, n, shape, rank, axes);
  if (rc) return rc;
  int64_t stride[4];
  row_major_strides(shape, rank, stride);
  int64_t total = 1;
  for (int a = 0; a < rank; ++a) total *= shape[a];
  if (total != symbol_bytes) return fail("symbols size must equal prod(source_shape)");
  if (offsets[n] > flat_bytes) return fail("chunk_offsets exceed the flat stream");
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
  for (int64_t k = 0; k < n; ++k) {
    const int64_t* s = specs + 6 * k;
    uint8_t* dst = flat + offsets[k];
    int64_t dst_bytes = offsets[k + 1] - offsets[k];
    int b = (int)bits[k];
    uint32_t mask = (1u << b) - 1u;
    int64_t Tc = s[5] - s[4], Cc = s[3] - s[2];
    int64_t per_head = Cc * Tc, cnt = spec_symbols(s);
    memset(dst, 0, (size_t)dst_bytes);
    for (int64_t i = 0; i < cnt; ++i) {
      int64_t h = s[0] + i / per_head;
      int64_t rem = i % per_head;
      int64_t c = s[2] + rem / Tc;
      int64_t t = s[4] + rem % Tc;
      uint32_t v = symbols[source_index(stride, axes, t, h, c)] & mask;
      int64_t bit_pos = i * (int64_t)b;
      int64_t byte = bit_pos >> 3;
      uint32_t w = v << (bit_pos & 7);
      dst[byte] |= (uint8_t)(w & 0xff);
      if (w >> 8) dst[byte + 1] |= (uint8_t)(w >> 8);
    }
  }
  return ORACLE_OK;
}

/* Paged scatter of a token-major K/V tensor into vLLM's paged cache.
 *   value: bytes of [2, T, H, C]   (C = head_dim * element size)
 *   cache: bytes of [2, NB, bs, H, C] (blocks_first = 0) or
 *                   [NB, 2, bs, H, C] (blocks_first = 1)
 * bu:350-444 (_normalize_kv_value / _assign_blocks): the value is zero-padded
 * to block_count*bs tokens, reshaped into blocks and index_copy_'d along the
 * block axis; cu:408-420 gives the same destination index in closed form.
 * A block id outside [0, NB) is an error, as index_copy_ raises on it. */
int oracle_scatter_kv_cache(const uint8_t* value, int64_t T, int64_t H,
                            int64_t C, const int64_t* block_ids,
                            int64_t block_count, uint8_t* cache, int64_t NB,
                            int64_t bs, int blocks_first) {
  if (T > block_count * bs) return fail("tokens exceed destination block capacity");
  for (int64_t b = 0; b < block_count; ++b)
    if (block_ids[b] < 0 || block_ids[b] >= NB) return fail("block id out of range");
  int64_t row = H * C;
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (int64_t b = 0; b < block_count; ++b) {
    int64_t p = block_ids[b];
    for (int kv = 0; kv < 2; ++kv) {
      for (int64_t off = 0; off < bs; ++off) {
        int64_t t = b * bs + off;
        int64_t dst_row = blocks_first ? ((p * 2 + kv) * bs + off)
                                       : ((kv * NB + p) * bs + off);
        uint8_t* d = cache + dst_row * row;
        if (t < T)
          memcpy(d, value + (kv * T + t) * row, (size_t)row);
        else
          memset(d, 0, (size_t)row);
      }
    }
  }
  return ORACLE_OK;
}

/* Block gather for the save path, wk:1881-1897 (_select_blocks:
 * index_select of whole blocks along the block axis) followed by the
 * token-major view of raw_tensor.py:100-123: the result holds bytes of
 * [2, block_count*bs, H, C], K blocks then V blocks. */
int oracle_gather_kv_cache(const uint8_t* cache, int64_t NB, int64_t bs,
                           int64_t H, int64_t C, int blocks_first,
                           const int64_t* block_ids, int64_t block_count,
                           uint8_t* value) {
  for (int64_t b = 0; b < block_count; ++b)
    if (block_ids[b] < 0 || block_ids[b] >= NB) return fail("block id out of range");
  int64_t row = H * C, Tt = block_count * bs;
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (int64_t b = 0; b < block_count; ++b) {
    int64_t p = block_ids[b];
    for (int kv = 0; kv < 2; ++kv) {
      for (int64_t off = 0; off < bs; ++off) {
        int64_t src_row = blocks_first ? ((p * 2 + kv) * bs + off)
                                       : ((kv * NB + p) * bs + off);
        memcpy(value + (kv * Tt + b * bs + off) * row, cache + src_row * row,
               (size_t)row);
      }
    }
  }
  return ORACLE_OK;
}
