/*
 * dequant_oracle.c -- CPU restatement of Origami's fused dequantize kernels:
 * CacheGen unpack+dequantize (to a dense tensor and into the paged KV cache)
 * and KIVI dequantize into the paged KV cache.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle that the HIP kernels of
 * origami_amd are checked against.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it, and only as the checker or as
 * the timed CPU baseline; the product path never calls it.
 *
 * Arithmetic is IEEE-754 binary32 throughout.  The Makefile compiles with
 * -ffp-contract=off, so a product and a sum are rounded separately except
 * where fmaf() is written out.  That is where the reference's CUDA kernel has
 * `a * b + c`, which nvcc's default --fmad=true contracts into one fused
 * multiply-add.
 *
 * Reference file: csrc/origami/bitpack_layout_cuda.cu (cu),
 *                 csrc/origami/bitpack_layout_cuda.cpp (cpp).
 *
 * Parity pinning (tests/test_dequant_oracle.py):
 *   oracle_half_to_float / oracle_float_to_half
 *                              -- numpy float16 casts over every half
 *                                 pattern and rounding edge cases
 *   oracle_float_to_bf16       -- torch bfloat16 casts (round to nearest
 *                                 even) over rounding edge cases
 *   oracle_cachegen_to_kv_cache
 *                              -- the reference's own unfused path restated
 *                                 with torch tensor ops (linear unpack,
 *                                 (q - c) / c * max, dtype cast, block
 *                                 assignment); closed-form symbols 0, c, 2c
 *                                 give -max, 0, +max exactly
 *   oracle_cachegen_unpack_dequantize
 *                              -- the same torch restatement, per layer,
 *                                 permuted to [layer, kv, head, token, dim]
 *   oracle_kivi_to_kv_cache    -- torch restatement of KIVI's unpack order
 *                                 (packers of kivi_adapter.py) with the
 *                                 multiply-add evaluated exactly in float64
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_EINVAL -1

uint8_t oracle_unpack_symbol(const uint8_t* src, int64_t src_bytes, int64_t i, int bits);

static char g_dq_err[512];

const char* oracle_dequant_last_error(void) { return g_dq_err; }

static int dq_fail(const char* msg) {
  snprintf(g_dq_err, sizeof(g_dq_err), "%s", msg);
  return ORACLE_EINVAL;
}

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* binary16 -> binary32, exact (subnormals, infinities and NaN payloads kept). */
float oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0x1f) return bits_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 is exact in binary32 */
    float v = (float)man * 0x1p-24f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest even; overflow -> infinity; NaN ->
 * quiet NaN with the sign kept. */
uint16_t oracle_float_to_half(float f) {
  uint32_t u = f32_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  uint32_t exp = (u >> 23) & 0xff;
  uint32_t man = u & 0x7fffff;
  if (exp == 0xff) return sign | (man ? 0x7e00 : 0x7c00);
  int32_t e = (int32_t)exp - 127;           /* unbiased exponent */
  if (e > 15) return sign | 0x7c00;
  if (e >= -14) {
    /* normal half: keep 10 fraction bits, round the 13 dropped bits */
    uint32_t m = man >> 13;
    uint32_t rest = man & 0x1fff;
    uint32_t h = ((uint32_t)(e + 15) << 10) | m;
    if (rest > 0x1000 || (rest == 0x1000 && (m & 1))) h += 1; /* may carry into exponent */
    return sign | (uint16_t)h;               /* carry past 0x7bff gives 0x7c00 = inf */
  }
  if (e < -25) return sign;                 /* below half of the smallest subnormal */
  /* subnormal half: value = full * 2^(e-23), full = 1.man (24 bits);
   * in units of 2^-24 that is full >> (-1 - e) with 0..24 dropped bits */
  uint32_t full = man | 0x800000u;
  int shift = -1 - e;                        /* 14..24 */
  uint32_t m = full >> shift;
  uint32_t rest = full & ((1u << shift) - 1);
  uint32_t half_ulp = 1u << (shift - 1);
  if (rest > half_ulp || (rest == half_ulp && (m & 1))) m += 1;
  return sign | (uint16_t)m;
}

/* binary32 -> bfloat16, round to nearest even; NaN -> quiet NaN. */
uint16_t oracle_float_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static float load_meta(const void* p, int is_half, int64_t i) {
  if (is_half) return oracle_half_to_float(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

static uint16_t store_out(float v, int out_is_bf16) {
  return out_is_bf16 ? oracle_float_to_bf16(v) : oracle_float_to_half(v);
}

/* cu:295-314 (unpack_symbol_direct) with one bound added: at b = 8 the
 * reference reads src[i] unchecked; here a byte past the stream reads as 0,
 * as it does for every other width. */
static uint8_t symbol_at(const uint8_t* src, int64_t src_bytes, int64_t i, int bits) {
  if (bits == 8) return i < src_bytes ? src[i] : 0;
  return oracle_unpack_symbol(src, src_bytes, i, bits);
}

/* kivi_adapter.py:39-43 / 71-76: the 3-bit KIVI stream keeps one symbol per
 * nibble (two per byte, low nibble first, upper bit of each nibble zero). */
static uint8_t kivi_symbol_at(const uint8_t* src, int64_t src_bytes, int64_t i, int bits,
                              int nibble3) {
  if (nibble3 && bits == 3) {
    int64_t k = i >> 1;
    if (k >= src_bytes) return 0;
    return (uint8_t)((src[k] >> (4 * (int)(i & 1))) & 0x7);
  }
  return symbol_at(src, src_bytes, i, bits);
}

/* cu:408-420: element index of (block p, half kv, offset, head, dim). */
static int64_t cache_index(int blocks_first, int64_t NB, int64_t bs, int64_t H, int64_t D,
                           int64_t p, int64_t kv, int64_t off, int64_t h, int64_t d) {
  if (blocks_first) return ((((p * 2 + kv) * bs + off) * H + h) * D + d);
  return ((((kv * NB + p) * bs + off) * H + h) * D + d);
}

static int check_streams(int64_t bytestream_bytes, int64_t key_offset, int64_t key_bytes,
                         int64_t value_offset, int64_t value_bytes) {
  if (key_offset < 0 || key_bytes < 0 || value_offset < 0 || value_bytes < 0)
    return dq_fail("invalid stream offsets");
  if (key_offset + key_bytes > bytestream_bytes || value_offset + value_bytes > bytestream_bytes)
    return dq_fail("stream ranges exceed bytestream length");
  return ORACLE_OK;
}

/* cu:349-423 (cachegen_unpack_dequantize_to_kv_cache_kernel): for every
 * destination element of the listed blocks with token < tokens, read symbol
 * token * C + channel of the K or V stream, dequantize
 * ((s - c) / c) * max[token] with c = bins / 2 - 1, and store it rounded to
 * float16 / bfloat16.  Tokens >= tokens and invalid block ids are skipped
 * (the cache keeps its contents there). */
int oracle_cachegen_to_kv_cache(const uint8_t* bytestream, int64_t bytestream_bytes,
                                int64_t key_offset, int64_t key_bytes, int64_t value_offset,
                                int64_t value_bytes, int key_bits, int value_bits,
                                int64_t key_bins, int64_t value_bins, const void* max_key,
                                const void* max_value, int max_is_half, uint16_t* kv_cache,
                                int out_is_bf16, int blocks_first, int64_t num_blocks,
                                int64_t block_size, const int64_t* block_ids,
                                int64_t block_count, int64_t tokens, int64_t heads,
                                int64_t head_dim) {
  if (check_streams(bytestream_bytes, key_offset, key_bytes, value_offset, value_bytes))
    return ORACLE_EINVAL;
  if (key_bits < 1 || key_bits > 8 || value_bits < 1 || value_bits > 8)
    return dq_fail("bits must be 1..8");
  if (key_bins <= 1 || value_bins <= 1) return dq_fail("CacheGen bins must be greater than one");
  if (tokens > block_count * block_size) return dq_fail("tokens exceed destination block capacity");
  const int64_t C = heads * head_dim;
  for (int64_t lb = 0; lb < block_count; ++lb) {
    const int64_t p = block_ids[lb];
    if (p < 0 || p >= num_blocks) continue;
    for (int64_t kv = 0; kv < 2; ++kv) {
      const uint8_t* stream = bytestream + (kv ? value_offset : key_offset);
      const int64_t stream_bytes = kv ? value_bytes : key_bytes;
      const int bits = kv ? value_bits : key_bits;
      const int64_t bins = kv ? value_bins : key_bins;
      const float center = (float)(bins / 2 - 1);
      const void* maxp = kv ? max_value : max_key;
      for (int64_t off = 0; off < block_size; ++off) {
        const int64_t token = lb * block_size + off;
        if (token >= tokens) continue;
        const float max_abs = load_meta(maxp, max_is_half, token);
        for (int64_t ch = 0; ch < C; ++ch) {
          const uint8_t s = symbol_at(stream, stream_bytes, token * C + ch, bits);
          const float v = (((float)s - center) / center) * max_abs;
          kv_cache[cache_index(blocks_first, num_blocks, block_size, heads, head_dim, p, kv, off,
                               ch / head_dim, ch % head_dim)] = store_out(v, out_is_bf16);
        }
      }
    }
  }
  return ORACLE_OK;
}

/* cu:141-186 (cachegen_unpack_dequantize_kernel): stream segment j of
 * offsets[] holds layer j's keys for j < L and layer j - L's values after
 * that, token-major at bits_per_layer[j] bits.  Output is float16
 * [layers, 2, heads, tokens, head_dim]; the per-token maxima are
 * [layers, tokens]. */
int oracle_cachegen_unpack_dequantize(const uint8_t* bytestream, int64_t bytestream_bytes,
                                      const int64_t* offsets, const int64_t* bits_per_layer,
                                      const int64_t* key_bins, const int64_t* value_bins,
                                      int64_t layers, const void* max_key, const void* max_value,
                                      int max_is_half, int64_t tokens, int64_t heads,
                                      int64_t head_dim, uint16_t* output) {
  const int64_t C = heads * head_dim;
  for (int64_t j = 0; j < 2 * layers; ++j) {
    if (offsets[j] < 0 || offsets[j + 1] < offsets[j] || offsets[j + 1] > bytestream_bytes)
      return dq_fail("stream offsets out of range");
    if (bits_per_layer[j] < 1 || bits_per_layer[j] > 8) return dq_fail("bits must be 1..8");
  }
  for (int64_t j = 0; j < 2 * layers; ++j) {
    const int is_value = j >= layers;
    const int64_t layer = is_value ? j - layers : j;
    const int64_t kv = is_value;
    const int bits = (int)bits_per_layer[j];
    const uint8_t* stream = bytestream + offsets[j];
    const int64_t stream_bytes = offsets[j + 1] - offsets[j];
    const int64_t bins = is_value ? value_bins[layer] : key_bins[layer];
    const float center = (float)(bins / 2 - 1);
    const void* maxp = is_value ? max_value : max_key;
    for (int64_t token = 0; token < tokens; ++token) {
      const float max_abs = load_meta(maxp, max_is_half, layer * tokens + token);
      for (int64_t ch = 0; ch < C; ++ch) {
        const int64_t h = ch / head_dim, d = ch % head_dim;
        const uint8_t s = symbol_at(stream, stream_bytes, token * C + ch, bits);
        const float v = (((float)s - center) / center) * max_abs;
        output[(((layer * 2 + kv) * heads + h) * tokens + token) * head_dim + d] =
            oracle_float_to_half(v);
      }
    }
  }
  return ORACLE_OK;
}

/* cu:578-683 (kivi_dequantize_to_kv_cache_kernel).  Tokens below
 * sink_tokens copy the float16/float32 sink values ([sink, C]); body token
 * bt = token - sink reads
 *   keys:   symbol (d * H + h) * body + bt, value s * key_scale[g][c] +
 *           key_zero[g][c] with g = bt / group_size (per-channel groups
 *           along tokens, [key_groups, C]);
 *   values: symbol (h * D + d) * body + bt, value s * value_scale[bt][g] +
 *           value_zero[bt][g] with g = c / group_size ([body, value_groups]).
 * nibble3 selects KIVI's 3-bit container (one symbol per nibble); otherwise
 * symbols are packed LSB-first at `bits` bits, as the reference kernel reads
 * them. */
int oracle_kivi_to_kv_cache(const uint8_t* bytestream, int64_t bytestream_bytes,
                            int64_t key_offset, int64_t key_bytes, int64_t value_offset,
                            int64_t value_bytes, int bits, int nibble3, int64_t group_size,
                            int64_t sink_tokens, const void* key_scale, const void* key_zero,
                            const void* value_scale, const void* value_zero,
                            const void* key_sink, const void* value_sink, int meta_is_half,
                            uint16_t* kv_cache, int out_is_bf16, int blocks_first,
                            int64_t num_blocks, int64_t block_size, const int64_t* block_ids,
                            int64_t block_count, int64_t tokens, int64_t heads,
                            int64_t head_dim) {
  if (check_streams(bytestream_bytes, key_offset, key_bytes, value_offset, value_bytes))
    return ORACLE_EINVAL;
  if (bits < 1 || bits > 8) return dq_fail("bits must be 1..8");
  if (group_size <= 0) return dq_fail("KIVI group_size must be positive");
  if (sink_tokens < 0 || sink_tokens > tokens) return dq_fail("KIVI sink_tokens must be in [0, tokens]");
  if (tokens > block_count * block_size) return dq_fail("tokens exceed destination block capacity");
  const int64_t C = heads * head_dim;
  const int64_t body = tokens - sink_tokens;
  const int64_t value_groups = (C + group_size - 1) / group_size;
  for (int64_t lb = 0; lb < block_count; ++lb) {
    const int64_t p = block_ids[lb];
    if (p < 0 || p >= num_blocks) continue;
    for (int64_t kv = 0; kv < 2; ++kv) {
      const uint8_t* stream = bytestream + (kv ? value_offset : key_offset);
      const int64_t stream_bytes = kv ? value_bytes : key_bytes;
      for (int64_t off = 0; off < block_size; ++off) {
        const int64_t token = lb * block_size + off;
        if (token >= tokens) continue;
        for (int64_t ch = 0; ch < C; ++ch) {
          const int64_t h = ch / head_dim, d = ch % head_dim;
          float v;
          if (token < sink_tokens) {
            v = load_meta(kv ? value_sink : key_sink, meta_is_half, token * C + ch);
          } else {
            const int64_t bt = token - sink_tokens;
            if (kv) {
              const uint8_t s =
                  kivi_symbol_at(stream, stream_bytes, (h * head_dim + d) * body + bt, bits, nibble3);
              const int64_t mi = bt * value_groups + ch / group_size;
              v = fmaf((float)s, load_meta(value_scale, meta_is_half, mi),
                       load_meta(value_zero, meta_is_half, mi));
            } else {
              const uint8_t s =
                  kivi_symbol_at(stream, stream_bytes, (d * heads + h) * body + bt, bits, nibble3);
              const int64_t mi = (bt / group_size) * C + ch;
              v = fmaf((float)s, load_meta(key_scale, meta_is_half, mi),
                       load_meta(key_zero, meta_is_half, mi));
            }
          }
          kv_cache[cache_index(blocks_first, num_blocks, block_size, heads, head_dim, p, kv, off,
                               h, d)] = store_out(v, out_is_bf16);
        }
      }
    }
  }
  return ORACLE_OK;
}
