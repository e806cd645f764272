// origami_dequant.hip -- MI355X (gfx950) kernels and C ABI for Origami's fused
// dequantize paths: CacheGen unpack + dequantize (into the paged KV cache, and
// into a dense [layers, 2, heads, tokens, head_dim] tensor).
//
// CacheGen streams (csrc/origami/bitpack_layout_cuda.cu:349-423) hold one
// half's symbols token-major, symbol token * C + channel at b bits LSB-first,
// C = heads * head_dim.  A value is ((s - c) / c) * max[token] in binary32,
// c = bins / 2 - 1, rounded to float16 / bfloat16.
//
// Kernel design (wave64):
//  * A lane owns 8 consecutive symbols of one token row.  When C % 8 == 0 the
//    group starts on a byte boundary and is exactly b bytes, so a lane reads
//    2-3 aligned dwords, funnel-shifts its b bytes out (v_alignbyte) and
//    splits them into 8 symbols with compile-time shifts.
//  * (s - c) / c depends only on s, so each workgroup tabulates it once in LDS
//    with correctly rounded division; a value is then one LDS read and one
//    multiply, bit-identical to evaluating the quotient per element.
//  * The 8 results are one 16-byte non-temporal store.  Consecutive lanes take
//    consecutive groups of a row, so every store instruction covers whole
//    128-byte lines of the destination block, which is contiguous
//    ([block_size, heads, head_dim] inside a paged block).
//  * One workgroup per destination block; a block's rows are contiguous in
//    both the stream and the cache.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <string>

#include "origami_internal.h"
#include "origami_layout.h"

using namespace origami_internal;

namespace {

constexpr int kDqThreads = 256;
constexpr int64_t kMaxDqGrid = 1 << 20;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// A byte stream read through aligned dwords.  `base` is the stream start
// rounded down to 4 bytes, `bias` the distance back to it, and `bytes` the
// readable length from `base` (bias + stream bytes).  Bytes at or past
// `bytes` read as 0 (bitpack_layout_cuda.cu:295-314).
struct ByteStream {
  const uint32_t* base;
  int64_t bytes;
  int32_t bias;
};

ByteStream make_stream(const uint8_t* start, int64_t nbytes) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(start);
  const uintptr_t aligned = addr & ~uintptr_t(3);
  ByteStream s;
  s.base = reinterpret_cast<const uint32_t*>(aligned);
  s.bias = static_cast<int32_t>(addr - aligned);
  s.bytes = nbytes > 0 ? nbytes + s.bias : 0;  // an empty stream reads no dword
  return s;
}

// The 8 bytes of the stream starting at byte `o` (relative to `base`), with
// bytes at or past s.bytes zeroed.  Only dwords holding at least one byte
// below s.bytes are read, so no read leaves the pages the stream occupies.
template <int NBYTES>
__device__ __forceinline__ uint64_t load_window(const ByteStream& s, int64_t o) {
  constexpr int NW = (3 + NBYTES + 3) / 4;
  const int64_t k0 = o >> 2;
  const int sh = static_cast<int>(o & 3);
  uint32_t w[3] = {0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if ((k0 + i) * 4 < s.bytes) w[i] = s.base[k0 + i];
  }
  const uint32_t lo = __builtin_amdgcn_alignbyte(w[1], w[0], sh);
  const uint32_t hi = NW > 2 ? __builtin_amdgcn_alignbyte(w[2], w[1], sh) : (w[1] >> (8 * sh));
  uint64_t x = (static_cast<uint64_t>(hi) << 32) | lo;
  const int64_t avail = s.bytes - o;
  if (avail < NBYTES) x = avail <= 0 ? 0 : (x & ((uint64_t(1) << (8 * avail)) - 1));
  return x;
}

template <bool HALF>
__device__ __forceinline__ float load_meta(const void* p, int64_t i) {
  if constexpr (HALF) {
    return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  } else {
    return static_cast<const float*>(p)[i];
  }
}

// Round the binary32 value `v` to nearest even into float16 / bfloat16 bits.
// The empty asm makes `v` an opaque, already-rounded binary32 register:
// without it the backend folds a preceding multiply (or fma) and the float16
// conversion into one v_fma_mix instruction that rounds only once, straight
// to float16, which is not the reference's fp32-then-fp16 rounding.
template <bool BF16>
__device__ __forceinline__ uint32_t out_bits(float v) {
  asm("" : "+v"(v));
  if constexpr (BF16) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  } else {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  }
}

// (s - c) / c for s in [0, 2^bits), correctly rounded (the reference's
// `((float)s - center) / center`, bitpack_layout_cuda.cu:401-403).
__device__ __forceinline__ float cachegen_level(int s, float center) {
  return __fdiv_rn(static_cast<float>(s) - center, center);
}

// ---------------------------------------------------------------------------
// CacheGen -> paged KV cache
// ---------------------------------------------------------------------------

struct CacheGenCacheParams {
  ByteStream s;
  const void* maxv;       // per-token maxima of this half
  uint16_t* cache;
  const int64_t* block_ids;
  int64_t num_blocks, block_count, bs;
  int64_t blk_stride, half_stride, half;  // in rows of C elements
  int64_t tokens;
  int64_t C;              // heads * head_dim, a multiple of 8
  float center;
};

template <int BITS, bool BF16, bool MAX_HALF>
__global__ __launch_bounds__(kDqThreads) void cachegen_cache_kernel(CacheGenCacheParams p) {
  __shared__ float lut[1 << BITS];
  for (int i = threadIdx.x; i < (1 << BITS); i += kDqThreads) lut[i] = cachegen_level(i, p.center);
  __syncthreads();

  const int32_t G = static_cast<int32_t>(p.C >> 3);  // groups per token row
  const int32_t t_step = kDqThreads / G, c_step = kDqThreads % G;
  const int32_t tt0 = static_cast<int32_t>(threadIdx.x) / G;
  const int32_t cg0 = static_cast<int32_t>(threadIdx.x) % G;
  constexpr uint32_t mask = (1u << BITS) - 1u;

  for (int64_t u = blockIdx.x; u < p.block_count; u += gridDim.x) {
    const int64_t pid = p.block_ids[u];
    if (pid < 0 || pid >= p.num_blocks) continue;
    const int64_t t0 = u * p.bs;
    int64_t nt64 = p.tokens - t0;
    if (nt64 <= 0) continue;
    const int32_t nt = static_cast<int32_t>(nt64 < p.bs ? nt64 : p.bs);
    uint16_t* dst = p.cache + (pid * p.blk_stride + p.half * p.half_stride) * p.C;
    const int64_t g0 = t0 * G;  // first 8-symbol group of the block's rows
    int32_t tt = tt0, cg = cg0;
    while (tt < nt) {
      const int64_t grp = g0 + static_cast<int64_t>(tt) * G + cg;
      const uint64_t w = load_window<BITS>(p.s, p.s.bias + grp * BITS);
      const float m = load_meta<MAX_HALF>(p.maxv, t0 + tt);
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t s0 = static_cast<uint32_t>(w >> ((2 * k) * BITS)) & mask;
        const uint32_t s1 = static_cast<uint32_t>(w >> ((2 * k + 1) * BITS)) & mask;
        o[k] = out_bits<BF16>(lut[s0] * m) | (out_bits<BF16>(lut[s1] * m) << 16);
      }
      const u32x4 x = {o[0], o[1], o[2], o[3]};
      __builtin_nontemporal_store(
          x, reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(tt) * p.C + cg * 8));
      cg += c_step;
      tt += t_step;
      if (cg >= G) {
        cg -= G;
        ++tt;
      }
    }
  }
}

// One thread per destination element, both halves: any C, any alignment.
struct CacheGenGenericParams {
  ByteStream s[2];
  const void* maxv[2];
  int32_t bits[2];
  float center[2];
  uint16_t* cache;
  const int64_t* block_ids;
  int64_t num_blocks, block_count, bs, blk_stride, half_stride;
  int64_t tokens, C;
};

__device__ __forceinline__ uint32_t symbol_at(const ByteStream& s, int64_t i, int bits) {
  const int64_t bit = i * bits;
  const int64_t o = s.bias + (bit >> 3);
  const uint64_t w = load_window<2>(s, o);
  return static_cast<uint32_t>(w >> (bit & 7)) & ((1u << bits) - 1u);
}

template <bool BF16, bool MAX_HALF>
__global__ __launch_bounds__(kDqThreads) void cachegen_cache_generic_kernel(
    CacheGenGenericParams p) {
  __shared__ float lut[2][256];
  for (int i = threadIdx.x; i < 512; i += kDqThreads) {
    const int h = i >> 8, s = i & 255;
    lut[h][s] = cachegen_level(s, p.center[h]);
  }
  __syncthreads();
  const int64_t per_half = p.bs * p.C;
  const int64_t total = p.block_count * 2 * per_half;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kDqThreads + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kDqThreads) {
    const int64_t lb = idx / (2 * per_half);
    const int64_t r0 = idx - lb * 2 * per_half;
    const int half = static_cast<int>(r0 / per_half);
    const int64_t r = r0 - half * per_half;
    const int64_t off = r / p.C;
    const int64_t ch = r - off * p.C;
    const int64_t token = lb * p.bs + off;
    if (token >= p.tokens) continue;
    const int64_t pid = p.block_ids[lb];
    if (pid < 0 || pid >= p.num_blocks) continue;
    const uint32_t s = symbol_at(p.s[half], token * p.C + ch, p.bits[half]);
    const float m = load_meta<MAX_HALF>(p.maxv[half], token);
    const int64_t row = pid * p.blk_stride + half * p.half_stride + off;
    p.cache[row * p.C + ch] = static_cast<uint16_t>(out_bits<BF16>(lut[half][s] * m));
  }
}

// ---------------------------------------------------------------------------
// CacheGen -> dense float16 [layers, 2, heads, tokens, head_dim]
// ---------------------------------------------------------------------------

struct CacheGenDenseParams {
  ByteStream s;
  const void* maxv;       // this segment's per-token maxima (already offset)
  uint16_t* out;          // this segment's [heads, tokens, head_dim] slab
  int64_t T, H, D, C;
  int32_t bits;
  float center;
};

// D % 8 == 0: a lane writes 8 consecutive head_dim values (one 16-byte store)
// of one (head, token) row; blockIdx.y is the head.
template <bool MAX_HALF>
__global__ __launch_bounds__(kDqThreads) void cachegen_dense_kernel(CacheGenDenseParams p) {
  __shared__ float lut[256];
  for (int i = threadIdx.x; i < 256; i += kDqThreads) lut[i] = cachegen_level(i, p.center);
  __syncthreads();
  const int64_t GD = p.D >> 3;
  const int64_t per_head = p.T * GD;
  const int64_t h = blockIdx.y;
  const uint32_t mask = (1u << p.bits) - 1u;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kDqThreads + threadIdx.x; i < per_head;
       i += static_cast<int64_t>(gridDim.x) * kDqThreads) {
    const int64_t t = i / GD;
    const int64_t dg = i - t * GD;
    const int64_t grp = (t * p.C + h * p.D) / 8 + dg;
    const uint64_t w = load_window<8>(p.s, p.s.bias + grp * p.bits);
    const float m = load_meta<MAX_HALF>(p.maxv, t);
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t s0 = static_cast<uint32_t>(w >> ((2 * k) * p.bits)) & mask;
      const uint32_t s1 = static_cast<uint32_t>(w >> ((2 * k + 1) * p.bits)) & mask;
      o[k] = out_bits<false>(lut[s0] * m) | (out_bits<false>(lut[s1] * m) << 16);
    }
    const u32x4 x = {o[0], o[1], o[2], o[3]};
    __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(p.out + (h * p.T + t) * p.D + dg * 8));
  }
}

// Any head_dim: one thread per output element.
template <bool MAX_HALF>
__global__ __launch_bounds__(kDqThreads) void cachegen_dense_generic_kernel(
    CacheGenDenseParams p) {
  __shared__ float lut[256];
  for (int i = threadIdx.x; i < 256; i += kDqThreads) lut[i] = cachegen_level(i, p.center);
  __syncthreads();
  const int64_t total = p.H * p.T * p.D;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kDqThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kDqThreads) {
    const int64_t d = i % p.D;
    const int64_t r = i / p.D;
    const int64_t t = r % p.T;
    const int64_t h = r / p.T;
    const uint32_t s = symbol_at(p.s, t * p.C + h * p.D + d, p.bits);
    p.out[i] = static_cast<uint16_t>(out_bits<false>(lut[s] * load_meta<MAX_HALF>(p.maxv, t)));
  }
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------

int check_bits(int64_t bits) {
  ORIGAMI_REQUIRE(bits >= 1 && bits <= 8, "Origami CUDA bitpack supports only 1..8 bit symbols");
  return ORIGAMI_OK;
}

int launch_cachegen_cache(const CacheGenCacheParams& p, int bits, bool bf16, bool max_half,
                          hipStream_t stream) {
  const dim3 grid(grid_for(p.block_count, 1, kMaxDqGrid)), block(kDqThreads);
#define ORIGAMI_CG_CASE(B)                                                                   \
  case B:                                                                                    \
    if (bf16) {                                                                              \
      if (max_half)                                                                          \
        hipLaunchKernelGGL((cachegen_cache_kernel<B, true, true>), grid, block, 0, stream, p); \
      else                                                                                   \
        hipLaunchKernelGGL((cachegen_cache_kernel<B, true, false>), grid, block, 0, stream, p); \
    } else {                                                                                 \
      if (max_half)                                                                          \
        hipLaunchKernelGGL((cachegen_cache_kernel<B, false, true>), grid, block, 0, stream, p); \
      else                                                                                   \
        hipLaunchKernelGGL((cachegen_cache_kernel<B, false, false>), grid, block, 0, stream, p); \
    }                                                                                        \
    break;
  switch (bits) {
    ORIGAMI_CG_CASE(1)
    ORIGAMI_CG_CASE(2)
    ORIGAMI_CG_CASE(3)
    ORIGAMI_CG_CASE(4)
    ORIGAMI_CG_CASE(5)
    ORIGAMI_CG_CASE(6)
    ORIGAMI_CG_CASE(7)
    ORIGAMI_CG_CASE(8)
    default:
      return check_bits(bits);
  }
#undef ORIGAMI_CG_CASE
  return check_launch("cachegen_cache_kernel");
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

int origami_cachegen_unpack_dequantize_to_kv_cache(
    const uint8_t* bytestream, int64_t bytestream_bytes, int64_t key_offset, int64_t key_bytes,
    int64_t value_offset, int64_t value_bytes, int64_t key_bits, int64_t value_bits,
    int64_t key_bins, int64_t value_bins, const void* max_key, const void* max_value,
    int64_t max_key_count, int64_t max_value_count, int64_t max_dtype, void* kv_cache,
    int64_t cache_dtype, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    const int64_t* block_ids, int64_t block_count, int64_t tokens, int64_t heads,
    int64_t head_dim, origami_stream_t stream) {
  ORIGAMI_REQUIRE(cache_dtype == ORIGAMI_DTYPE_FLOAT16 || cache_dtype == ORIGAMI_DTYPE_BFLOAT16,
                  "kv_cache must be float16 or bfloat16");
  ORIGAMI_REQUIRE(max_dtype == ORIGAMI_DTYPE_FLOAT16 || max_dtype == ORIGAMI_DTYPE_FLOAT32,
                  "max tensors must be float16 or float32");
  if (int rc = check_bits(key_bits)) return rc;
  if (int rc = check_bits(value_bits)) return rc;
  ORIGAMI_REQUIRE(tokens > 0 && heads > 0 && head_dim > 0,
                  "tokens, heads, and head_dim must be positive");
  ORIGAMI_REQUIRE(key_bins > 1 && value_bins > 1, "CacheGen bins must be greater than one");
  ORIGAMI_REQUIRE(key_offset >= 0 && key_bytes >= 0 && value_offset >= 0 && value_bytes >= 0,
                  "invalid CacheGen stream offsets");
  ORIGAMI_REQUIRE(key_offset + key_bytes <= bytestream_bytes &&
                      value_offset + value_bytes <= bytestream_bytes,
                  "CacheGen stream ranges exceed bytestream length");
  ORIGAMI_REQUIRE(max_key_count >= tokens && max_value_count >= tokens,
                  "max tensors must contain at least tokens values");
  ORIGAMI_REQUIRE(block_size > 0, "kv_cache block size must be positive");
  ORIGAMI_REQUIRE(num_blocks > 0, "kv_cache must hold at least one block");
  ORIGAMI_REQUIRE(block_count > 0, "block_ids must be non-empty");
  ORIGAMI_REQUIRE(tokens <= block_count * block_size, "tokens exceed destination block capacity");
  const int64_t C = heads * head_dim;
  ORIGAMI_REQUIRE(C <= (int64_t(1) << 24), "heads * head_dim exceeds 2^24");
  int64_t blk_stride = 0, half_stride = 0;
  if (int rc = cache_geometry(cache_layout, num_blocks, block_size, &blk_stride, &half_stride))
    return rc;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool bf16 = cache_dtype == ORIGAMI_DTYPE_BFLOAT16;
  const bool max_half = max_dtype == ORIGAMI_DTYPE_FLOAT16;
  const int64_t offs[2] = {key_offset, value_offset};
  const int64_t lens[2] = {key_bytes, value_bytes};
  const int64_t bits[2] = {key_bits, value_bits};
  const int64_t bins[2] = {key_bins, value_bins};
  const void* maxes[2] = {max_key, max_value};

  if (C % 8 == 0 && aligned16(kv_cache)) {
    for (int half = 0; half < 2; ++half) {
      CacheGenCacheParams p{};
      p.s = make_stream(bytestream + offs[half], lens[half]);
      p.maxv = maxes[half];
      p.cache = static_cast<uint16_t*>(kv_cache);
      p.block_ids = block_ids;
      p.num_blocks = num_blocks;
      p.block_count = block_count;
      p.bs = block_size;
      p.blk_stride = blk_stride;
      p.half_stride = half_stride;
      p.half = half;
      p.tokens = tokens;
      p.C = C;
      p.center = static_cast<float>(bins[half] / 2 - 1);
      if (int rc = launch_cachegen_cache(p, static_cast<int>(bits[half]), bf16, max_half, st))
        return rc;
    }
    return ORIGAMI_OK;
  }

  CacheGenGenericParams p{};
  for (int half = 0; half < 2; ++half) {
    p.s[half] = make_stream(bytestream + offs[half], lens[half]);
    p.maxv[half] = maxes[half];
    p.bits[half] = static_cast<int32_t>(bits[half]);
    p.center[half] = static_cast<float>(bins[half] / 2 - 1);
  }
  p.cache = static_cast<uint16_t*>(kv_cache);
  p.block_ids = block_ids;
  p.num_blocks = num_blocks;
  p.block_count = block_count;
  p.bs = block_size;
  p.blk_stride = blk_stride;
  p.half_stride = half_stride;
  p.tokens = tokens;
  p.C = C;
  const dim3 grid(grid_for(block_count * 2 * block_size * C, kDqThreads, 65536)), block(kDqThreads);
  if (bf16) {
    if (max_half)
      hipLaunchKernelGGL((cachegen_cache_generic_kernel<true, true>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((cachegen_cache_generic_kernel<true, false>), grid, block, 0, st, p);
  } else {
    if (max_half)
      hipLaunchKernelGGL((cachegen_cache_generic_kernel<false, true>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((cachegen_cache_generic_kernel<false, false>), grid, block, 0, st, p);
  }
  return check_launch("cachegen_cache_generic_kernel");
}

int origami_cachegen_unpack_dequantize(const uint8_t* bytestream, int64_t bytestream_bytes,
                                       const int64_t* offsets, const int64_t* bits_per_layer,
                                       const int64_t* key_bins, const int64_t* value_bins,
                                       int64_t layers, const void* max_key,
                                       const void* max_value, int64_t max_key_count,
                                       int64_t max_value_count, int64_t max_dtype, int64_t tokens,
                                       int64_t heads, int64_t head_dim, void* output,
                                       int64_t output_bytes, origami_stream_t stream) {
  ORIGAMI_REQUIRE(max_dtype == ORIGAMI_DTYPE_FLOAT16 || max_dtype == ORIGAMI_DTYPE_FLOAT32,
                  "max tensors must be float16 or float32");
  ORIGAMI_REQUIRE(layers >= 0, "layers must be non-negative");
  ORIGAMI_REQUIRE(max_key_count == layers * tokens, "max_key must have layers * tokens values");
  ORIGAMI_REQUIRE(max_value_count == layers * tokens,
                  "max_value must have layers * tokens values");
  ORIGAMI_REQUIRE(tokens > 0 && heads > 0 && head_dim > 0,
                  "tokens, heads, and head_dim must be positive");
  for (int64_t j = 0; j < 2 * layers; ++j) {
    if (int rc = check_bits(bits_per_layer[j])) return rc;
  }
  for (int64_t j = 0; j < 2 * layers; ++j) {
    ORIGAMI_REQUIRE(offsets[j] >= 0 && offsets[j + 1] >= offsets[j] &&
                        offsets[j + 1] <= bytestream_bytes,
                    "CacheGen stream offsets must be non-decreasing and within the bytestream");
  }
  const int64_t C = heads * head_dim;
  const int64_t slab = heads * tokens * head_dim;  // elements per (layer, half)
  ORIGAMI_REQUIRE(output_bytes >= layers * 2 * slab * 2, "output is smaller than the result");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool max_half = max_dtype == ORIGAMI_DTYPE_FLOAT16;
  const size_t esize = max_half ? 2 : 4;
  const bool fast = head_dim % 8 == 0 && aligned16(output);
  for (int64_t j = 0; j < 2 * layers; ++j) {
    const bool is_value = j >= layers;
    const int64_t layer = is_value ? j - layers : j;
    CacheGenDenseParams p{};
    p.s = make_stream(bytestream + offsets[j], offsets[j + 1] - offsets[j]);
    p.maxv = static_cast<const uint8_t*>(is_value ? max_value : max_key) + layer * tokens * esize;
    p.out = static_cast<uint16_t*>(output) + (layer * 2 + (is_value ? 1 : 0)) * slab;
    p.T = tokens;
    p.H = heads;
    p.D = head_dim;
    p.C = C;
    p.bits = static_cast<int32_t>(bits_per_layer[j]);
    p.center = static_cast<float>((is_value ? value_bins[layer] : key_bins[layer]) / 2 - 1);
    if (fast) {
      ORIGAMI_REQUIRE(heads <= 65535, "heads exceeds the launch grid");
      const dim3 grid(grid_for(tokens * (head_dim / 8), kDqThreads, 65536),
                      static_cast<unsigned>(heads));
      if (max_half)
        hipLaunchKernelGGL((cachegen_dense_kernel<true>), grid, dim3(kDqThreads), 0, st, p);
      else
        hipLaunchKernelGGL((cachegen_dense_kernel<false>), grid, dim3(kDqThreads), 0, st, p);
    } else {
      const dim3 grid(grid_for(slab, kDqThreads, 65536));
      if (max_half)
        hipLaunchKernelGGL((cachegen_dense_generic_kernel<true>), grid, dim3(kDqThreads), 0, st, p);
      else
        hipLaunchKernelGGL((cachegen_dense_generic_kernel<false>), grid, dim3(kDqThreads), 0, st,
                           p);
    }
    if (int rc = check_launch("cachegen_dense_kernel")) return rc;
  }
  return ORIGAMI_OK;
}

}  // extern "C"
