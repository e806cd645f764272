// origami_dequant.hip -- MI355X (gfx950) kernels and C ABI for Origami's fused
// dequantize paths: CacheGen unpack + dequantize (into the paged KV cache, and
// into a dense [layers, 2, heads, tokens, head_dim] tensor) and KIVI
// dequantize into the paged KV cache.
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
// CacheGen row kernel: one workgroup per destination block.  512 threads give
// each thread 4 rows of a 16-token bf16 block at 1024 channels (measured 3%
// faster than 256 threads, 7% faster than 1024).
constexpr int kCgThreads = 512;
constexpr int kCgBatch = 4;  // groups a CacheGen thread loads before expanding
constexpr uint32_t kXcds = 8;  // MI355X: 8 accelerator complex dies, one L2 each
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

// Two binary32 values rounded to nearest even and packed (a low, b high);
// one v_cvt_pk conversion for both.  The empty asm serves as in out_bits.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Eight binary32 values rounded and packed into four dwords (pairs low,
// high).  One empty asm over all eight keeps the rounding barrier of
// out_bits2 without tying each conversion to the two fma results just
// before it (which made the compiler pad every pair with wait states).
template <bool BF16>
__device__ __forceinline__ void out_bits8(float (&v)[8], uint32_t (&o)[4]) {
  asm("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),
      "+v"(v[7]));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x2 x = {v[2 * k], v[2 * k + 1]};
    if constexpr (BF16) {
      o[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2));
    } else {
      o[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
    }
  }
}

template <bool BF16>
__device__ __forceinline__ uint32_t out_bits2(float a, float b) {
  asm("" : "+v"(a), "+v"(b));
  const f32x2 v = {a, b};
  if constexpr (BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
}

// fmaf(a, b, c) as a three-address v_fma_f32: the addend (a zero point shared
// by many elements) stays in its register instead of being copied into the
// accumulator of a two-address v_fmac for every element.
__device__ __forceinline__ float fma3(float a, float b, float c) {
  float r;
  asm("v_fma_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
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
__global__ __launch_bounds__(kCgThreads) void cachegen_cache_kernel(CacheGenCacheParams p) {
  __shared__ float lut[1 << BITS];
  for (int i = threadIdx.x; i < (1 << BITS); i += kCgThreads) lut[i] = cachegen_level(i, p.center);
  __syncthreads();

  const int32_t G = static_cast<int32_t>(p.C >> 3);  // groups per token row
  const int32_t t_step = kCgThreads / G, c_step = kCgThreads % G;
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
    // kCgBatch groups at a time: every group's dwords and maximum are
    // requested before the first group is expanded, so a thread's loads
    // overlap (load_window and load_meta, split into loads and arithmetic)
    constexpr int NW = (3 + BITS + 3) / 4;
    while (tt < nt) {
      int32_t bt[kCgBatch], bc[kCgBatch];
      int64_t bo[kCgBatch];
      uint32_t w[kCgBatch][3];
      uint32_t mraw[kCgBatch];
#pragma unroll
      for (int j = 0; j < kCgBatch; ++j) {
        bt[j] = tt;
        bc[j] = cg;
        bo[j] = 0;
        w[j][0] = w[j][1] = w[j][2] = 0;
        mraw[j] = 0;
        if (tt < nt) {
          const int64_t o = p.s.bias + (g0 + static_cast<int64_t>(tt) * G + cg) * BITS;
          bo[j] = o;
          const int64_t k0 = o >> 2;
#pragma unroll
          for (int i = 0; i < NW; ++i)
            if ((k0 + i) * 4 < p.s.bytes) w[j][i] = p.s.base[k0 + i];
          if constexpr (MAX_HALF)
            mraw[j] = static_cast<const uint16_t*>(p.maxv)[t0 + tt];
          else
            mraw[j] = static_cast<const uint32_t*>(p.maxv)[t0 + tt];
        }
        cg += c_step;
        tt += t_step;
        if (cg >= G) {
          cg -= G;
          ++tt;
        }
      }
#pragma unroll
      for (int j = 0; j < kCgBatch; ++j) {
        if (bt[j] >= nt) break;
        // load_window's arithmetic on the loaded dwords
        const int sh = static_cast<int>(bo[j] & 3);
        const uint32_t lo = __builtin_amdgcn_alignbyte(w[j][1], w[j][0], sh);
        const uint32_t hi = NW > 2 ? __builtin_amdgcn_alignbyte(w[j][2], w[j][1], sh)
                                   : (w[j][1] >> (8 * sh));
        uint64_t x64 = (static_cast<uint64_t>(hi) << 32) | lo;
        const int64_t avail = p.s.bytes - bo[j];
        if (avail < BITS) x64 = avail <= 0 ? 0 : (x64 & ((uint64_t(1) << (8 * avail)) - 1));
        float m;
        if constexpr (MAX_HALF)
          m = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(mraw[j])));
        else
          m = __builtin_bit_cast(float, mraw[j]);
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t s0 = static_cast<uint32_t>(x64 >> ((2 * k) * BITS)) & mask;
          const uint32_t s1 = static_cast<uint32_t>(x64 >> ((2 * k + 1) * BITS)) & mask;
          o[k] = out_bits2<BF16>(lut[s0] * m, lut[s1] * m);
        }
        const u32x4 x = {o[0], o[1], o[2], o[3]};
        __builtin_nontemporal_store(
            x, reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(bt[j]) * p.C + bc[j] * 8));
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
// KIVI -> paged KV cache
// ---------------------------------------------------------------------------
//
// KIVI streams (bitpack_layout_cuda.cu:578-683, kivi_adapter.py:97-122) hold
// the body tokens [sink, tokens) plane-major with the token axis fastest:
// keys in plane order (head_dim, head), values in (head, head_dim).  Plane
// p's run starts at bit p * body * b.  Keys are dequantized per channel with
// groups along tokens (scale[bt / group][c]), values per token with groups
// along channels (scale[bt][c / group]); value = fmaf(s, scale, zero).
//
// Row kernel (C and head_dim multiples of 8, group a multiple of 16, block
// size >= 16): a lane owns 8 channels x LT body tokens (LT = 8 at widths up
// to 2 bits, else 16).  It reads its run of each of its 8 planes with dword
// loads (funnel-shifted when the run does not start on a dword), keeps it
// packed, and for every token extracts
// the 8 symbols, dequantizes them and writes one 16-byte store.  Eight lanes
// along channels cover a 128-byte line of a destination row; eight lanes
// along tokens read 8 * LT consecutive tokens of a plane.  A workgroup (2
// waves along channels) is 8 * LT tokens x 128 channels; the value metadata
// of its tokens is staged in LDS.

// Waves along channels per workgroup: 4 (256 channels) at widths up to 2
// bits, else 2.  Measured on a 32768-token Llama-3-8B layer in separate
// processes: at b = 2, 4 waves 37.0-38.4 us against 40.3-41.8 for 2; at
// b = 3, 2 waves 42.1-42.7 against 46.2-47.2 for 4; 8 and 16 waves (whole
// 2 KiB rows per workgroup) were slower at both widths.
constexpr int kivi_waves_c(int sbits) { return sbits <= 2 ? 4 : 2; }

// Body tokens per lane at `sbits` stored bits per symbol.  Fewer tokens per
// lane means more waves and shorter store bursts; more means longer plane
// runs.  Measured on a 32768-token Llama-3-8B layer: 16 tokens rather than 32
// at b = 3 (37.5-41.4 us against 48.0-48.2); 8 rather than 16 at b = 2 is
// within run-to-run variation.
constexpr int kivi_lane_tokens(int sbits) { return sbits <= 2 ? 8 : 16; }

struct KiviHalf {
  const uint8_t* sbase;  // 4-byte aligned base of the half's stream
  int64_t sbytes;        // readable bytes from sbase
  int64_t bit_bias;      // (stream start - sbase) * 8
  const void* scale;
  const void* zero;
  const void* sink;
};

struct KiviParams {
  KiviHalf half[2];      // 0: keys, 1: values
  uint16_t* cache;
  const int64_t* block_ids;
  int64_t num_blocks, bs, blk_stride, half_stride;
  int64_t sink, body;
  int64_t C, H, D;
  int64_t group, vgroups;
  int32_t nct;           // workgroups along channels
  int32_t ntiles;        // row-kernel tiles per half; workgroups past them copy sink rows
};

// Row index of token t of `half`, or -1 when its block id is outside the cache.
__device__ __forceinline__ int64_t kivi_row(const KiviParams& p, int half, int64_t blk,
                                            int64_t off) {
  const int64_t pid = p.block_ids[blk];
  if (pid < 0 || pid >= p.num_blocks) return -1;
  return pid * p.blk_stride + half * p.half_stride + off;
}

// Sink tokens [0, sink) of one half, 8 channels per thread (C % 8 == 0):
// workgroup `wg` of the extra workgroups that follow the row tiles.
template <bool BF16, bool META_HALF>
__device__ __forceinline__ void kivi_sink_rows(const KiviParams& p, int half, int64_t wg) {
  const int64_t G = p.C >> 3;
  const int64_t i = wg * blockDim.x + threadIdx.x;
  if (i >= p.sink * G) return;
  const int64_t t = i / G, g = i - t * G;
  const int64_t blk = t / p.bs;
  const int64_t row = kivi_row(p, half, blk, t - blk * p.bs);
  if (row < 0) return;
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e = t * p.C + g * 8 + 2 * k;
    o[k] = out_bits2<BF16>(load_meta<META_HALF>(p.half[half].sink, e),
                           load_meta<META_HALF>(p.half[half].sink, e + 1));
  }
  const u32x4 x = {o[0], o[1], o[2], o[3]};
  __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(p.cache + row * p.C + g * 8));
}

template <int SBITS>
struct KiviTileShape {
  static constexpr int kThreads = 64 * kivi_waves_c(SBITS);
  static constexpr int kChannels = kThreads;          // 8 channels x 8 lanes per wave
  static constexpr int kMaxGroups = kChannels / 16;   // value groups per tile (group >= 16)
  static constexpr int LT = kivi_lane_tokens(SBITS);
  static constexpr int TILE_T = 8 * LT;
};

// One row-kernel tile of half HALF (0 keys, 1 values).  The half is a template
// parameter so that no per-element branch on it remains in the store loop.
template <int HALF, int SBITS, bool NIB3, bool BF16, bool META_HALF>
__device__ __forceinline__ void kivi_tile(
    const KiviParams& p,
    float (&vmeta)[2][KiviTileShape<SBITS>::kMaxGroups][KiviTileShape<SBITS>::TILE_T]) {
  using Shape = KiviTileShape<SBITS>;
  constexpr int kKiviThreads = Shape::kThreads;
  constexpr int kKiviTileChannels = Shape::kChannels;
  constexpr int LT = Shape::LT;
  constexpr int NU = (LT * SBITS + 31) / 32;  // dwords holding a lane's plane run
  constexpr int CH = LT < 16 ? LT : 16;        // tokens per store chunk
  constexpr int TILE_T = Shape::TILE_T;
  constexpr uint32_t mask = NIB3 ? 0x7u : (1u << SBITS) - 1u;
  constexpr int half = HALF;
  const KiviHalf& hs = p.half[half];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Workgroups go to the 8 XCDs round-robin and each XCD has its own L2.
  // Give each XCD a contiguous range of tiles, so that the channel tiles of
  // one token range (which share their value metadata lines) and the token
  // tiles that share plane lines meet in the same L2.
  uint32_t tile = blockIdx.x;
  if (p.ntiles % kXcds == 0) tile = (tile % kXcds) * (p.ntiles / kXcds) + tile / kXcds;
  const int ct = static_cast<int>(tile % p.nct);
  const int64_t tile_bt0 = static_cast<int64_t>(tile / p.nct) * TILE_T;
  const int64_t tile_c0 = static_cast<int64_t>(ct) * kKiviTileChannels;
  const int64_t c0 = tile_c0 + wave * 64 + (lane & 7) * 8;
  const int64_t bt0 = tile_bt0 + (lane >> 3) * LT;

  // Value metadata of the tile: [scale / zero][group][token], staged once
  // (consecutive threads read consecutive groups of a token).
  const int64_t g_first = tile_c0 / p.group;
  if constexpr (HALF == 1) {
    const int64_t c_last = min(tile_c0 + kKiviTileChannels, p.C) - 1;
    const int ng = static_cast<int>(c_last / p.group - g_first + 1);
    for (int i = threadIdx.x; i < ng * TILE_T; i += kKiviThreads) {
      const int tt = i / ng, gi = i - tt * ng;
      const int64_t bt = tile_bt0 + tt;
      float sc = 0.f, ze = 0.f;
      if (bt < p.body) {
        const int64_t mi = bt * p.vgroups + g_first + gi;
        sc = load_meta<META_HALF>(hs.scale, mi);
        ze = load_meta<META_HALF>(hs.zero, mi);
      }
      vmeta[0][gi][tt] = sc;
      vmeta[1][gi][tt] = ze;
    }
    __syncthreads();
  }
  if (c0 >= p.C || bt0 >= p.body) return;

  // The lane's runs of its 8 planes, packed.  Key planes of consecutive
  // channels are H planes apart, value planes adjacent.
  const int64_t h = c0 / p.D, d0 = c0 - h * p.D;  // D % 8 == 0: one head
  const int64_t plane0 = half == 0 ? d0 * p.H + h : c0;
  const int64_t pstep = (half == 0 ? p.H : 1) * p.body * SBITS;
  const int64_t P0 = hs.bit_bias + (plane0 * p.body + bt0) * SBITS;
  // Every plane's dwords are requested before any funnel shift: with the
  // shift next to each plane's loads, the compiler waited for each plane's
  // data before requesting the next plane's.  A run whose dwords would pass
  // the end of the stream is read again dword by dword afterwards.
  uint32_t w[8][NU + 1];
  uint32_t tail = 0;     // bit i: plane i's dwords pass the end of the stream
  uint32_t shp[2] = {};  // byte i & 3 of shp[i >> 2]: plane i's funnel shift
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t P = P0 + i * pstep;
    const int64_t byte0 = (P >> 5) * 4;
    shp[i >> 2] |= static_cast<uint32_t>(P & 31) << (8 * (i & 3));
    if (byte0 + 4 * (NU + 1) <= hs.sbytes) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(hs.sbase + byte0);
#pragma unroll
      for (int k = 0; k <= NU; ++k) w[i][k] = src[k];
    } else {
      tail |= 1u << i;
    }
  }
  uint32_t u[8][NU];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t sh = (shp[i >> 2] >> (8 * (i & 3))) & 31u;
    if (tail & (1u << i)) {
      const int64_t byte0 = ((P0 + i * pstep) >> 5) * 4;
#pragma unroll
      for (int k = 0; k <= NU; ++k)
        w[i][k] = load_dword_guarded(hs.sbase, byte0 + 4 * k, hs.sbytes);
    }
#pragma unroll
    for (int k = 0; k < NU; ++k) u[i][k] = __builtin_amdgcn_alignbit(w[i][k + 1], w[i][k], sh);
  }

  const int nj = static_cast<int>(min<int64_t>(LT, p.body - bt0));
  const int gi = static_cast<int>(c0 / p.group - g_first);
  const int tt0 = static_cast<int>(bt0 - tile_bt0);

  // CH-token chunks: each lies in one key group (group % 16 == 0) and in at
  // most two blocks (block_size >= 16).
#pragma unroll
  for (int jb = 0; jb < LT / CH; ++jb) {
    if (CH * jb >= nj) break;
    float ks[8] = {}, kz[8] = {};
    if constexpr (HALF == 0) {
      const int64_t g = (bt0 + CH * jb) / p.group;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ks[i] = load_meta<META_HALF>(hs.scale, g * p.C + c0 + i);
        kz[i] = load_meta<META_HALF>(hs.zero, g * p.C + c0 + i);
      }
    }
    const int64_t t0 = p.sink + bt0 + CH * jb;
    const int64_t blk0 = t0 / p.bs;
    const int64_t off0 = t0 - blk0 * p.bs;
    const int jsplit = static_cast<int>(min<int64_t>(CH, p.bs - off0));
    const int64_t row_a = kivi_row(p, half, blk0, off0);
    const int64_t row_b = jsplit < nj - CH * jb ? kivi_row(p, half, blk0 + 1, 0) : -1;
    // the chunk's value metadata, read before its stores
    float vs[CH], vz[CH];
    if constexpr (HALF == 1) {
#pragma unroll
      for (int jj = 0; jj < CH; ++jj) {
        vs[jj] = vmeta[0][gi][tt0 + CH * jb + jj];
        vz[jj] = vmeta[1][gi][tt0 + CH * jb + jj];
      }
    }
    // the 8 dequantized values of token j, as 4 packed pairs
    auto token_bits = [&](int j, int jj, uint32_t (&o)[4]) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int bp = j * SBITS;
        const int dw = bp >> 5, off = bp & 31;
        uint32_t sym = u[i][dw] >> off;
        if (off + SBITS > 32) sym |= u[i][dw + 1] << (32 - off);
        const float s = static_cast<float>(sym & mask);
        if constexpr (HALF == 0) {
          v[i] = fma3(s, ks[i], kz[i]);
        } else {
          v[i] = fma3(s, vs[jj], vz[jj]);
        }
      }
      out_bits8<BF16>(v, o);
    };
    if (jsplit == CH) {
      // the chunk lies in one block: one row pointer, advanced a row per token
      if (row_a >= 0) {
        uint16_t* dst = p.cache + row_a * p.C + c0;
#pragma unroll
        for (int jj = 0; jj < CH; ++jj, dst += p.C) {
          const int j = CH * jb + jj;
          if (j < nj) {
            uint32_t o[4];
            token_bits(j, jj, o);
            const u32x4 x = {o[0], o[1], o[2], o[3]};
            __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dst));
          }
        }
      }
    } else {
      uint16_t* const dst_a = p.cache + row_a * p.C + c0;
      uint16_t* const dst_b = p.cache + row_b * p.C + c0;
#pragma unroll
      for (int jj = 0; jj < CH; ++jj) {
        const int j = CH * jb + jj;
        const bool second = jj >= jsplit;
        if (j < nj && (second ? row_b : row_a) >= 0) {
          uint32_t o[4];
          token_bits(j, jj, o);
          uint16_t* dst = second ? dst_b + (jj - jsplit) * p.C : dst_a + jj * p.C;
          const u32x4 x = {o[0], o[1], o[2], o[3]};
          __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dst));
        }
      }
    }
  }
}

template <int SBITS, bool NIB3, bool BF16, bool META_HALF>
__global__ __launch_bounds__(64 * kivi_waves_c(SBITS)) void kivi_cache_kernel(KiviParams p) {
  using Shape = KiviTileShape<SBITS>;
  __shared__ float vmeta[2][Shape::kMaxGroups][Shape::TILE_T];
  if (static_cast<int32_t>(blockIdx.x) >= p.ntiles) {
    kivi_sink_rows<BF16, META_HALF>(p, blockIdx.y, blockIdx.x - p.ntiles);
    return;
  }
  if (blockIdx.y == 0)
    kivi_tile<0, SBITS, NIB3, BF16, META_HALF>(p, vmeta);
  else
    kivi_tile<1, SBITS, NIB3, BF16, META_HALF>(p, vmeta);
}

// One thread per destination element of both halves: any shape, any group,
// any alignment (the reference kernel's mapping).
template <bool BF16, bool META_HALF>
__global__ __launch_bounds__(kDqThreads) void kivi_generic_kernel(KiviParams p, int32_t bits,
                                                                  int32_t nib3,
                                                                  int64_t block_count) {
  const int64_t per_half = p.bs * p.C;
  const int64_t total = block_count * 2 * per_half;
  const int64_t tokens = p.sink + p.body;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kDqThreads + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kDqThreads) {
    const int64_t lb = idx / (2 * per_half);
    const int64_t r0 = idx - lb * 2 * per_half;
    const int half = static_cast<int>(r0 / per_half);
    const int64_t r = r0 - half * per_half;
    const int64_t off = r / p.C;
    const int64_t ch = r - off * p.C;
    const int64_t t = lb * p.bs + off;
    if (t >= tokens) continue;
    const int64_t row = kivi_row(p, half, lb, off);
    if (row < 0) continue;
    const KiviHalf& hs = p.half[half];
    float v;
    if (t < p.sink) {
      v = load_meta<META_HALF>(hs.sink, t * p.C + ch);
    } else {
      const int64_t bt = t - p.sink;
      const int64_t h = ch / p.D, d = ch - h * p.D;
      const int64_t idx_s = (half == 0 ? d * p.H + h : h * p.D + d) * p.body + bt;
      uint32_t sv;
      if (nib3) {
        const int64_t o = (hs.bit_bias >> 3) + (idx_s >> 1);
        const uint32_t w = static_cast<uint32_t>(load_window<1>(
            ByteStream{reinterpret_cast<const uint32_t*>(hs.sbase), hs.sbytes, 0}, o));
        sv = (w >> (4 * (idx_s & 1))) & 0x7u;
      } else {
        const int64_t bit = hs.bit_bias + idx_s * bits;
        const uint64_t w = load_window<2>(
            ByteStream{reinterpret_cast<const uint32_t*>(hs.sbase), hs.sbytes, 0}, bit >> 3);
        sv = static_cast<uint32_t>(w >> (bit & 7)) & ((1u << bits) - 1u);
      }
      int64_t mi;
      if (half == 0) {
        mi = (bt / p.group) * p.C + ch;
      } else {
        mi = bt * p.vgroups + ch / p.group;
      }
      v = __builtin_fmaf(static_cast<float>(sv), load_meta<META_HALF>(hs.scale, mi),
                         load_meta<META_HALF>(hs.zero, mi));
    }
    p.cache[row * p.C + ch] = static_cast<uint16_t>(out_bits<BF16>(v));
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
  const dim3 grid(grid_for(p.block_count, 1, kMaxDqGrid)), block(kCgThreads);
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

template <int SBITS, bool NIB3, bool BF16, bool META_HALF>
int launch_kivi_rows(const KiviParams& params, int64_t body, hipStream_t stream) {
  constexpr int64_t tile_t = 8 * kivi_lane_tokens(SBITS);
  constexpr int threads = 64 * kivi_waves_c(SBITS);
  const int64_t nst = (body + tile_t - 1) / tile_t;
  const int64_t sink_wgs = (params.sink * (params.C / 8) + threads - 1) / threads;
  KiviParams p = params;
  p.nct = static_cast<int32_t>((p.C + threads - 1) / threads);
  ORIGAMI_REQUIRE(p.nct * nst + sink_wgs <= INT32_MAX, "KIVI layer exceeds the launch grid");
  p.ntiles = static_cast<int32_t>(p.nct * nst);
  const dim3 grid(static_cast<unsigned>(p.ntiles + sink_wgs), 2);
  hipLaunchKernelGGL((kivi_cache_kernel<SBITS, NIB3, BF16, META_HALF>), grid, dim3(threads),
                     0, stream, p);
  return check_launch("kivi_cache_kernel");
}

template <bool BF16, bool META_HALF>
int launch_kivi_cache(const KiviParams& p, int64_t body, int sbits, bool nib3,
                      hipStream_t stream) {
  if (nib3) return launch_kivi_rows<4, true, BF16, META_HALF>(p, body, stream);
  switch (sbits) {
    case 1: return launch_kivi_rows<1, false, BF16, META_HALF>(p, body, stream);
    case 2: return launch_kivi_rows<2, false, BF16, META_HALF>(p, body, stream);
    case 3: return launch_kivi_rows<3, false, BF16, META_HALF>(p, body, stream);
    case 4: return launch_kivi_rows<4, false, BF16, META_HALF>(p, body, stream);
    case 5: return launch_kivi_rows<5, false, BF16, META_HALF>(p, body, stream);
    case 6: return launch_kivi_rows<6, false, BF16, META_HALF>(p, body, stream);
    case 7: return launch_kivi_rows<7, false, BF16, META_HALF>(p, body, stream);
    case 8: return launch_kivi_rows<8, false, BF16, META_HALF>(p, body, stream);
    default: return check_bits(sbits);
  }
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

int origami_kivi_dequantize_to_kv_cache(
    const uint8_t* bytestream, int64_t bytestream_bytes, int64_t key_offset, int64_t key_bytes,
    int64_t value_offset, int64_t value_bytes, int64_t bits, int64_t symbol_packing,
    int64_t group_size, int64_t sink_tokens, const void* key_scale, const void* key_zero,
    const void* value_scale, const void* value_zero, const void* key_sink,
    const void* value_sink, const int64_t* meta_counts, int64_t meta_dtype, void* kv_cache,
    int64_t cache_dtype, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    const int64_t* block_ids, int64_t block_count, int64_t tokens, int64_t heads,
    int64_t head_dim, origami_stream_t stream) {
  ORIGAMI_REQUIRE(cache_dtype == ORIGAMI_DTYPE_FLOAT16 || cache_dtype == ORIGAMI_DTYPE_BFLOAT16,
                  "kv_cache must be float16 or bfloat16");
  ORIGAMI_REQUIRE(meta_dtype == ORIGAMI_DTYPE_FLOAT16 || meta_dtype == ORIGAMI_DTYPE_FLOAT32,
                  "KIVI metadata tensors must be float16 or float32");
  if (int rc = check_bits(bits)) return rc;
  ORIGAMI_REQUIRE(symbol_packing == ORIGAMI_KIVI_PACKED_LSB ||
                      symbol_packing == ORIGAMI_KIVI_NIBBLE3,
                  "unknown KIVI symbol packing");
  ORIGAMI_REQUIRE(group_size > 0, "KIVI group_size must be positive");
  ORIGAMI_REQUIRE(sink_tokens >= 0 && sink_tokens <= tokens,
                  "KIVI sink_tokens must be in [0, tokens]");
  ORIGAMI_REQUIRE(tokens > 0 && heads > 0 && head_dim > 0,
                  "tokens, heads, and head_dim must be positive");
  ORIGAMI_REQUIRE(key_offset >= 0 && key_bytes >= 0 && value_offset >= 0 && value_bytes >= 0,
                  "invalid KIVI stream offsets");
  ORIGAMI_REQUIRE(key_offset + key_bytes <= bytestream_bytes &&
                      value_offset + value_bytes <= bytestream_bytes,
                  "KIVI stream ranges exceed bytestream length");
  const int64_t body = tokens - sink_tokens;
  const int64_t C = heads * head_dim;
  ORIGAMI_REQUIRE(C <= (int64_t(1) << 24), "heads * head_dim exceeds 2^24");
  const int64_t key_groups = (body + group_size - 1) / group_size;
  const int64_t value_groups = (C + group_size - 1) / group_size;
  ORIGAMI_REQUIRE(meta_counts[0] >= key_groups * C && meta_counts[1] >= key_groups * C,
                  "KIVI key metadata is too small");
  ORIGAMI_REQUIRE(meta_counts[2] >= body * value_groups && meta_counts[3] >= body * value_groups,
                  "KIVI value metadata is too small");
  ORIGAMI_REQUIRE(meta_counts[4] >= sink_tokens * C && meta_counts[5] >= sink_tokens * C,
                  "KIVI sink metadata is too small");
  const size_t esize = meta_dtype == ORIGAMI_DTYPE_FLOAT16 ? 2 : 4;
  const void* metas[6] = {key_scale, key_zero, value_scale, value_zero, key_sink, value_sink};
  for (const void* m : metas) {
    ORIGAMI_REQUIRE(reinterpret_cast<uintptr_t>(m) % esize == 0,
                    "KIVI metadata must be aligned to its element size");
  }
  ORIGAMI_REQUIRE(block_size > 0, "kv_cache block size must be positive");
  ORIGAMI_REQUIRE(num_blocks > 0, "kv_cache must hold at least one block");
  ORIGAMI_REQUIRE(block_count > 0, "block_ids must be non-empty");
  ORIGAMI_REQUIRE(tokens <= block_count * block_size, "tokens exceed destination block capacity");
  KiviParams p{};
  if (int rc = cache_geometry(cache_layout, num_blocks, block_size, &p.blk_stride,
                              &p.half_stride))
    return rc;
  const int64_t offs[2] = {key_offset, value_offset};
  const int64_t lens[2] = {key_bytes, value_bytes};
  for (int half = 0; half < 2; ++half) {
    const ByteStream bs = make_stream(bytestream + offs[half], lens[half]);
    p.half[half].sbase = reinterpret_cast<const uint8_t*>(bs.base);
    p.half[half].sbytes = bs.bytes;
    p.half[half].bit_bias = static_cast<int64_t>(bs.bias) * 8;
    p.half[half].scale = half == 0 ? key_scale : value_scale;
    p.half[half].zero = half == 0 ? key_zero : value_zero;
    p.half[half].sink = half == 0 ? key_sink : value_sink;
  }
  p.cache = static_cast<uint16_t*>(kv_cache);
  p.block_ids = block_ids;
  p.num_blocks = num_blocks;
  p.bs = block_size;
  p.sink = sink_tokens;
  p.body = body;
  p.C = C;
  p.H = heads;
  p.D = head_dim;
  p.group = group_size;
  p.vgroups = value_groups;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool bf16 = cache_dtype == ORIGAMI_DTYPE_BFLOAT16;
  const bool mhalf = meta_dtype == ORIGAMI_DTYPE_FLOAT16;
  const bool nib3 = symbol_packing == ORIGAMI_KIVI_NIBBLE3 && bits == 3;
  const int sbits = nib3 ? 4 : static_cast<int>(bits);

  const bool rows = C % 8 == 0 && head_dim % 8 == 0 && group_size % 16 == 0 &&
                    block_size >= 16 && aligned16(kv_cache);
  if (!rows) {
    const dim3 grid(grid_for(block_count * 2 * block_size * C, kDqThreads, 65536));
#define ORIGAMI_KIVI_GENERIC(BF, MH)                                                          \
  hipLaunchKernelGGL((kivi_generic_kernel<BF, MH>), grid, dim3(kDqThreads), 0, st, p,          \
                     static_cast<int32_t>(bits), static_cast<int32_t>(nib3), block_count)
    if (bf16) {
      if (mhalf) ORIGAMI_KIVI_GENERIC(true, true); else ORIGAMI_KIVI_GENERIC(true, false);
    } else {
      if (mhalf) ORIGAMI_KIVI_GENERIC(false, true); else ORIGAMI_KIVI_GENERIC(false, false);
    }
#undef ORIGAMI_KIVI_GENERIC
    return check_launch("kivi_generic_kernel");
  }
  if (bf16) {
    return mhalf ? launch_kivi_cache<true, true>(p, body, sbits, nib3, st)
                 : launch_kivi_cache<true, false>(p, body, sbits, nib3, st);
  }
  return mhalf ? launch_kivi_cache<false, true>(p, body, sbits, nib3, st)
               : launch_kivi_cache<false, false>(p, body, sbits, nib3, st);
}

}  // extern "C"
