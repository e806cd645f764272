// origami_layout.hip -- MI355X (gfx950) kernels and C ABI for Origami's
// canonical KV codec layout: pack, unpack, fused unpack+scatter into the paged
// KV cache, fused gather+pack from it, and paged block copies.
//
// Canonical format (the reference decoder, csrc/origami/bitpack_layout_cuda.cu
// :70-128): a layer's uint8 symbol tensor is cut into chunks
// [head range x channel range x token range]; inside a chunk symbols run
// head-major, then channel, token fastest, packed LSB-first at b bits
// (b = 8 is the identity).  A "plane" is one (head, channel) pair: its token
// run is contiguous in the stream.
//
// Kernel design (wave64, 16-byte lanes):
//  * rows kernels (the hot path).  A lane owns a 16-channel x 16-token byte
//    tile.  It reads the 16 planes' 16-token runs (2b bytes each: one vector
//    load per run, see RowsMode), transposes the 16x16 bytes in registers
//    with v_perm_b32, and writes 16 destination rows of 16 bytes.  Eight
//    lanes share a channel group and cover 128 consecutive tokens (a full
//    128-byte line of a plane per load instruction at b = 8); eight lanes
//    share a token and cover 128 consecutive channels (a full 128-byte line
//    of a destination row per store instruction).  No LDS is needed for the
//    data; LDS holds only the plane descriptors a workgroup shares.
//  * generic kernels: one thread per symbol / per output byte, for layouts the
//    rows kernels do not serve (irregular chunk plans, channel-major layouts).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "origami_internal.h"
#include "origami_layout.h"

// ---------------------------------------------------------------------------
// Errors and shared host helpers (declared in origami_internal.h)
// ---------------------------------------------------------------------------

namespace origami_internal {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(ORIGAMI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
  }
  return ORIGAMI_OK;
}

int cache_geometry(int64_t cache_layout, int64_t num_blocks, int64_t block_size,
                   int64_t* blk_stride, int64_t* half_stride) {
  if (cache_layout == ORIGAMI_CACHE_KV_FIRST) {
    *blk_stride = block_size;               // [2, NB, bs, H, D]
    *half_stride = num_blocks * block_size;
  } else if (cache_layout == ORIGAMI_CACHE_BLOCKS_FIRST) {
    *blk_stride = 2 * block_size;           // [NB, 2, bs, H, D]
    *half_stride = block_size;
  } else {
    return fail(ORIGAMI_ERR_INVALID,
                "kv_cache must be [num_blocks,2,block,heads,dim] or [2,num_blocks,block,heads,dim]");
  }
  return ORIGAMI_OK;
}

}  // namespace origami_internal

using namespace origami_internal;

namespace {

// Upper bound on the workgroups of one rows-kernel launch on this thread
// (0: one workgroup per tile).  A restore that runs hidden behind other work
// can be spread thinner over the GPU with it.
thread_local int64_t g_rows_grid_limit = 0;

// ---------------------------------------------------------------------------
// Host-side layout helpers
// ---------------------------------------------------------------------------

struct Strides {
  int64_t token, head, channel;
};

int64_t spec_symbols(const int64_t* s) {
  return (s[1] - s[0]) * (s[3] - s[2]) * (s[5] - s[4]);
}

// Validation the reference performs in read_source_layout / read_chunk_specs
// / check_bits / the byte-size loop (bitpack_layout_cuda.cpp:43-185, 326-362),
// with the same messages, plus stream bounds the reference does not check.
int validate_layout(const int64_t* offsets, const int64_t* bits,
                    const int64_t* specs, int64_t n, const int64_t* shape,
                    int64_t rank, const int64_t* axes, int64_t token_count,
                    int64_t num_heads, int64_t head_dim, int64_t flat_bytes,
                    Strides* strides) {
  ORIGAMI_REQUIRE(n >= 0, "chunk count must be non-negative");
  ORIGAMI_REQUIRE(token_count > 0 && num_heads > 0 && head_dim > 0,
                  "canonical symbol shape must be positive");
  ORIGAMI_REQUIRE(rank == 3 || rank == 4,
                  "Origami source layout supports rank 3 or rank 4");
  int64_t stride[4] = {1, 1, 1, 1};
  for (int64_t a = 0; a < rank; ++a)
    ORIGAMI_REQUIRE(shape[a] > 0, "source_shape dimensions must be positive");
  for (int64_t a = rank - 2; a >= 0; --a) stride[a] = stride[a + 1] * shape[a + 1];
  ORIGAMI_REQUIRE(axes[0] >= 0 && axes[0] < rank,
                  "token axis must be present in source layout");
  ORIGAMI_REQUIRE(axes[1] >= 0 && axes[1] < rank,
                  "head axis must be present in source layout");
  ORIGAMI_REQUIRE(axes[2] >= 0 && axes[2] < rank,
                  "head_dim axis must be present in source layout");
  ORIGAMI_REQUIRE(axes[3] == -1 || (axes[3] >= 0 && axes[3] < rank),
                  "layer axis must be -1 or present in source layout");
  ORIGAMI_REQUIRE(shape[axes[0]] == token_count,
                  "source token axis size must match token_count");
  ORIGAMI_REQUIRE(shape[axes[1]] == num_heads,
                  "source head axis size must match num_heads");
  ORIGAMI_REQUIRE(shape[axes[2]] == head_dim,
                  "source head_dim axis size must match head_dim");
  if (axes[3] != -1)
    ORIGAMI_REQUIRE(shape[axes[3]] == 1,
                    "per-layer Origami native layout requires layer axis size 1");
  {
    // the four axes must be distinct
    bool seen[4] = {false, false, false, false};
    for (int i = 0; i < 4; ++i) {
      if (axes[i] < 0) continue;
      ORIGAMI_REQUIRE(!seen[axes[i]], "source layout axes must be unique");
      seen[axes[i]] = true;
    }
  }
  if (n > 0) ORIGAMI_REQUIRE(offsets[0] >= 0, "chunk_offsets must be non-negative");
  for (int64_t k = 0; k < n; ++k) {
    const int64_t* s = specs + 6 * k;
    ORIGAMI_REQUIRE(0 <= s[0] && s[0] < s[1] && s[1] <= num_heads,
                    "invalid head range in Origami chunk spec");
    ORIGAMI_REQUIRE(0 <= s[2] && s[2] < s[3] && s[3] <= head_dim,
                    "invalid channel range in Origami chunk spec");
    ORIGAMI_REQUIRE(0 <= s[4] && s[4] < s[5] && s[5] <= token_count,
                    "invalid token range in Origami chunk spec");
    ORIGAMI_REQUIRE(bits[k] >= 1 && bits[k] <= 8,
                    "Origami CUDA bitpack supports only 1..8 bit symbols");
    ORIGAMI_REQUIRE(offsets[k + 1] - offsets[k] == (spec_symbols(s) * bits[k] + 7) / 8,
                    "Origami CUDA packed chunk byte size mismatch");
  }
  if (n > 0)
    ORIGAMI_REQUIRE(offsets[n] <= flat_bytes,
                    "chunk_offsets exceed the flat stream length");
  if (strides) {
    strides->token = stride[axes[0]];
    strides->head = stride[axes[1]];
    strides->channel = stride[axes[2]];
  }
  return ORIGAMI_OK;
}

// ---------------------------------------------------------------------------
// Plans: host plane table + device copies of the metadata, cached per layout
// ---------------------------------------------------------------------------

constexpr int64_t kMaxPlaneTable = int64_t(1) << 20;  // planes per plan (8 MiB)
constexpr size_t kMaxPlans = 256;

struct PlanInfo {
  bool regular = false;      // full token span per chunk, no plane twice
  int bits = 0;              // uniform symbol width, 0 when mixed
  bool aligned16 = false;    // every plane starts on a 16-byte boundary
  bool byte_aligned = false; // every plane starts on a byte boundary
  bool planes_even = false;  // every plane starts on a 2-byte boundary
  bool planes_dword = false; // every plane starts on a 4-byte boundary
  bool lines128 = false;     // every plane starts on a 128-byte line (b = 8)
  bool planes16 = false;     // every plane starts on a 16-byte boundary (any b)
  bool planes_lines = false; // every plane starts on a 128-byte line (any b)
  // Every plane p = h * C + c is covered and starts at bit dense_base + p * T *
  // bits: the plane table is a closed form (what the chunk planner produces),
  // so the row kernels compute descriptors instead of reading a table.
  bool dense = false;
  int64_t dense_base = 0;
};

// Builds the plane table: table[h*C + c] = bit offset of token 0 of plane
// (h, c), or -1.  Local plane order inside a chunk is head-major then channel
// (bitpack_layout_cuda.cu:110-124), so plane (h, c) of chunk k starts at
// symbol ((h - hs) * Cc + (c - cs)) * Tc.
PlanInfo build_plane_table(const int64_t* offsets, const int64_t* bits,
                           const int64_t* specs, int64_t n, int64_t T,
                           int64_t H, int64_t C, int64_t* table) {
  PlanInfo info;
  std::fill(table, table + H * C, int64_t(-1));
  info.regular = n > 0;
  info.bits = n > 0 ? static_cast<int>(bits[0]) : 0;
  info.aligned16 = true;
  info.byte_aligned = true;
  info.planes_even = true;
  info.planes_dword = true;
  info.lines128 = true;
  info.planes16 = info.planes_lines = true;
  for (int64_t k = 0; k < n; ++k) {
    const int64_t* s = specs + 6 * k;
    if (bits[k] != info.bits) info.bits = 0;
    if (s[4] != 0 || s[5] != T) {
      info.regular = false;
      continue;
    }
    const int64_t Cc = s[3] - s[2];
    for (int64_t h = s[0]; h < s[1]; ++h) {
      for (int64_t c = s[2]; c < s[3]; ++c) {
        const int64_t local = (h - s[0]) * Cc + (c - s[2]);
        const int64_t bit_off = offsets[k] * 8 + local * T * bits[k];
        int64_t& slot = table[h * C + c];
        if (slot != -1) info.regular = false;
        slot = bit_off;
        if (bit_off % 128 != 0) info.aligned16 = info.planes16 = false;
        if (bit_off % 1024 != 0) info.lines128 = info.planes_lines = false;
        if (bit_off % 8 != 0) info.byte_aligned = false;
        if (bit_off % 16 != 0) info.planes_even = false;
        if (bit_off % 32 != 0) info.planes_dword = false;
      }
    }
  }
  if (info.bits != 8) info.aligned16 = false;
  if (!info.aligned16) info.lines128 = false;
  if (!info.planes16) info.planes_lines = false;
  if (!info.regular) {
    info.aligned16 = false;
    info.lines128 = false;
    info.planes16 = info.planes_lines = false;
    info.byte_aligned = false;
    info.planes_even = false;
    info.planes_dword = false;
  }
  if (info.regular && info.bits != 0 && H * C > 0) {
    info.dense = true;
    info.dense_base = table[0];
    const int64_t stride = T * info.bits;
    for (int64_t p = 0; p < H * C && info.dense; ++p)
      info.dense = table[p] == info.dense_base + p * stride;
  }
  return info;
}

struct Plan {
  Plan() = default;
  Plan(const Plan&) = delete;
  Plan& operator=(const Plan&) = delete;
  ~Plan() {
    if (dev) (void)hipFree(dev);  // hipFree waits for work still reading it
  }
  int device = -1;
  bool want_table = false;
  int64_t n = 0, T = 0, H = 0, C = 0, max_symbols = 0;
  PlanInfo info;
  bool has_table = false;    // info was computed (row-kernel layout)
  std::vector<int64_t> host; // offsets | bits | specs | table (table only if not dense)
  void* dev = nullptr;       // device copy of `host`, made on first need
  const int64_t* d_offsets = nullptr;
  const int64_t* d_bits = nullptr;
  const int64_t* d_specs = nullptr;
  const int64_t* d_table = nullptr;
};

std::mutex g_plan_mutex;
std::unordered_map<uint64_t, std::vector<std::shared_ptr<Plan>>> g_plans;
size_t g_plan_count = 0;         // plans in the cache
size_t g_plan_device_count = 0;  // of which hold device memory
// Totals since the library was loaded (origami_debug_counters).
std::atomic<int64_t> g_plans_created{0};
std::atomic<int64_t> g_device_allocations{0};
constexpr size_t kMaxHostPlans = 4096;

uint64_t hash_words(uint64_t h, const int64_t* w, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    h ^= static_cast<uint64_t>(w[i]);
    h *= 1099511628211ull;
    h ^= h >> 29;
  }
  return h;
}

// True when `plan` was built from exactly this metadata (its host copy holds
// offsets | bits | specs).
bool plan_matches(const Plan& plan, const int64_t* offsets, const int64_t* bits,
                  const int64_t* specs, int64_t n, int64_t T, int64_t H, int64_t C,
                  int device, bool want_table) {
  if (plan.n != n || plan.T != T || plan.H != H || plan.C != C || plan.device != device ||
      plan.want_table != want_table)
    return false;
  const int64_t* h = plan.host.data();
  const size_t w = sizeof(int64_t);
  return std::memcmp(h, offsets, (n + 1) * w) == 0 &&
         std::memcmp(h + (n + 1), bits, n * w) == 0 &&
         std::memcmp(h + (n + 1) + n, specs, 6 * n * w) == 0;
}

void drop_all_plans() {
  // Kernels may still read cached metadata: wait for the device first (only
  // when some plan holds device memory; dense row layouts never do).
  if (g_plan_device_count > 0) (void)hipDeviceSynchronize();
  g_plans.clear();  // plans a caller still holds live on until it lets go
  g_plan_count = 0;
  g_plan_device_count = 0;
}

// Uploads the plan's metadata (chunk offsets, bits, specs and, unless the
// layout is dense, the plane table) on first need: one hipMalloc and one
// synchronous copy per distinct layout.
int plan_device(const std::shared_ptr<const Plan>& cplan) {
  Plan* plan = const_cast<Plan*>(cplan.get());
  std::lock_guard<std::mutex> lock(g_plan_mutex);
  if (plan->dev) return ORIGAMI_OK;
  const size_t words = plan->host.size();
  if (hipMalloc(&plan->dev, words * sizeof(int64_t)) != hipSuccess) {
    plan->dev = nullptr;
    return fail(ORIGAMI_ERR_HIP, "hipMalloc of the layout plan failed");
  }
  g_device_allocations.fetch_add(1, std::memory_order_relaxed);
  if (hipMemcpy(plan->dev, plan->host.data(), words * sizeof(int64_t), hipMemcpyHostToDevice) !=
      hipSuccess) {
    (void)hipFree(plan->dev);
    plan->dev = nullptr;
    return fail(ORIGAMI_ERR_HIP, "upload of the layout plan failed");
  }
  const int64_t n = plan->n;
  const int64_t* base = static_cast<const int64_t*>(plan->dev);
  plan->d_offsets = base;
  plan->d_bits = base + (n + 1);
  plan->d_specs = base + (n + 1) + n;
  plan->d_table = words > static_cast<size_t>(8 * n + 1) ? base + (n + 1) + n + 6 * n : nullptr;
  ++g_plan_device_count;
  return ORIGAMI_OK;
}

// Returns the cached plan for this metadata on the current device, creating
// its host part on first use.  Device copies are made by plan_device(), only
// for paths that read metadata on the device (generic kernels, row kernels
// over a non-dense plane table).
int get_plan(const int64_t* offsets, const int64_t* bits, const int64_t* specs,
             int64_t n, int64_t T, int64_t H, int64_t C, bool want_table,
             std::shared_ptr<const Plan>* out) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess)
    return fail(ORIGAMI_ERR_HIP, "hipGetDevice failed");
  const int64_t dims[6] = {n, T, H, C, device, want_table ? 1 : 0};
  uint64_t h = hash_words(1469598103934665603ull, dims, 6);
  h = hash_words(h, offsets, n + 1);
  h = hash_words(h, bits, n);
  h = hash_words(h, specs, 6 * n);

  std::lock_guard<std::mutex> lock(g_plan_mutex);
  auto it = g_plans.find(h);
  if (it != g_plans.end()) {
    for (auto& p : it->second) {
      if (plan_matches(*p, offsets, bits, specs, n, T, H, C, device, want_table)) {
        *out = p;
        return ORIGAMI_OK;
      }
    }
  }
  if (g_plan_device_count >= kMaxPlans || g_plan_count >= kMaxHostPlans) drop_all_plans();

  auto plan = std::make_shared<Plan>();
  plan->want_table = want_table;
  plan->device = device;
  plan->n = n;
  plan->T = T;
  plan->H = H;
  plan->C = C;
  for (int64_t k = 0; k < n; ++k)
    plan->max_symbols = std::max(plan->max_symbols, spec_symbols(specs + 6 * k));
  std::vector<int64_t> table;
  if (want_table && H * C <= kMaxPlaneTable) {
    table.resize(static_cast<size_t>(H * C));
    plan->info = build_plane_table(offsets, bits, specs, n, T, H, C, table.data());
    plan->has_table = true;
    if (plan->info.dense) table.clear();  // the kernels compute it
  }
  std::vector<int64_t>& host = plan->host;
  host.reserve(static_cast<size_t>((n + 1) + n + 6 * n) + table.size());
  host.insert(host.end(), offsets, offsets + n + 1);
  host.insert(host.end(), bits, bits + n);
  host.insert(host.end(), specs, specs + 6 * n);
  host.insert(host.end(), table.begin(), table.end());
  *out = plan;
  g_plans[h].push_back(std::move(plan));
  ++g_plan_count;
  g_plans_created.fetch_add(1, std::memory_order_relaxed);
  return ORIGAMI_OK;
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

constexpr int kThreads = 256;          // generic and block-copy kernels

// Rows kernels: a lane owns 16 channels x 16 tokens; a wave tile is 8 lanes
// along channels x 8 lanes along tokens (128 channels x 128 tokens); a
// workgroup is normally 16 wave tiles arranged wq x (16 / wq), wq <= 2, i.e.
// up to 256 channels x 1024 tokens.  Large tiles keep both the plane runs read
// (1 KiB) and the row segments written (256 B) long, which is what HBM
// rewards; 2 x 8 measured 0.4-2% faster than 4 x 4 and 1 x 16.  A launch with too few such tiles to give every CU two uses 8- or
// 4-wave workgroups (wq <= 2) instead: a CU only moves about 1/256 of HBM
// bandwidth, so idle CUs cost more than short runs.
constexpr int kRowsMaxWaves = 16;
constexpr int kRowsThreads = kRowsMaxWaves * 64;  // launch bound
// A restore launch with at least kRowsSplitTiles tiles per CU dispatches each
// tile as waves / kRowsSplitWaves workgroups of kRowsSplitWaves waves, each a
// column of wave tiles along tokens (same tile geometry and order).  Per layer:
// 70B layer (8 tiles per CU) 233.9 -> 224.0 us against whole-tile workgroups.
// Launches of 2 tiles per CU stay whole-tile: the 32768-token layer ran 53.7 us
// whole against 58.4 us in 4-wave slices (8-wave slices: 59.7 us), and batched
// restores gained nothing.
constexpr int kRowsSplitWaves = 4;
constexpr int kRowsSplitTiles = 4;
constexpr int kSegTokens = 16;         // tokens per lane
constexpr int kLaneSegs = 8;           // lanes along tokens in a wave tile
constexpr int kLaneGroups = 8;         // lanes along 16-channel groups
constexpr int kWavePlanes = kLaneGroups * 16;  // channels per wave tile (128)
constexpr int kMaxWq = 16;
constexpr int kRowsWq = 2;  // wave tiles along channels when the row is wide enough
constexpr int kTilePlanes = kMaxWq * kWavePlanes;  // descriptor slots per workgroup

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Multi-dword vectors at 4-byte alignment (one global load or store each).
typedef unsigned int u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef unsigned int u32x3a4 __attribute__((ext_vector_type(3), aligned(4)));
typedef unsigned int u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// How the row kernels address a lane's run of 16 packed symbols (2 * b bytes
// at bit P of the stream).
enum RowsMode : int {
  kRowsWindow = 1,     // runs start on even bytes (odd b) or dwords (even b)
  kRowsAligned16 = 2,  // b = 8 and runs start on 16-byte boundaries
  kRowsShift = 3,      // unpack: runs start at any bit, any token count
  kRowsBytes = 4,      // pack: runs start on bytes, any token count
  // b = 8, runs on 16-byte boundaries but not all on 128-byte lines: the
  // 128 bytes that 8 lanes read or write then span two lines, each shared
  // with the neighbouring wave, so the stream goes through the L2 normally
  // (non-temporal loads here ran a 32784-token layer in 71.7 us, cached
  // ones in 64.1 us; on 128-byte lines non-temporal is faster: 53.8 vs 56.3).
  kRowsAligned16Cached = 5,
  // pack, b = 8, runs not all on 128-byte lines: through LDS, each stream
  // line written whole by one wave (rows_pack_staged8_kernel)
  kRowsStaged8 = 6,
  // restore, b = 1, 2 or 4, runs on 16-byte boundaries, T % (128 / b) == 0:
  // 16-byte runs of 128 / b tokens per lane (rows_unpack_wide_kernel),
  // non-temporal when every group's 8 runs are one 128-byte line
  kRowsWide = 7,
  kRowsWideCached = 8,
  // pack, b < 8, planes not all on bytes (T * b % 8 != 0 or unaligned chunk
  // planes): runs start at any bit and are ORed into the cleared stream
  kRowsBits = 9,
};

struct RowsParams {
  uint8_t* stream;           // 4-byte aligned base of the flat stream
  int64_t stream_bytes;      // bytes addressable from `stream`
  int64_t bit_bias;          // (caller's stream pointer - stream) * 8
  const int64_t* planes;     // [H*C] plane bit offsets (caller pointer based), or
                             // nullptr: plane p starts at plane_base + p * plane_bits
  int64_t plane_base, plane_bits;
  uint8_t* rows;             // row base: destination (unpack) or source (pack)
  const int64_t* block_ids;  // nullptr: identity rows
  int64_t num_blocks;        // valid block ids are [0, num_blocks)
  int64_t T;                 // valid tokens per half
  int64_t row_tokens;        // destination tokens per half
  int64_t C;                 // channels (bytes) per head
  int64_t row_pitch;         // bytes between consecutive rows
  int64_t head_pitch;        // bytes between heads inside a row
  int64_t bs;                // rows per block
  int64_t blk_stride;        // rows per block-id step
  int64_t half_stride;       // rows per half step
  int32_t H;
  int32_t nq;                // C / 16
  int32_t waves;             // waves per workgroup (16, 8 or 4)
  int32_t wq;                // wave tiles along channels per workgroup (1, 2, 4)
  int32_t ws;                // wave tiles along tokens per workgroup (waves / wq)
  int32_t nqt;               // workgroups along channels
  int32_t nst;               // workgroups along tokens
  int64_t ntiles;            // workgroup tiles; a workgroup loops over tiles
  int32_t partial_last;      // the last token tile is partial: order those tiles last
  int64_t token0;            // first destination token of the tiles (a multiple of 16)
  int32_t nt_stores;         // staged pack: whole 16-byte chunks as non-temporal stores
  int32_t own_lines;         // staged pack: each stream line written by one tile (16 waves)
};

// Per-request fields of a batched restore (one layer of several requests
// into one cache, one launch); the rest of RowsParams is shared.
struct RowsRequest {
  uint8_t* stream;
  int64_t stream_bytes, bit_bias;
  const int64_t* planes;
  int64_t plane_base, plane_bits;
  const int64_t* block_ids;
  int64_t T, row_tokens;
  int64_t token0;  // tokens [token0, row_tokens) are restored
  int64_t tile0;   // first full-token-tile workgroup tile of the request
  int64_t ptile0;  // first partial-token-tile workgroup tile of the request
  int32_t nst;
  int32_t partial;  // 1: the last token tile is partial
  int32_t nt;       // aligned16 batches: 1 = non-temporal loads (runs on 128-byte lines)
};

constexpr int kBatchRequests = 16;  // requests per batched launch (kernel arguments)

struct RowsBatch {
  RowsParams common;
  int64_t nfull;  // tiles [0, nfull) are full token tiles
  int32_t nreq;
  RowsRequest req[kBatchRequests];
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4x4 byte transpose: o_r byte i = a_i byte r.
__device__ __forceinline__ void transpose4x4(uint32_t a0, uint32_t a1, uint32_t a2,
                                             uint32_t a3, uint32_t& o0, uint32_t& o1,
                                             uint32_t& o2, uint32_t& o3) {
  const uint32_t t0 = perm(a1, a0, 0x05010400u);  // a0.b0 a1.b0 a0.b1 a1.b1
  const uint32_t t1 = perm(a1, a0, 0x07030602u);  // a0.b2 a1.b2 a0.b3 a1.b3
  const uint32_t t2 = perm(a3, a2, 0x05010400u);
  const uint32_t t3 = perm(a3, a2, 0x07030602u);
  o0 = perm(t2, t0, 0x05040100u);
  o1 = perm(t2, t0, 0x07060302u);
  o2 = perm(t3, t1, 0x05040100u);
  o3 = perm(t3, t1, 0x07060302u);
}

// 16x16 byte transpose: out[j] byte i = in[i] byte j, with rows stored as
// 4 dwords (byte i of row r lives in dword i/4, byte i%4).
__device__ __forceinline__ void transpose16(const uint32_t (&in)[16][4],
                                            uint32_t (&out)[16][4]) {
#pragma unroll
  for (int n = 0; n < 4; ++n) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      transpose4x4(in[4 * n][m], in[4 * n + 1][m], in[4 * n + 2][m], in[4 * n + 3][m],
                   out[4 * m][n], out[4 * m + 1][n], out[4 * m + 2][n], out[4 * m + 3][n]);
    }
  }
}

// Packs 16 bytes (symbols, masked to b bits) LSB-first into u[].
template <int BITS>
__device__ __forceinline__ void compress16(const uint32_t (&in)[4], uint32_t* u) {
  constexpr int NU = (16 * BITS + 31) / 32;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = in[i];
  } else {
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int i = 0; i < NU; ++i) u[i] = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t s = (in[j >> 2] >> (8 * (j & 3))) & mask;
      const int bp = j * BITS;
      const int dw = bp >> 5, off = bp & 31;
      u[dw] |= s << off;
      if (off + BITS > 32) u[dw + 1] |= s >> (32 - off);
    }
  }
}

// Window-mode runs are 2b bytes, so one instruction covers less than a
// 128-byte line per plane and the rest of each line is read or written by
// neighbouring waves: these accesses go through the L2 normally (measured
// up to 2x faster for the pack, and 1.2x for the restore at b = 1, than
// non-temporal ones).
#define ORIGAMI_RUN_LOAD(T, src) (*reinterpret_cast<const T*>(src))
#define ORIGAMI_RUN_STORE(T, v, dst) (*reinterpret_cast<T*>(dst) = static_cast<T>(v))

// Loads NU dwords from a 4-byte aligned stream address.
template <int NU>
__device__ __forceinline__ void load_run_dwords(const uint8_t* src, uint32_t* w) {
  if constexpr (NU == 1) {
    w[0] = ORIGAMI_RUN_LOAD(uint32_t, src);
  } else if constexpr (NU == 2) {
    const u32x2a4 x = ORIGAMI_RUN_LOAD(u32x2a4, src);
    w[0] = x.x;
    w[1] = x.y;
  } else if constexpr (NU == 3) {
    const u32x3a4 x = ORIGAMI_RUN_LOAD(u32x3a4, src);
    w[0] = x.x;
    w[1] = x.y;
    w[2] = x.z;
  } else {
    static_assert(NU == 4, "a lane run is at most 4 dwords");
    const u32x4a4 x = ORIGAMI_RUN_LOAD(u32x4a4, src);
    w[0] = x.x;
    w[1] = x.y;
    w[2] = x.z;
    w[3] = x.w;
  }
}

// The window and shift modes of load_planes16 (below).
template <int BITS, int MODE, bool SERIAL>
__device__ __forceinline__ void load_runs16(const RowsParams& p, const int64_t* desc,
                                            int64_t sym0, bool any, uint32_t (&v)[16][4]) {
  static_assert(MODE == kRowsWindow || MODE == kRowsShift, "restore addressing mode");
  constexpr int NU = (16 * BITS + 31) / 32;  // = ceil(b / 2): dwords of a run
  // kRowsWindow: the run's 2b bytes start on an even byte (on a dword when b
  // is even), so the NU dwords from the dword at or below it hold it.
  // kRowsShift: the run starts at any bit, so the NU + 1 dwords from the one
  // holding its first bit hold it.
  constexpr int NW = MODE == kRowsShift ? NU + 1 : NU;
  if constexpr (SERIAL) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t d = desc[k];
      v[k][0] = v[k][1] = v[k][2] = v[k][3] = 0;
      if (d < 0 || !any) continue;
      const int64_t P = d + p.bit_bias + sym0 * BITS;
      const int64_t byte0 = MODE == kRowsShift ? (P >> 5) * 4 : (P >> 3) & ~int64_t(3);
      uint32_t w[NU + 1], u[NU > 4 ? NU : 4];
      uint32_t sh;
      if (byte0 + 4 * NW <= p.stream_bytes) {
        if constexpr (NW == 5) {
          load_run_dwords<4>(p.stream + byte0, w);
          load_run_dwords<1>(p.stream + byte0 + 16, w + 4);
        } else {
          load_run_dwords<NW>(p.stream + byte0, w);
        }
        if constexpr (NW == NU) w[NU] = 0;
        sh = MODE == kRowsShift ? static_cast<uint32_t>(P & 31)
             : (BITS % 2 == 1 && ((P >> 3) & 2)) ? 16u
                                                 : 0u;
      } else {  // as below: the NU + 1 dwords from the one holding bit P
        const int64_t d0 = P >> 5;
        sh = static_cast<uint32_t>(P & 31);
#pragma unroll
        for (int i = 0; i <= NU; ++i)
          w[i] = load_dword_guarded(p.stream, (d0 + i) * 4, p.stream_bytes);
      }
#pragma unroll
      for (int i = 0; i < NU; ++i) u[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], sh);
      expand16<BITS>(u, v[k]);
    }
  } else {
    uint32_t w[16][NW];
    uint32_t tail = 0;    // bit k: plane k's dwords pass the end of the stream
    uint32_t shp[4] = {};  // byte k & 3 of shp[k >> 2]: plane k's funnel shift
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t d = desc[k];
#pragma unroll
      for (int i = 0; i < NW; ++i) w[k][i] = 0;
      if (d >= 0 && any) {
        const int64_t P = d + p.bit_bias + sym0 * BITS;
        const int64_t byte0 = MODE == kRowsShift ? (P >> 5) * 4 : (P >> 3) & ~int64_t(3);
        const uint32_t sh = MODE == kRowsShift ? static_cast<uint32_t>(P & 31)
                            : (BITS % 2 == 1 && ((P >> 3) & 2)) ? 16u
                                                                : 0u;
        shp[k >> 2] |= sh << (8 * (k & 3));
        if (byte0 + 4 * NW <= p.stream_bytes) {
          if constexpr (NW == 5) {
            load_run_dwords<4>(p.stream + byte0, w[k]);
            load_run_dwords<1>(p.stream + byte0 + 16, w[k] + 4);
          } else {
            load_run_dwords<NW>(p.stream + byte0, w[k]);
          }
        } else {
          tail |= 1u << k;
        }
      }
    }
    // keeps the descriptors from staying live in registers until the tail
    // reloads below (they are read from LDS again there)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      uint32_t u[NU > 4 ? NU : 4];
      if (tail & (1u << k)) {
        // the NU + 1 dwords from the one holding bit P, those past the end of
        // the stream read as zeros
        const int64_t P = desc[k] + p.bit_bias + sym0 * BITS;
        const int64_t d0 = P >> 5;
        const uint32_t sh = static_cast<uint32_t>(P & 31);
        uint32_t t[NU + 1];
#pragma unroll
        for (int i = 0; i <= NU; ++i)
          t[i] = load_dword_guarded(p.stream, (d0 + i) * 4, p.stream_bytes);
#pragma unroll
        for (int i = 0; i < NU; ++i) u[i] = __builtin_amdgcn_alignbit(t[i + 1], t[i], sh);
      } else {
        const uint32_t sh = (shp[k >> 2] >> (8 * (k & 3))) & 31u;
#pragma unroll
        for (int i = 0; i < NU; ++i)
          u[i] = __builtin_amdgcn_alignbit(i + 1 < NW ? w[k][i + 1] : 0u, w[k][i], sh);
      }
      expand16<BITS>(u, v[k]);
    }
  }
}

// Loads a lane's 16 symbols of each of its 16 planes (plane k at stream bit
// P_k = desc[k] + bit_bias + sym0 * b; a plane with desc[k] < 0, or every
// plane when `any` is false, reads as zeros) into v[k], one byte per symbol.
// Every plane's dwords are requested before any of them is used, so a lane
// has all 16 loads in flight at once: with the funnel shift of each plane
// next to its loads, the compiler waited for every plane's data before
// requesting the next plane's (16 round trips per lane, 2053 tokens restored
// in 15.9 us against 8.5 for 2048).  A run whose dwords would pass the end
// of the stream is read again dword by dword afterwards.  SERIAL keeps the
// funnel shift next to each plane's loads (window and shift modes): with two
// loads per plane (b = 7, 8 in shift mode) and more than 12 waves per CU that
// order restored faster (15000 tokens 28.2 us, against 30.5 with every load
// in flight).
template <int BITS, int MODE, bool SERIAL = false>
__device__ __forceinline__ void load_planes16(const RowsParams& p, const int64_t* desc,
                                              int64_t sym0, bool any, uint32_t (&v)[16][4]) {
  if constexpr (MODE == kRowsAligned16 || MODE == kRowsAligned16Cached) {
    static_assert(BITS == 8, "aligned loads are for 8-bit symbols");
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t d = desc[k];
      v[k][0] = v[k][1] = v[k][2] = v[k][3] = 0;
      if (d >= 0 && any) {
        // the stream is read once: non-temporal when each 8-lane run is one line
        const u32x4* src = reinterpret_cast<const u32x4*>(p.stream + ((d + p.bit_bias + sym0 * 8) >> 3));
        const u32x4 x = MODE == kRowsAligned16 ? __builtin_nontemporal_load(src) : *src;
        v[k][0] = x.x;
        v[k][1] = x.y;
        v[k][2] = x.z;
        v[k][3] = x.w;
      }
    }
  } else {
    load_runs16<BITS, MODE, SERIAL>(p, desc, sym0, any, v);
  }
}

// Writes nbytes of u[] (little-endian) to dst, a byte address in the stream.
// kRowsWindow: nbytes is the whole run, 2b bytes at an even address (a dword
// address when b is even), written as dwords plus at most one 2-byte store.
// kRowsBytes: any byte address and any nbytes <= 2b.
template <int BITS, int MODE>
__device__ __forceinline__ void store_stream(uint8_t* dst, const uint32_t* u, int nbytes) {
  constexpr int NU = (16 * BITS + 31) / 32;
  if constexpr (MODE == kRowsAligned16) {
    const u32x4 x = {u[0], u[1], u[2], u[3]};
    __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dst));
  } else if constexpr (MODE == kRowsWindow && BITS % 2 == 0) {
    if constexpr (NU == 1) {
      ORIGAMI_RUN_STORE(uint32_t, u[0], dst);
    } else if constexpr (NU == 2) {
      ORIGAMI_RUN_STORE(u32x2a4, (u32x2a4{u[0], u[1]}), dst);
    } else if constexpr (NU == 3) {
      ORIGAMI_RUN_STORE(u32x3a4, (u32x3a4{u[0], u[1], u[2]}), dst);
    } else {
      ORIGAMI_RUN_STORE(u32x4a4, (u32x4a4{u[0], u[1], u[2], u[3]}), dst);
    }
  } else if constexpr (MODE == kRowsWindow) {
    // odd b: 2b = 4 * (NU - 1) + 2 bytes
    uint32_t d[NU];
    uint8_t* words = dst;
    uint16_t* half = reinterpret_cast<uint16_t*>(dst + 4 * (NU - 1));
    if ((reinterpret_cast<uintptr_t>(dst) & 2) == 0) {
#pragma unroll
      for (int i = 0; i < NU - 1; ++i) d[i] = u[i];
      d[NU - 1] = u[NU - 1];
    } else {  // a 2-byte head, then dwords
      half = reinterpret_cast<uint16_t*>(dst);
      words = dst + 2;
#pragma unroll
      for (int i = 0; i < NU - 1; ++i) d[i] = __builtin_amdgcn_alignbit(u[i + 1], u[i], 16);
      d[NU - 1] = u[0];
    }
    if constexpr (NU - 1 == 1) {
      ORIGAMI_RUN_STORE(uint32_t, d[0], words);
    } else if constexpr (NU - 1 == 2) {
      ORIGAMI_RUN_STORE(u32x2a4, (u32x2a4{d[0], d[1]}), words);
    } else if constexpr (NU - 1 == 3) {
      ORIGAMI_RUN_STORE(u32x3a4, (u32x3a4{d[0], d[1], d[2]}), words);
    }
    ORIGAMI_RUN_STORE(uint16_t, d[NU - 1], half);
  } else {
    static_assert(MODE == kRowsBytes, "pack modes: aligned16, window, bytes");
    // nbytes <= 2b bytes at any byte address: up to 3 head bytes to the next
    // dword, whole dwords, then up to 3 tail bytes.  Byte j of the run is
    // byte j & 3 of u[j >> 2].
    uint32_t w[NU + 1];
#pragma unroll
    for (int i = 0; i < NU; ++i) w[i] = u[i];
    w[NU] = 0;
    const int head =
        min(static_cast<int>((4u - (reinterpret_cast<uintptr_t>(dst) & 3u)) & 3u), nbytes);
    if (head == 0 && nbytes == 4 * NU) {  // a whole run of even b at a dword address
      if constexpr (NU == 1) {
        ORIGAMI_RUN_STORE(uint32_t, u[0], dst);
      } else if constexpr (NU == 2) {
        ORIGAMI_RUN_STORE(u32x2a4, (u32x2a4{u[0], u[1]}), dst);
      } else if constexpr (NU == 3) {
        ORIGAMI_RUN_STORE(u32x3a4, (u32x3a4{u[0], u[1], u[2]}), dst);
      } else {
        ORIGAMI_RUN_STORE(u32x4a4, (u32x4a4{u[0], u[1], u[2], u[3]}), dst);
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (j < head) dst[j] = static_cast<uint8_t>(w[0] >> (8 * j));
    const uint32_t sh = 8u * static_cast<uint32_t>(head);
    const int ndw = (nbytes - head) >> 2;
#pragma unroll
    for (int k = 0; k < NU; ++k)
      if (k < ndw)
        *reinterpret_cast<uint32_t*>(dst + head + 4 * k) =
            __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
    const int tail0 = head + 4 * ndw;
#pragma unroll
    for (int j = 0; j < 2 * BITS; ++j)
      if (j >= tail0 && j < nbytes) dst[j] = static_cast<uint8_t>(w[j >> 2] >> (8 * (j & 3)));
  }
}

struct TileCoord {
  int h, half, slot, q;  // slot: this lane's descriptor group in the workgroup
  int64_t t0;
};

// Tile order: token tiles fastest, then channel tiles, heads, halves; when the
// last token tile is partial, the full token tiles of every (channel tile,
// head, half) come first and the partial ones after them, so that the small
// tiles finish the launch instead of unbalancing its full rounds.
// A tile is its token tile `st` and the rest (channel tile fastest, then
// head, then half).
struct TileIndex {
  int st;
  int64_t rest;
};

// Splits a tile index of a single-request launch.
__device__ __forceinline__ TileIndex split_tile(const RowsParams& p, int64_t tile) {
  if (p.partial_last) {
    const int full = p.nst - 1;
    const int64_t nfull = p.ntiles / p.nst * full;
    if (tile >= nfull) return {full, tile - nfull};
    return {static_cast<int>(tile % full), tile / full};
  }
  return {static_cast<int>(tile % p.nst), tile / p.nst};
}

// Workgroups are dealt to the 8 XCDs round-robin (workgroup b runs on XCD
// b mod 8), each XCD with its own L2.  xcd_run_order(i, n, run) is a
// bijection on [0, n) that gives each XCD runs of `run` consecutive indices:
// index i of a group of 8 * run goes to member (i / 8) mod run of XCD slot
// i mod 8; a last partial group keeps its order.
__device__ __forceinline__ int64_t xcd_run_order(int64_t i, int64_t n, int run) {
  const int64_t group = 8 * static_cast<int64_t>(run);
  if (run <= 1 || i >= n / group * group) return i;
  const int64_t r = i % group;
  return i - r + (r % 8) * run + r / 8;
}

// Inside a tile, whole-tile workgroups order wave tiles along channels
// fastest; with SPLIT, workgroup `slice` holds waves [4 slice, 4 slice + 4)
// and wave tiles run along tokens fastest, so a workgroup is one channel
// column of the tile.
// SEG: tokens of a lane's run (16; 128 / b in the wide restore).
template <bool SPLIT = false, int SEG = kSegTokens>
__device__ __forceinline__ TileCoord tile_coord(const RowsParams& p, TileIndex ti,
                                                int slice = 0) {
  const int st = ti.st;
  int64_t tile = ti.rest;
  const int qt = static_cast<int>(tile % p.nqt);
  tile /= p.nqt;
  TileCoord tc;
  tc.h = static_cast<int>(tile % p.H);
  tc.half = static_cast<int>(tile / p.H);
  const int lane = threadIdx.x & 63;
  int wqi, wsi;
  if constexpr (SPLIT) {
    const int wave = slice * kRowsSplitWaves + (threadIdx.x >> 6);
    wqi = wave / p.ws;
    wsi = wave % p.ws;
  } else {
    const int wave = threadIdx.x >> 6;
    wqi = wave % p.wq;
    wsi = wave / p.wq;
  }
  tc.slot = wqi * kLaneGroups + (lane >> 3);
  tc.q = qt * p.wq * kLaneGroups + tc.slot;
  tc.t0 = p.token0 + (static_cast<int64_t>(st * p.ws + wsi) * kLaneSegs + (lane & 7)) * SEG;
  return tc;
}

// Stages the tile's plane descriptors in LDS.  The leading barrier keeps a
// workgroup that loops over tiles from overwriting descriptors another wave
// is still reading.
__device__ __forceinline__ void load_descriptors(const RowsParams& p, TileIndex ti,
                                                 int64_t* desc) {
  const int qt = static_cast<int>(ti.rest % p.nqt);
  const int h = static_cast<int>((ti.rest / p.nqt) % p.H);
  const int n = p.wq * kWavePlanes;
  __syncthreads();
  for (int i = static_cast<int>(threadIdx.x); i < n; i += static_cast<int>(blockDim.x)) {
    const int64_t c = static_cast<int64_t>(qt) * n + i;
    const int64_t plane = static_cast<int64_t>(h) * p.C + c;
    desc[i] = c >= p.C ? -1 : p.planes ? p.planes[plane] : p.plane_base + plane * p.plane_bits;
  }
  __syncthreads();
}

// Row cursor over the 16 tokens of a lane: follows the block table.
struct RowCursor {
  int64_t blk, off, pid;
};

__device__ __forceinline__ void cursor_init(const RowsParams& p, int64_t t0, RowCursor& rc) {
  if (p.block_ids) {
    rc.blk = t0 / p.bs;
    rc.off = t0 - rc.blk * p.bs;
    rc.pid = p.block_ids[rc.blk];
  } else {
    rc.blk = 0;
    rc.off = t0;
    rc.pid = 0;
  }
}

// Advances to the next token (call for j > 0 only, with that token < row_tokens).
__device__ __forceinline__ void cursor_next(const RowsParams& p, RowCursor& rc) {
  ++rc.off;
  if (p.block_ids && rc.off == p.bs) {
    rc.off = 0;
    ++rc.blk;
    rc.pid = p.block_ids[rc.blk];
  }
}

// Row index of the cursor's token, or -1 for a block id outside the cache.
__device__ __forceinline__ int64_t cursor_row(const RowsParams& p, int half, const RowCursor& rc) {
  if (!p.block_ids) return half * p.half_stride + rc.off;
  if (rc.pid < 0 || rc.pid >= p.num_blocks) return -1;
  return rc.pid * p.blk_stride + half * p.half_stride + rc.off;
}

// Calls f(j, row) for each token t0 + j (t0 % 16 == 0, j < 16 and j < nrows)
// whose block is in the cache, with its row index.  ONEBLK: every block holds
// a multiple of 16 rows, or there is no block table, so the 16 tokens are
// consecutive rows of one block: one table load, then fixed strides.
// Otherwise a cursor follows the table; its table load, taken only when the
// rows cross into the next block, makes the compiler wait for every
// outstanding memory access of the wave (stores included) before each row,
// so a lane's 16 row accesses go one at a time.  That costs the split
// restores 2-8% (131072 tokens of Llama-3-70B geometry: 0.601 -> 0.649 of
// HBM peak) and launches of few waves per CU up to half their time, while
// whole-tile launches of 8 or more waves per CU run 1-4% faster with it: the
// host picks by launch size (waves_per_cu).
template <bool ONEBLK, class F>
__device__ __forceinline__ void for_rows16(const RowsParams& p, int half, int64_t t0,
                                           int64_t nrows, F&& f) {
  RowCursor rc;
  cursor_init(p, t0, rc);
  if constexpr (ONEBLK) {
    const int64_t row0 = cursor_row(p, half, rc);
    if (row0 < 0) return;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < nrows) f(j, row0 + j);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (j < nrows) {
        if (j > 0) cursor_next(p, rc);
        const int64_t row = cursor_row(p, half, rc);
        if (row >= 0) f(j, row);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Rows kernels
// ---------------------------------------------------------------------------

template <int BITS, int MODE, bool SPLIT = false, bool ONEBLK = false, bool SERIAL = false>
__device__ __forceinline__ void unpack_tile(const RowsParams& p, TileIndex ti,
                                            const int64_t* desc, int slice = 0) {
  const TileCoord tc = tile_coord<SPLIT>(p, ti, slice);
  if (tc.q >= p.nq || tc.t0 >= p.row_tokens) return;
  const int64_t nv = p.T - tc.t0;  // tokens of this segment that hold symbols
  const int64_t sym0 = static_cast<int64_t>(tc.half) * p.T + tc.t0;

  uint32_t v[16][4];
  load_planes16<BITS, MODE, SERIAL>(p, desc + tc.slot * 16, sym0, nv > 0, v);
  if (MODE == kRowsShift && nv < 16) {  // other modes: T % 16 == 0
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int64_t keep = nv - 4 * m;
      const uint32_t mask = keep >= 4 ? 0xffffffffu
                            : keep <= 0 ? 0u
                                        : ((1u << (8 * keep)) - 1u);
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k][m] &= mask;
    }
  }
  uint32_t o[16][4];
  transpose16(v, o);

  uint8_t* col = p.rows + static_cast<int64_t>(tc.h) * p.head_pitch + tc.q * 16;
  // each row is written once: non-temporal
  for_rows16<ONEBLK>(p, tc.half, tc.t0, p.row_tokens - tc.t0, [&](int j, int64_t row) {
    const u32x4 x = {o[j][0], o[j][1], o[j][2], o[j][3]};
    __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(col + row * p.row_pitch));
  });
}

// ONEBLK as for for_rows16, SERIAL as for load_planes16; the host picks both
// by launch size.
template <int BITS, int MODE, bool ONEBLK, bool SERIAL>
__global__ __launch_bounds__(kRowsThreads) void rows_unpack_kernel(RowsParams p) {
  __shared__ int64_t desc[kTilePlanes];
  for (int64_t tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const TileIndex ti = split_tile(p, tile);
    load_descriptors(p, ti, desc);
    unpack_tile<BITS, MODE, false, ONEBLK, SERIAL>(p, ti, desc);
  }
}

// The same restore with each tile dispatched as 2^sh workgroups of
// kRowsSplitWaves waves (p.waves = kRowsSplitWaves << sh); ONEBLK as for
// for_rows16.
template <int BITS, int MODE, bool ONEBLK>
__global__ __launch_bounds__(kRowsSplitWaves * 64) void rows_unpack_split_kernel(RowsParams p,
                                                                                 int sh) {
  __shared__ int64_t desc[kTilePlanes];
  const int64_t slots = p.ntiles << sh;
  for (int64_t s = blockIdx.x; s < slots; s += gridDim.x) {
    const int64_t tile = s >> sh;
    const TileIndex ti = split_tile(p, tile);
    load_descriptors(p, ti, desc);
    unpack_tile<BITS, MODE, true, ONEBLK>(p, ti, desc, static_cast<int>(s & ((1 << sh) - 1)));
  }
}

// Restore at b = 1, 2 or 4 with runs on 16-byte boundaries (kRowsWide): a
// lane's run of a plane is one 16-byte load, 128 / b tokens, so the 8 lanes
// of a group read a whole 128-byte line per plane (the window mode reads 2b
// bytes per lane: at b = 4 two waves each read half of every line).  The lane
// then restores its run as 16-token sub-tiles: expand, transpose, 16 row
// stores each.  Needs T % (128 / b) == 0, so a run holds symbols either
// throughout or not at all.
template <int BITS, bool NT, bool ONEBLK>
__device__ __forceinline__ void unpack_tile_wide(const RowsParams& p, TileIndex ti,
                                                 const int64_t* desc) {
  static_assert(BITS == 1 || BITS == 2 || BITS == 4, "wide runs are 16 bytes of 1, 2 or 4-bit symbols");
  constexpr int SEG = 128 / BITS, SUB = SEG / kSegTokens;
  const TileCoord tc = tile_coord<false, SEG>(p, ti);
  if (tc.q >= p.nq || tc.t0 >= p.row_tokens) return;
  const bool has_symbols = tc.t0 < p.T;
  const int64_t sym0 = static_cast<int64_t>(tc.half) * p.T + tc.t0;

  uint32_t w[16][4];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t d = desc[tc.slot * 16 + k];
    w[k][0] = w[k][1] = w[k][2] = w[k][3] = 0;
    if (d >= 0 && has_symbols) {
      const u32x4* src = reinterpret_cast<const u32x4*>(p.stream + ((d + p.bit_bias + sym0 * BITS) >> 3));
      const u32x4 x = NT ? __builtin_nontemporal_load(src) : *src;
      w[k][0] = x.x;
      w[k][1] = x.y;
      w[k][2] = x.z;
      w[k][3] = x.w;
    }
  }
  uint8_t* const col = p.rows + static_cast<int64_t>(tc.h) * p.head_pitch + tc.q * 16;
#pragma unroll
  for (int m = 0; m < SUB; ++m) {
    const int64_t t0 = tc.t0 + m * kSegTokens;
    if (t0 >= p.row_tokens) break;
    // sub-tile m: bits [16 b m, 16 b (m + 1)) of each run
    uint32_t v[16][4];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      uint32_t u[2];
      if constexpr (BITS == 4) {
        u[0] = w[k][2 * m];
        u[1] = w[k][2 * m + 1];
      } else if constexpr (BITS == 2) {
        u[0] = w[k][m];
      } else {
        u[0] = w[k][m >> 1] >> (16 * (m & 1));
      }
      expand16<BITS>(u, v[k]);
    }
    uint32_t o[16][4];
    transpose16(v, o);
    for_rows16<ONEBLK>(p, tc.half, t0, p.row_tokens - t0, [&](int j, int64_t row) {
      const u32x4 x = {o[j][0], o[j][1], o[j][2], o[j][3]};
      __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(col + row * p.row_pitch));
    });
  }
}

// Wide-run workgroups have at most kWideMaxWaves waves: the 16-byte runs of
// 16 planes stay in registers while the sub-tiles are restored.
constexpr int kWideMaxWaves = 8;

template <int BITS, bool NT, bool ONEBLK>
__global__ __launch_bounds__(kWideMaxWaves * 64) void rows_unpack_wide_kernel(RowsParams p) {
  __shared__ int64_t desc[kTilePlanes];
  for (int64_t tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const TileIndex ti = split_tile(p, tile);
    load_descriptors(p, ti, desc);
    unpack_tile_wide<BITS, NT, ONEBLK>(p, ti, desc);
  }
}

// One layer of several requests.  The full token tiles of all requests come
// first (request by request), then every request's partial last token tile;
// the workgroup's tile picks its request with a uniform scan of at most
// kBatchRequests tile offsets (a request with no tiles in a range has the next
// request's offset, so the scan passes it).
// Restores tile `tile` of a batched launch (slice `slice` of it with SPLIT).
template <int BITS, int MODE, bool SPLIT, bool ONEBLK, bool SERIAL>
__device__ __forceinline__ void batch_tile(const RowsBatch& b, int64_t tile, int64_t* desc,
                                           int slice) {
  int r = 0;
  TileIndex ti;
  if (tile < b.nfull) {
    while (r + 1 < b.nreq && tile >= b.req[r + 1].tile0) ++r;
    const int full = b.req[r].nst - b.req[r].partial;
    const int64_t local = tile - b.req[r].tile0;
    ti = {static_cast<int>(local % full), local / full};
  } else {
    while (r + 1 < b.nreq && tile >= b.req[r + 1].ptile0) ++r;
    ti = {b.req[r].nst - 1, tile - b.req[r].ptile0};
  }
  const RowsRequest& q = b.req[r];
  RowsParams p = b.common;
  p.stream = q.stream;
  p.stream_bytes = q.stream_bytes;
  p.bit_bias = q.bit_bias;
  p.planes = q.planes;
  p.plane_base = q.plane_base;
  p.plane_bits = q.plane_bits;
  p.block_ids = q.block_ids;
  p.T = q.T;
  p.row_tokens = q.row_tokens;
  p.nst = q.nst;
  p.token0 = q.token0;
  load_descriptors(p, ti, desc);
  if constexpr (MODE == kRowsAligned16) {
    // one launch for the batch, the load policy per request
    if (q.nt)
      unpack_tile<BITS, kRowsAligned16, SPLIT, ONEBLK>(p, ti, desc, slice);
    else
      unpack_tile<BITS, kRowsAligned16Cached, SPLIT, ONEBLK>(p, ti, desc, slice);
  } else {
    unpack_tile<BITS, MODE, SPLIT, ONEBLK, SERIAL>(p, ti, desc, slice);
  }
}

template <int BITS, int MODE, bool ONEBLK, bool SERIAL>
__global__ __launch_bounds__(kRowsThreads) void rows_unpack_batch_kernel(RowsBatch b) {
  __shared__ int64_t desc[kTilePlanes];
  for (int64_t tile = blockIdx.x; tile < b.common.ntiles; tile += gridDim.x)
    batch_tile<BITS, MODE, false, ONEBLK, SERIAL>(b, tile, desc, 0);
}

// The batched restore with each tile dispatched as 2^sh workgroups of
// kRowsSplitWaves waves, as rows_unpack_split_kernel does for one request.
template <int BITS, int MODE, bool ONEBLK>
__global__ __launch_bounds__(kRowsSplitWaves * 64) void rows_unpack_batch_split_kernel(
    RowsBatch b, int sh) {
  __shared__ int64_t desc[kTilePlanes];
  const int64_t slots = b.common.ntiles << sh;
  for (int64_t s = blockIdx.x; s < slots; s += gridDim.x)
    batch_tile<BITS, MODE, true, ONEBLK, false>(b, s >> sh, desc,
                                               static_cast<int>(s & ((1 << sh) - 1)));
}

// Calls f(std::integral_constant<int, i>) for i = 0 .. N - 1, in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// The dword of c holding byte j (0 <= j < 16), by selects on scalars (an
// indexed read of c would put it in scratch memory).
__device__ __forceinline__ uint32_t chunk_word(uint32_t c0, uint32_t c1, uint32_t c2,
                                               uint32_t c3, int j) {
  const uint32_t lo = (j & 4) ? c1 : c0, hi = (j & 4) ? c3 : c2;
  return (j & 8) ? hi : lo;
}

// Writes bytes [lo, hi) of the 16-byte aligned chunk at dst (0 <= lo < hi
// <= 16, not the whole chunk; byte j of the chunk is byte j & 3 of c[j >> 2]):
// at most a byte, a short, the whole dwords, a short and a byte.
__device__ __forceinline__ void store_chunk_part(uint8_t* dst, uint32_t c0, uint32_t c1,
                                                 uint32_t c2, uint32_t c3, int lo, int hi) {
  asm("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
  int a = lo;
  if (a & 1) {
    dst[a] = static_cast<uint8_t>(chunk_word(c0, c1, c2, c3, a) >> (8 * (a & 3)));
    ++a;
  }
  if (a + 2 <= hi && (a & 2)) {
    *reinterpret_cast<uint16_t*>(dst + a) =
        static_cast<uint16_t>(chunk_word(c0, c1, c2, c3, a) >> 16);
    a += 2;
  }
  const uint32_t cw[4] = {c0, c1, c2, c3};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (4 * i >= a && 4 * i + 4 <= hi) *reinterpret_cast<uint32_t*>(dst + 4 * i) = cw[i];
  int t = hi & ~3;
  if (t < a) t = a;
  if (t + 2 <= hi) {  // t is even here
    *reinterpret_cast<uint16_t*>(dst + t) =
        static_cast<uint16_t>(chunk_word(c0, c1, c2, c3, t) >> (8 * (t & 2)));
    t += 2;
  }
  if (t < hi) dst[t] = static_cast<uint8_t>(chunk_word(c0, c1, c2, c3, t) >> (8 * (t & 3)));
}

// Gathers a lane's 16 rows x 16 bytes (tokens t0 .. t0 + nv - 1 of its
// 16-byte channel column) through the block table; missing rows read as 0.
// ONEBLK as for for_rows16: without it the row loads are requested one after
// another, which is faster only in launches of more than 12 waves per CU
// (6 for the staged pack).
template <bool ONEBLK>
__device__ __forceinline__ void load_tile_rows(const RowsParams& p, const TileCoord& tc, int nv,
                                               uint32_t (&r)[16][4]) {
  const uint8_t* col = p.rows + static_cast<int64_t>(tc.h) * p.head_pitch + tc.q * 16;
#pragma unroll
  for (int j = 0; j < 16; ++j) r[j][0] = r[j][1] = r[j][2] = r[j][3] = 0;
  if (nv <= 0) return;
  for_rows16<ONEBLK>(p, tc.half, tc.t0, nv, [&](int j, int64_t row) {
    const u32x4 x =
        __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(col + row * p.row_pitch));
    r[j][0] = x.x;
    r[j][1] = x.y;
    r[j][2] = x.z;
    r[j][3] = x.w;
  });
}

// 8-bit pack of planes off 128-byte lines (kRowsStaged8), staged through LDS.
// In a tile, the runs of one plane for one 16-channel slot are one stretch of
// the stream: its region, bytes [R0, R0 + n) for the tile's n tokens.  Lanes
// put their 16-token runs into LDS at their offset in the region; after a
// barrier, wave wsi writes the region's 128-byte stream line wsi (and one
// wave the line after the last), whole except where the region starts or
// ends inside it.  Each line is then written by one wave.  Writing each run
// in place instead leaves most lines written in two parts by two waves, which
// measured 88.0 us per 32753-token layer against 59.7 us with the same work
// on whole lines.  Planes go through LDS kStagePlanes at a time, in two
// buffers, so one barrier per round separates writers and readers.
constexpr int kStagePlanes = 4;
constexpr int kStageFront = 16, kStageBack = 32;  // pad bytes around a region
// A round: kStagePlanes x (wq * 8 slots) regions of ws * 128 + pad bytes, for
// a workgroup of `waves` waves.
constexpr int stage_round_bytes(int waves) {
  return kStagePlanes * (waves * 1024 + kRowsWq * kLaneGroups * (kStageFront + kStageBack));
}
static_assert(2 * stage_round_bytes(kRowsMaxWaves) + kRowsWq * kWavePlanes * 8 <= 160 * 1024,
              "LDS of the staged pack");

// Writes this lane's 16-byte chunk of region line j: stream bytes
// [line0 + 128 j + 16 s, + 16), region bytes [o, o + 16), o = 128 j + 16 s - M
// (M = R0 mod 128); only the bytes inside the region [0, n).  Reads at most
// 16 bytes before and 20 after the region's bytes in LDS (its pads).  `nt`:
// whole chunks as non-temporal stores (the parts of the shared edge lines stay
// plain stores either way).
__device__ __forceinline__ void store_region_chunk(uint8_t* line0, const uint8_t* reg, int M,
                                                   int n, int j, int s, bool nt) {
  const int o = 128 * j + 16 * s - M;
  const int lo = o < 0 ? -o : 0, hi = n - o < 16 ? n - o : 16;
  if (lo >= hi) return;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(reg + (o & ~3));
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
  const uint32_t sh = static_cast<uint32_t>(o & 3);
  const uint32_t c0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
  const uint32_t c1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
  const uint32_t c2 = __builtin_amdgcn_alignbyte(w3, w2, sh);
  const uint32_t c3 = __builtin_amdgcn_alignbyte(w4, w3, sh);
  uint8_t* const dst = line0 + 128 * j + 16 * s;
  if (lo == 0 && hi == 16) {
    if (nt)
      __builtin_nontemporal_store(u32x4{c0, c1, c2, c3}, reinterpret_cast<u32x4*>(dst));
    else
      *reinterpret_cast<u32x4*>(dst) = u32x4{c0, c1, c2, c3};
  } else {
    store_chunk_part(dst, c0, c1, c2, c3, lo, hi);
  }
}

// Every wave of the workgroup runs this for every tile (no early exit: the
// rounds hold barriers); lanes outside the tile's channels or tokens only
// take part in the barriers.
template <int WAVES, bool ONEBLK>
__device__ __forceinline__ void pack_tile_staged8(const RowsParams& p, TileIndex ti,
                                                  const int64_t* desc, uint8_t* stage) {
  const TileCoord tc = tile_coord(p, ti);
  const int s = static_cast<int>(threadIdx.x & 7);
  const int wsi = static_cast<int>(threadIdx.x >> 6) / p.wq;
  const int64_t T0 = tc.t0 - (static_cast<int64_t>(wsi) * kLaneSegs + s) * kSegTokens;
  const bool slot_ok = tc.q < p.nq;
  const bool run_ok = slot_ok && tc.t0 < p.T;
  const int nv = run_ok ? static_cast<int>(p.T - tc.t0 < 16 ? p.T - tc.t0 : 16) : 0;

  uint32_t r[16][4];
  load_tile_rows<ONEBLK>(p, tc, nv, r);
  uint32_t v[16][4];
  transpose16(r, v);

  const int n = static_cast<int>(p.T - T0 < p.ws * 128 ? p.T - T0 : p.ws * 128);
  const int RS = p.ws * 128 + kStageFront + kStageBack;
  const int slots = p.wq * kLaneGroups;
  const int64_t sym0 = static_cast<int64_t>(tc.half) * p.T + T0;
  const int run_off = kStageFront + (wsi * kLaneSegs + s) * kSegTokens;
  static_for<16 / kStagePlanes>([&](auto rc) {
    constexpr int round = decltype(rc)::value;
    uint8_t* const buf = stage + (round & 1) * stage_round_bytes(WAVES);
    static_for<kStagePlanes>([&](auto kc) {
      constexpr int kk = decltype(kc)::value, k = round * kStagePlanes + kk;
      if (run_ok && desc[tc.slot * 16 + k] >= 0)
        *reinterpret_cast<u32x4*>(buf + (kk * slots + tc.slot) * RS + run_off) =
            u32x4{v[k][0], v[k][1], v[k][2], v[k][3]};
    });
    __syncthreads();
    static_for<kStagePlanes>([&](auto kc) {
      constexpr int kk = decltype(kc)::value, k = round * kStagePlanes + kk;
      const int64_t d = desc[tc.slot * 16 + k];
      if (!slot_ok || d < 0) return;
      uint8_t* const r0 = p.stream + ((d + p.bit_bias + sym0 * 8) >> 3);
      const int M = static_cast<int>(reinterpret_cast<uintptr_t>(r0) & 127);
      const uint8_t* const reg = buf + (kk * slots + tc.slot) * RS + kStageFront;
      const bool nt = p.nt_stores != 0;
      store_region_chunk(r0 - M, reg, M, n, wsi, s, nt);
      // the line past the waves' own (when the region is off a line): one
      // wave per plane, a different one for each plane
      if (wsi == (k & (p.ws - 1))) store_region_chunk(r0 - M, reg, M, n, p.ws, s, nt);
    });
  });
}

// Single-owner variant of the staged pack (own_lines, 16-wave tiles).  A tile
// holds kOwnTokens = 15 * 128 tokens of its half, [T0, T0 + n); wave 0
// gathers the 128 tokens before T0 as well (the K half's last 128 for the V
// half's first tile), so that the LDS region reg[i] holds the plane byte of
// token T0 - 128 + i, i in [0, 2048).  In the stream a plane's region starts
// M = R0 mod 128 bytes into its first line; the tile writes every line whose
// last byte is in its region, whole, the M bytes before R0 included, and
// leaves the line holding its region's end to the tile after it.  So each
// stream line is written by one tile in one piece, except the two lines at
// each plane's start and end, whose other bytes belong to another plane:
// there the tile writes its own bytes only, as the two-part scheme does.
// Against 2048-token tiles writing a region's first and last lines in two
// parts (one by each neighbouring tile), us per layer: 24001 tokens 54.9 ->
// 51.3, 49217 tokens 111.2 -> 103.2, 12001 tokens 31.0 -> 27.5.
constexpr int kOwnTokens = 15 * 128;

// Writes the bytes [a, b) of this lane's chunk s of line j (offsets from the
// line's start line0, a plane's region starting M bytes into line 0): stream
// bytes [line0 + 128 j + 16 s, + 16) from LDS bytes reg[128 - M + 128 j + 16 s
// ...] (5 dwords read, at most 20 bytes past the chunk).
__device__ __forceinline__ void store_owned_chunk(uint8_t* line0, const uint8_t* reg, int M,
                                                  int j, int s, int a, int b, bool nt) {
  const int o = 128 * j + 16 * s;
  const int lo = a > o ? a - o : 0, hi = b - o < 16 ? b - o : 16;
  if (lo >= hi) return;
  const int i = 128 - M + o;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(reg + (i & ~3));
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
  const uint32_t sh = static_cast<uint32_t>(i & 3);
  const uint32_t c0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
  const uint32_t c1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
  const uint32_t c2 = __builtin_amdgcn_alignbyte(w3, w2, sh);
  const uint32_t c3 = __builtin_amdgcn_alignbyte(w4, w3, sh);
  uint8_t* const dst = line0 + o;
  if (lo == 0 && hi == 16) {
    if (nt)
      __builtin_nontemporal_store(u32x4{c0, c1, c2, c3}, reinterpret_cast<u32x4*>(dst));
    else
      *reinterpret_cast<u32x4*>(dst) = u32x4{c0, c1, c2, c3};
  } else {
    store_chunk_part(dst, c0, c1, c2, c3, lo, hi);
  }
}

// pack_tile_staged8 with own_lines: every wave of the workgroup runs this for
// every tile (the rounds hold barriers).  p.T >= 128 (the V half's first tile
// reads the K half's last 128 tokens, whose runs start at any token, so rows
// are gathered through the block-table walk; 16-wave staged tiles only run at
// 8 or more waves per CU, where the walk is the faster order anyway).
__device__ __forceinline__ void pack_tile_owned(const RowsParams& p, TileIndex ti,
                                                const int64_t* desc, uint8_t* stage) {
  constexpr int WAVES = 16;
  TileCoord tc = tile_coord(p, ti);
  const int s = static_cast<int>(threadIdx.x & 7);
  const int wsi = static_cast<int>(threadIdx.x >> 6);  // wq == 1: the wave's token row
  const int64_t T0 = static_cast<int64_t>(ti.st) * kOwnTokens;
  const bool slot_ok = tc.q < p.nq;
  const bool kv_halo = tc.half == 1 && T0 == 0;  // wave 0 reads the K half's tail
  tc.t0 = T0 - 128 + (static_cast<int64_t>(wsi) * kLaneSegs + s) * kSegTokens;
  int nv = 0;
  if (wsi == 0) {
    if (kv_halo) {
      tc.half = 0;
      tc.t0 += p.T;
    }
    if (slot_ok && (T0 > 0 || kv_halo)) nv = 16;
  } else if (slot_ok && tc.t0 < p.T) {
    nv = static_cast<int>(p.T - tc.t0 < 16 ? p.T - tc.t0 : 16);
  }

  uint32_t r[16][4];
  load_tile_rows<false>(p, tc, nv, r);
  uint32_t v[16][4];
  transpose16(r, v);

  const int64_t half = kv_halo ? 1 : tc.half;
  const int n = static_cast<int>(p.T - T0 < kOwnTokens ? p.T - T0 : kOwnTokens);
  const bool first_part = half == 0 && T0 == 0;         // the plane's first line
  const bool last_part = half == 1 && T0 + n == p.T;    // the plane's last line
  const int RS = WAVES * 128 + kStageFront + kStageBack;
  const int slots = p.wq * kLaneGroups;
  const int64_t sym0 = half * p.T + T0;
  const int run_off = kStageFront + (wsi * kLaneSegs + s) * kSegTokens;
  const bool nt = p.nt_stores != 0;
  static_for<16 / kStagePlanes>([&](auto rc) {
    constexpr int round = decltype(rc)::value;
    uint8_t* const buf = stage + (round & 1) * stage_round_bytes(WAVES);
    static_for<kStagePlanes>([&](auto kc) {
      constexpr int kk = decltype(kc)::value, k = round * kStagePlanes + kk;
      if (nv > 0 && desc[tc.slot * 16 + k] >= 0)
        *reinterpret_cast<u32x4*>(buf + (kk * slots + tc.slot) * RS + run_off) =
            u32x4{v[k][0], v[k][1], v[k][2], v[k][3]};
    });
    __syncthreads();
    static_for<kStagePlanes>([&](auto kc) {
      constexpr int kk = decltype(kc)::value, k = round * kStagePlanes + kk;
      const int64_t d = desc[tc.slot * 16 + k];
      if (!slot_ok || d < 0) return;
      uint8_t* const r0 = p.stream + ((d + p.bit_bias + sym0 * 8) >> 3);
      const int M = static_cast<int>(reinterpret_cast<uintptr_t>(r0) & 127);
      const uint8_t* const reg = buf + (kk * slots + tc.slot) * RS + kStageFront;
      // bytes [a, b) from the region's first line: whole lines up to the
      // last one that ends inside the region, the plane's ends only in part
      const int a = first_part ? M : 0;
      const int b = last_part ? M + n : 128 * ((M + n) >> 7);
      store_owned_chunk(r0 - M, reg, M, wsi, s, a, b, nt);
    });
  });
}

// Writes the low `nbits` bits (> 0) of u[] into the stream at bit P
// (kRowsBits).  The 8 lanes of a group hold consecutive runs of one plane,
// lane i at P0 + 16 b i, and the group's bits are [P0, Pend).  A dword wholly
// inside that range is stored by the lane holding its first bit, with the
// next lane's leading bits merged in (a dword spans at most two runs for
// b >= 2).  The dwords at the range's ends are shared with other groups
// (other waves, tiles or planes): their bits go in with atomic ORs into the
// stream, which the launch clears first.  Below b = 5 every dword does: the
// plain stores then cost more than the ORs they replace (32753 tokens, GB/s
// with / without the merge: b = 7 719 / 469, 6 721 / 581, 5 654 / 618,
// 3 656 / 851, 2 937 / 1235).  Every lane of the group with symbols must call
// this (the merge reads the next lane's first dword); no bit outside the run
// is set and no dword past its last bit is touched.
template <int BITS>
__device__ __forceinline__ void put_run_bits(uint8_t* stream, int64_t P, const uint32_t* u,
                                             int nbits, int64_t P0, int64_t Pend) {
  constexpr int NU = (16 * BITS + 31) / 32;
  const int64_t D0 = P >> 5;
  uint32_t* const base = reinterpret_cast<uint32_t*>(stream) + D0;
  const uint32_t s = static_cast<uint32_t>(P & 31);
  const int last = static_cast<int>((s + nbits - 1) >> 5);  // last dword index touched
  uint32_t g[NU + 1];
#pragma unroll
  for (int i = 0; i <= NU; ++i) {
    const uint64_t hi = i < NU ? u[i] : 0u, lo = i > 0 ? u[i - 1] : 0u;
    g[i] = static_cast<uint32_t>(((hi << 32) | lo) >> (32 - s));
  }
  const uint32_t next0 = __shfl_down(g[0], 1, 8);  // the next run's first dword
  const int64_t Pn = P + 16 * BITS;
#pragma unroll
  for (int i = 0; i <= NU; ++i) {
    if (i > last) break;
    const int64_t D = D0 + i;
    const bool inside = BITS >= 5 && 32 * D >= P0 && 32 * D + 32 <= Pend;
    if (!inside) {
      if (g[i] != 0) atomicOr(base + i, g[i]);
    } else if (32 * D >= P) {  // else the previous lane holds its first bit
      const bool merge = (Pn & 31) != 0 && (Pn >> 5) == D;
      base[i] = merge ? (g[i] | next0) : g[i];
    }
  }
}

template <int BITS, int MODE, bool ONEBLK>
__device__ __forceinline__ void pack_tile(const RowsParams& p, TileIndex ti,
                                          const int64_t* desc) {
  const TileCoord tc = tile_coord(p, ti);
  if (tc.q >= p.nq || tc.t0 >= p.T) return;
  const int nv = static_cast<int>(p.T - tc.t0 < 16 ? p.T - tc.t0 : 16);

  uint32_t r[16][4];
  load_tile_rows<ONEBLK>(p, tc, nv, r);
  uint32_t v[16][4];
  transpose16(r, v);

  constexpr int NU = (16 * BITS + 31) / 32;
  const int nbytes = (nv * BITS) >> 3;
  const int64_t sym0 = static_cast<int64_t>(tc.half) * p.T + tc.t0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t d = desc[tc.slot * 16 + k];
    if (d < 0) continue;
    const int64_t P = d + p.bit_bias + sym0 * BITS;  // byte aligned unless kRowsBits
    uint32_t u[NU > 4 ? NU : 4];
    compress16<BITS>(v[k], u);
    if constexpr (MODE == kRowsBits) {
      // the group's runs: 8 lanes from token t0g, those below T hold symbols
      const int64_t t0g = tc.t0 - static_cast<int64_t>(threadIdx.x & 7) * kSegTokens;
      const int64_t ng = p.T - t0g < 8 * kSegTokens ? p.T - t0g : 8 * kSegTokens;
      const int64_t P0 = P - (tc.t0 - t0g) * BITS;
      put_run_bits<BITS>(p.stream, P, u, nv * BITS, P0, P0 + ng * BITS);
    } else {
      store_stream<BITS, MODE>(p.stream + (P >> 3), u, nbytes);
    }
  }
}

template <int BITS, int MODE, bool ONEBLK>
__global__ __launch_bounds__(kRowsThreads) void rows_pack_kernel(RowsParams p) {
  __shared__ int64_t desc[kTilePlanes];
  for (int64_t tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const TileIndex ti = split_tile(p, tile);
    load_descriptors(p, ti, desc);
    pack_tile<BITS, MODE, ONEBLK>(p, ti, desc);
  }
}

// The 8-bit pack off 128-byte lines (kRowsStaged8), for workgroups of WAVES
// waves (p.waves == WAVES): LDS in proportion, so that the smaller workgroups
// of short launches still share a CU.
// The staged pack's regions share their
// first and last stream lines with the token-neighbouring tiles, so those
// lines are written in two parts.  Dealing runs of kStagedXcdRun consecutive
// token tiles to one XCD (workgroups b, b + 8, ... of a group of 8 runs) puts
// both parts of most shared lines into one L2 at about the same time.  Pack
// GB/s, runs of 1 / 4 / 16 / 32 / 64 tiles: 32753 tokens 3894 / 4247 / 4448 /
// 4411 / 4470; 49217 tokens 3340 / - / 3638 / 3622 / 3496; launches with
// fewer tiles than a group (8199, 4100 tokens) unchanged.
constexpr int kStagedXcdRun = 16;
constexpr int kStagedNtTiles = 4;

template <int WAVES, bool ONEBLK, bool OWN = false>
__global__ __launch_bounds__(WAVES * 64) void rows_pack_staged8_kernel(RowsParams p) {
  static_assert(!OWN || (WAVES == 16 && !ONEBLK), "single-owner tiles: 16 waves, row walk");
  __shared__ int64_t desc[kRowsWq * kWavePlanes];
  __shared__ __align__(16) uint8_t stage[2 * stage_round_bytes(WAVES)];
  for (int64_t t = blockIdx.x; t < p.ntiles; t += gridDim.x) {
    const int64_t tile = xcd_run_order(t, p.ntiles, kStagedXcdRun);
    const TileIndex ti = split_tile(p, tile);
    load_descriptors(p, ti, desc);
    if constexpr (OWN)
      pack_tile_owned(p, ti, desc, stage);
    else
      pack_tile_staged8<WAVES, ONEBLK>(p, ti, desc, stage);
  }
}

// ---------------------------------------------------------------------------
// Generic kernels (any layout, any plan)
// ---------------------------------------------------------------------------

struct GenericLayout {
  int64_t st, sh, sc;  // element strides of the token / head / head_dim axes
};

// bitpack_layout_cuda.cu:70-89: 16-bit LE window, bytes past the chunk read 0.
__device__ __forceinline__ uint8_t unpack_symbol(const uint8_t* src, int64_t nbytes,
                                                 int64_t i, int bits) {
  if (bits == 8) return src[i];
  const int64_t bp = i * bits;
  const int64_t k = bp >> 3;
  uint32_t w = 0;
  if (k < nbytes) w = src[k];
  if (k + 1 < nbytes) w |= static_cast<uint32_t>(src[k + 1]) << 8;
  return static_cast<uint8_t>((w >> (bp & 7)) & ((1u << bits) - 1u));
}

__global__ __launch_bounds__(kThreads) void generic_unpack_kernel(
    const uint8_t* __restrict__ flat, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ bits, const int64_t* __restrict__ specs,
    GenericLayout L, uint8_t* __restrict__ out) {
  const int64_t k = blockIdx.y;
  const int64_t* s = specs + 6 * k;
  const int64_t Tc = s[5] - s[4], Cc = s[3] - s[2];
  const int64_t per_head = Tc * Cc, n = (s[1] - s[0]) * per_head;
  const int b = static_cast<int>(bits[k]);
  const uint8_t* src = flat + offsets[k];
  const int64_t nbytes = offsets[k + 1] - offsets[k];
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const int64_t hh = i / per_head;
    const int64_t rem = i - hh * per_head;
    const int64_t cc = rem / Tc;
    const int64_t tt = rem - cc * Tc;
    out[(s[4] + tt) * L.st + (s[0] + hh) * L.sh + (s[2] + cc) * L.sc] =
        unpack_symbol(src, nbytes, i, b);
  }
}

// One thread per output byte: ORs in the (at most 8) symbols overlapping it.
__global__ __launch_bounds__(kThreads) void generic_pack_kernel(
    const uint8_t* __restrict__ symbols, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ bits, const int64_t* __restrict__ specs,
    GenericLayout L, uint8_t* __restrict__ flat) {
  const int64_t k = blockIdx.y;
  const int64_t* s = specs + 6 * k;
  const int64_t Tc = s[5] - s[4], Cc = s[3] - s[2];
  const int64_t per_head = Tc * Cc, n = (s[1] - s[0]) * per_head;
  const int b = static_cast<int>(bits[k]);
  const uint32_t mask = (1u << b) - 1u;
  uint8_t* dst = flat + offsets[k];
  const int64_t nbytes = offsets[k + 1] - offsets[k];
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t byte = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; byte < nbytes;
       byte += step) {
    const int64_t first = (byte * 8) / b;
    int64_t last = (byte * 8 + 7) / b;
    if (last > n - 1) last = n - 1;
    uint32_t acc = 0;
    for (int64_t i = first; i <= last; ++i) {
      const int64_t hh = i / per_head;
      const int64_t rem = i - hh * per_head;
      const int64_t cc = rem / Tc;
      const int64_t tt = rem - cc * Tc;
      const uint32_t sym =
          symbols[(s[4] + tt) * L.st + (s[0] + hh) * L.sh + (s[2] + cc) * L.sc] & mask;
      const int64_t shift = i * b - byte * 8;
      acc |= shift >= 0 ? (sym << shift) : (sym >> (-shift));
    }
    dst[byte] = static_cast<uint8_t>(acc & 0xffu);
  }
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(uint8_t* __restrict__ p, int64_t n) {
  // p is 16-byte aligned by the caller; the tail is written bytewise.
  const int64_t nvec = n >> 4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = tid; i < nvec; i += step)
    reinterpret_cast<uint4*>(p)[i] = make_uint4(0, 0, 0, 0);
  const int64_t tail = n - (nvec << 4);
  if (tid < tail) p[(nvec << 4) + tid] = 0;
}

__global__ __launch_bounds__(kThreads) void fill_zero_bytes_kernel(uint8_t* __restrict__ p, int64_t n) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step)
    p[i] = 0;
}

// ---------------------------------------------------------------------------
// Paged block copies (token-major K/V <-> cache)
// ---------------------------------------------------------------------------

struct BlockCopyParams {
  const uint8_t* src;
  uint8_t* dst;
  const int64_t* block_ids;
  int64_t num_blocks;
  int64_t T;           // valid tokens per half in the token-major tensor
  int64_t Tt;          // token-major tokens per half (T for scatter, block_count*bs for gather)
  int64_t block_count, bs, blk_stride, half_stride;
  int64_t row_bytes;   // H * head_bytes
};

// SCATTER: token-major value -> cache rows (zero rows for t >= T).
// GATHER:  cache rows -> token-major value.
// Byte path (rows not a multiple of 16 bytes, or unaligned buffers): one
// thread per byte.
template <bool SCATTER>
__global__ __launch_bounds__(kThreads) void block_copy_bytes_kernel(BlockCopyParams p) {
  const int64_t rows_per_half = p.block_count * p.bs;
  const int64_t total = 2 * rows_per_half * p.row_bytes;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += step) {
    const int64_t v = idx % p.row_bytes;
    const int64_t r = idx / p.row_bytes;
    const int64_t t = r % rows_per_half;
    const int64_t half = r / rows_per_half;
    const int64_t blk = t / p.bs;
    const int64_t pid = p.block_ids[blk];
    if (pid < 0 || pid >= p.num_blocks) continue;
    const int64_t cache_off =
        (pid * p.blk_stride + half * p.half_stride + (t - blk * p.bs)) * p.row_bytes + v;
    if constexpr (SCATTER)
      p.dst[cache_off] = t < p.T ? p.src[(half * p.T + t) * p.row_bytes + v] : 0;
    else
      p.dst[(half * p.Tt + t) * p.row_bytes + v] = p.src[cache_off];
  }
}

// 16-byte path: one workgroup per (half, block) pair.  A block's bs rows are
// one contiguous run of the cache (both layouts) and of the token-major
// value, so the workgroup copies bs * row_bytes contiguous bytes, 16 per
// lane, kBlockCopyUnroll loads in flight per lane before their stores; rows
// past T are written as zeros.  Each byte is read and written once:
// non-temporal accesses.
constexpr int kBlockCopyUnroll = 8;

template <bool SCATTER>
__global__ __launch_bounds__(kThreads) void block_copy_kernel(BlockCopyParams p) {
  const int64_t items = 2 * p.block_count;
  const int64_t run = p.bs * p.row_bytes;  // bytes of one block-half
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int64_t half = item / p.block_count;
    const int64_t blk = item - half * p.block_count;
    const int64_t pid = p.block_ids[blk];
    if (pid < 0 || pid >= p.num_blocks) continue;
    uint8_t* const cache = SCATTER ? p.dst : const_cast<uint8_t*>(p.src);
    uint8_t* const crun = cache + (pid * p.blk_stride + half * p.half_stride) * p.row_bytes;
    const int64_t t0 = blk * p.bs;
    // value bytes of this block-half that hold tokens (scatter: rows below T)
    const int64_t valid =
        SCATTER ? (p.T - t0 >= p.bs ? run : p.T > t0 ? (p.T - t0) * p.row_bytes : 0) : run;
    const uint8_t* const src =
        SCATTER ? p.src + (half * p.T + t0) * p.row_bytes : crun;
    uint8_t* const dst = SCATTER ? crun : p.dst + (half * p.Tt + t0) * p.row_bytes;
    constexpr int64_t kStep = static_cast<int64_t>(kThreads) * 16;
    for (int64_t base = static_cast<int64_t>(threadIdx.x) * 16; base < run;
         base += kStep * kBlockCopyUnroll) {
      u32x4 x[kBlockCopyUnroll];
#pragma unroll
      for (int u = 0; u < kBlockCopyUnroll; ++u) {
        const int64_t off = base + u * kStep;
        x[u] = u32x4{0u, 0u, 0u, 0u};
        if (off < valid) x[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + off));
      }
#pragma unroll
      for (int u = 0; u < kBlockCopyUnroll; ++u) {
        const int64_t off = base + u * kStep;
        if (off < run) __builtin_nontemporal_store(x[u], reinterpret_cast<u32x4*>(dst + off));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Launch helpers
// ---------------------------------------------------------------------------

int launch_fill_zero(uint8_t* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return ORIGAMI_OK;
  if (aligned16(p)) {
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n >> 4, kThreads, 65536)), dim3(kThreads), 0,
                       stream, p, n);
  } else {
    hipLaunchKernelGGL(fill_zero_bytes_kernel, dim3(grid_for(n, kThreads, 65536)), dim3(kThreads),
                       0, stream, p, n);
  }
  return check_launch("fill_zero_kernel");
}

// Fills the stream fields of RowsParams: `flat` may have any alignment.
void set_stream(RowsParams& p, const uint8_t* flat, int64_t flat_bytes) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(flat);
  const uintptr_t base = addr & ~uintptr_t(3);
  p.stream = reinterpret_cast<uint8_t*>(base);
  p.bit_bias = static_cast<int64_t>(addr - base) * 8;
  p.stream_bytes = flat_bytes + static_cast<int64_t>(addr - base);
}

// A kRowsBits pack ORs its runs into the stream, so the chunks' bytes
// [offsets[0], offsets[n]) are cleared first; bytes of the caller's buffer
// outside them are left as they are.
int clear_bits_stream(int mode, uint8_t* flat, const int64_t* offsets, int64_t n,
                      hipStream_t stream) {
  if (mode != kRowsBits || n <= 0) return ORIGAMI_OK;
  return launch_fill_zero(flat + offsets[0], offsets[n] - offsets[0], stream);
}

// Points the row kernels at the plan's plane offsets: the closed form of a
// dense plan (no device memory), or its uploaded plane table.
int set_planes(RowsParams& p, const std::shared_ptr<const Plan>& plan) {
  if (plan->info.dense) {
    p.planes = nullptr;
    p.plane_base = plan->info.dense_base;
    p.plane_bits = plan->T * plan->info.bits;
    return ORIGAMI_OK;
  }
  if (int rc = plan_device(plan)) return rc;
  p.planes = plan->d_table;
  return ORIGAMI_OK;
}

// Compute units of the current device (cached per device).
int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Grid of the rows kernels.  When heads are contiguous inside a row
// (head_pitch == C) and the plane table is indexed h * C + c, the heads are
// folded into one row of H * C channels so a workgroup can span them.  The
// workgroup is the largest of 16, 8 or 4 waves that still gives at least two
// workgroups per CU over `nhalf` halves of `tile_tokens_total` tokens.
void set_grid_dims(RowsParams& p, int64_t H, int64_t C, int64_t tile_tokens_total,
                   int64_t nhalf, int wq_max = kRowsWq, int seg_tokens = kSegTokens,
                   int max_waves = kRowsMaxWaves, int64_t want_tiles = 0) {
  if (H > 1 && p.head_pitch == C) {
    C *= H;
    H = 1;
  }
  p.H = static_cast<int32_t>(H);
  p.C = C;
  p.nq = static_cast<int32_t>(C / 16);
  const int nqg = (p.nq + kLaneGroups - 1) / kLaneGroups;
  const int64_t segs = (tile_tokens_total + seg_tokens - 1) / seg_tokens;
  const int64_t cus = device_cu_count();
  const int64_t want = want_tiles > 0 ? want_tiles : 2 * cus;
  // tiles of a `waves`-wave workgroup shape (sets the shape fields of p)
  auto shape = [&](int waves) {
    const int wq_cap = std::min(waves == kRowsMaxWaves ? kRowsWq : 2, wq_max);
    int wq = 1;
    while (wq < wq_cap && wq * 2 <= nqg && wq * 2 <= waves) wq *= 2;
    p.waves = waves;
    p.wq = wq;
    p.ws = waves / wq;
    p.nqt = (nqg + wq - 1) / wq;
    const int64_t segs_per_wg = static_cast<int64_t>(p.ws) * kLaneSegs;
    p.nst = static_cast<int32_t>((segs + segs_per_wg - 1) / segs_per_wg);
    return nhalf * H * static_cast<int64_t>(p.nqt) * p.nst;
  };
  int waves = max_waves;
  int64_t tiles = shape(waves);
  while (tiles < want && waves > 4) tiles = shape(waves /= 2);
  // Short of `want` at 4 waves: 2-wave tiles when they lower the most work a
  // CU gets (tiles per CU rounded up, times waves per tile).  Restore / pack
  // of Llama-3-8B geometry, us / GB/s: 2048 tokens 6.87 -> 5.61 / 2515 ->
  // 2793, 6144 tokens 14.1 -> 12.0 / 3650 -> 4644; where it is a tie (4096,
  // 7168 tokens) 2-wave tiles ran up to 15% slower.  Not for the staged pack
  // (wq_max 1), whose workgroups hold LDS rounds for 4 waves or more.
  if (tiles < want && waves == 4 && wq_max != 1) {
    const int64_t load4 = (tiles + cus - 1) / cus * 4;
    const int64_t tiles2 = shape(2);
    if ((tiles2 + cus - 1) / cus * 2 < load4)
      tiles = tiles2;
    else
      tiles = shape(4);
  }
  const int64_t segs_per_wg = static_cast<int64_t>(p.ws) * kLaneSegs;
  p.partial_last = p.nst > 1 && segs % segs_per_wg != 0;
}

// Workgroup shape of a batched restore: set_grid_dims' rule with the launch
// size summed over the requests (each request has its own token tiles), then
// each request's tile count and first tile.
void set_batch_grid(RowsBatch& b, int64_t H, int64_t C) {
  RowsParams& p = b.common;
  p.partial_last = 0;  // tile_coord's order is per request here
  if (H > 1 && p.head_pitch == C) {
    C *= H;
    H = 1;
  }
  p.H = static_cast<int32_t>(H);
  p.C = C;
  p.nq = static_cast<int32_t>(C / 16);
  const int nqg = (p.nq + kLaneGroups - 1) / kLaneGroups;
  const int64_t want = 2 * static_cast<int64_t>(device_cu_count());
  auto nst_of = [&](int64_t row_tokens) {
    const int64_t segs = (row_tokens + kSegTokens - 1) / kSegTokens;
    const int64_t segs_per_wg = static_cast<int64_t>(p.ws) * kLaneSegs;
    return (segs + segs_per_wg - 1) / segs_per_wg;
  };
  auto shape = [&](int waves) {
    const int wq_cap = waves == kRowsMaxWaves ? kRowsWq : 2;
    int wq = 1;
    while (wq < wq_cap && wq * 2 <= nqg && wq * 2 <= waves) wq *= 2;
    p.waves = waves;
    p.wq = wq;
    p.ws = waves / wq;
    p.nqt = (nqg + wq - 1) / wq;
    int64_t tiles = 0;
    for (int r = 0; r < b.nreq; ++r)
      tiles += 2 * H * p.nqt * nst_of(b.req[r].row_tokens - b.req[r].token0);
    return tiles;
  };
  int waves = kRowsMaxWaves;
  int64_t tiles = shape(waves);
  while (tiles < want && waves > 4) tiles = shape(waves /= 2);
  // short of `want` at 4 waves: 2-wave tiles when they lower the most work a
  // CU gets, as set_grid_dims does for one request
  if (tiles < want && waves == 4) {
    const int64_t cus = device_cu_count();
    const int64_t load4 = (tiles + cus - 1) / cus * 4;
    const int64_t tiles2 = shape(2);
    if ((tiles2 + cus - 1) / cus * 2 >= load4) shape(4);
  }
  const int64_t per = 2 * H * static_cast<int64_t>(p.nqt);  // tiles per token tile
  const int64_t tile_tokens = static_cast<int64_t>(p.ws) * kLaneSegs * kSegTokens;
  int64_t tile0 = 0;
  for (int r = 0; r < b.nreq; ++r) {
    const int64_t n = b.req[r].row_tokens - b.req[r].token0;
    b.req[r].nst = static_cast<int32_t>(nst_of(n));
    b.req[r].partial = n % tile_tokens != 0 ? 1 : 0;
    b.req[r].tile0 = tile0;
    tile0 += per * (b.req[r].nst - b.req[r].partial);
  }
  b.nfull = tile0;
  for (int r = 0; r < b.nreq; ++r) {
    b.req[r].ptile0 = tile0;
    tile0 += per * b.req[r].partial;
  }
  p.ntiles = tile0;
}

// Average waves per CU over a launch of `ntiles` workgroups of `waves` waves,
// at most the 16 a CU holds at once.
double waves_per_cu(int64_t ntiles, int waves) {
  const double w = static_cast<double>(ntiles) * waves / device_cu_count();
  return w < 16.0 ? w : 16.0;
}

// Row order of the whole-tile row kernels by launch size (waves per CU).
// One-block rows (for_rows16) for restores and staged packs up to 6 waves per
// CU (4096 tokens of Llama-3-8B: 9.6 -> 8.0 us; 8192 tokens: 14.0 -> 14.6, so
// not above), for the other packs up to 12 (4096 tokens: 2.07 -> 4.03 TB/s;
// 12288: 4.50 -> 4.74; 16384 tokens at 16: 5.07 -> 4.83).  Serial plane loads
// (load_planes16) for b = 7, 8 shift restores above 12 waves per CU.
constexpr double kOneBlockWaves = 6;
constexpr double kOneBlockPackWaves = 12;
constexpr double kSerialLoadWaves = 12;

bool one_block_rows(const RowsParams& p) { return !p.block_ids || (p.bs & 15) == 0; }

// A batched restore: split (sh > 0) into 4-wave slices, or whole-tile
// workgroups with the row order of launch_unpack_tiles.
template <int BITS, int MODE>
void launch_batch_tiles(dim3 grid, dim3 block, hipStream_t stream, const RowsBatch& b, int sh,
                        bool oneblk, bool serial) {
  if (sh > 0) {
    if (oneblk)
      hipLaunchKernelGGL((rows_unpack_batch_split_kernel<BITS, MODE, true>), grid, block, 0,
                         stream, b, sh);
    else
      hipLaunchKernelGGL((rows_unpack_batch_split_kernel<BITS, MODE, false>), grid, block, 0,
                         stream, b, sh);
    return;
  }
  if constexpr (MODE == kRowsShift && BITS >= 7) {
    if (serial && !oneblk) {
      hipLaunchKernelGGL((rows_unpack_batch_kernel<BITS, MODE, false, true>), grid, block, 0,
                         stream, b);
      return;
    }
  }
  if (oneblk)
    hipLaunchKernelGGL((rows_unpack_batch_kernel<BITS, MODE, true, false>), grid, block, 0,
                       stream, b);
  else
    hipLaunchKernelGGL((rows_unpack_batch_kernel<BITS, MODE, false, false>), grid, block, 0,
                       stream, b);
}

int launch_rows_batch(const RowsBatch& b, int bits, int mode, hipStream_t stream) {
  if (b.common.ntiles <= 0) return ORIGAMI_OK;
  // At least kRowsSplitTiles tiles per CU: each tile as 4-wave workgroups,
  // as launch_rows does for one request.
  int sh = 0;
  if (b.common.waves > kRowsSplitWaves &&
      b.common.ntiles >= kRowsSplitTiles * static_cast<int64_t>(device_cu_count()))
    while ((kRowsSplitWaves << sh) < b.common.waves) ++sh;
  const bool split = sh > 0;
  bool rows1 = true;  // one-block rows (for_rows16) possible for every request
  for (int r = 0; r < b.nreq; ++r)
    if (b.req[r].block_ids && (b.common.bs & 15) != 0) rows1 = false;
  // whole-tile workgroups: the single-request rules by launch size
  const double wpc = waves_per_cu(b.common.ntiles, b.common.waves);
  const bool oneblk = rows1 && (split || wpc <= kOneBlockWaves);
  const bool serial = !split && wpc > kSerialLoadWaves;
  int64_t blocks = b.common.ntiles << sh;
  if (g_rows_grid_limit > 0 && blocks > g_rows_grid_limit) blocks = g_rows_grid_limit;
  if (blocks > INT32_MAX) blocks = INT32_MAX;
  const dim3 grid(static_cast<unsigned>(blocks)),
      block(static_cast<unsigned>(64 * (split ? kRowsSplitWaves : b.common.waves)));
  if (bits == 8 && mode == kRowsAligned16) {
    launch_batch_tiles<8, kRowsAligned16>(grid, block, stream, b, sh, oneblk, serial);
    return check_launch("rows_unpack_batch_kernel");
  }
  const bool window = mode == kRowsWindow;
#define ORIGAMI_BATCH_CASE(B)                                                          \
  case B:                                                                              \
    if (window)                                                                        \
      launch_batch_tiles<B, kRowsWindow>(grid, block, stream, b, sh, oneblk, serial);  \
    else                                                                               \
      launch_batch_tiles<B, kRowsShift>(grid, block, stream, b, sh, oneblk, serial);   \
    break;
  switch (bits) {
    ORIGAMI_BATCH_CASE(1)
    ORIGAMI_BATCH_CASE(2)
    ORIGAMI_BATCH_CASE(3)
    ORIGAMI_BATCH_CASE(4)
    ORIGAMI_BATCH_CASE(5)
    ORIGAMI_BATCH_CASE(6)
    ORIGAMI_BATCH_CASE(7)
    ORIGAMI_BATCH_CASE(8)
    default:
      return fail(ORIGAMI_ERR_INVALID, "Origami CUDA bitpack supports only 1..8 bit symbols");
  }
#undef ORIGAMI_BATCH_CASE
  return check_launch("rows_unpack_batch_kernel");
}

// Addressing mode of the row kernels for this plan and stream: `T` is the
// symbol count per half (a multiple of 16 keeps every lane run inside its
// plane).  The rows pack is only launched for byte-aligned planes with T * b
// a multiple of 8, so its runs always start on bytes.
int rows_mode(const PlanInfo& info, const RowsParams& p, int64_t T, bool pack,
              int64_t token0 = 0, bool allow_wide = false) {
  if (allow_wide && !pack && p.bit_bias == 0 && aligned16(p.stream) && info.planes16 &&
      (info.bits == 1 || info.bits == 2 || info.bits == 4)) {
    const int64_t seg = 128 / info.bits;
    if (T % seg == 0 && token0 % seg == 0) {
      const bool lines = info.planes_lines && (reinterpret_cast<uintptr_t>(p.stream) & 127) == 0 &&
                         (T * info.bits) % 1024 == 0 && (token0 * info.bits) % 1024 == 0;
      return lines ? kRowsWide : kRowsWideCached;
    }
  }
  if (p.bit_bias == 0 && T % 16 == 0) {
    if (info.aligned16 && aligned16(p.stream)) {
      // Non-temporal when every plane starts on a 128-byte line and, for the
      // restore, the V half too (T % 128 == 0).  The pack kept non-temporal
      // stores faster with only the V half off the line: 4136 against 3794
      // GB/s at T = 32832.  (A pack of planes off the line is staged through
      // LDS instead: pack_mode.)
      const bool lines = info.lines128 && (reinterpret_cast<uintptr_t>(p.stream) & 127) == 0;
      // Lane runs start at token0 + 16 k: a batched request restored past
      // its shared prefix needs token0 % 128 == 0 too.
      return lines && (pack || (T % 128 == 0 && token0 % 128 == 0)) ? kRowsAligned16
                                                                    : kRowsAligned16Cached;
    }
    const bool runs_ok = info.bits % 2 == 0 ? info.planes_dword : info.planes_even;
    if (runs_ok) return kRowsWindow;
  }
  return pack ? kRowsBytes : kRowsShift;
}

// Workgroup grid of a single-request restore in `mode`: wide runs hold
// 128 / b tokens and their workgroups at most kWideMaxWaves waves.
void set_restore_grid(RowsParams& p, int mode, int bits, int64_t H, int64_t C,
                      int64_t tile_tokens_total, int64_t nhalf) {
  if (mode == kRowsWide || mode == kRowsWideCached)
    set_grid_dims(p, H, C, tile_tokens_total, nhalf, kRowsWq, 128 / bits, kWideMaxWaves);
  else
    set_grid_dims(p, H, C, tile_tokens_total, nhalf);
}

// Mode of the rows pack: 8-bit planes off 128-byte lines go through LDS so
// that every stream line is written whole (32753 tokens: 3062 -> 3766 GB/s;
// 32784, planes 32 bytes off: 3163 -> 3399).  Planes on lines keep in-place
// non-temporal stores even when the V half is not: 3874 against 3608 staged
// at 32832 tokens.
int pack_mode(const PlanInfo& info, const RowsParams& p, int64_t T) {
  if (info.bits < 8 && (!info.byte_aligned || (T * info.bits) % 8 != 0)) return kRowsBits;
  const int mode = rows_mode(info, p, T, true);
  if (info.bits == 8 && mode != kRowsAligned16) return kRowsStaged8;
  return mode;
}

// Channel columns per workgroup tile of the staged pack: 1, 128 channels x
// 2048 tokens, so a plane's region in a tile spans 17 lines, 2 of them shared
// with the neighbouring tiles (3766 GB/s at 32753 tokens, against 3436 for
// 256 x 1024 tiles).
constexpr int kStagedWq = 1;

// Workgroup grid of a pack in `mode`.  The staged pack takes the largest
// workgroups that still give half a tile per CU (the rows kernels want two):
// its LDS rounds and barriers favour fewer, larger tiles.  GB/s with 4-, 8-
// and 16-wave workgroups: 4100 tokens 1550 / 1649 / 1375, 8200 tokens 2320 /
// 2315 / 2482, 15000 tokens 3235 / 3565 / 3824; at 2053 tokens 4-wave tiles
// stay fastest (955 against 901 / 699).
void set_pack_grid(RowsParams& p, int mode, int64_t H, int64_t C, int64_t T, int64_t nhalf) {
  p.own_lines = 0;
  if (mode == kRowsStaged8) {
    set_grid_dims(p, H, C, T, nhalf, kStagedWq, kSegTokens, kRowsMaxWaves,
                  std::max<int64_t>(1, device_cu_count() / 2));
    // 16-wave tiles write each stream line from one tile (kOwnTokens per
    // tile) when that takes no more rounds of tiles per CU (one 16-wave tile
    // per CU at a time): the smaller tiles are more of them, and a further
    // round cost more than single ownership saves.  µs per layer, two-part
    // lines -> single owner: 49217 tokens 111.0 -> 103.4 (4 rounds either
    // way); 32753 tokens 62.9 -> 73.3 and 16383 tokens 30.5 -> 46.5 (2 -> 3
    // and 1 -> 2 rounds: not taken).
    if (p.waves == 16 && p.wq == 1 && T >= 128 && nhalf == 2) {
      const int64_t nst_own = (T + kOwnTokens - 1) / kOwnTokens;
      const int64_t per_st = nhalf * p.H * static_cast<int64_t>(p.nqt);
      const int64_t cus = device_cu_count();
      if ((per_st * nst_own + cus - 1) / cus <= (per_st * p.nst + cus - 1) / cus) {
        p.own_lines = 1;
        p.nst = static_cast<int32_t>(nst_own);
        p.partial_last = 0;
      }
    }
  } else {
    set_grid_dims(p, H, C, T, nhalf);
  }
}

template <int BITS, int MODE>
void launch_unpack_tiles(dim3 grid, dim3 block, hipStream_t stream, const RowsParams& p,
                         bool oneblk, bool serial) {
  if constexpr (MODE == kRowsShift && BITS >= 7) {
    if (serial && !oneblk) {
      hipLaunchKernelGGL((rows_unpack_kernel<BITS, MODE, false, true>), grid, block, 0, stream, p);
      return;
    }
  }
  if (oneblk)
    hipLaunchKernelGGL((rows_unpack_kernel<BITS, MODE, true, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((rows_unpack_kernel<BITS, MODE, false, false>), grid, block, 0, stream, p);
}

template <int BITS, int MODE>
void launch_pack_tiles(dim3 grid, dim3 block, hipStream_t stream, const RowsParams& p,
                       bool oneblk) {
  if (oneblk)
    hipLaunchKernelGGL((rows_pack_kernel<BITS, MODE, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((rows_pack_kernel<BITS, MODE, false>), grid, block, 0, stream, p);
}

template <int WAVES>
void launch_staged_tiles(dim3 grid, dim3 block, hipStream_t stream, const RowsParams& p,
                         bool oneblk) {
  if constexpr (WAVES == 16) {
    if (p.own_lines) {  // the row walk whatever `oneblk` says (pack_tile_owned)
      hipLaunchKernelGGL((rows_pack_staged8_kernel<16, false, true>), grid, block, 0, stream, p);
      return;
    }
  }
  if (oneblk)
    hipLaunchKernelGGL((rows_pack_staged8_kernel<WAVES, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((rows_pack_staged8_kernel<WAVES, false>), grid, block, 0, stream, p);
}

template <int BITS>
void launch_wide_tiles(dim3 grid, dim3 block, hipStream_t stream, const RowsParams& p, bool nt,
                       bool oneblk) {
  if (nt && oneblk)
    hipLaunchKernelGGL((rows_unpack_wide_kernel<BITS, true, true>), grid, block, 0, stream, p);
  else if (nt)
    hipLaunchKernelGGL((rows_unpack_wide_kernel<BITS, true, false>), grid, block, 0, stream, p);
  else if (oneblk)
    hipLaunchKernelGGL((rows_unpack_wide_kernel<BITS, false, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((rows_unpack_wide_kernel<BITS, false, false>), grid, block, 0, stream, p);
}

template <int BITS, int MODE>
int launch_split(dim3 grid, dim3 block, hipStream_t stream, const RowsParams& p, int sh,
                 bool oneblk) {
  if (oneblk)
    hipLaunchKernelGGL((rows_unpack_split_kernel<BITS, MODE, true>), grid, block, 0, stream, p, sh);
  else
    hipLaunchKernelGGL((rows_unpack_split_kernel<BITS, MODE, false>), grid, block, 0, stream, p,
                       sh);
  return check_launch("rows_unpack_split_kernel");
}

// Restore launch in kRowsSplitWaves-wave workgroups, 2^sh per tile.
int launch_rows_split(const RowsParams& p, int bits, int mode, hipStream_t stream) {
  int sh = 0;
  while ((kRowsSplitWaves << sh) < p.waves) ++sh;
  int64_t blocks = p.ntiles << sh;
  if (g_rows_grid_limit > 0 && blocks > g_rows_grid_limit) blocks = g_rows_grid_limit;
  if (blocks > INT32_MAX) blocks = INT32_MAX;
  const dim3 grid(static_cast<unsigned>(blocks)), block(64 * kRowsSplitWaves);
  const bool oneblk = !p.block_ids || (p.bs & 15) == 0;
  if (bits == 8 && mode == kRowsAligned16)
    return launch_split<8, kRowsAligned16>(grid, block, stream, p, sh, oneblk);
  if (bits == 8 && mode == kRowsAligned16Cached)
    return launch_split<8, kRowsAligned16Cached>(grid, block, stream, p, sh, oneblk);
  const bool window = mode == kRowsWindow;
#define ORIGAMI_SPLIT_CASE(B)                                                    \
  case B:                                                                        \
    return window ? launch_split<B, kRowsWindow>(grid, block, stream, p, sh, oneblk) \
                  : launch_split<B, kRowsShift>(grid, block, stream, p, sh, oneblk);
  switch (bits) {
    ORIGAMI_SPLIT_CASE(1)
    ORIGAMI_SPLIT_CASE(2)
    ORIGAMI_SPLIT_CASE(3)
    ORIGAMI_SPLIT_CASE(4)
    ORIGAMI_SPLIT_CASE(5)
    ORIGAMI_SPLIT_CASE(6)
    ORIGAMI_SPLIT_CASE(7)
    ORIGAMI_SPLIT_CASE(8)
    default:
      return fail(ORIGAMI_ERR_INVALID, "Origami CUDA bitpack supports only 1..8 bit symbols");
  }
#undef ORIGAMI_SPLIT_CASE
}

int launch_rows(bool pack, const RowsParams& params, int64_t nhalf, int bits, int mode,
                hipStream_t stream) {
  RowsParams p = params;
  p.ntiles = nhalf * p.H * static_cast<int64_t>(p.nqt) * p.nst;
  if (p.ntiles <= 0) return ORIGAMI_OK;
  // partial token tiles last: restore 32784 tokens 64.0 -> 61.4 us, 49216
  // tokens 96.8 -> 94.8 us; the pack ran 2-5% slower that way
  if (pack) p.partial_last = 0;
  if (!pack && mode != kRowsWide && mode != kRowsWideCached && p.waves > kRowsSplitWaves &&
      p.ntiles >= kRowsSplitTiles * static_cast<int64_t>(device_cu_count()))
    return launch_rows_split(p, bits, mode, stream);
  int64_t blocks = p.ntiles;
  if (g_rows_grid_limit > 0 && blocks > g_rows_grid_limit) blocks = g_rows_grid_limit;
  if (blocks > INT32_MAX) blocks = INT32_MAX;
  const dim3 grid(static_cast<unsigned>(blocks)), block(static_cast<unsigned>(64 * p.waves));
  const double wpc = waves_per_cu(p.ntiles, p.waves);
  const bool staged = mode == kRowsStaged8;
  const bool oneblk =
      one_block_rows(p) && wpc <= (pack && !staged ? kOneBlockPackWaves : kOneBlockWaves);
  const bool serial = wpc > kSerialLoadWaves;
  if (mode == kRowsWide || mode == kRowsWideCached) {
    if (pack || p.waves > kWideMaxWaves)
      return fail(ORIGAMI_ERR_INVALID, "wide rows mode is a restore of at most 8-wave tiles");
    const bool nt = mode == kRowsWide;
    switch (bits) {
      case 1:
        launch_wide_tiles<1>(grid, block, stream, p, nt, oneblk);
        break;
      case 2:
        launch_wide_tiles<2>(grid, block, stream, p, nt, oneblk);
        break;
      case 4:
        launch_wide_tiles<4>(grid, block, stream, p, nt, oneblk);
        break;
      default:
        return fail(ORIGAMI_ERR_INVALID, "wide rows mode takes 1, 2 or 4-bit symbols");
    }
    return check_launch("rows_unpack_wide_kernel");
  }
  if (bits == 8 && mode == kRowsAligned16) {
    if (pack)
      launch_pack_tiles<8, kRowsAligned16>(grid, block, stream, p, oneblk);
    else
      launch_unpack_tiles<8, kRowsAligned16>(grid, block, stream, p, oneblk, serial);
    return check_launch(pack ? "rows_pack_kernel" : "rows_unpack_kernel");
  }
  if (pack && bits == 8 && !staged)  // pack_mode: aligned16 or staged
    return fail(ORIGAMI_ERR_INVALID, "8-bit rows pack modes are aligned16 and staged");
  if (bits == 8 && mode == kRowsAligned16Cached) {
    launch_unpack_tiles<8, kRowsAligned16Cached>(grid, block, stream, p, oneblk, serial);
    return check_launch("rows_unpack_kernel");
  }
  if (staged) {
    if (!pack || bits != 8) return fail(ORIGAMI_ERR_INVALID, "staged rows mode is the 8-bit pack");
    // Non-temporal chunk stores below kStagedNtTiles tiles per CU.  Pack
    // GB/s, plain -> non-temporal (same box, two runs each): 4100 tokens
    // 1696 / 1697 -> 1802 / 1762, 8199: 2368 / 2366 -> 2584 / 2606, 16383:
    // 4429 / 4375 -> 4637 / 4795, 32753: 4292 / 4303 -> 4308 / 4333, 49217:
    // 3638 / 3645 -> 3766 / 3776; 65521 tokens (4 tiles per CU): 4203 / 4201
    // -> 4135 / 4119.
    p.nt_stores = p.ntiles < kStagedNtTiles * static_cast<int64_t>(device_cu_count());
    if (p.waves == 16)
      launch_staged_tiles<16>(grid, block, stream, p, oneblk);
    else if (p.waves == 8)
      launch_staged_tiles<8>(grid, block, stream, p, oneblk);
    else if (p.waves == 4)
      launch_staged_tiles<4>(grid, block, stream, p, oneblk);
    else
      return fail(ORIGAMI_ERR_INVALID, "staged pack workgroups have 4, 8 or 16 waves");
    return check_launch("rows_pack_staged8_kernel");
  }
  if (mode == kRowsBits && (!pack || bits >= 8))
    return fail(ORIGAMI_ERR_INVALID, "bit rows mode is a sub-byte pack");
  const bool window = mode == kRowsWindow;
#define ORIGAMI_ROWS_CASE(B)                                                          \
  case B:                                                                             \
    if (pack && window)                                                               \
      launch_pack_tiles<B, kRowsWindow>(grid, block, stream, p, oneblk);              \
    else if (pack && mode == kRowsBits)                                               \
      launch_pack_tiles<B, kRowsBits>(grid, block, stream, p, oneblk);                \
    else if (pack)                                                                    \
      launch_pack_tiles<B, kRowsBytes>(grid, block, stream, p, oneblk);               \
    else if (window)                                                                  \
      launch_unpack_tiles<B, kRowsWindow>(grid, block, stream, p, oneblk, serial);    \
    else                                                                              \
      launch_unpack_tiles<B, kRowsShift>(grid, block, stream, p, oneblk, serial);     \
    break;
  switch (bits) {
    ORIGAMI_ROWS_CASE(1)
    ORIGAMI_ROWS_CASE(2)
    ORIGAMI_ROWS_CASE(3)
    ORIGAMI_ROWS_CASE(4)
    ORIGAMI_ROWS_CASE(5)
    ORIGAMI_ROWS_CASE(6)
    ORIGAMI_ROWS_CASE(7)
    case 8:  // restore only: the 8-bit pack is aligned16 or staged
      if (window)
        launch_unpack_tiles<8, kRowsWindow>(grid, block, stream, p, oneblk, serial);
      else
        launch_unpack_tiles<8, kRowsShift>(grid, block, stream, p, oneblk, serial);
      break;
    default:
      return fail(ORIGAMI_ERR_INVALID, "Origami CUDA bitpack supports only 1..8 bit symbols");
  }
#undef ORIGAMI_ROWS_CASE
  return check_launch(pack ? "rows_pack_kernel" : "rows_unpack_kernel");
}

const int64_t kKvAxes[4] = {0, 1, 2, -1};

// Checks shared by the fused restore entry points (sizes, cache geometry,
// chunk metadata against the [2 * tokens, heads, head_bytes] symbol view).
int check_fused_restore(const int64_t* offsets, const int64_t* bits, const int64_t* specs,
                        int64_t n, int64_t flat_bytes, int64_t tokens, const void* kv_cache,
                        int64_t cache_layout, int64_t num_blocks, int64_t block_size,
                        int64_t num_heads, int64_t head_bytes, int64_t block_count,
                        int64_t* blk_stride, int64_t* half_stride) {
  ORIGAMI_REQUIRE(tokens > 0 && num_heads > 0 && head_bytes > 0,
                  "tokens, heads, and head_dim must be positive");
  ORIGAMI_REQUIRE(block_size > 0, "kv_cache block size must be positive");
  ORIGAMI_REQUIRE(num_blocks > 0, "kv_cache must hold at least one block");
  ORIGAMI_REQUIRE(block_count > 0, "block_ids must be non-empty");
  ORIGAMI_REQUIRE(tokens <= block_count * block_size, "tokens exceed destination block capacity");
  const int64_t shape[3] = {2 * tokens, num_heads, head_bytes};
  int rc = validate_layout(offsets, bits, specs, n, shape, 3, kKvAxes, 2 * tokens, num_heads,
                           head_bytes, flat_bytes, nullptr);
  if (rc) return rc;
  rc = cache_geometry(cache_layout, num_blocks, block_size, blk_stride, half_stride);
  if (rc) return rc;
  if (head_bytes % 16 != 0 || !aligned16(kv_cache) || num_heads * head_bytes > kMaxPlaneTable)
    return fail(ORIGAMI_ERR_UNSUPPORTED, "fused restore needs 16-byte head rows");
  return ORIGAMI_OK;
}

// Row-kernel parameters of a fused restore (planes are set by the caller).
RowsParams fused_restore_params(const uint8_t* flat, int64_t flat_bytes, int64_t tokens,
                                void* kv_cache, int64_t num_blocks, int64_t block_size,
                                int64_t num_heads, int64_t head_bytes, const int64_t* block_ids,
                                int64_t block_count, int64_t blk_stride, int64_t half_stride) {
  RowsParams p{};
  set_stream(p, flat, flat_bytes);
  p.rows = static_cast<uint8_t*>(kv_cache);
  p.block_ids = block_ids;
  p.num_blocks = num_blocks;
  p.T = tokens;
  p.row_tokens = block_count * block_size;
  p.row_pitch = num_heads * head_bytes;
  p.head_pitch = head_bytes;
  p.bs = block_size;
  p.blk_stride = blk_stride;
  p.half_stride = half_stride;
  return p;
}

// ---------------------------------------------------------------------------
// Allocation-free fused restore: the plane table of a reordered chunk plan
// lives in `scratch`, a fixed device array, instead of library-allocated
// memory, and the plan is analysed per call without the plan cache.
// ---------------------------------------------------------------------------

constexpr int64_t kScratchPlanes = 131072;  // int64 plane offsets: 1 MiB per GPU
constexpr int kScratchDevices = 64;

static __device__ __align__(256) int64_t scratch[kScratchPlanes];

// Per-device state of `scratch`: its device address, looked up once per
// device (each GPU holds its own copy of the array; host code must use this
// address, never the array's name, which is only a host-side stand-in), and
// an event recorded after the last call that wrote it, with that call's
// stream, so a call from another stream can see that the array is still in
// use.  Both are set up on a device's first call.
struct ScratchState {
  int64_t* ptr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool pending = false;
};

// Holds the scratch array of the current device from acquire() to its
// destruction, under a lock, so two host threads cannot interleave their
// table fills and launches.  acquire() refuses the array while work of a
// call on another stream is still pending (the two would race on it); in a
// stream that is being captured into a graph it neither checks nor records
// (a graph's replays are ordered by the caller).
class ScratchLease {
 public:
  ~ScratchLease() {
    if (state_ && !capturing_) {
      (void)hipEventRecord(state_->done, stream_);
      state_->last = stream_;
      state_->pending = true;
    }
  }

  int acquire(hipStream_t stream, int64_t** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
      return fail(ORIGAMI_ERR_HIP, "hipGetDevice failed (or device index above 63)");
    lock_ = std::unique_lock<std::mutex>(mutex());
    ScratchState& st = states()[dev];
    if (st.ptr == nullptr) {
      void* p = nullptr;
      const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess || p == nullptr)
        return fail(ORIGAMI_ERR_HIP, std::string("hipGetSymbolAddress of the restore scratch "
                                                 "table failed: ") + hipGetErrorString(err));
      hipEvent_t ev = nullptr;
      if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
        return fail(ORIGAMI_ERR_HIP, "event creation for the restore scratch table failed");
      st.ptr = static_cast<int64_t*>(p);
      st.done = ev;
    }
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) != hipSuccess)
      return fail(ORIGAMI_ERR_HIP, "hipStreamIsCapturing failed");
    capturing_ = status != hipStreamCaptureStatusNone;
    if (!capturing_ && st.pending && st.last != stream) {
      const hipError_t q = hipEventQuery(st.done);
      if (q == hipErrorNotReady)
        return fail(ORIGAMI_ERR_INVALID,
                    "an allocation-free restore of a reordered chunk plan is still running on "
                    "another stream of this GPU; such calls share one scratch plane table and "
                    "must not overlap");
      if (q != hipSuccess) return fail(ORIGAMI_ERR_HIP, "hipEventQuery failed");
    }
    state_ = &st;
    stream_ = stream;
    *out = st.ptr;
    return ORIGAMI_OK;
  }

 private:
  static std::mutex& mutex() {
    static std::mutex mu;
    return mu;
  }
  static ScratchState* states() {
    static ScratchState s[kScratchDevices];
    return s;
  }
  std::unique_lock<std::mutex> lock_;
  ScratchState* state_ = nullptr;
  hipStream_t stream_ = nullptr;
  bool capturing_ = false;
};

// The PlanInfo build_plane_table would give, from the chunk list alone: O(n),
// plus an O(n^2) box-overlap test when the chunks are not in plane order.
PlanInfo analyze_plan(const int64_t* offsets, const int64_t* bits, const int64_t* specs,
                      int64_t n, int64_t T, int64_t H, int64_t C) {
  PlanInfo info;
  info.regular = n > 0;
  info.bits = n > 0 ? static_cast<int>(bits[0]) : 0;
  info.aligned16 = info.byte_aligned = info.planes_even = info.planes_dword = true;
  info.lines128 = true;
  info.planes16 = info.planes_lines = true;
  bool in_order = true;  // chunk k holds planes [next, next + planes_k) in h * C + c order
  int64_t next = 0;
  for (int64_t k = 0; k < n; ++k) {
    const int64_t* s = specs + 6 * k;
    if (bits[k] != info.bits) info.bits = 0;
    if (s[4] != 0 || s[5] != T) {
      info.regular = false;
      continue;
    }
    const int64_t planes = (s[1] - s[0]) * (s[3] - s[2]);
    const int64_t first = offsets[k] * 8, step = T * bits[k];
    auto all_multiple = [&](int64_t m) { return first % m == 0 && (planes == 1 || step % m == 0); };
    if (!all_multiple(128)) info.aligned16 = info.planes16 = false;
    if (!all_multiple(1024)) info.lines128 = info.planes_lines = false;
    if (!all_multiple(8)) info.byte_aligned = false;
    if (!all_multiple(16)) info.planes_even = false;
    if (!all_multiple(32)) info.planes_dword = false;
    if (in_order) {
      const bool one_run = s[1] - s[0] == 1 || (s[2] == 0 && s[3] == C);
      in_order = one_run && s[0] * C + s[2] == next && first == offsets[0] * 8 + next * step;
      next += planes;
    }
  }
  if (info.regular && !in_order) {
    // reordered boxes: a plane covered twice makes the plan irregular
    for (int64_t a = 0; a < n && info.regular; ++a) {
      const int64_t* sa = specs + 6 * a;
      for (int64_t b = a + 1; b < n; ++b) {
        const int64_t* sb = specs + 6 * b;
        if (sa[0] < sb[1] && sb[0] < sa[1] && sa[2] < sb[3] && sb[2] < sa[3]) {
          info.regular = false;
          break;
        }
      }
    }
  }
  if (info.bits != 8) info.aligned16 = false;
  if (!info.aligned16) info.lines128 = false;
  if (!info.planes16) info.planes_lines = false;
  if (!info.regular) {
    info.aligned16 = info.byte_aligned = info.planes_even = info.planes_dword = false;
    info.lines128 = false;
    info.planes16 = info.planes_lines = false;
  }
  if (info.regular && info.bits != 0 && in_order && next == H * C && H * C > 0) {
    info.dense = true;
    info.dense_base = offsets[0] * 8;
  }
  return info;
}

constexpr int kFillChunks = 32;  // chunk boxes per table-fill launch (kernel arguments)

struct PlaneFill {
  int64_t C;           // channels per head
  int64_t plane_bits;  // T * b: bits per plane
  int32_t n;           // chunks in this launch
  int64_t first_bit[kFillChunks];  // bit offset of each chunk's first symbol
  int32_t box[kFillChunks][4];     // head_start, head_end, channel_start, channel_end
};

__global__ __launch_bounds__(kThreads) void fill_i64_kernel(int64_t* __restrict__ p, int64_t n,
                                                            int64_t value) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step)
    p[i] = value;
}

// table[h * C + c] = bit offset of plane (h, c) for the chunks of one launch
// (local plane order head-major, then channel: bitpack_layout_cuda.cu:110-124).
__global__ __launch_bounds__(kThreads) void plane_table_kernel(PlaneFill f,
                                                               int64_t* __restrict__ table) {
  const int j = static_cast<int>(blockIdx.y);
  if (j >= f.n) return;
  const int64_t hs = f.box[j][0], cs = f.box[j][2];
  const int64_t cc = f.box[j][3] - cs;
  const int64_t planes = (f.box[j][1] - hs) * cc;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < planes;
       i += step) {
    const int64_t h = hs + i / cc, c = cs + i % cc;
    table[h * f.C + c] = f.first_bit[j] + i * f.plane_bits;
  }
}

// Writes the plane table of a regular, uniform-width plan into `table`
// (H * C entries, -1 for planes no chunk covers), on `stream`.
int fill_plane_table(int64_t* table, const int64_t* offsets, const int64_t* specs, int64_t n,
                     int64_t T, int64_t H, int64_t C, int bits, hipStream_t stream) {
  hipLaunchKernelGGL(fill_i64_kernel, dim3(grid_for(H * C, kThreads, 1024)), dim3(kThreads), 0,
                     stream, table, H * C, int64_t(-1));
  if (int rc = check_launch("fill_i64_kernel")) return rc;
  for (int64_t k0 = 0; k0 < n; k0 += kFillChunks) {
    PlaneFill f{};
    f.C = C;
    f.plane_bits = T * bits;
    f.n = static_cast<int32_t>(std::min<int64_t>(kFillChunks, n - k0));
    int64_t most = 0;
    for (int j = 0; j < f.n; ++j) {
      const int64_t* s = specs + 6 * (k0 + j);
      f.first_bit[j] = offsets[k0 + j] * 8;
      for (int a = 0; a < 4; ++a) f.box[j][a] = static_cast<int32_t>(s[a]);
      most = std::max(most, (s[1] - s[0]) * (s[3] - s[2]));
    }
    hipLaunchKernelGGL(plane_table_kernel, dim3(grid_for(most, kThreads, 1024), f.n),
                       dim3(kThreads), 0, stream, f, table);
    if (int rc = check_launch("plane_table_kernel")) return rc;
  }
  return ORIGAMI_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

// A prepared fused restore (origami_restore_plan_create): everything but the
// stream and cache pointers, shared read-only by every launch.
struct origami_restore_plan {
  std::shared_ptr<const Plan> plan;  // keeps a reordered plan's device table alive
  RowsParams p;                      // stream and rows set per launch
  RowsParams pw;                     // the same with the wide-run grid (b = 1, 2, 4)
  bool has_wide = false;
  int64_t stream_bytes = 0;          // chunk_offsets[num_chunks]
  int64_t tokens = 0;
  int device = 0;
};

extern "C" {

const char* origami_last_error(void) { return g_last_error.c_str(); }

int origami_abi_version(void) { return 3; }

void origami_debug_counters(int64_t* plans_created, int64_t* device_allocations) {
  if (plans_created) *plans_created = g_plans_created.load(std::memory_order_relaxed);
  if (device_allocations)
    *device_allocations = g_device_allocations.load(std::memory_order_relaxed);
}

int64_t origami_set_rows_grid_limit(int64_t max_workgroups) {
  const int64_t previous = g_rows_grid_limit;
  g_rows_grid_limit = max_workgroups > 0 ? max_workgroups : 0;
  return previous;
}

int origami_validate_chunks(const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
                            const int64_t* chunk_specs, int64_t num_chunks,
                            const int64_t* source_shape, int64_t rank,
                            const int64_t* axis_positions, int64_t token_count,
                            int64_t num_heads, int64_t head_dim, int64_t flat_bytes) {
  return validate_layout(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, source_shape,
                         rank, axis_positions, token_count, num_heads, head_dim, flat_bytes,
                         nullptr);
}

int origami_plan_planes(const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
                        const int64_t* chunk_specs, int64_t num_chunks, int64_t token_count,
                        int64_t num_heads, int64_t head_dim, int64_t* table, int64_t table_len,
                        int64_t* info) {
  ORIGAMI_REQUIRE(token_count > 0 && num_heads > 0 && head_dim > 0,
                  "canonical symbol shape must be positive");
  ORIGAMI_REQUIRE(table_len == num_heads * head_dim, "table_len must be num_heads * head_dim");
  const int64_t shape[3] = {token_count, num_heads, head_dim};
  const int64_t last = num_chunks > 0 ? chunk_offsets[num_chunks] : 0;
  int rc = validate_layout(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, shape, 3,
                           kKvAxes, token_count, num_heads, head_dim, last, nullptr);
  if (rc) return rc;
  const PlanInfo pi = build_plane_table(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks,
                                        token_count, num_heads, head_dim, table);
  info[0] = pi.regular;
  info[1] = pi.bits;
  info[2] = pi.aligned16;
  info[3] = pi.byte_aligned;
  return ORIGAMI_OK;
}

int origami_unpack_canonical_storage_chunks(
    const uint8_t* flat_chunks, int64_t flat_bytes, const int64_t* chunk_offsets,
    const int64_t* bits_per_chunk, const int64_t* chunk_specs, int64_t num_chunks,
    const int64_t* source_shape, int64_t rank, const int64_t* axis_positions,
    int64_t token_count, int64_t num_heads, int64_t head_dim, uint8_t* output,
    int64_t output_bytes, origami_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  Strides st;
  int rc = validate_layout(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, source_shape,
                           rank, axis_positions, token_count, num_heads, head_dim, flat_bytes,
                           &st);
  if (rc) return rc;
  int64_t total = 1;
  for (int64_t a = 0; a < rank; ++a) total *= source_shape[a];
  ORIGAMI_REQUIRE(output_bytes == total, "output size must equal prod(source_shape)");
  if (num_chunks == 0) return launch_fill_zero(output, output_bytes, stream);

  const int64_t T = token_count, H = num_heads, C = head_dim;
  const bool rows_layout = st.channel == 1 && C % 16 == 0 && st.token % 16 == 0 &&
                           st.head % 16 == 0 && aligned16(output) && T >= 16 &&
                           H * C <= kMaxPlaneTable;
  std::shared_ptr<const Plan> plan;
  rc = get_plan(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, T, H, C, rows_layout, &plan);
  if (rc) return rc;

  if (rows_layout && plan->has_table && plan->info.regular && plan->info.bits != 0) {
    RowsParams p{};
    set_stream(p, flat_chunks, flat_bytes);
    if (int rc2 = set_planes(p, plan)) return rc2;
    p.rows = output;
    p.block_ids = nullptr;
    p.num_blocks = 0;
    p.T = T;
    p.row_tokens = T;
    p.row_pitch = st.token;
    p.head_pitch = st.head;
    p.bs = T;
    p.blk_stride = 0;
    p.half_stride = 0;
    const int mode = rows_mode(plan->info, p, T, false, 0, true);
    set_restore_grid(p, mode, plan->info.bits, H, C, T, 1);
    return launch_rows(false, p, 1, plan->info.bits, mode, stream);
  }

  rc = launch_fill_zero(output, output_bytes, stream);
  if (rc) return rc;
  rc = plan_device(plan);
  if (rc) return rc;
  const GenericLayout L{st.token, st.head, st.channel};
  const dim3 grid(grid_for(plan->max_symbols, kThreads, 4096), static_cast<unsigned>(num_chunks));
  hipLaunchKernelGGL(generic_unpack_kernel, grid, dim3(kThreads), 0, stream, flat_chunks,
                     plan->d_offsets, plan->d_bits, plan->d_specs, L, output);
  return check_launch("generic_unpack_kernel");
}

int origami_pack_canonical_storage_chunks(
    const uint8_t* symbols, int64_t symbol_bytes, const int64_t* chunk_offsets,
    const int64_t* bits_per_chunk, const int64_t* chunk_specs, int64_t num_chunks,
    const int64_t* source_shape, int64_t rank, const int64_t* axis_positions,
    int64_t token_count, int64_t num_heads, int64_t head_dim, uint8_t* flat_chunks,
    int64_t flat_bytes, origami_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  Strides st;
  int rc = validate_layout(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, source_shape,
                           rank, axis_positions, token_count, num_heads, head_dim, flat_bytes,
                           &st);
  if (rc) return rc;
  int64_t total = 1;
  for (int64_t a = 0; a < rank; ++a) total *= source_shape[a];
  ORIGAMI_REQUIRE(symbol_bytes == total, "symbols size must equal prod(source_shape)");
  if (num_chunks == 0) return ORIGAMI_OK;

  const int64_t T = token_count, H = num_heads, C = head_dim;
  const bool rows_layout = st.channel == 1 && C % 16 == 0 && st.token % 16 == 0 &&
                           st.head % 16 == 0 && aligned16(symbols) && T >= 16 &&
                           H * C <= kMaxPlaneTable;
  std::shared_ptr<const Plan> plan;
  rc = get_plan(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, T, H, C, rows_layout, &plan);
  if (rc) return rc;

  if (rows_layout && plan->has_table && plan->info.regular && plan->info.bits != 0 &&
      (plan->info.bits < 8 || (plan->info.byte_aligned && (T * plan->info.bits) % 8 == 0))) {
    RowsParams p{};
    set_stream(p, flat_chunks, flat_bytes);
    if (int rc2 = set_planes(p, plan)) return rc2;
    p.rows = const_cast<uint8_t*>(symbols);
    p.T = T;
    p.row_tokens = T;
    p.row_pitch = st.token;
    p.head_pitch = st.head;
    p.bs = T;
    const int mode = pack_mode(plan->info, p, T);
    set_pack_grid(p, mode, H, C, T, 1);
    if (int rc2 = clear_bits_stream(mode, flat_chunks, chunk_offsets, num_chunks, stream))
      return rc2;
    return launch_rows(true, p, 1, plan->info.bits, mode, stream);
  }

  rc = plan_device(plan);
  if (rc) return rc;
  const GenericLayout L{st.token, st.head, st.channel};
  int64_t max_bytes = 0;
  for (int64_t k = 0; k < num_chunks; ++k)
    max_bytes = std::max(max_bytes, chunk_offsets[k + 1] - chunk_offsets[k]);
  const dim3 grid(grid_for(max_bytes, kThreads, 4096), static_cast<unsigned>(num_chunks));
  hipLaunchKernelGGL(generic_pack_kernel, grid, dim3(kThreads), 0, stream, symbols,
                     plan->d_offsets, plan->d_bits, plan->d_specs, L, flat_chunks);
  return check_launch("generic_pack_kernel");
}

int origami_unpack_canonical_to_kv_cache(
    const uint8_t* flat_chunks, int64_t flat_bytes, const int64_t* chunk_offsets,
    const int64_t* bits_per_chunk, const int64_t* chunk_specs, int64_t num_chunks, int64_t tokens,
    void* kv_cache, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    int64_t num_heads, int64_t head_bytes, const int64_t* block_ids, int64_t block_count,
    origami_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  int64_t blk_stride = 0, half_stride = 0;
  int rc = check_fused_restore(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, flat_bytes,
                               tokens, kv_cache, cache_layout, num_blocks, block_size, num_heads,
                               head_bytes, block_count, &blk_stride, &half_stride);
  if (rc) return rc;
  std::shared_ptr<const Plan> plan;
  rc = get_plan(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, 2 * tokens, num_heads,
                head_bytes, true, &plan);
  if (rc) return rc;
  if (!plan->has_table || !plan->info.regular || plan->info.bits == 0)
    return fail(ORIGAMI_ERR_UNSUPPORTED,
                "fused restore needs chunks spanning all tokens with one bit width");
  RowsParams p = fused_restore_params(flat_chunks, flat_bytes, tokens, kv_cache, num_blocks,
                                      block_size, num_heads, head_bytes, block_ids, block_count,
                                      blk_stride, half_stride);
  if (int rc2 = set_planes(p, plan)) return rc2;
  const int mode = rows_mode(plan->info, p, tokens, false, 0, true);
  set_restore_grid(p, mode, plan->info.bits, num_heads, head_bytes, p.row_tokens, 2);
  return launch_rows(false, p, 2, plan->info.bits, mode, stream);
}

int origami_restore_plan_create(const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
                                const int64_t* chunk_specs, int64_t num_chunks, int64_t tokens,
                                int64_t cache_layout, int64_t num_blocks, int64_t block_size,
                                int64_t num_heads, int64_t head_bytes, const int64_t* block_ids,
                                int64_t block_count, origami_restore_plan_t* out) {
  ORIGAMI_REQUIRE(out != nullptr, "plan output pointer is null");
  *out = nullptr;
  ORIGAMI_REQUIRE(chunk_offsets != nullptr || num_chunks == 0, "chunk_offsets is null");
  const int64_t need = num_chunks > 0 ? chunk_offsets[num_chunks] : 0;
  int64_t blk_stride = 0, half_stride = 0;
  // a 16-byte aligned stand-in for the cache pointer: the launch checks the real one
  alignas(16) static const uint8_t kAligned[16] = {};
  int rc = check_fused_restore(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, need,
                               tokens, kAligned, cache_layout, num_blocks, block_size, num_heads,
                               head_bytes, block_count, &blk_stride, &half_stride);
  if (rc) return rc;
  std::shared_ptr<const Plan> plan;
  rc = get_plan(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, 2 * tokens, num_heads,
                head_bytes, true, &plan);
  if (rc) return rc;
  if (!plan->has_table || !plan->info.regular || plan->info.bits == 0)
    return fail(ORIGAMI_ERR_UNSUPPORTED,
                "fused restore needs chunks spanning all tokens with one bit width");
  auto rp = std::make_unique<origami_restore_plan>();
  rp->plan = plan;
  rp->stream_bytes = need;
  rp->tokens = tokens;
  if (hipGetDevice(&rp->device) != hipSuccess) return fail(ORIGAMI_ERR_HIP, "hipGetDevice failed");
  rp->p = fused_restore_params(nullptr, 0, tokens, nullptr, num_blocks, block_size, num_heads,
                               head_bytes, block_ids, block_count, blk_stride, half_stride);
  if (int rc2 = set_planes(rp->p, plan)) return rc2;
  const int bits = plan->info.bits;
  if (bits == 1 || bits == 2 || bits == 4) {
    // the wide 16-byte-run restore applies when the stream pointer passed to
    // a launch is aligned (rows_mode decides per launch)
    rp->pw = rp->p;
    set_restore_grid(rp->pw, kRowsWide, bits, num_heads, head_bytes, rp->p.row_tokens, 2);
    rp->has_wide = true;
  }
  set_grid_dims(rp->p, num_heads, head_bytes, rp->p.row_tokens, 2);
  *out = rp.release();
  return ORIGAMI_OK;
}

int origami_restore_plan_launch(origami_restore_plan_t plan, const uint8_t* flat_chunks,
                                int64_t flat_bytes, void* kv_cache, origami_stream_t stream) {
  ORIGAMI_REQUIRE(plan != nullptr, "restore plan is null");
  ORIGAMI_REQUIRE(flat_chunks != nullptr || plan->stream_bytes == 0, "flat_chunks is null");
  ORIGAMI_REQUIRE(flat_bytes >= plan->stream_bytes,
                  "Origami CUDA packed chunk offsets exceed flat_chunks length");
  ORIGAMI_REQUIRE(kv_cache != nullptr && aligned16(kv_cache),
                  "fused restore needs a 16-byte aligned kv_cache");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(ORIGAMI_ERR_INVALID, "restore plan launched on another device than it was made on");
  RowsParams p = plan->p;
  set_stream(p, flat_chunks, flat_bytes);
  const int mode = rows_mode(plan->plan->info, p, plan->tokens, false, 0, plan->has_wide);
  if (mode == kRowsWide || mode == kRowsWideCached) {
    p = plan->pw;
    set_stream(p, flat_chunks, flat_bytes);
  }
  p.rows = static_cast<uint8_t*>(kv_cache);
  return launch_rows(false, p, 2, plan->plan->info.bits, mode,
                     reinterpret_cast<hipStream_t>(stream));
}

void origami_restore_plan_destroy(origami_restore_plan_t plan) { delete plan; }

int origami_unpack_canonical_to_kv_cache_noalloc(
    const uint8_t* flat_chunks, int64_t flat_bytes, const int64_t* chunk_offsets,
    const int64_t* bits_per_chunk, const int64_t* chunk_specs, int64_t num_chunks, int64_t tokens,
    void* kv_cache, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    int64_t num_heads, int64_t head_bytes, const int64_t* block_ids, int64_t block_count,
    origami_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  int64_t blk_stride = 0, half_stride = 0;
  int rc = check_fused_restore(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, flat_bytes,
                               tokens, kv_cache, cache_layout, num_blocks, block_size, num_heads,
                               head_bytes, block_count, &blk_stride, &half_stride);
  if (rc) return rc;
  const PlanInfo info = analyze_plan(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks,
                                     2 * tokens, num_heads, head_bytes);
  if (!info.regular || info.bits == 0)
    return fail(ORIGAMI_ERR_UNSUPPORTED,
                "fused restore needs chunks spanning all tokens with one bit width");
  RowsParams p = fused_restore_params(flat_chunks, flat_bytes, tokens, kv_cache, num_blocks,
                                      block_size, num_heads, head_bytes, block_ids, block_count,
                                      blk_stride, half_stride);
  if (info.dense) {
    p.planes = nullptr;
    p.plane_base = info.dense_base;
    p.plane_bits = 2 * tokens * info.bits;
  } else {
    if (num_heads * head_bytes > kScratchPlanes)
      return fail(ORIGAMI_ERR_UNSUPPORTED,
                  "allocation-free restore of a reordered chunk plan supports at most 131072 "
                  "(head, channel) planes (num_heads * head_bytes)");
    // the table fill and the launch happen under the lease; its release
    // records their completion for calls from other streams
    ScratchLease lease;
    int64_t* table = nullptr;
    if (int rc2 = lease.acquire(stream, &table)) return rc2;
    if (int rc2 = fill_plane_table(table, chunk_offsets, chunk_specs, num_chunks, 2 * tokens,
                                   num_heads, head_bytes, info.bits, stream))
      return rc2;
    p.planes = table;
    const int mode = rows_mode(info, p, tokens, false, 0, true);
    set_restore_grid(p, mode, info.bits, num_heads, head_bytes, p.row_tokens, 2);
    return launch_rows(false, p, 2, info.bits, mode, stream);
  }
  const int mode = rows_mode(info, p, tokens, false, 0, true);
  set_restore_grid(p, mode, info.bits, num_heads, head_bytes, p.row_tokens, 2);
  return launch_rows(false, p, 2, info.bits, mode, stream);
}

int origami_unpack_canonical_to_kv_cache_batch(
    int64_t num_requests, const uint8_t* const* flat_chunks, const int64_t* flat_bytes,
    const int64_t* const* chunk_offsets, const int64_t* const* bits_per_chunk,
    const int64_t* const* chunk_specs, const int64_t* num_chunks, const int64_t* tokens,
    void* kv_cache, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    int64_t num_heads, int64_t head_bytes, const int64_t* const* block_ids,
    const int64_t* block_counts, const int64_t* first_tokens, origami_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  ORIGAMI_REQUIRE(num_requests >= 0, "request count must be non-negative");
  // validate and plan every request before anything is launched
  struct Item {
    RowsRequest q;
    int bits, mode;
  };
  std::vector<Item> items;
  items.reserve(static_cast<size_t>(num_requests));
  RowsParams common{};
  for (int64_t r = 0; r < num_requests; ++r) {
    int64_t blk_stride = 0, half_stride = 0;
    int rc = check_fused_restore(chunk_offsets[r], bits_per_chunk[r], chunk_specs[r],
                                 num_chunks[r], flat_bytes[r], tokens[r], kv_cache, cache_layout,
                                 num_blocks, block_size, num_heads, head_bytes, block_counts[r],
                                 &blk_stride, &half_stride);
    if (rc) return rc;
    std::shared_ptr<const Plan> plan;
    rc = get_plan(chunk_offsets[r], bits_per_chunk[r], chunk_specs[r], num_chunks[r],
                  2 * tokens[r], num_heads, head_bytes, true, &plan);
    if (rc) return rc;
    if (!plan->has_table || !plan->info.regular || plan->info.bits == 0)
      return fail(ORIGAMI_ERR_UNSUPPORTED,
                  "fused restore needs chunks spanning all tokens with one bit width");
    RowsParams p = fused_restore_params(flat_chunks[r], flat_bytes[r], tokens[r], kv_cache,
                                        num_blocks, block_size, num_heads, head_bytes,
                                        block_ids[r], block_counts[r], blk_stride, half_stride);
    if (int rc2 = set_planes(p, plan)) return rc2;
    if (r == 0) common = p;
    Item it{};
    it.q.stream = p.stream;
    it.q.stream_bytes = p.stream_bytes;
    it.q.bit_bias = p.bit_bias;
    it.q.planes = p.planes;
    it.q.plane_base = p.plane_base;
    it.q.plane_bits = p.plane_bits;
    it.q.block_ids = p.block_ids;
    it.q.T = p.T;
    it.q.row_tokens = p.row_tokens;
    const int64_t first = first_tokens ? first_tokens[r] : 0;
    ORIGAMI_REQUIRE(first >= 0 && first <= p.row_tokens,
                    "first_tokens must lie in [0, block_count * block_size]");
    ORIGAMI_REQUIRE(first % 16 == 0 && first % block_size == 0,
                    "first_tokens must be a multiple of the block size and of 16");
    it.q.token0 = first;
    it.bits = plan->info.bits;
    it.mode = rows_mode(plan->info, p, tokens[r], false, first);
    // both aligned16 policies share a launch; the kernel picks per request
    it.q.nt = it.mode == kRowsAligned16;
    if (it.mode == kRowsAligned16Cached) it.mode = kRowsAligned16;
    items.push_back(it);
  }
  // one launch per (width, addressing mode) group of up to kBatchRequests
  std::vector<bool> done(items.size(), false);
  for (size_t i = 0; i < items.size(); ++i) {
    if (done[i]) continue;
    RowsBatch b{};
    b.common = common;
    for (size_t j = i; j < items.size() && b.nreq < kBatchRequests; ++j) {
      if (done[j] || items[j].bits != items[i].bits || items[j].mode != items[i].mode) continue;
      b.req[b.nreq++] = items[j].q;
      done[j] = true;
    }
    set_batch_grid(b, num_heads, head_bytes);
    if (int rc = launch_rows_batch(b, items[i].bits, items[i].mode, stream)) return rc;
  }
  return ORIGAMI_OK;
}

int origami_pack_canonical_from_kv_cache(
    const void* kv_cache, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    int64_t num_heads, int64_t head_bytes, const int64_t* block_ids, int64_t block_count,
    int64_t tokens, const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks, uint8_t* flat_chunks, int64_t flat_bytes,
    origami_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  ORIGAMI_REQUIRE(tokens > 0 && num_heads > 0 && head_bytes > 0,
                  "tokens, heads, and head_dim must be positive");
  ORIGAMI_REQUIRE(block_size > 0, "kv_cache block size must be positive");
  ORIGAMI_REQUIRE(num_blocks > 0, "kv_cache must hold at least one block");
  ORIGAMI_REQUIRE(block_count > 0, "block_ids must be non-empty");
  ORIGAMI_REQUIRE(tokens <= block_count * block_size, "tokens exceed source block capacity");
  const int64_t shape[3] = {2 * tokens, num_heads, head_bytes};
  int rc = validate_layout(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, shape, 3,
                           kKvAxes, 2 * tokens, num_heads, head_bytes, flat_bytes, nullptr);
  if (rc) return rc;
  int64_t blk_stride = 0, half_stride = 0;
  rc = cache_geometry(cache_layout, num_blocks, block_size, &blk_stride, &half_stride);
  if (rc) return rc;
  if (head_bytes % 16 != 0 || !aligned16(kv_cache) ||
      num_heads * head_bytes > kMaxPlaneTable)
    return fail(ORIGAMI_ERR_UNSUPPORTED, "fused save needs 16-byte head rows");
  std::shared_ptr<const Plan> plan;
  rc = get_plan(chunk_offsets, bits_per_chunk, chunk_specs, num_chunks, 2 * tokens, num_heads,
                head_bytes, true, &plan);
  if (rc) return rc;
  if (!plan->has_table || !plan->info.regular || plan->info.bits == 0 ||
      (plan->info.bits == 8 && !plan->info.byte_aligned))
    return fail(ORIGAMI_ERR_UNSUPPORTED,
                "fused save needs regular planes with one bit width");
  RowsParams p{};
  set_stream(p, flat_chunks, flat_bytes);
  if (int rc2 = set_planes(p, plan)) return rc2;
  p.rows = static_cast<uint8_t*>(const_cast<void*>(kv_cache));
  p.block_ids = block_ids;
  p.num_blocks = num_blocks;
  p.T = tokens;
  p.row_tokens = block_count * block_size;
  p.row_pitch = num_heads * head_bytes;
  p.head_pitch = head_bytes;
  p.bs = block_size;
  p.blk_stride = blk_stride;
  p.half_stride = half_stride;
  const int mode = pack_mode(plan->info, p, tokens);
  set_pack_grid(p, mode, num_heads, head_bytes, tokens, 2);
  if (int rc2 = clear_bits_stream(mode, flat_chunks, chunk_offsets, num_chunks, stream))
    return rc2;
  return launch_rows(true, p, 2, plan->info.bits, mode, stream);
}

static int block_copy(bool scatter, const uint8_t* src, uint8_t* dst, int64_t tokens,
                      int64_t cache_layout, int64_t num_blocks, int64_t block_size,
                      int64_t num_heads, int64_t head_bytes, const int64_t* block_ids,
                      int64_t block_count, hipStream_t stream) {
  ORIGAMI_REQUIRE(num_heads > 0 && head_bytes > 0, "heads and head_dim must be positive");
  ORIGAMI_REQUIRE(block_size > 0, "kv_cache block size must be positive");
  ORIGAMI_REQUIRE(num_blocks > 0, "kv_cache must hold at least one block");
  ORIGAMI_REQUIRE(block_count >= 0, "block count must be non-negative");
  ORIGAMI_REQUIRE(tokens >= 0 && tokens <= block_count * block_size,
                  "tokens exceed destination block capacity");
  if (block_count == 0) return ORIGAMI_OK;
  BlockCopyParams p{};
  p.src = src;
  p.dst = dst;
  p.block_ids = block_ids;
  p.num_blocks = num_blocks;
  p.T = tokens;
  p.Tt = block_count * block_size;
  p.block_count = block_count;
  p.bs = block_size;
  p.row_bytes = num_heads * head_bytes;
  int rc = cache_geometry(cache_layout, num_blocks, block_size, &p.blk_stride, &p.half_stride);
  if (rc) return rc;
  const bool vec = p.row_bytes % 16 == 0 && aligned16(src) && aligned16(dst);
  const dim3 block(kThreads);
  if (vec) {
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(2 * block_count, 1 << 20)));
    if (scatter)
      hipLaunchKernelGGL(block_copy_kernel<true>, grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL(block_copy_kernel<false>, grid, block, 0, stream, p);
    return check_launch("block_copy_kernel");
  }
  const dim3 grid(grid_for(2 * p.Tt * p.row_bytes, kThreads, 65536));
  if (scatter)
    hipLaunchKernelGGL(block_copy_bytes_kernel<true>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(block_copy_bytes_kernel<false>, grid, block, 0, stream, p);
  return check_launch("block_copy_bytes_kernel");
}

int origami_scatter_kv_blocks(const uint8_t* value, int64_t tokens, void* kv_cache,
                              int64_t cache_layout, int64_t num_blocks, int64_t block_size,
                              int64_t num_heads, int64_t head_bytes, const int64_t* block_ids,
                              int64_t block_count, origami_stream_t stream) {
  return block_copy(true, value, static_cast<uint8_t*>(kv_cache), tokens, cache_layout,
                    num_blocks, block_size, num_heads, head_bytes, block_ids, block_count,
                    reinterpret_cast<hipStream_t>(stream));
}

int origami_gather_kv_blocks(const void* kv_cache, int64_t cache_layout, int64_t num_blocks,
                             int64_t block_size, int64_t num_heads, int64_t head_bytes,
                             const int64_t* block_ids, int64_t block_count, uint8_t* value,
                             origami_stream_t stream) {
  return block_copy(false, static_cast<const uint8_t*>(kv_cache), value,
                    block_count * block_size, cache_layout, num_blocks, block_size, num_heads,
                    head_bytes, block_ids, block_count, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
