/*
 * origami_layout.h -- C ABI of the MI355X (gfx950) Origami KV codec-layout
 * library, liborigami_layout.so.
 *
 * The library replaces the layout/bitpack and fused-dequantize parts of
 * Origami's CUDA extension (csrc/origami/bitpack_layout_cuda.cpp +
 * bitpack_layout_cuda.cu, loaded as `origami_bitpack_cuda_v6` by
 * lossless/native_gpu.py:35-49).  Every entry
 * point takes plain pointers and sizes: device buffers are raw device
 * addresses, metadata arrays are host memory, and the stream is a hipStream_t.
 * No torch types cross this boundary.
 *
 * Conventions (mirroring the reference's torch extension):
 *  - Return value: ORIGAMI_OK (0) or an error code; origami_last_error()
 *    returns the message of the last failure on the calling thread.  The
 *    reference raised RuntimeError from TORCH_CHECK with these messages.
 *  - Chunk metadata follows the reference wire format: chunk_specs is
 *    [num_chunks, 6] int64 rows (head_start, head_end, channel_start,
 *    channel_end, token_start, token_end); chunk_offsets is [num_chunks + 1]
 *    byte offsets into the flat stream; bits_per_chunk is [num_chunks] with
 *    values 1..8.  Symbols are LSB-first, head-major, then channel, token
 *    fastest (bitpack_layout_cuda.cu:70-128).
 *  - source_shape is the rank-3/4 symbol tensor shape and axis_positions is
 *    [token_axis, head_axis, head_dim_axis, layer_axis or -1]
 *    (lossless/native_cpu.py:102-130).
 *  - Metadata is read on the host only: unlike the reference
 *    (bitpack_layout_cuda.cpp:156, 350-351) no call copies device memory
 *    back to the host.  Device copies of the metadata the kernels need are
 *    made once per distinct layout and cached inside the library.
 *  - All device work is enqueued on `stream` and is asynchronous.  Inputs
 *    must stay alive until that work completes.
 *  - kv_cache layout codes: ORIGAMI_CACHE_KV_FIRST is [2, num_blocks,
 *    block_size, num_heads, head_dim]; ORIGAMI_CACHE_BLOCKS_FIRST is
 *    [num_blocks, 2, block_size, num_heads, head_dim]
 *    (bitpack_layout_cuda.cpp:526-552).  head_bytes = head_dim * element size.
 *  - Block ids are int64 device arrays.  Ids outside [0, num_blocks) are
 *    skipped by the kernels, as the reference's fused kernels do
 *    (bitpack_layout_cuda.cu:389-392); callers validate them beforehand.
 */
#ifndef ORIGAMI_LAYOUT_H_
#define ORIGAMI_LAYOUT_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* origami_stream_t; /* == hipStream_t */

#define ORIGAMI_OK 0
#define ORIGAMI_ERR_INVALID 1     /* invalid argument (reference: TORCH_CHECK) */
#define ORIGAMI_ERR_UNSUPPORTED 2 /* layout not served by the requested fused path */
#define ORIGAMI_ERR_HIP 3         /* HIP runtime failure */

#define ORIGAMI_CACHE_KV_FIRST 0
#define ORIGAMI_CACHE_BLOCKS_FIRST 1

/* element types of dequantize inputs and outputs */
#define ORIGAMI_DTYPE_FLOAT16 1
#define ORIGAMI_DTYPE_BFLOAT16 2
#define ORIGAMI_DTYPE_FLOAT32 3

/* KIVI symbol packing: LSB-first at `bits` bits (what the reference kernel
 * reads), or KIVI's own container, where 3-bit symbols sit one per nibble
 * (kivi_adapter.py:39-43) and other widths are LSB-first. */
#define ORIGAMI_KIVI_PACKED_LSB 0
#define ORIGAMI_KIVI_NIBBLE3 1

/* Message of the last failing call on this thread ("" if none). */
const char* origami_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int origami_abi_version(void);

/*
 * Totals since the library was loaded: chunk plans created (one per distinct
 * chunk metadata seen by an allocating entry point) and device allocations
 * the library made (plan metadata uploads).  Either pointer may be null.
 * New; no reference counterpart: lets a caller (and the tests) check that a
 * call such as the allocation-free restore created no plan and allocated
 * no device memory.
 */
void origami_debug_counters(int64_t* plans_created, int64_t* device_allocations);

/*
 * Caps the number of workgroups of the row kernels (the fused restore / save
 * and the fast unpack / pack paths) launched later on the calling thread;
 * each workgroup then loops over several tiles.  0 restores the default (one
 * workgroup per tile).  Returns the previous cap.  New; no reference
 * counterpart: a restore that runs hidden behind host-to-device copies uses it
 * to take a smaller share of HBM bandwidth at a time.
 */
int64_t origami_set_rows_grid_limit(int64_t max_workgroups);

/*
 * Host-only validation of a canonical chunk layout.  Replaces the checks of
 * read_source_layout / read_chunk_specs / check_bits /
 * packed_bytes_for_symbols and the byte-size loop of
 * unpack_canonical_storage_chunks_cuda (bitpack_layout_cuda.cpp:43-185,
 * 326-362), plus a bound the reference lacks: chunk_offsets must be
 * non-decreasing and end within flat_bytes.
 */
int origami_validate_chunks(const int64_t* chunk_offsets,
                            const int64_t* bits_per_chunk,
                            const int64_t* chunk_specs, int64_t num_chunks,
                            const int64_t* source_shape, int64_t rank,
                            const int64_t* axis_positions, int64_t token_count,
                            int64_t num_heads, int64_t head_dim,
                            int64_t flat_bytes);

/*
 * Host-only plane plan (new; no reference counterpart, used by tests and
 * diagnostics).  A plane is one (head, channel) pair; its symbols are the
 * token run of that pair inside its chunk.  Writes table[h * head_dim + c] =
 * bit offset of token 0 of plane (h, c) in the flat stream, or -1 when no
 * chunk covers it, and info[0..3] = {regular, uniform bits or 0,
 * planes 16-byte aligned, planes byte aligned}.  "regular" means every chunk
 * spans the whole token axis and no plane is covered twice, which is what
 * the fused row kernels need.  table_len must be num_heads * head_dim.
 */
int origami_plan_planes(const int64_t* chunk_offsets,
                        const int64_t* bits_per_chunk,
                        const int64_t* chunk_specs, int64_t num_chunks,
                        int64_t token_count, int64_t num_heads,
                        int64_t head_dim, int64_t* table, int64_t table_len,
                        int64_t* info);

/*
 * Unpack a flat stream of canonical chunks into a zero-initialised uint8
 * symbol tensor of prod(source_shape) bytes in the source layout.
 * Replaces unpack_canonical_storage_chunks_cuda (bitpack_layout_cuda.cpp:
 * 316-400) and origami_unpack_canonical_storage_chunks_launch
 * (bitpack_layout_cuda.cu:190-243).  Bytes no chunk covers are 0.
 */
int origami_unpack_canonical_storage_chunks(
    const uint8_t* flat_chunks, int64_t flat_bytes,
    const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks,
    const int64_t* source_shape, int64_t rank, const int64_t* axis_positions,
    int64_t token_count, int64_t num_heads, int64_t head_dim,
    uint8_t* output, int64_t output_bytes, origami_stream_t stream);

/*
 * Pack a uint8 symbol tensor (source layout) into the flat canonical stream:
 * the inverse of origami_unpack_canonical_storage_chunks, with zero pad bits
 * after each chunk's last symbol.  Replaces the stub
 * native_cpu.pack_canonical_storage_chunks (lossless/native_cpu.py:144-151),
 * which raises in the reference.  flat_bytes must be >= chunk_offsets[N].
 */
int origami_pack_canonical_storage_chunks(
    const uint8_t* symbols, int64_t symbol_bytes,
    const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks,
    const int64_t* source_shape, int64_t rank, const int64_t* axis_positions,
    int64_t token_count, int64_t num_heads, int64_t head_dim,
    uint8_t* flat_chunks, int64_t flat_bytes, origami_stream_t stream);

/*
 * Fused restore: unpack one layer's canonical stream and scatter it into the
 * paged KV cache through the block table, in one pass.  The layer's symbols
 * are the bytes of its token-major K/V, viewed as [2 * tokens, num_heads,
 * head_bytes] (K tokens, then V tokens; chunk_specs index that tensor).
 * Destination tokens [0, block_count * block_size) of K and V are written;
 * tokens >= `tokens` are written as zero (the tail padding of
 * benchmark_utils.py:378-392).  Replaces the chain
 * unpack_canonical_storage_chunks_cuda -> RawBytesTensorAdapter.dequantize
 * -> copy_kv_to_hbm (worker.py:1087-1248, raw_tensor.py:125-157,
 * benchmark_utils.py:350-444); the destination index is that of
 * bitpack_layout_cuda.cu:408-420.  Returns ORIGAMI_ERR_UNSUPPORTED when the
 * chunk plan is not regular or head_bytes is not a multiple of 16; the caller
 * then unpacks and scatters in two steps.
 */
int origami_unpack_canonical_to_kv_cache(
    const uint8_t* flat_chunks, int64_t flat_bytes,
    const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks, int64_t tokens,
    void* kv_cache, int64_t cache_layout, int64_t num_blocks,
    int64_t block_size, int64_t num_heads, int64_t head_bytes,
    const int64_t* block_ids, int64_t block_count, origami_stream_t stream);

/*
 * Allocation-free variant of origami_unpack_canonical_to_kv_cache: same
 * arguments, same results.  It has no counterpart in the reference.  It is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): it calls no
 * hipMalloc, hipFree or other allocating routine and keeps no plan cache.
 * A chunk plan in the planner's order needs no device metadata; the plane
 * table of a reordered plan is written into a fixed 1 MiB device array per
 * GPU (at most 131072 (head, channel) planes, i.e. num_heads * head_bytes;
 * larger reordered plans return ORIGAMI_ERR_UNSUPPORTED).  That array is
 * shared by every call on the GPU and keeps the last call's contents, so
 * reordered-plan calls on one GPU must not overlap: calls from several host
 * threads are serialised on the host, and a call from another stream while
 * the previous call's work is still pending returns ORIGAMI_ERR_INVALID
 * (nothing is launched).  Inside graph capture the check is skipped; replays
 * of captured calls must not overlap other calls on the GPU.  The device
 * state (array address, one event) is set up on a device's first call.
 */
int origami_unpack_canonical_to_kv_cache_noalloc(
    const uint8_t* flat_chunks, int64_t flat_bytes,
    const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks, int64_t tokens,
    void* kv_cache, int64_t cache_layout, int64_t num_blocks,
    int64_t block_size, int64_t num_heads, int64_t head_bytes,
    const int64_t* block_ids, int64_t block_count, origami_stream_t stream);

/*
 * Prepared fused restore: origami_unpack_canonical_to_kv_cache split into a
 * setup done once per request (the chunk metadata validated and its plan
 * looked up or built, a reordered plan's plane table uploaded, the cache
 * geometry checked, the launch shape computed) and a launch per layer that
 * takes only the layer's stream and destination cache.  It has no
 * counterpart in the reference; it is for callers that restore every layer
 * of a request with the same chunk plan, tokens, cache geometry and block
 * table (the layer-wise restore of worker.py:718-1248), where the per-call
 * host cost of the full entry point (argument checks, the plan lookup, which
 * hashes the chunk metadata) would otherwise be paid per layer.  Results are
 * those of origami_unpack_canonical_to_kv_cache with the same arguments.
 * block_ids is a device array the caller keeps alive and unchanged while the
 * plan is in use; the plan is used on the device current at creation.  The
 * launch needs flat_bytes >= chunk_offsets[num_chunks] and a 16-byte aligned
 * kv_cache of the geometry given at creation.  A plan may be launched from
 * several threads; destroy it once no launch can still use it (pending
 * kernels keep nothing of it).  create returns ORIGAMI_ERR_UNSUPPORTED where
 * origami_unpack_canonical_to_kv_cache would.
 */
typedef struct origami_restore_plan* origami_restore_plan_t;

int origami_restore_plan_create(
    const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks, int64_t tokens,
    int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    int64_t num_heads, int64_t head_bytes, const int64_t* block_ids,
    int64_t block_count, origami_restore_plan_t* plan);
int origami_restore_plan_launch(origami_restore_plan_t plan, const uint8_t* flat_chunks,
                                int64_t flat_bytes, void* kv_cache, origami_stream_t stream);
void origami_restore_plan_destroy(origami_restore_plan_t plan);

/*
 * Batched fused restore: one layer of several requests into one paged cache.
 * Request r is exactly the argument set of origami_unpack_canonical_to_kv_cache
 * (stream flat_chunks[r] of flat_bytes[r] bytes, its chunk metadata arrays,
 * tokens[r], device block table block_ids[r] of block_counts[r] ids); the
 * cache geometry is shared.  Requests whose plans share a symbol width and
 * addressing mode go to one launch (up to 16 per launch), so a batch of short
 * requests fills the GPU like one long one.  Replaces the per-request loop of
 * the reference's layer restore (worker.py:796-897 and 1087-1248, one
 * unpack + copy_kv_to_hbm per request and layer).  The requests of one call
 * run concurrently: two requests must not carry different bytes for the same
 * destination block (vLLM's shared prefix blocks hold the same bytes).  Block
 * ids outside [0, num_blocks) are skipped, as in the single restore.
 * first_tokens (NULL: all 0) starts request r at destination token
 * first_tokens[r], a multiple of block_size and of 16: its earlier blocks are
 * neither read nor written, so a shared prefix that an earlier request of
 * the batch restores is moved once.  All requests are validated before
 * anything is launched.
 */
int origami_unpack_canonical_to_kv_cache_batch(
    int64_t num_requests, const uint8_t* const* flat_chunks, const int64_t* flat_bytes,
    const int64_t* const* chunk_offsets, const int64_t* const* bits_per_chunk,
    const int64_t* const* chunk_specs, const int64_t* num_chunks, const int64_t* tokens,
    void* kv_cache, int64_t cache_layout, int64_t num_blocks, int64_t block_size,
    int64_t num_heads, int64_t head_bytes, const int64_t* const* block_ids,
    const int64_t* block_counts, const int64_t* first_tokens, origami_stream_t stream);

/*
 * Fused save: gather a layer's K/V through the block table from the paged
 * cache and pack it into the canonical stream, in one pass; the inverse of
 * origami_unpack_canonical_to_kv_cache.  Replaces _select_blocks +
 * RawBytesTensorAdapter.quantize + the packer of _pack_quantized_symbols
 * (worker.py:1881-2040, raw_tensor.py:100-123).  Tokens are [0, tokens) of
 * the blocks listed.  Returns ORIGAMI_ERR_UNSUPPORTED unless the plan is
 * regular, every plane starts on a byte boundary and tokens * bits is a
 * multiple of 8.
 */
int origami_pack_canonical_from_kv_cache(
    const void* kv_cache, int64_t cache_layout, int64_t num_blocks,
    int64_t block_size, int64_t num_heads, int64_t head_bytes,
    const int64_t* block_ids, int64_t block_count, int64_t tokens,
    const int64_t* chunk_offsets, const int64_t* bits_per_chunk,
    const int64_t* chunk_specs, int64_t num_chunks, uint8_t* flat_chunks,
    int64_t flat_bytes, origami_stream_t stream);

/*
 * Paged scatter of a token-major K/V tensor (bytes of [2, tokens, num_heads,
 * head_bytes]) into the cache, zero-padding to whole blocks.  Replaces
 * copy_kv_to_hbm / _assign_blocks / _normalize_kv_value
 * (benchmark_utils.py:350-444) for device-resident values.
 */
int origami_scatter_kv_blocks(const uint8_t* value, int64_t tokens,
                              void* kv_cache, int64_t cache_layout,
                              int64_t num_blocks, int64_t block_size,
                              int64_t num_heads, int64_t head_bytes,
                              const int64_t* block_ids, int64_t block_count,
                              origami_stream_t stream);

/*
 * Block gather from the cache into a token-major K/V tensor (bytes of
 * [2, block_count * block_size, num_heads, head_bytes]).  Replaces
 * _select_blocks (worker.py:1881-1897) + the byte view of
 * RawBytesTensorAdapter.quantize (raw_tensor.py:100-123).
 */
int origami_gather_kv_blocks(const void* kv_cache, int64_t cache_layout,
                             int64_t num_blocks, int64_t block_size,
                             int64_t num_heads, int64_t head_bytes,
                             const int64_t* block_ids, int64_t block_count,
                             uint8_t* value, origami_stream_t stream);

/* ---------------------------------------------------------------------------
 * Fused dequantize paths (CacheGen, KIVI).  Element types use the
 * ORIGAMI_DTYPE_* codes; arithmetic is IEEE binary32 and results are
 * rounded to nearest even into float16 / bfloat16.
 * ------------------------------------------------------------------------- */

/*
 * CacheGen unpack + dequantize + paged scatter.  Replaces
 * cachegen_unpack_dequantize_to_kv_cache_cuda (bitpack_layout_cuda.cpp:
 * 475-581) and its kernel (bitpack_layout_cuda.cu:349-575).  The K and V
 * streams are bytestream[key_offset, +key_bytes) and
 * bytestream[value_offset, +value_bytes): symbol token * (heads * head_dim) +
 * channel at key_bits / value_bits bits, LSB-first.  Destination element
 * (block_ids[t / block_size], half, t % block_size, head, dim) becomes
 * ((s - c) / c) * max[t] with c = bins / 2 - 1, for t < tokens; other tokens
 * and ids outside [0, num_blocks) are left untouched.  max_key / max_value
 * are device arrays of max_dtype (FLOAT16 or FLOAT32) with at least `tokens`
 * values; kv_cache is FLOAT16 or BFLOAT16.  Stream bytes past key_bytes /
 * value_bytes read as 0 at every width (the reference reads past the range
 * unchecked at 8 bits).
 */
int origami_cachegen_unpack_dequantize_to_kv_cache(
    const uint8_t* bytestream, int64_t bytestream_bytes, int64_t key_offset,
    int64_t key_bytes, int64_t value_offset, int64_t value_bytes,
    int64_t key_bits, int64_t value_bits, int64_t key_bins, int64_t value_bins,
    const void* max_key, const void* max_value, int64_t max_key_count,
    int64_t max_value_count, int64_t max_dtype, void* kv_cache,
    int64_t cache_dtype, int64_t cache_layout, int64_t num_blocks,
    int64_t block_size, const int64_t* block_ids, int64_t block_count,
    int64_t tokens, int64_t heads, int64_t head_dim, origami_stream_t stream);

/*
 * CacheGen unpack + dequantize of several layers into a dense float16 tensor
 * [layers, 2, heads, tokens, head_dim].  Replaces
 * cachegen_unpack_dequantize_cuda (bitpack_layout_cuda.cpp:402-473) and its
 * kernel (bitpack_layout_cuda.cu:141-186).  Host arrays: offsets[2 * layers +
 * 1] (segment j < layers is layer j's keys, segment layers + j its values),
 * bits_per_layer[2 * layers], key_bins[layers], value_bins[layers].  max_key
 * and max_value are device arrays [layers, tokens] of max_dtype.  Offsets
 * must be non-decreasing and within bytestream_bytes (a bound the reference
 * lacks).
 */
int origami_cachegen_unpack_dequantize(
    const uint8_t* bytestream, int64_t bytestream_bytes, const int64_t* offsets,
    const int64_t* bits_per_layer, const int64_t* key_bins,
    const int64_t* value_bins, int64_t layers, const void* max_key,
    const void* max_value, int64_t max_key_count, int64_t max_value_count,
    int64_t max_dtype, int64_t tokens, int64_t heads, int64_t head_dim,
    void* output, int64_t output_bytes, origami_stream_t stream);

/*
 * KIVI dequantize + paged scatter.  Replaces kivi_dequantize_to_kv_cache_cuda
 * (bitpack_layout_cuda.cpp:583-714) and its kernel (bitpack_layout_cuda.cu:
 * 578-853).  Tokens [0, sink_tokens) copy key_sink / value_sink ([sink, C]);
 * body token bt = t - sink_tokens reads, for keys, symbol (d * heads + h) *
 * body + bt and dequantizes fmaf(s, key_scale[bt / group][c],
 * key_zero[bt / group][c]); for values, symbol (h * head_dim + d) * body + bt
 * and fmaf(s, value_scale[bt][c / group], value_zero[bt][c / group]), with
 * body = tokens - sink_tokens and C = heads * head_dim.  The reference's
 * `s * scale + zero` is one fused multiply-add as nvcc compiles it.
 * meta_counts (host, [6]) are the element counts of key_scale, key_zero,
 * value_scale, value_zero, key_sink, value_sink; the metadata arrays are
 * device arrays of meta_dtype (FLOAT16 or FLOAT32), aligned to their element
 * size.  symbol_packing is ORIGAMI_KIVI_PACKED_LSB or ORIGAMI_KIVI_NIBBLE3.
 * Destination handling is that of the CacheGen entry point: tokens >= tokens
 * and invalid block ids are left untouched.
 */
int origami_kivi_dequantize_to_kv_cache(
    const uint8_t* bytestream, int64_t bytestream_bytes, int64_t key_offset,
    int64_t key_bytes, int64_t value_offset, int64_t value_bytes, int64_t bits,
    int64_t symbol_packing, int64_t group_size, int64_t sink_tokens,
    const void* key_scale, const void* key_zero, const void* value_scale,
    const void* value_zero, const void* key_sink, const void* value_sink,
    const int64_t* meta_counts, int64_t meta_dtype, void* kv_cache,
    int64_t cache_dtype, int64_t cache_layout, int64_t num_blocks,
    int64_t block_size, const int64_t* block_ids, int64_t block_count,
    int64_t tokens, int64_t heads, int64_t head_dim, origami_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ORIGAMI_LAYOUT_H_ */
