// origami_torch_ext.cpp -- PyTorch-ROCm extension module over the C ABI of
// liborigami_layout.so (include/origami_layout.h).
//
// It exports the function names of the reference's extension module
// origami_bitpack_cuda_v6 (csrc/origami/bitpack_layout_cuda.cpp:894-903) with
// their argument lists, plus the fused paths this library adds.  Tensors are
// checked and unwrapped here; the work is done by the extern "C" entry points
// on the calling thread's current HIP stream of the tensors' device, and a
// non-zero status becomes a RuntimeError carrying origami_last_error(), the
// way the reference's TORCH_CHECKs raise.  There is no device code here.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <string>
#include <vector>

#include "origami_layout.h"

namespace {

void check(int rc) {
  TORCH_CHECK(rc == ORIGAMI_OK, origami_last_error());
}

// ORIGAMI_ERR_UNSUPPORTED is returned to Python as False (the caller takes
// the two-step path); every other failure raises.
bool check_supported(int rc) {
  if (rc == ORIGAMI_ERR_UNSUPPORTED) return false;
  check(rc);
  return true;
}

origami_stream_t current_stream(const at::Tensor& t) {
  return reinterpret_cast<origami_stream_t>(
      c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void require_device(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

void require_byte(const at::Tensor& t, const char* name) {
  require_device(t, name);
  TORCH_CHECK(t.scalar_type() == at::kByte, name, " must be uint8");
}

// Host int64 copy of a metadata tensor (no copy when it already is one).
// Device metadata costs one device-to-host copy, as in the reference
// (bitpack_layout_cuda.cpp:156, 350-351).
at::Tensor host_i64(const at::Tensor& t) {
  at::Tensor h = t;
  if (h.device().type() != at::kCPU || h.scalar_type() != at::kLong)
    h = h.to(at::kCPU, at::kLong);
  return h.contiguous();
}

const int64_t* i64p(const at::Tensor& t) { return t.data_ptr<int64_t>(); }

// Paged cache geometry of the layout entry points: [2, NB, bs, H, D] is
// recognised first, then [NB, 2, bs, H, D] (benchmark_utils.py:357,
// bitpack_layout_cuda.cpp:810-831).
struct CacheGeom {
  int64_t layout, num_blocks, block_size, heads, head_bytes;
};

CacheGeom layout_cache_geometry(const at::Tensor& c) {
  TORCH_CHECK(c.dim() == 5, "kv_cache must have rank 5");
  CacheGeom g{};
  if (c.size(0) == 2) {
    g.layout = ORIGAMI_CACHE_KV_FIRST;
    g.num_blocks = c.size(1);
  } else if (c.size(1) == 2) {
    g.layout = ORIGAMI_CACHE_BLOCKS_FIRST;
    g.num_blocks = c.size(0);
  } else {
    TORCH_CHECK(false, "kv_cache must be [num_blocks,2,block,heads,dim] or "
                       "[2,num_blocks,block,heads,dim]");
  }
  g.block_size = c.size(2);
  g.heads = c.size(3);
  g.head_bytes = c.size(4) * static_cast<int64_t>(c.element_size());
  return g;
}

// The dequantize entry points follow bitpack_layout_cuda.cpp:526-552, which
// recognises [NB, 2, bs, H, D] first.
CacheGeom dequant_cache_geometry(const at::Tensor& c, int64_t heads, int64_t head_dim) {
  TORCH_CHECK(c.dim() == 5, "kv_cache must have rank 5");
  CacheGeom g{};
  if (c.size(1) == 2) {
    g.layout = ORIGAMI_CACHE_BLOCKS_FIRST;
    g.num_blocks = c.size(0);
  } else if (c.size(0) == 2) {
    g.layout = ORIGAMI_CACHE_KV_FIRST;
    g.num_blocks = c.size(1);
  } else {
    TORCH_CHECK(false, "kv_cache must be [num_blocks,2,block,heads,dim] or "
                       "[2,num_blocks,block,heads,dim]");
  }
  TORCH_CHECK(c.size(3) == heads && c.size(4) == head_dim, "kv_cache head shape mismatch");
  g.block_size = c.size(2);
  return g;
}

int64_t dtype_code(at::ScalarType t, const char* name) {
  switch (t) {
    case at::kHalf:
      return ORIGAMI_DTYPE_FLOAT16;
    case at::kBFloat16:
      return ORIGAMI_DTYPE_BFLOAT16;
    case at::kFloat:
      return ORIGAMI_DTYPE_FLOAT32;
    default:
      TORCH_CHECK(false, name, " has an unsupported dtype");
  }
  return 0;
}

void require_block_ids(const at::Tensor& ids, const at::Tensor& cache) {
  require_device(ids, "block_ids");
  TORCH_CHECK(ids.scalar_type() == at::kLong, "block_ids must be int64");
  TORCH_CHECK(ids.device() == cache.device(), "block_ids must be on the kv_cache device");
}

// ---------------------------------------------------------------------------
// Reference names (bitpack_layout_cuda.cpp:894-903)
// ---------------------------------------------------------------------------

// bitpack_layout_cuda.cpp:316-400: flat chunks -> new uint8 symbol tensor.
at::Tensor unpack_canonical_storage_chunks_cuda(at::Tensor flat_chunks, at::Tensor chunk_offsets,
                                                at::Tensor bits_per_chunk, at::Tensor source_shape,
                                                at::Tensor axis_positions, int64_t token_count,
                                                int64_t num_heads, int64_t head_dim,
                                                at::Tensor chunk_specs) {
  require_byte(flat_chunks, "flat_chunks");
  const at::Tensor offs = host_i64(chunk_offsets), bits = host_i64(bits_per_chunk);
  const at::Tensor specs = host_i64(chunk_specs), shape = host_i64(source_shape);
  const at::Tensor axes = host_i64(axis_positions);
  TORCH_CHECK(axes.numel() == 4,
              "axis_positions must be [token_axis, head_axis, head_dim_axis, layer_axis]");
  const int64_t n = bits.numel();
  TORCH_CHECK(offs.numel() == n + 1, "chunk_offsets length must be chunk count + 1");
  TORCH_CHECK(specs.numel() == 6 * n, "chunk_specs must be [num_chunks, 6]");
  int64_t total = 1;
  for (int64_t a = 0; a < shape.numel(); ++a) total *= std::max<int64_t>(i64p(shape)[a], 0);
  const c10::OptionalDeviceGuard guard(flat_chunks.device());
  at::Tensor out = at::empty({total}, flat_chunks.options());
  check(origami_unpack_canonical_storage_chunks(
      flat_chunks.data_ptr<uint8_t>(), flat_chunks.numel(), i64p(offs), i64p(bits), i64p(specs),
      n, i64p(shape), shape.numel(), i64p(axes), token_count, num_heads, head_dim,
      out.data_ptr<uint8_t>(), out.numel(), current_stream(flat_chunks)));
  return out;
}

// bitpack_layout_cuda.cpp:402-473: CacheGen layers -> float16 [L, 2, H, T, D].
at::Tensor cachegen_unpack_dequantize_cuda(at::Tensor bytestream, at::Tensor offsets,
                                           at::Tensor bits_per_layer, at::Tensor key_bins,
                                           at::Tensor value_bins, at::Tensor max_key,
                                           at::Tensor max_value, int64_t tokens, int64_t heads,
                                           int64_t head_dim) {
  at::Tensor flat = bytestream.reshape(-1).contiguous();
  require_byte(flat, "bytestream");
  const at::Tensor offs = host_i64(offsets), bits = host_i64(bits_per_layer);
  const at::Tensor kb = host_i64(key_bins), vb = host_i64(value_bins);
  TORCH_CHECK(bits.numel() % 2 == 0, "bits_per_layer length must be even");
  const int64_t layers = bits.numel() / 2;
  TORCH_CHECK(kb.numel() == layers, "key_bins length must match layers");
  TORCH_CHECK(vb.numel() == layers, "value_bins length must match layers");
  TORCH_CHECK(offs.numel() == bits.numel() + 1,
              "offsets length must be bits_per_layer length + 1");
  const at::Tensor mk = max_key.contiguous(), mv = max_value.contiguous();
  require_device(mk, "max_key");
  require_device(mv, "max_value");
  TORCH_CHECK(mk.scalar_type() == mv.scalar_type(),
              "max_key and max_value must have the same dtype");
  const c10::OptionalDeviceGuard guard(flat.device());
  at::Tensor out = at::empty({layers, 2, heads, tokens, head_dim},
                             flat.options().dtype(at::kHalf));
  check(origami_cachegen_unpack_dequantize(
      flat.data_ptr<uint8_t>(), flat.numel(), i64p(offs), i64p(bits), i64p(kb), i64p(vb), layers,
      mk.data_ptr(), mv.data_ptr(), mk.numel(), mv.numel(), dtype_code(mk.scalar_type(), "max_key"),
      tokens, heads, head_dim, out.data_ptr(), out.numel() * 2, current_stream(flat)));
  return out;
}

// bitpack_layout_cuda.cpp:475-581: CacheGen K/V streams -> paged cache.
void cachegen_unpack_dequantize_to_kv_cache_cuda(
    at::Tensor bytestream, int64_t key_offset, int64_t key_bytes, int64_t value_offset,
    int64_t value_bytes, int64_t key_bits, int64_t value_bits, int64_t key_bins,
    int64_t value_bins, at::Tensor max_key, at::Tensor max_value, at::Tensor kv_cache,
    at::Tensor block_ids, int64_t tokens, int64_t heads, int64_t head_dim) {
  at::Tensor flat = bytestream.reshape(-1).contiguous();
  require_byte(flat, "bytestream");
  require_device(kv_cache, "kv_cache");
  require_block_ids(block_ids, kv_cache);
  const at::Tensor mk = max_key.contiguous(), mv = max_value.contiguous();
  require_device(mk, "max_key");
  require_device(mv, "max_value");
  TORCH_CHECK(mk.scalar_type() == mv.scalar_type(),
              "max_key and max_value must have the same dtype");
  const CacheGeom g = dequant_cache_geometry(kv_cache, heads, head_dim);
  const c10::OptionalDeviceGuard guard(kv_cache.device());
  check(origami_cachegen_unpack_dequantize_to_kv_cache(
      flat.data_ptr<uint8_t>(), flat.numel(), key_offset, key_bytes, value_offset, value_bytes,
      key_bits, value_bits, key_bins, value_bins, mk.data_ptr(), mv.data_ptr(), mk.numel(),
      mv.numel(), dtype_code(mk.scalar_type(), "max_key"), kv_cache.data_ptr(),
      dtype_code(kv_cache.scalar_type(), "kv_cache"), g.layout, g.num_blocks, g.block_size,
      block_ids.data_ptr<int64_t>(), block_ids.numel(), tokens, heads, head_dim,
      current_stream(kv_cache)));
}

void kivi_to_kv_cache(at::Tensor bytestream, int64_t key_offset, int64_t key_bytes,
                      int64_t value_offset, int64_t value_bytes, int64_t bits,
                      int64_t symbol_packing, int64_t group_size, int64_t sink_tokens,
                      at::Tensor key_scale, at::Tensor key_zero, at::Tensor value_scale,
                      at::Tensor value_zero, at::Tensor key_sink, at::Tensor value_sink,
                      at::Tensor kv_cache, at::Tensor block_ids, int64_t tokens, int64_t heads,
                      int64_t head_dim) {
  at::Tensor flat = bytestream.reshape(-1).contiguous();
  require_byte(flat, "bytestream");
  require_device(kv_cache, "kv_cache");
  require_block_ids(block_ids, kv_cache);
  const at::Tensor metas[6] = {key_scale.contiguous(), key_zero.contiguous(),
                               value_scale.contiguous(), value_zero.contiguous(),
                               key_sink.contiguous(), value_sink.contiguous()};
  const char* names[6] = {"key_scale", "key_zero", "value_scale", "value_zero", "key_sink",
                          "value_sink"};
  int64_t counts[6];
  for (int i = 0; i < 6; ++i) {
    require_device(metas[i], names[i]);
    TORCH_CHECK(metas[i].scalar_type() == metas[0].scalar_type(),
                "KIVI metadata tensors must have the same dtype");
    counts[i] = metas[i].numel();
  }
  const CacheGeom g = dequant_cache_geometry(kv_cache, heads, head_dim);
  const c10::OptionalDeviceGuard guard(kv_cache.device());
  check(origami_kivi_dequantize_to_kv_cache(
      flat.data_ptr<uint8_t>(), flat.numel(), key_offset, key_bytes, value_offset, value_bytes,
      bits, symbol_packing, group_size, sink_tokens, metas[0].data_ptr(), metas[1].data_ptr(),
      metas[2].data_ptr(), metas[3].data_ptr(), metas[4].data_ptr(), metas[5].data_ptr(), counts,
      dtype_code(metas[0].scalar_type(), "KIVI metadata"), kv_cache.data_ptr(),
      dtype_code(kv_cache.scalar_type(), "kv_cache"), g.layout, g.num_blocks, g.block_size,
      block_ids.data_ptr<int64_t>(), block_ids.numel(), tokens, heads, head_dim,
      current_stream(kv_cache)));
}

// bitpack_layout_cuda.cpp:583-714: LSB-first symbols, as the reference kernel reads.
void kivi_dequantize_to_kv_cache_cuda(at::Tensor bytestream, int64_t key_offset,
                                      int64_t key_bytes, int64_t value_offset,
                                      int64_t value_bytes, int64_t bits, int64_t group_size,
                                      int64_t sink_tokens, at::Tensor key_scale,
                                      at::Tensor key_zero, at::Tensor value_scale,
                                      at::Tensor value_zero, at::Tensor key_sink,
                                      at::Tensor value_sink, at::Tensor kv_cache,
                                      at::Tensor block_ids, int64_t tokens, int64_t heads,
                                      int64_t head_dim) {
  kivi_to_kv_cache(bytestream, key_offset, key_bytes, value_offset, value_bytes, bits,
                   ORIGAMI_KIVI_PACKED_LSB, group_size, sink_tokens, key_scale, key_zero,
                   value_scale, value_zero, key_sink, value_sink, kv_cache, block_ids, tokens,
                   heads, head_dim);
}

void fused_prefix_attention_cuda(py::args, py::kwargs) {
  TORCH_CHECK(false, "fused prefix attention is outside the layout path");
}

// ---------------------------------------------------------------------------
// Fused paths (no reference counterpart under these names); chunk metadata
// as host int64 tensors.
// ---------------------------------------------------------------------------

// Packs a symbol tensor into `out` (the stub native_cpu.pack_canonical_storage_chunks).
void pack_canonical_storage_chunks(at::Tensor symbols, at::Tensor chunk_offsets,
                                   at::Tensor bits_per_chunk, at::Tensor chunk_specs,
                                   at::Tensor source_shape, at::Tensor axis_positions,
                                   int64_t token_count, int64_t num_heads, int64_t head_dim,
                                   at::Tensor out) {
  require_byte(symbols, "symbols");
  require_byte(out, "flat_chunks");
  const at::Tensor offs = host_i64(chunk_offsets), bits = host_i64(bits_per_chunk);
  const at::Tensor specs = host_i64(chunk_specs), shape = host_i64(source_shape);
  const at::Tensor axes = host_i64(axis_positions);
  TORCH_CHECK(offs.numel() == bits.numel() + 1, "chunk_offsets length must be chunk count + 1");
  const c10::OptionalDeviceGuard guard(symbols.device());
  check(origami_pack_canonical_storage_chunks(
      symbols.data_ptr<uint8_t>(), symbols.numel(), i64p(offs), i64p(bits), i64p(specs),
      bits.numel(), i64p(shape), shape.numel(), i64p(axes), token_count, num_heads, head_dim,
      out.data_ptr<uint8_t>(), out.numel(), current_stream(symbols)));
}

// One layer's stream -> paged cache through the block table.  Returns False
// when the chunk plan is not served by the fused kernel.
bool unpack_canonical_to_kv_cache(at::Tensor flat, at::Tensor chunk_offsets,
                                  at::Tensor bits_per_chunk, at::Tensor chunk_specs,
                                  int64_t tokens, at::Tensor kv_cache, at::Tensor block_ids) {
  require_byte(flat, "flat_chunks");
  require_device(kv_cache, "kv_cache");
  require_block_ids(block_ids, kv_cache);
  const CacheGeom g = layout_cache_geometry(kv_cache);
  const at::Tensor offs = host_i64(chunk_offsets), bits = host_i64(bits_per_chunk);
  const at::Tensor specs = host_i64(chunk_specs);
  TORCH_CHECK(offs.numel() == bits.numel() + 1, "chunk_offsets length must be chunk count + 1");
  const c10::OptionalDeviceGuard guard(kv_cache.device());
  return check_supported(origami_unpack_canonical_to_kv_cache(
      flat.data_ptr<uint8_t>(), flat.numel(), i64p(offs), i64p(bits), i64p(specs), bits.numel(),
      tokens, kv_cache.data_ptr(), g.layout, g.num_blocks, g.block_size, g.heads, g.head_bytes,
      block_ids.data_ptr<int64_t>(), block_ids.numel(), current_stream(kv_cache)));
}

// Paged cache -> one layer's stream (`out`).  Returns False when the chunk
// plan is not served by the fused kernel.
bool pack_canonical_from_kv_cache(at::Tensor kv_cache, at::Tensor block_ids, int64_t tokens,
                                  at::Tensor chunk_offsets, at::Tensor bits_per_chunk,
                                  at::Tensor chunk_specs, at::Tensor out) {
  require_device(kv_cache, "kv_cache");
  require_block_ids(block_ids, kv_cache);
  require_byte(out, "flat_chunks");
  const CacheGeom g = layout_cache_geometry(kv_cache);
  const at::Tensor offs = host_i64(chunk_offsets), bits = host_i64(bits_per_chunk);
  const at::Tensor specs = host_i64(chunk_specs);
  TORCH_CHECK(offs.numel() == bits.numel() + 1, "chunk_offsets length must be chunk count + 1");
  const c10::OptionalDeviceGuard guard(kv_cache.device());
  return check_supported(origami_pack_canonical_from_kv_cache(
      kv_cache.data_ptr(), g.layout, g.num_blocks, g.block_size, g.heads, g.head_bytes,
      block_ids.data_ptr<int64_t>(), block_ids.numel(), tokens, i64p(offs), i64p(bits),
      i64p(specs), bits.numel(), out.data_ptr<uint8_t>(), out.numel(),
      current_stream(kv_cache)));
}

// One layer of several requests into one cache.  Returns False when a plan
// is not served by the fused kernel.
bool unpack_canonical_to_kv_cache_batch(std::vector<at::Tensor> flats,
                                        std::vector<at::Tensor> chunk_offsets,
                                        std::vector<at::Tensor> bits_per_chunk,
                                        std::vector<at::Tensor> chunk_specs,
                                        std::vector<int64_t> tokens, at::Tensor kv_cache,
                                        std::vector<at::Tensor> block_ids,
                                        std::vector<int64_t> first_tokens) {
  const size_t n = flats.size();
  TORCH_CHECK(chunk_offsets.size() == n && bits_per_chunk.size() == n &&
                  chunk_specs.size() == n && tokens.size() == n && block_ids.size() == n &&
                  (first_tokens.empty() || first_tokens.size() == n),
              "one entry per request is required");
  require_device(kv_cache, "kv_cache");
  const CacheGeom g = layout_cache_geometry(kv_cache);
  std::vector<at::Tensor> offs(n), bits(n), specs(n);
  std::vector<const uint8_t*> fp(n);
  std::vector<const int64_t*> op(n), bp(n), sp(n), ip(n);
  std::vector<int64_t> fb(n), nc(n), bc(n);
  for (size_t r = 0; r < n; ++r) {
    require_byte(flats[r], "flat_chunks");
    require_block_ids(block_ids[r], kv_cache);
    offs[r] = host_i64(chunk_offsets[r]);
    bits[r] = host_i64(bits_per_chunk[r]);
    specs[r] = host_i64(chunk_specs[r]);
    TORCH_CHECK(offs[r].numel() == bits[r].numel() + 1,
                "chunk_offsets length must be chunk count + 1");
    fp[r] = flats[r].data_ptr<uint8_t>();
    fb[r] = flats[r].numel();
    op[r] = i64p(offs[r]);
    bp[r] = i64p(bits[r]);
    sp[r] = i64p(specs[r]);
    nc[r] = bits[r].numel();
    ip[r] = block_ids[r].data_ptr<int64_t>();
    bc[r] = block_ids[r].numel();
  }
  const c10::OptionalDeviceGuard guard(kv_cache.device());
  return check_supported(origami_unpack_canonical_to_kv_cache_batch(
      static_cast<int64_t>(n), fp.data(), fb.data(), op.data(), bp.data(), sp.data(), nc.data(),
      tokens.data(), kv_cache.data_ptr(), g.layout, g.num_blocks, g.block_size, g.heads,
      g.head_bytes, ip.data(), bc.data(), first_tokens.empty() ? nullptr : first_tokens.data(),
      current_stream(kv_cache)));
}

// A prepared restore (origami_restore_plan_create) with the cache geometry it
// was made for and its device block table, which it keeps alive.
struct PreparedRestore {
  origami_restore_plan_t plan = nullptr;
  std::vector<int64_t> sizes;
  at::ScalarType dtype;
  at::Device device;
  at::Tensor block_ids;
  ~PreparedRestore() { origami_restore_plan_destroy(plan); }
};

// Returns a handle (an integer), or 0 when the chunk plan is not served by the
// fused kernel.
int64_t restore_plan_create(at::Tensor chunk_offsets, at::Tensor bits_per_chunk,
                            at::Tensor chunk_specs, int64_t tokens, at::Tensor kv_cache,
                            at::Tensor block_ids) {
  require_device(kv_cache, "kv_cache");
  require_block_ids(block_ids, kv_cache);
  const CacheGeom g = layout_cache_geometry(kv_cache);
  const at::Tensor offs = host_i64(chunk_offsets), bits = host_i64(bits_per_chunk);
  const at::Tensor specs = host_i64(chunk_specs);
  TORCH_CHECK(offs.numel() == bits.numel() + 1, "chunk_offsets length must be chunk count + 1");
  const c10::OptionalDeviceGuard guard(kv_cache.device());
  origami_restore_plan_t plan = nullptr;
  if (!check_supported(origami_restore_plan_create(
          i64p(offs), i64p(bits), i64p(specs), bits.numel(), tokens, g.layout, g.num_blocks,
          g.block_size, g.heads, g.head_bytes, block_ids.data_ptr<int64_t>(), block_ids.numel(),
          &plan)))
    return 0;
  auto* r = new PreparedRestore{plan, kv_cache.sizes().vec(), kv_cache.scalar_type(),
                                kv_cache.device(), block_ids};
  return reinterpret_cast<int64_t>(r);
}

// One layer: `flat` (this layer's stream) into `kv_cache` (a cache of the
// geometry the plan was made for), on the current stream.
void restore_plan_launch(int64_t handle, const at::Tensor& flat, const at::Tensor& kv_cache) {
  TORCH_CHECK(handle != 0, "restore plan is closed");
  const auto* r = reinterpret_cast<const PreparedRestore*>(handle);
  TORCH_CHECK(kv_cache.device() == r->device && kv_cache.scalar_type() == r->dtype &&
                  kv_cache.sizes().equals(r->sizes) && kv_cache.is_contiguous(),
              "kv_cache geometry differs from the prepared restore");
  TORCH_CHECK(flat.device() == r->device && flat.scalar_type() == at::kByte &&
                  flat.is_contiguous(),
              "flat_chunks must be a contiguous uint8 tensor on the cache's device");
  const c10::OptionalDeviceGuard guard(r->device);
  check(origami_restore_plan_launch(r->plan, flat.data_ptr<uint8_t>(), flat.numel(),
                                    kv_cache.data_ptr(), current_stream(kv_cache)));
}

void restore_plan_destroy(int64_t handle) {
  delete reinterpret_cast<PreparedRestore*>(handle);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Origami KV codec-layout path on MI355X (liborigami_layout.so)";
  m.def("unpack_canonical_storage_chunks_cuda", &unpack_canonical_storage_chunks_cuda);
  m.def("cachegen_unpack_dequantize_cuda", &cachegen_unpack_dequantize_cuda);
  m.def("cachegen_unpack_dequantize_to_kv_cache_cuda",
        &cachegen_unpack_dequantize_to_kv_cache_cuda);
  m.def("kivi_dequantize_to_kv_cache_cuda", &kivi_dequantize_to_kv_cache_cuda);
  m.def("fused_prefix_attention_cuda", &fused_prefix_attention_cuda);
  m.def("kivi_dequantize_to_kv_cache", &kivi_to_kv_cache);
  m.def("pack_canonical_storage_chunks", &pack_canonical_storage_chunks);
  m.def("unpack_canonical_to_kv_cache", &unpack_canonical_to_kv_cache);
  m.def("pack_canonical_from_kv_cache", &pack_canonical_from_kv_cache);
  m.def("unpack_canonical_to_kv_cache_batch", &unpack_canonical_to_kv_cache_batch);
  m.def("restore_plan_create", &restore_plan_create);
  m.def("restore_plan_launch", &restore_plan_launch);
  m.def("restore_plan_destroy", &restore_plan_destroy);
  m.def("abi_version", &origami_abi_version);
}
