"""MI355X-native (gfx950, HIP) implementation of Origami's KV codec-layout path.

Layout path: the canonical chunked, plane-major, LSB-first bit-packed stream of
one layer's KV (pack / unpack), fused unpack+scatter into vLLM's paged KV cache
through the block table, fused gather+pack from it, and the layer-wise restore
pipeline behind the connector API.  Device work runs in liborigami_layout.so
(origami_amd/csrc/origami_layout.hip), reached through a C ABI
(include/origami_layout.h).
"""

__version__ = "0.1.0"
