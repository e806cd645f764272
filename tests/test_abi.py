"""The C ABI library loads without a GPU, exports every symbol the header
declares, and its host-only entry points (validation, plane plan) behave."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle
from origami_amd import _native
from origami_amd.lossless.chunking import plan_head_channel_chunks

HEADER = Path(__file__).resolve().parents[1] / "include" / "origami_layout.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(origami_\w+)\(", text, re.M)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert "origami_unpack_canonical_storage_chunks" in names
    assert "origami_unpack_canonical_to_kv_cache" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(_native.EXPORTED_SYMBOLS)


def test_abi_version():
    assert _native.lib().origami_abi_version() == _native.ABI_VERSION


def _validate(offsets, bits, specs, shape, axes, T, H, C, flat_bytes):
    offsets, bits, specs = (_native.i64_array(x) for x in (offsets, bits, specs))
    shape, axes = _native.i64_array(shape), _native.i64_array(axes)
    return _native.call("origami_validate_chunks", offsets.ctypes.data, bits.ctypes.data,
                        specs.ctypes.data, specs.size // 6, shape.ctypes.data, shape.size,
                        axes.ctypes.data, T, H, C, flat_bytes)


def test_validation_accepts_planner_layout():
    specs = [[0, 1, 0, 4, 0, 10], [0, 1, 4, 8, 0, 10]]
    assert _validate([0, 40, 80], [8, 8], specs, [10, 1, 8], [0, 1, 2, -1], 10, 1, 8, 80) == 0


@pytest.mark.parametrize("mutate,msg", [
    (dict(bits=[0, 8]), "1..8 bit"),
    (dict(offsets=[0, 40, 79]), "byte size mismatch"),
    (dict(flat_bytes=79), "exceed the flat stream"),
    (dict(specs=[[0, 2, 0, 4, 0, 10], [0, 1, 4, 8, 0, 10]]), "head range"),
    (dict(shape=[10, 1, 8, 2], axes=[0, 1, 2, 3]), "layer axis size 1"),
    (dict(T=11), "token axis size"),
    (dict(axes=[0, 0, 2, -1]), "axes must be unique|head axis size"),
    (dict(T=0, shape=[0, 1, 8]), "shape must be positive"),
    (dict(shape=[10, 0, 8]), "must be positive"),
    (dict(specs=[[0, 1, 0, 4, 0, 11], [0, 1, 4, 8, 0, 10]]), "token range"),
    (dict(specs=[[0, 1, 4, 4, 0, 10], [0, 1, 4, 8, 0, 10]]), "channel range"),
    (dict(offsets=[-40, 0, 40]), "non-negative"),
    (dict(bits=[8, 9]), "1..8 bit"),
    (dict(axes=[0, 1, 5, -1]), "head_dim axis must be present"),
])
def test_validation_messages(mutate, msg):
    args = dict(offsets=[0, 40, 80], bits=[8, 8],
                specs=[[0, 1, 0, 4, 0, 10], [0, 1, 4, 8, 0, 10]],
                shape=[10, 1, 8], axes=[0, 1, 2, -1], T=10, H=1, C=8, flat_bytes=80)
    args.update(mutate)
    with pytest.raises(_native.OrigamiNativeError, match=msg) as ei:
        _validate(**args)
    assert ei.value.code == _native.ORIGAMI_ERR_INVALID


def _plan(specs, bits, T, H, C):
    specs = _native.i64_array(specs).reshape(-1, 6)
    bits_a = _native.i64_array(np.broadcast_to(bits, (specs.shape[0],)))
    offsets = oracle.chunk_offsets(specs, bits_a)
    table = np.zeros(H * C, np.int64)
    info = np.zeros(4, np.int64)
    _native.call("origami_plan_planes", offsets.ctypes.data, bits_a.ctypes.data,
                 specs.ctypes.data, specs.shape[0], T, H, C, table.ctypes.data, table.size,
                 info.ctypes.data)
    return table, info, offsets


@pytest.mark.parametrize("bits", [8, 5, 3])
def test_plane_table_points_at_each_planes_token_run(bits):
    """The host plan's bit offsets locate every (head, channel) token run in a
    stream packed by the oracle: read back with the bit-list reference."""
    rng = np.random.default_rng(bits)
    T, H, C = 40, 3, 32
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, 0, T]
             for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                               token_count=T, bytes_per_symbol=1,
                                               min_bytes=300, target_bytes=300,
                                               max_bytes=300)]
    sym = rng.integers(0, 1 << bits, (T, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
    table, info, offsets = _plan(specs, bits, T, H, C)
    assert np.array_equal(offsets, offs)
    assert info[0] == 1 and info[1] == bits
    bitsarr = np.unpackbits(flat, bitorder="little")
    for h in range(H):
        for c in range(C):
            start = int(table[h * C + c])
            run = bitsarr[start:start + T * bits].reshape(T, bits)
            vals = (run.astype(np.uint32) @ (1 << np.arange(bits))).astype(np.uint8)
            assert np.array_equal(vals, sym[:, h, c])
    assert info[3] == int(all(int(x) % 8 == 0 for x in table))


def test_plane_plan_flags_irregular_layouts():
    # token-split chunk -> not regular
    _, info, _ = _plan([[0, 1, 0, 16, 0, 8], [0, 1, 0, 16, 8, 16]], 8, 16, 1, 16)
    assert info[0] == 0
    # overlapping planes -> not regular
    _, info, _ = _plan([[0, 1, 0, 16, 0, 16], [0, 1, 8, 16, 0, 16]], 8, 16, 1, 16)
    assert info[0] == 0
    # uncovered planes are allowed (-1 entries), aligned16 for 16-token runs
    table, info, _ = _plan([[0, 1, 0, 8, 0, 16]], 8, 16, 1, 16)
    assert info[0] == 1 and info[2] == 1 and (table[8:] == -1).all()
    # mixed bit widths -> bits 0
    specs = [[0, 1, 0, 8, 0, 16], [0, 1, 8, 16, 0, 16]]
    sp = _native.i64_array(specs)
    bits_a = _native.i64_array([8, 4])
    offs = oracle.chunk_offsets(sp, bits_a)
    table = np.zeros(16, np.int64)
    info = np.zeros(4, np.int64)
    _native.call("origami_plan_planes", offs.ctypes.data, bits_a.ctypes.data, sp.ctypes.data,
                 2, 16, 1, 16, table.ctypes.data, 16, info.ctypes.data)
    assert info[1] == 0


def test_extension_module_exports_reference_names():
    """origami_bitpack_hip loads without a GPU and exports the reference
    module's functions (bitpack_layout_cuda.cpp:894-903) and the fused paths."""
    from origami_amd import _ext

    m = _ext.ext()
    for name in ("unpack_canonical_storage_chunks_cuda", "cachegen_unpack_dequantize_cuda",
                 "cachegen_unpack_dequantize_to_kv_cache_cuda",
                 "kivi_dequantize_to_kv_cache_cuda", "fused_prefix_attention_cuda",
                 "unpack_canonical_to_kv_cache", "pack_canonical_from_kv_cache",
                 "unpack_canonical_to_kv_cache_batch", "pack_canonical_storage_chunks",
                 "kivi_dequantize_to_kv_cache", "restore_plan_create", "restore_plan_launch",
                 "restore_plan_destroy"):
        assert callable(getattr(m, name)), name
    assert m.abi_version() == _native.ABI_VERSION
    with pytest.raises(RuntimeError, match="outside the layout path"):
        m.fused_prefix_attention_cuda()


def test_restore_plan_host_checks():
    """origami_restore_plan_create validates the chunk metadata and the cache
    geometry before it needs a GPU, with the messages of the fused restore;
    origami_restore_plan_launch refuses a null plan."""
    specs = _native.i64_array([[0, 1, 0, 16, 0, 64], [0, 1, 16, 32, 0, 64]])
    bits = _native.i64_array([8, 8])
    out = ctypes.c_void_p()

    def create(offsets, block_size=16, num_blocks=4, block_count=2):
        offs = _native.i64_array(offsets)
        return _native.call("origami_restore_plan_create", offs.ctypes.data, bits.ctypes.data,
                            specs.ctypes.data, 2, 32, _native.CACHE_KV_FIRST, num_blocks,
                            block_size, 1, 32, None, block_count, ctypes.byref(out))

    with pytest.raises(_native.OrigamiNativeError, match="byte size mismatch"):
        create([0, 1024, 2047])
    with pytest.raises(_native.OrigamiNativeError, match="tokens exceed destination block"):
        create([0, 1024, 2048], block_count=1)
    with pytest.raises(_native.OrigamiNativeError, match="block size must be positive"):
        create([0, 1024, 2048], block_size=0)
    assert out.value is None
    with pytest.raises(_native.OrigamiNativeError, match="restore plan is null"):
        _native.call("origami_restore_plan_launch", None, None, 0, None, None)
    _native.lib().origami_restore_plan_destroy(None)  # a null plan is a no-op
