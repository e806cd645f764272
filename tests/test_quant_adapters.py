"""CPU checks of the CacheGen and KIVI adapters (origami_amd/quantization).

Pinned by:
  * hand-worked values of the reference's bin schedule, width rule and layer
    index (cachegen_adapter.py:49-57, 99-114);
  * numpy restatements of the quantizers (float32 numpy arithmetic, round
    half to even), independent of torch;
  * the KIVI packers restated in tests/dqref.py;
  * quantization error bounds and exact sink tokens on round trips, for every
    KV layout the adapters accept.
"""
import numpy as np
import pytest
import torch

from origami_amd.quantization import create_quantizer_adapter
from origami_amd.quantization.cachegen_adapter import (CacheGenAdapter, bits_for_bins,
                                                       cachegen_bins, canonicalize, layer_index,
                                                       restore_layout)
from origami_amd.quantization.kivi_adapter import (KiviAdapter, pack_lowbit, pack_ordered,
                                                   unpack_lowbit, unpack_ordered)
from tests import dqref


def test_bin_schedule_and_widths():
    a = CacheGenAdapter({"quant_level": "2"})
    assert [a.key_bins(i) for i in (0, 9, 10, 19, 20, 31)] == [32, 32, 16, 16, 16, 16]
    assert [a.value_bins(i) for i in (0, 1, 2, 31)] == [32, 32, 16, 16]
    b = CacheGenAdapter({"quant_level": "1"})
    assert [b.key_bins(i) for i in (0, 10, 20)] == [16, 16, 12]
    assert [b.value_bins(i) for i in (1, 2)] == [16, 12]
    assert cachegen_bins("/m/Qwen3-8B", "3").key_third_layers == 36
    assert cachegen_bins("mistral", "3").key_third_layers == 32
    with pytest.raises(ValueError):
        cachegen_bins("m", "4")
    assert [bits_for_bins(n) for n in (1, 2, 3, 4, 12, 16, 17, 32, 256, 300)] == \
        [1, 1, 2, 2, 4, 4, 5, 5, 8, 8]
    assert [layer_index(x) for x in ("model.layers.17.self_attn", "layers.3", "abc", None,
                                     "l12x34y")] == [17, 3, 0, 0, 34]


KV_SHAPES = [(2, 3, 4, 2, 8), (3, 2, 4, 2, 8), (3, 4, 2, 2, 8), (2, 12, 2, 8), (12, 2, 2, 8),
             (2, 2, 130, 8)]


@pytest.mark.parametrize("shape", KV_SHAPES)
def test_canonicalize_round_trip(shape):
    kv = torch.randn(shape)
    canonical, layout = canonicalize(kv)
    assert canonical.shape[0] == 2 and canonical.dim() == 4
    back = restore_layout(canonical, {"shape": list(shape), "kv_layout": layout})
    assert torch.equal(back, kv)


def _np_cachegen_plane(x: np.ndarray, bins: int):
    """cachegen_adapter.py:246-257 in numpy float32."""
    x = x.reshape(x.shape[0], -1).astype(np.float32)
    max_abs = np.maximum(np.abs(x).max(axis=1, keepdims=True), np.float32(1e-6))
    c = bins // 2 - 1
    q = np.round(x * (np.float32(c) / max_abs) + np.float32(c))
    return np.clip(q, 0, 2 * c).astype(np.uint8), max_abs.astype(np.float16)


@pytest.mark.parametrize("bins", [4, 12, 16, 32, 256])
def test_cachegen_quantize_plane_matches_numpy(bins):
    x = torch.randn(64, 4, 16) * torch.rand(64, 1, 1) * 5
    x[3] = 0  # an all-zero token: max clamped to 1e-6
    q, mx = CacheGenAdapter.quantize_plane(x, bins)
    qn, mxn = _np_cachegen_plane(x.numpy(), bins)
    assert np.array_equal(q.numpy(), qn)
    assert np.array_equal(mx.numpy().view(np.uint16), mxn.view(np.uint16))


@pytest.mark.parametrize("shape", KV_SHAPES[:3])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_cachegen_structured_round_trip_cpu(shape, dtype):
    torch.manual_seed(0)
    kv = (torch.randn(shape) * 3).to(dtype)
    a = CacheGenAdapter({"bitpacked": False, "dequant_device": "cpu"})
    q = a.quantize(kv, layer_group="model.layers.12.attn")
    m = q.metadata
    assert m["format"] == "cachegen_structured_blob" and m["key_bins"] == 16
    assert m["origami_symbol_shape"] == [1, 1, q.symbols.numel()]
    assert m["key_max_offset"] % 2 == 0 and m["value_max_offset"] % 2 == 0
    back = a.dequantize(q.symbols, m)
    assert back.shape == kv.shape and back.dtype == dtype
    canonical, _ = canonicalize(kv.float())
    got, _ = canonicalize(back.float())
    for h, bins in ((0, m["key_bins"]), (1, m["value_bins"])):
        c = bins // 2 - 1
        mx = canonical[h].reshape(canonical.shape[1], -1).abs().amax(1, keepdim=True)
        err = (got[h] - canonical[h]).reshape(canonical.shape[1], -1).abs()
        # half a level plus the float16 rounding of max and of the output
        assert torch.all(err <= mx / c * 0.5 + mx * 2 ** -7 + 1e-6)


def test_kivi_packers_match_reference_packers():
    rng = np.random.default_rng(0)
    for bits in (2, 3, 4, 8):
        for n in (1, 2, 3, 5, 64, 97):
            v = rng.integers(0, 1 << bits, n, dtype=np.uint8)
            packed = pack_lowbit(torch.from_numpy(v), bits)
            assert np.array_equal(packed.numpy(), dqref.kivi_pack(v, bits)), (bits, n)
            assert np.array_equal(unpack_lowbit(packed, bits, n).numpy(), v)
    with pytest.raises(ValueError):
        pack_lowbit(torch.zeros(4, dtype=torch.uint8), 5)


def test_kivi_stream_orders():
    rng = np.random.default_rng(1)
    body, H, D = 7, 3, 4
    q = rng.integers(0, 16, (body, H * D), dtype=np.uint8)
    data = torch.from_numpy(q).reshape(1, body, H, D)
    ks = pack_ordered(data, ("head_dim", "layer", "head", "token"), 8)
    vs = pack_ordered(data, ("head", "layer", "head_dim", "token"), 8)
    assert np.array_equal(ks.numpy(), dqref.kivi_key_order(q, H, D))
    assert np.array_equal(vs.numpy(), dqref.kivi_value_order(q, H, D))
    back = unpack_ordered(ks, (1, body, H, D), ("head_dim", "layer", "head", "token"), 8)
    assert torch.equal(back, data)


def _np_kivi_key(m: np.ndarray, group: int, bits: int):
    rows, cols = m.shape
    groups = -(-rows // group)
    padded = np.concatenate([m, np.repeat(m[-1:], groups * group - rows, axis=0)])
    g = padded.reshape(groups, group, cols)
    zero = g.min(axis=1)
    levels = np.float32((1 << bits) - 1)
    scale = np.maximum((g.max(axis=1) - zero) / levels, np.finfo(np.float32).tiny)
    q = np.clip(np.round((g - zero[:, None]) / scale[:, None]), 0, levels)
    return (q.astype(np.uint8).reshape(-1, cols)[:rows], scale.astype(np.float16),
            zero.astype(np.float16))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_kivi_key_quantizer_matches_numpy(bits):
    m = torch.randn(37, 24) * 2
    q, s, z = KiviAdapter.quantize_key_per_channel(m, 8, bits)
    qn, sn, zn = _np_kivi_key(m.numpy(), 8, bits)
    assert np.array_equal(q.numpy(), qn)
    assert np.array_equal(s.numpy().view(np.uint16), sn.view(np.uint16))
    assert np.array_equal(z.numpy().view(np.uint16), zn.view(np.uint16))
    qv, sv, zv = KiviAdapter.quantize_value_per_token(m.T.contiguous(), 8, bits)
    assert np.array_equal(qv.numpy(), qn.T)
    assert np.array_equal(sv.numpy().view(np.uint16), sn.T.view(np.uint16))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("shape", KV_SHAPES[:3])
def test_kivi_round_trip_cpu(bits, shape):
    torch.manual_seed(bits)
    kv = (torch.randn(shape) * 2).to(torch.float16)
    a = create_quantizer_adapter("kivi", {"bits": bits, "group_size": 4, "sink_tokens": 3,
                                          "dequant_device": "cpu"})
    q = a.quantize(kv)
    m = q.metadata
    assert m["format"] == "kivi_structured_blob" and m["sink_tokens"] == 3
    for k in ("key_scale", "key_zero", "value_scale", "value_zero", "key_sink", "value_sink"):
        assert m[f"{k}_offset"] % 2 == 0
    back = a.dequantize(q.symbols, m)
    assert back.shape == kv.shape
    c_in, _ = canonicalize(kv.float())
    c_out, _ = canonicalize(back.float())
    assert torch.equal(c_out[:, :3], c_in[:, :3])  # sink tokens are kept exactly
    span = c_in.amax() - c_in.amin()
    assert torch.all((c_out - c_in).abs() <= span / ((1 << bits) - 1) * 0.5 + 0.02)
