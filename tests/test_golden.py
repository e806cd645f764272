"""Committed golden fixtures (tests/golden/, made by make_golden.py from the
format definition): the oracle on the CPU and the HIP path on the GPU must
reproduce them byte for byte."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = [c for c in (GOLDEN / "CASES.txt").read_text().split() if c != "scatter_kv_first"]
NAMES = {0: "token", 1: "head", 2: "head_dim", 3: "layer"}


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def layout_names(shape, axes):
    names = [""] * len(shape)
    for role, pos in enumerate(axes):
        if pos >= 0:
            names[int(pos)] = NAMES[role]
    return names


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    g = load(name)
    flat, offs = oracle.pack_canonical(g["symbols"], g["bits"], g["specs"], g["shape"], g["axes"])
    assert np.array_equal(offs, g["offsets"]) and np.array_equal(flat, g["stream"])
    out = oracle.unpack_canonical(g["stream"], g["offsets"], g["bits"], g["specs"], g["shape"],
                                  g["axes"])
    assert np.array_equal(out, g["unpacked"])


def test_oracle_scatter_golden():
    g = load("scatter_kv_first")
    cache = g["cache"].copy()
    T, H, C = int(g["tokens"]), g["value"].shape[2], g["value"].shape[3]
    oracle.scatter_kv_cache(g["value"], T, H, C, g["ids"], cache)
    assert np.array_equal(cache, g["expect"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_reproduces_golden(cuda_device, name):
    import torch

    from origami_amd.lossless import native_gpu

    g = load(name)
    names = layout_names(g["shape"], g["axes"])
    bits = [int(b) for b in g["bits"]]
    flat, lay = native_gpu.pack_canonical_storage_flat(
        torch.from_numpy(g["symbols"]).to(cuda_device), bits, g["shape"].tolist(), names,
        g["specs"])
    assert np.array_equal(lay.offsets, g["offsets"])
    assert np.array_equal(flat.cpu().numpy(), g["stream"])
    out = native_gpu.unpack_canonical_storage_chunks(
        torch.from_numpy(g["stream"]).to(cuda_device), bits, g["shape"].tolist(), names,
        g["specs"], device=cuda_device)
    assert np.array_equal(out.cpu().numpy(), g["unpacked"])


@pytest.mark.gpu
def test_hip_scatter_golden(cuda_device):
    import torch

    from origami_amd.lossless import native_gpu

    g = load("scatter_kv_first")
    cache = torch.from_numpy(g["cache"].copy()).to(cuda_device)
    ids = native_gpu.block_ids_tensor(g["ids"], cuda_device, cache.shape[1])
    native_gpu.scatter_kv_blocks(torch.from_numpy(g["value"]).to(cuda_device),
                                 int(g["tokens"]), cache, ids)
    assert np.array_equal(cache.cpu().numpy(), g["expect"])
