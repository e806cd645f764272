"""The benchmark's CPU-side contract: one GPU only, the closed-form restore
check its GPU legs rely on, and the committed traffic figure it reports."""
import argparse
import subprocess
import sys
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert not r.stdout.strip()


def _restored(T, H, C, bs, seed):
    """A b = 8 planner-layout stream of random tokens and the paged cache a
    correct restore leaves: the stream is plane-major (plane h * C + c holds
    that channel's 2T symbols), the cache holds the tokens at the table's
    blocks and zeros past T."""
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randint(0, 256, (2, T, H * C), dtype=torch.uint8, generator=g)
    stream = tokens.reshape(2 * T, H * C).t().contiguous().reshape(-1)
    nblk = -(-T // bs)
    NB = nblk + 3
    ids = torch.randperm(NB, generator=g)[:nblk]
    cache = torch.zeros((2, NB, bs, H, C), dtype=torch.uint8)
    rows = torch.zeros((2, nblk * bs, H * C), dtype=torch.uint8)
    rows[:, :T] = tokens
    cache[:, ids] = rows.reshape(2, nblk, bs, H, C)
    return stream, tokens, cache, ids


def test_closed_form_check_accepts_a_correct_restore():
    T, H, C = 40, 2, 16
    stream, tokens, cache, ids = _restored(T, H, C, 16, 1)
    assert bench._closed_form_ok(stream, tokens, cache, ids, T, H, C)


def test_closed_form_check_catches_mistakes():
    T, H, C = 40, 2, 16
    stream, tokens, cache, ids = _restored(T, H, C, 16, 2)
    bad_stream = stream.clone()
    bad_stream[123] ^= 1  # one symbol of the stream
    assert not bench._closed_form_ok(bad_stream, tokens, cache, ids, T, H, C)
    bad_cache = cache.clone()
    bad_cache[1, ids[0], 3, 1, 5] ^= 0x80  # one restored V byte
    assert not bench._closed_form_ok(stream, tokens, bad_cache, ids, T, H, C)
    tail = cache.clone()
    tail[0, ids[-1], 15, 0, 0] = 7  # a byte past T in the last block
    assert not bench._closed_form_ok(stream, tokens, tail, ids, T, H, C)
    swapped = cache.clone()
    swapped[:, ids[[0, 1]]] = cache[:, ids[[1, 0]]]  # two blocks exchanged
    assert not bench._closed_form_ok(stream, tokens, swapped, ids, T, H, C)


def test_committed_traffic_is_the_profiles_figure():
    args = argparse.Namespace(layers=32, tokens=32768, heads=8, head_dim=128, block_size=16,
                              bits=8)
    line = next(l for l in (REPO / "profiles" / "rows_unpack_llama3_8b_32k.txt")
                .read_text().splitlines()
                if l.startswith("traffic_bytes_per_launch rows_unpack_kernel<8, 2, false, false>:"))
    assert bench.committed_traffic(args) == int(line.split(":")[1].split()[0])
    # a workload the summary does not cover reports no traffic
    args.tokens = 4096
    assert bench.committed_traffic(args) is None
