"""Synthetic KV generators for the benchmark workloads.

K = N(0, 1) * per-channel scale, scale ~ LogNormal(0, 1), with 4 outlier
channels per head multiplied by 20; V = N(0, sigma=0.5).  fp8 caches draw
N(0, 1) scaled by a per-head scale and cast to float8_e4m3fn.  Values are
generated directly into the paged cache blocks a block table names.
"""
from __future__ import annotations

import torch


def _k_scale(gen: torch.Generator, heads: int, head_dim: int, device) -> torch.Tensor:
    scale = torch.exp(torch.randn(heads, head_dim, generator=gen, device=device))
    for h in range(heads):
        idx = torch.randperm(head_dim, generator=gen, device=device)[:4]
        scale[h, idx] *= 20.0
    return scale


def fill_layer(cache: torch.Tensor, block_ids: torch.Tensor, gen: torch.Generator) -> None:
    """Writes synthetic K/V into the blocks `block_ids` of a [2, NB, bs, H, D]
    cache (bf16/fp16/fp32 or float8_e4m3fn)."""
    _, _, bs, H, D = cache.shape
    n = int(block_ids.numel())
    dev = cache.device
    if cache.dtype == torch.float8_e4m3fn:
        head_scale = torch.exp(torch.randn(H, generator=gen, device=dev))
        kv = torch.randn(2, n, bs, H, D, generator=gen, device=dev) * head_scale[:, None]
    else:
        k = torch.randn(n, bs, H, D, generator=gen, device=dev) * _k_scale(gen, H, D, dev)
        v = torch.randn(n, bs, H, D, generator=gen, device=dev) * 0.5
        kv = torch.stack((k, v))
    cache[:, block_ids] = kv.to(cache.dtype)
