#!/usr/bin/env python3
"""Layer-wise KV restore benchmark (fused unpack + paged scatter) on one GPU.

Workload: Llama-3-8B KV geometry, 32 layers x one 32768-token request,
8 KV heads, head_dim 128, bf16, block_size 16, each layer's blocks at a
randomly permuted block table (seed 1), 1 MiB chunks from the chunk planner,
bits 8.  Each layer's codec stream (K/V bytes in plane-major chunk order) is
packed once from a synthetic source cache and kept in HBM; one step restores
all 32 layers into the paged destination cache.

Prints one JSON line.  `value` is whole-step restore throughput in GB/s
(10^9 bytes/s) of algorithmic bytes: stream bytes read + cache bytes written +
block-table bytes, per layer.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBPS = 8000.0
METRIC = "KV restore GB/s (unpack+scatter) and % of HBM peak; per-layer restore µs"
CAL_BYTES = 256 << 20

# launch-bound single-request geometries: the configs leg adds a same-size
# device copy beside them
SHORT_CONFIGS = ("llama3-8b-4k", "llama3-8b-32k-tp8-rank")

CONFIG_NAMES = ("llama3-8b-4k", "qwen2.5-7b-batch", "llama3-8b-fp8-16x16k", "llama3-70b-128k",
                "llama3-8b-32k-tp8-rank")

# name -> (layers, tokens); both: 8 KV heads, head_dim 128, bf16, block_size 16
WORKLOADS = {
    "llama3-8b-32k": (32, 32768),      # Llama-3-8B geometry, one 32768-token request
    "llama3-70b-128k": (80, 131072),   # Llama-3-70B geometry, one 131072-token request
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="llama3-8b-32k")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--block-size", type=int, default=16)
    ap.add_argument("--bits", type=int, default=8)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=10)
    ap.add_argument("--no-pipeline", action="store_true")
    ap.add_argument("--no-pack-ragged", action="store_true",
                    help="skip the fused save at a ragged length (32753 tokens)")
    ap.add_argument("--no-dequant", action="store_true",
                    help="skip the CacheGen / KIVI fused dequantize legs")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the restore legs at the other KV geometries")
    ap.add_argument("--config-layers", type=int, default=4,
                    help="layers per geometry in the configs leg")
    ap.add_argument("--no-connector", action="store_true",
                    help="skip the end-to-end save/restore through the connector")
    ap.add_argument("--connector-layers", type=int, default=8)
    ap.add_argument("--profile-only", action="store_true",
                    help="only the timed restore loop (for rocprofv3 runs)")
    ap.add_argument("--profile-dequant", action="store_true",
                    help="with --profile-only: also run the dequantize legs")
    ap.add_argument("--profile-config", choices=sorted(CONFIG_NAMES), default=None,
                    help="only the restore loop of one of the other geometries (for "
                         "rocprofv3 runs), then the calibration copy")
    return ap.parse_args()


def main() -> int:
    args = parse_args()
    wl_layers, wl_tokens = WORKLOADS[args.workload]
    args.layers = args.layers or wl_layers
    args.tokens = args.tokens or wl_tokens
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the restore "
              "path needs no cross-GPU exchange and this build measures one GPU's share.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from origami_amd.layout import kv_symbol_layout
    from origami_amd.lossless import native_gpu
    from origami_amd.lossless.chunking import plan_head_channel_chunks
    from origami_amd.synthetic import fill_layer

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.profile_config:
        res = configs_leg(dev, args.steps, args.config_layers, only=args.profile_config,
                          min_launches=0)
        calibration_copy(dev)
        print(json.dumps(res), flush=True)
        return 0

    L, T, H, D, bs, bits = (args.layers, args.tokens, args.heads, args.head_dim,
                            args.block_size, args.bits)
    esize = 2  # bf16
    C = D * esize
    nblk = -(-T // bs)
    NB = nblk + nblk // 4
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    layout = kv_symbol_layout(T, H, C, bits, specs)

    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    src_cache = torch.empty((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev)
    streams, dst_ids, dst_caches = [], [], []
    src_tokens0 = None
    for layer in range(L):
        src_ids = torch.randperm(NB, generator=gen, device=dev)[:nblk].contiguous()
        fill_layer(src_cache, src_ids, gen)
        streams.append(native_gpu.pack_from_kv_cache(src_cache, src_ids, T, layout))
        if layer == 0:  # layer 0's source tokens, for the check below
            src_tokens0 = (src_cache.view(torch.uint8)[:, src_ids].reshape(2, -1, H * C)[:, :T]
                           .contiguous())
        dst_ids.append(torch.randperm(NB, generator=gen, device=dev)[:nblk].contiguous())
        dst_caches.append(torch.zeros((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev))
    torch.cuda.synchronize()

    stream_bytes = layout.stream_bytes
    cache_bytes = 2 * nblk * bs * H * C  # whole blocks written
    table_bytes = nblk * 8
    layer_bytes = stream_bytes + cache_bytes + table_bytes

    def restore_all():
        for layer in range(L):
            native_gpu.unpack_to_kv_cache(streams[layer], layout, T, dst_caches[layer],
                                          dst_ids[layer])

    # correctness check before timing, independent of the kernels: layer 0's
    # stream is the plane-major transpose of its source tokens and the
    # restored blocks hold those tokens (b = 8 planner layout)
    restore_all()
    torch.cuda.synchronize()
    if bits == 8 and not _closed_form_ok(streams[0], src_tokens0,
                                         dst_caches[0].view(torch.uint8), dst_ids[0], T, H, C):
        print("restore check failed: layer 0 differs from its source tokens", file=sys.stderr)
        return 1
    del src_tokens0

    for _ in range(args.warmup):
        restore_all()
    torch.cuda.synchronize()

    cur = torch.cuda.current_stream(dev)
    step_start = torch.cuda.Event(enable_timing=True)
    step_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    step_start.record(cur)
    for _ in range(args.steps):
        restore_all()
    step_end.record(cur)
    torch.cuda.synchronize()
    total_ms = step_start.elapsed_time(step_end)
    ms_per_step = total_ms / args.steps
    value = L * layer_bytes / (ms_per_step * 1e-3) / 1e9
    # the timed region is back-to-back launches of the restore kernel on one
    # stream: its average launch duration is the region over the launch count
    avg_launch_ms = total_ms / (args.steps * L)
    achieved = layer_bytes / (avg_launch_ms * 1e-3) / 1e9

    if args.profile_only:
        if args.profile_dequant:
            dequant_leg(src_cache, T, bs, torch.zeros_like(dst_caches[0]), dst_ids[0], gen, dev,
                        args.steps)
        calibration_copy(dev)
        print(json.dumps({"ms_per_step": ms_per_step, "value_gbps": value,
                          "avg_launch_us": avg_launch_ms * 1e3,
                          "calibration_copy_bytes": CAL_BYTES}), flush=True)
        return 0

    # --- pack throughput (fused gather + pack, the save direction) ---
    pack_out = [torch.empty_like(s) for s in streams]
    for _ in range(2):
        for layer in range(L):
            native_gpu.pack_from_kv_cache(dst_caches[layer], dst_ids[layer], T, layout,
                                          pack_out[layer])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    pack_steps = max(3, args.steps // 2)
    e0.record(cur)
    for _ in range(pack_steps):
        for layer in range(L):
            native_gpu.pack_from_kv_cache(dst_caches[layer], dst_ids[layer], T, layout,
                                          pack_out[layer])
    e1.record(cur)
    torch.cuda.synchronize()
    pack_ms = e0.elapsed_time(e1) / pack_steps
    pack_gbps = L * layer_bytes / (pack_ms * 1e-3) / 1e9
    pack_ok = all(torch.equal(a, b) for a, b in zip(pack_out, streams))

    # --- device copy ceiling in the same run (read + write bytes); 1 GiB
    # buffers so the 256 MB last-level cache cannot serve them ---
    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    e0.record(cur)
    for _ in range(20):
        b.copy_(a)
    e1.record(cur)
    torch.cuda.synchronize()
    copy_gbps = 2 * a.numel() * 20 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del a, b

    ceilings = same_pattern_leg(streams, layout, dst_caches, dst_ids, T, layer_bytes,
                                max(3, args.steps // 2))
    for c in dst_caches:  # back to the permuted-table restore for the legs below
        c.zero_()
    restore_all()

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": (f"{args.workload} KV geometry layer-wise restore: {L} layers x {T} tokens, "
                         f"{H} KV heads, head_dim {D}, bf16, block_size {bs}, permuted block "
                         f"table, 1 MiB chunks, bits {bits}; streams resident in HBM"),
            "layers": L, "tokens": T, "kv_heads": H, "head_dim": D, "block_size": bs,
            "bits": bits, "kv_dtype": "bf16", "chunks_per_layer": layout.num_chunks,
            "parallelism": "single GPU",
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "per_layer_restore_us": round(1e3 * ms_per_step / L, 2),
        "algorithmic_bytes_per_layer": layer_bytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": committed_traffic(args),
            "traffic_source": ("profiles/rows_unpack_llama3_8b_32k.txt: EA read/write requests "
                               "by size from rocprofv3 --pmc runs of bench.py --profile-only "
                               "(not measured in this run)"),
            "kernel": "rows_unpack_kernel<8, 2, false, false> (b = 8, 16-byte aligned runs)",
            "avg_launch_us": round(avg_launch_ms * 1e3, 2),
            # a copy of the same bytes with the restore's destination pattern
            # (whole blocks through the same permuted tables), this run
            "same_pattern_copy_gbps": ceilings["block_scatter"]["gbps"],
            "frac_of_same_pattern_copy": round(achieved / ceilings["block_scatter"]["gbps"], 4),
        },
        "ceilings": ceilings,
        "pack_gbps": round(pack_gbps, 2),
        "pack_ok": pack_ok,
        "d2d_copy_gbps": round(copy_gbps, 2),
    }

    if not args.no_pipeline:
        host = [torch.empty(layout.stream_bytes, dtype=torch.uint8, pin_memory=True)
                for _ in range(L)]
        for h, s_ in zip(host, streams):
            h.copy_(s_)
        result["pipeline"] = pipeline_leg(host, layout, T, dst_caches, dst_ids, dev,
                                          avg_launch_ms)
        del host
        result["pipeline_llama3_70b_128k"] = pipeline_70b_leg(dev)

    if not args.no_pack_ragged:
        result["pack_ragged"] = pack_ragged_leg(dev, max(3, args.steps // 2), H=H, D=D, bs=bs)
        # a ragged length whose staged pack takes single-owner tiles, in whole
        # rounds of tiles per CU as pack_ragged's 32753 tokens are (2 rounds)
        result["pack_ragged_single_owner"] = pack_ragged_leg(
            dev, max(3, args.steps // 2), T=30001, H=H, D=D, bs=bs)

    if not args.no_dequant:
        result["dequant"] = dequant_leg(src_cache, T, bs, torch.zeros_like(dst_caches[0]),
                                        dst_ids[0], gen, dev, args.steps)

    if not args.no_configs:
        result["configs"] = configs_leg(dev, max(3, args.steps // 2), args.config_layers)
        result["host_cost"] = host_cost_leg(dev)

    if not args.no_connector:
        result["connector"] = connector_leg(dev, args.connector_layers, T, H, D, bs)
        cb = connector_batch_leg(dev)
        qwen = result.get("configs", {}).get("qwen2.5-7b-batch")
        if qwen:
            cb["kernel_vs_configs_batched"] = round(
                cb["batched"]["kernel_us_per_layer"] / qwen["per_layer_us"], 4)
        result["connector_batch"] = cb

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(streams[0], layout, specs, T, H, C, bs, NB,
                                              dst_ids[0], dst_caches[0], layer_bytes,
                                              args.cpu_reps, dev)
    print(json.dumps(result), flush=True)
    return 0


def same_pattern_leg(streams, layout, dst_caches, dst_ids, T, layer_bytes, steps):
    """Copies of the workload's bytes with the restore's access patterns, in
    the same run, over the same layers and destination caches:

    * block_scatter: origami_scatter_kv_blocks (block_copy_kernel) of each
      layer's stream bytes taken as a token-major [2, T, H, C] value, read
      sequentially, into the layer's permuted destination blocks (each block
      written whole): the restore's destination pattern with sequential reads
      and no layout transform;
    * identity_table_restore: the restore kernel itself with block table
      0..nblk-1: the restore's plane-run reads, destination rows written in
      address order.

    Bytes per layer as for the restore.  The caches are left holding the
    identity-table restore (callers zero or rewrite them afterwards)."""
    import torch

    from origami_amd.lossless import native_gpu

    L = len(streams)
    dev = streams[0].device
    nblk = int(dst_ids[0].numel())
    ident = torch.arange(nblk, dtype=torch.int64, device=dev)

    def scatter_pass():
        for layer in range(L):
            native_gpu.scatter_kv_blocks(streams[layer], T, dst_caches[layer], dst_ids[layer])

    def ident_pass():
        for layer in range(L):
            native_gpu.unpack_to_kv_cache(streams[layer], layout, T, dst_caches[layer], ident)

    out = {}
    for name, fn, what in (
            ("block_scatter", scatter_pass,
             "block_copy_kernel: sequential reads, whole blocks written through the "
             "permuted tables"),
            ("identity_table_restore", ident_pass,
             "the restore kernel with block table 0..nblk-1 (rows written in address order)")):
        ms = _time_passes(fn, dev, steps) / L
        gbps = layer_bytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_layer": round(ms * 1e3, 2), "gbps": round(gbps, 2),
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "what": what}
    return out


def pack_ragged_leg(dev, steps, T=32753, layers=4, H=8, D=128, bs=16):
    """Fused save (block gather + pack) at a ragged length: `layers` layers of
    T tokens (odd, so runs start at any byte and the planes sit off 128-byte
    lines; the 8-bit pack then stages through LDS), bf16, permuted source
    tables, 1 MiB planner chunks, bits 8.  Bytes per layer: the stream, the
    gathered blocks and the table.  Layer 0 is checked in closed form: its
    stream is the plane-major transpose of its source tokens."""
    import torch

    from origami_amd.layout import kv_symbol_layout
    from origami_amd.lossless import native_gpu
    from origami_amd.lossless.chunking import plan_head_channel_chunks
    from origami_amd.synthetic import fill_layer

    C = 2 * D
    nblk = -(-T // bs)
    NB = nblk + nblk // 4
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    layout = kv_symbol_layout(T, H, C, 8, specs)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    caches, ids, outs = [], [], []
    for _ in range(layers):
        c = torch.empty((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev)
        i = torch.randperm(NB, generator=gen, device=dev)[:nblk].contiguous()
        fill_layer(c, i, gen)
        caches.append(c)
        ids.append(native_gpu.block_ids_tensor(i, dev, NB))
        outs.append(torch.empty(layout.stream_bytes, dtype=torch.uint8, device=dev))

    def one_pass():
        for c, i, o in zip(caches, ids, outs):
            native_gpu.pack_from_kv_cache(c, i, T, layout, o)

    for _ in range(2):
        one_pass()
    cur = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(cur)
    for _ in range(steps):
        one_pass()
    e1.record(cur)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    layer_bytes = layout.stream_bytes + 2 * nblk * bs * H * C + 8 * nblk
    src_tokens = caches[0].view(torch.uint8)[:, ids[0]].reshape(2, -1, H * C)[:, :T]
    ok = bool(torch.equal(outs[0].view(H * C, 2 * T), src_tokens.reshape(2 * T, H * C).t()))
    gbps = layers * layer_bytes / (ms * 1e-3) / 1e9
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    return {"tokens": T, "layers": layers, "us_per_layer": round(1e3 * ms / layers, 2),
            "algorithmic_bytes_per_layer": layer_bytes, "gbps": round(gbps, 2),
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "pack_ok": ok,
            "kernel": _staged_pack_kernel(T, H, C, cus)}


def _staged_pack_kernel(T, H, C, cus):
    """The staged pack kernel the library picks for T tokens of H heads x C
    bytes on `cus` CUs (the host rule in set_pack_grid, restated for the
    label): 16-wave tiles once they give half a tile per CU, single-owner
    tiles of 1920 tokens when those take no more rounds of tiles per CU."""
    cols = 2 * -(-H * C // 128)
    tiles16 = cols * -(-T // 2048)
    if tiles16 < max(1, cus // 2):
        return "rows_pack_staged8_kernel (8- or 4-wave tiles; 8-bit runs off 128-byte lines)"
    if -(-cols * -(-T // 1920) // cus) <= -(-tiles16 // cus):
        return ("rows_pack_staged8_kernel<16, false, true> (single-owner tiles: each stream "
                "line written by one tile)")
    return "rows_pack_staged8_kernel<16, false> (8-bit runs off 128-byte lines)"


def dequant_leg(src_cache, T, bs, dst_cache, dst_ids, gen, dev, steps, layers=4):
    """Fused dequantize-to-cache restores of one layer at the workload's
    geometry, from payloads the CacheGen and KIVI adapters produce for
    synthetic layers: CacheGen quant level 2 at layer 12 (16 bins, 4-bit K and
    V) and KIVI 2-bit, group 32, 128 sink tokens.  `layers` distinct layers
    (own K/V, payload and destination cache each; 4 x ~190 MB, past the
    256 MB MALL) are restored in turn, so no launch finds its inputs or
    outputs in the memory-side cache.  Algorithmic bytes per layer: the K and V
    symbol streams and the metadata the kernels read, the bf16 cache rows
    written, and the block table.  Each kernel is timed with events on the
    stream it is launched on, over `steps` passes of back-to-back launches."""
    import torch

    from origami_amd.quantization import create_quantizer_adapter

    from origami_amd.synthetic import fill_layer

    nblk = -(-T // bs)
    H, D = int(src_cache.shape[3]), int(src_cache.shape[4])
    out_bytes = 2 * T * H * D * 2
    kvs = []
    for _ in range(layers):
        ids = torch.randperm(src_cache.shape[1], generator=gen, device=dev)[:nblk].contiguous()
        fill_layer(src_cache, ids, gen)
        kvs.append(src_cache[:, ids].contiguous())
    dsts = [dst_cache] + [torch.zeros_like(dst_cache) for _ in range(layers - 1)]
    legs = {}
    for name, quantizer, cfg in (
            ("cachegen", "cachegen", {"quant_level": "2"}),
            ("kivi", "kivi", {"bits": 2, "group_size": 32, "sink_tokens": 128})):
        a = create_quantizer_adapter(quantizer, cfg)
        payloads = []
        for kv in kvs:
            q = a.quantize(kv, layer_group="model.layers.12.self_attn")
            payloads.append((q.symbols, q.metadata))
        m = payloads[0][1]
        if name == "cachegen":
            read = (m["key_stream_bytes"] + m["value_stream_bytes"]
                    + 2 * (m["key_max_numel"] + m["value_max_numel"]))
            kernel = "cachegen_cache_kernel<4, bf16, f16 max>"
        else:
            read = (m["key_stream_bytes"] + m["value_stream_bytes"]
                    + 2 * sum(m[f"{k}_numel"] for k in ("key_scale", "key_zero", "value_scale",
                                                        "value_zero", "key_sink", "value_sink")))
            kernel = "kivi_cache_kernel<2, nibble=false, bf16, f16 meta> (sink rows included)"
        alg = read + out_bytes + nblk * 8

        def run():
            for (blob, meta), dst in zip(payloads, dsts):
                a.dequantize_to_cache(blob, meta, dst, dst_ids, T)

        for _ in range(2):
            run()
        cur = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(cur)
        for _ in range(steps):
            run()
        e1.record(cur)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (steps * layers)
        gbps = alg / (ms * 1e-3) / 1e9
        legs[name] = {
            "kernel": kernel, "bits": [m.get("key_bits", m.get("bits")),
                                       m.get("value_bits", m.get("bits"))],
            "layers": layers,
            "per_layer_us": round(ms * 1e3, 2), "algorithmic_bytes_per_layer": int(alg),
            "gbps": round(gbps, 2), "frac": round(gbps / HBM_PEAK_GBPS, 4),
        }
        del payloads
    del kvs, dsts
    torch.cuda.empty_cache()
    legs["cachegen_dense"] = _cachegen_dense_leg(T, H, D, dev, steps, layers)
    return legs


def _cachegen_dense_leg(T, H, D, dev, steps, layers):
    """CacheGen unpack + dequantize into the float16 [layers, 2, H, T, D]
    tensor (cachegen_dense_kernel, one launch per K or V stream segment):
    `layers` layers at 4-bit keys and values, 16 bins, float16 per-token
    maxima.  The streams are zeros, so every value must come out as minus
    its token's maximum (symbol 0 dequantizes to (0 - c) / c * max, c = 7),
    which checks the output in closed form.  Algorithmic bytes: the streams,
    the maxima and the float16 output."""
    import torch

    from origami_amd.lossless import native_gpu

    seg = T * H * D * 4 // 8
    offs = torch.arange(2 * layers + 1, dtype=torch.int64) * seg
    stream = torch.zeros(2 * layers * seg, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    mk = (torch.rand(layers * T, generator=g, device=dev) * 2 + 0.1).half()
    mv = (torch.rand(layers * T, generator=g, device=dev) * 2 + 0.1).half()
    bits = torch.full((2 * layers,), 4, dtype=torch.int64)
    bins = torch.full((layers,), 16, dtype=torch.int64)

    def run():
        return native_gpu.cachegen_unpack_dequantize(stream, offs, bits, bins, bins, mk, mv,
                                                     tokens=T, heads=H, head_dim=D)

    out = run()
    ok = bool(torch.equal(out[:, 0], (-mk).view(layers, 1, T, 1).expand(-1, H, -1, D))
              and torch.equal(out[:, 1], (-mv).view(layers, 1, T, 1).expand(-1, H, -1, D)))
    del out
    run()
    cur = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(cur)
    for _ in range(steps):
        run()
    e1.record(cur)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (steps * layers)
    alg = 2 * seg + 2 * T * 2 + 2 * H * T * D * 2
    gbps = alg / (ms * 1e-3) / 1e9
    return {"kernel": "cachegen_dense_kernel<4> (float16 [L, 2, H, T, D] output)",
            "bits": [4, 4], "layers": layers, "per_layer_us": round(ms * 1e3, 2),
            "algorithmic_bytes_per_layer": int(alg), "gbps": round(gbps, 2),
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "output_ok": ok}


def host_cost_leg(dev, calls=200, reps=7, tokens=4096):
    """Host time per restore call: wall time of `calls` back-to-back calls
    of one 4096-token layer (8 KV heads, head_dim 128, bf16, bs 16, planner
    chunks of 1 MiB) from Python, through native_gpu.unpack_to_kv_cache (the
    full entry point: tensor checks, chunk metadata, plan lookup) and through
    a PreparedRestore made once for the request.  Each of `reps` loops is
    timed on the host from a synchronized start without waiting for the GPU;
    the median is reported (and the fastest loop); `gpu_us_per_call` (events
    over the same calls) shows the GPU was not what limited it."""
    import time

    import numpy as np
    import torch

    from origami_amd.lossless import native_gpu
    from origami_amd.synthetic import fill_layer

    H, D, bs = 8, 128, 16
    C = 2 * D
    nblk = -(-tokens // bs)
    layout = _planner_layout(tokens, H, C)
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    src = torch.zeros((2, nblk, bs, H, D), dtype=torch.bfloat16, device=dev)
    fill_layer(src, torch.arange(nblk, device=dev), gen)
    ids = torch.arange(nblk, device=dev, dtype=torch.int64)
    flat = native_gpu.pack_from_kv_cache(src, ids, tokens, layout)
    cache = torch.zeros_like(src)
    prep = native_gpu.PreparedRestore(layout, tokens, cache, ids)
    cur = torch.cuda.current_stream(dev)
    out = {"calls": calls, "reps": reps,
           "sample": f"one {tokens}-token layer, 8 KV heads, head_dim 128, bf16"}
    for name, fn in (("unpack_to_kv_cache", lambda: native_gpu.unpack_to_kv_cache(
                          flat, layout, tokens, cache, ids)),
                     ("prepared_restore", lambda: prep.restore(flat, cache))):
        for _ in range(50):
            fn()
        host, gpu = [], []
        for _ in range(reps):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cur)
            t0 = time.perf_counter()
            for _ in range(calls):
                fn()
            t1 = time.perf_counter()
            e1.record(cur)
            torch.cuda.synchronize()
            host.append((t1 - t0) * 1e6 / calls)
            gpu.append(e0.elapsed_time(e1) * 1e3 / calls)
        out[f"{name}_host_us"] = round(float(np.median(host)), 2)
        out[f"{name}_host_us_min"] = round(min(host), 2)
        out[f"{name}_gpu_us_per_call"] = round(float(np.median(gpu)), 2)
    ok = bool(torch.equal(cache.view(torch.uint8), src.view(torch.uint8)))
    out["restore_ok"] = ok
    prep.close()
    return out


def calibration_copy(dev):
    """A plain device copy of a known size (256 MiB read + 256 MiB written per
    launch, three launches) at the end of a profiling run: the memory
    counters of the same run must read these bytes for it."""
    import torch

    cal_a = torch.empty(CAL_BYTES, dtype=torch.uint8, device=dev)
    cal_b = torch.empty_like(cal_a)
    for _ in range(3):
        cal_b.copy_(cal_a)
    torch.cuda.synchronize()


def _planner_layout(T, H, C):
    from origami_amd.layout import kv_symbol_layout
    from origami_amd.lossless.chunking import plan_head_channel_chunks

    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    return kv_symbol_layout(T, H, C, 8, specs)


def _time_passes(one_pass, dev, steps):
    """ms per call of one_pass(), with events on the launch stream, after two
    warm-up calls."""
    import torch

    for _ in range(2):
        one_pass()
    cur = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(cur)
    for _ in range(steps):
        one_pass()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _closed_form_ok(stream, src_tokens, cache, ids, T, H, C):
    """Checks a b = 8 planner-layout restore without the kernels' own
    inverse: the stream is the plane-major transpose of the source tokens
    (plane h * C + c holds that channel's 2T symbols, K then V), and the
    restored blocks hold the source tokens, zeros past T.  `src_tokens` is
    uint8 [2, T, H * C]; `cache` a uint8 view of a [2, NB, bs, H, D] cache."""
    import torch

    sym = src_tokens.reshape(2 * T, H * C)
    if not torch.equal(stream.view(H * C, 2 * T), sym.t()):
        return False
    got = cache[:, ids].reshape(2, -1, H * C)
    return bool(torch.equal(got[:, :T], src_tokens)) and not bool(got[:, T:].any())


def configs_leg(dev, steps, layers, only=None, min_launches=200):
    """Restore throughput at the other KV geometries, `layers` layers each
    (every layer has its own paged cache and streams):

    * qwen2.5-7b-batch: 4 KV heads, head_dim 128, bf16, bs 16; 8 requests of
      U[8192, 65536] tokens (seed 2) whose first floor(T/2/bs) blocks come
      from a prefix pool shared by all block tables (the same destination
      blocks in every request).  One batched launch per layer; a shared
      prefix block is read and written once.  Bytes count what the job needs:
      each request's stream except its shared-prefix blocks past the first
      occurrence, each destination block once, the tables (`gbps`);
      `gbps_with_repeats` counts every request's full stream and blocks;
    * llama3-8b-fp8-16x16k: 8 KV heads, head_dim 128, float8_e4m3fn (128-byte
      head rows), 16 requests of 16384 tokens, one batched launch per layer;
    * llama3-70b-128k: 8 KV heads, head_dim 128, bf16, one 131072-token
      request per layer;
    * llama3-8b-4k: one 4096-token request, 8 KV heads, head_dim 128,
      bf16, block table 0..255 (a launch-bound size); 16 layers in rotation
      (537 MB of streams and caches), so no launch finds its layer in the
      256 MB MALL;
    * llama3-8b-32k-tp8-rank: one tensor-parallel rank's share of the
      32768-token Llama-3-8B layer at TP = 8: 1 KV head (256-byte rows),
      head_dim 128, bf16, 16 chunks of 1 MiB per layer; 16 layers, so the
      caches and streams (576 MiB) do not fit the 256 MB MALL.

    All use 1 MiB planner chunks and bits 8; the tables are permuted except
    for the 4096-token case.  For the batches, `per_request_us` times the
    same layers restored one launch per request.  Each geometry's last layer
    is checked in closed form (_closed_form_ok)."""
    import numpy as np
    import torch

    from origami_amd.lossless import native_gpu
    from origami_amd.synthetic import fill_layer

    bs = 16
    out = {}

    def build(name, H, D, dtype, lengths, seed, shared_pool, identity=False, nlayers=layers,
              batch=False):
        esize = torch.empty((), dtype=dtype).element_size()
        C = D * esize
        rng = np.random.default_rng(seed)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        lengths = [int(T) for T in lengths]
        nblks = [-(-T // bs) for T in lengths]
        pool = max(T // 2 // bs for T in lengths) if shared_pool else 0
        shared = [T // 2 // bs if shared_pool else 0 for T in lengths]
        NB = pool + sum(n - k for n, k in zip(nblks, shared)) + 64
        layouts = {T: _planner_layout(T, H, C) for T in set(lengths)}
        src = torch.zeros((2, NB, bs, H, D), dtype=dtype, device=dev)
        layers_items, alg_unique, alg_repeats, ok = [], 0, 0, True
        batches = []

        def tables():
            perm = np.arange(NB) if identity else rng.permutation(NB)
            cur, ts = pool, []
            for n, k in zip(nblks, shared):
                ts.append(np.concatenate([perm[:k], perm[cur:cur + n - k]]).astype(np.int64))
                cur += n - k
            return ts

        for layer in range(nlayers):
            fill_layer(src, torch.arange(NB, device=dev), gen)
            src_tables, dst_tables = tables(), tables()
            cache = torch.zeros((2, NB, bs, H, D), dtype=dtype, device=dev)
            reqs = []
            for T, st, dt in zip(lengths, src_tables, dst_tables):
                stream = native_gpu.pack_from_kv_cache(
                    src, native_gpu.block_ids_tensor(st, dev, NB), T, layouts[T])
                reqs.append((stream, layouts[T], T, dt))
            rb = native_gpu.KVRestoreBatch([r[1] for r in reqs], lengths,
                                           [r[3] for r in reqs], cache,
                                           dedup_shared_blocks=shared_pool)
            batches.append(rb)
            ids_dev = [native_gpu.block_ids_tensor(dt, dev, NB) for dt in dst_tables]
            layers_items.append((reqs, cache, ids_dev))
            stream_bytes = sum(r[1].stream_bytes for r in reqs)
            table_bytes = 8 * sum(r[3].size for r in reqs)
            written = len(np.unique(np.concatenate(dst_tables)))
            # a skipped (shared) block is neither read nor written again
            skipped_read = rb.skipped_blocks * 2 * bs * H * C
            alg_unique += stream_bytes - skipped_read + 2 * written * bs * H * C + table_bytes
            alg_repeats += stream_bytes + 2 * sum(nblks) * bs * H * C + table_bytes
            if layer == nlayers - 1:
                # closed-form check of this layer (restored once up front)
                if batch:
                    rb.restore([r[0] for r in reqs], cache)
                else:
                    for (stream, lay, T, _), ids in zip(reqs, ids_dev):
                        native_gpu.unpack_to_kv_cache(stream, lay, T, cache, ids)
                cu8 = cache.view(torch.uint8)
                su8 = src.view(torch.uint8)
                for (stream, lay, T, dt), st in zip(reqs, src_tables):
                    tok = su8[:, torch.from_numpy(st).to(dev)].reshape(2, -1, H * C)[:, :T]
                    ok = ok and _closed_form_ok(stream, tok.contiguous(), cu8,
                                                torch.from_numpy(dt).to(dev), T, H, C)
        del src

        def batched_pass():
            for rb, (reqs, cache, _) in zip(batches, layers_items):
                rb.restore([r[0] for r in reqs], cache)

        def per_request_pass():
            for reqs, cache, ids_dev in layers_items:
                for (stream, lay, T, _), ids in zip(reqs, ids_dev):
                    native_gpu.unpack_to_kv_cache(stream, lay, T, cache, ids)

        # at least ~min_launches launches per timing, so short layers reach
        # steady state
        passes = max(steps, -(-min_launches // (nlayers * (1 if batch else len(lengths)))))
        ms = _time_passes(batched_pass if batch else per_request_pass, dev, passes)
        res = {
            "layers": nlayers, "requests_per_layer": len(lengths),
            "tokens_per_layer": int(sum(lengths)),
            "kv_heads": H, "head_dim": D, "kv_dtype": str(dtype).replace("torch.", ""),
            "launch": ("one batched launch per layer" if batch
                       else "one launch per request and layer"),
            "per_layer_us": round(1e3 * ms / nlayers, 2),
            "algorithmic_bytes_per_layer": int(alg_unique // nlayers),
            "gbps": round(alg_unique / (ms * 1e-3) / 1e9, 2),
            "frac": round(alg_unique / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "restore_ok": bool(ok),
        }
        if batch:
            ms_req = _time_passes(per_request_pass, dev, passes)
            res["per_request_us"] = round(1e3 * ms_req / nlayers, 2)
        elif name in SHORT_CONFIGS:
            # a device copy of the same bytes (each layer's stream into a
            # buffer of its size), rotating over the same number of layers:
            # what one launch of this size reaches at all
            bufs = [torch.empty_like(reqs[0][0]) for reqs, _, _ in layers_items]

            def copy_pass():
                for (reqs, _, _), b in zip(layers_items, bufs):
                    b.copy_(reqs[0][0])

            ms_copy = _time_passes(copy_pass, dev, passes)
            copy_bytes = 2 * layers_items[0][0][0][0].numel()
            res["same_size_copy_us"] = round(1e3 * ms_copy / nlayers, 2)
            res["same_size_copy_frac"] = round(
                copy_bytes / (ms_copy / nlayers * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
            del bufs
        if shared_pool:
            res["gbps_with_repeats"] = round(alg_repeats / (ms * 1e-3) / 1e9, 2)
            res["algorithmic_bytes_per_layer_with_repeats"] = int(alg_repeats // nlayers)
            res["shared_blocks_skipped_per_layer"] = int(batches[0].skipped_blocks)
        out[name] = res
        del layers_items, batches
        torch.cuda.empty_cache()

    geometries = {
        "llama3-8b-4k": lambda: build("llama3-8b-4k", 8, 128, torch.bfloat16, [4096], 0, False,
                                      identity=True, nlayers=max(layers, 16)),
        "qwen2.5-7b-batch": lambda: build(
            "qwen2.5-7b-batch", 4, 128, torch.bfloat16,
            np.random.default_rng(2).integers(8192, 65537, 8), 2, True, batch=True),
        "llama3-8b-fp8-16x16k": lambda: build("llama3-8b-fp8-16x16k", 8, 128,
                                              torch.float8_e4m3fn, [16384] * 16, 3, False,
                                              batch=True),
        "llama3-70b-128k": lambda: build("llama3-70b-128k", 8, 128, torch.bfloat16, [131072], 4,
                                         False),
        "llama3-8b-32k-tp8-rank": lambda: build("llama3-8b-32k-tp8-rank", 1, 128, torch.bfloat16,
                                                [32768], 1, False, nlayers=max(layers, 16)),
    }
    for name in CONFIG_NAMES:
        if only is None or only == name:
            geometries[name]()
    return out


def connector_leg(dev, layers, T, H, D, bs):
    """Save and restore `layers` layers of one T-token request end to end
    through the connector (OrigamiConnector, worker role): raw_byte_planes
    symbols, 1 MiB chunks, the zlib CPU codec on 16 threads, the in-memory
    store.  Save: save_kv_layer for every layer, then wait_for_save (fused
    gather + pack, device-to-host, compression).  Restore: start_load_kv,
    then wait_for_layer_load for every layer (decompression into pinned
    staging, host-to-device, fused unpack + scatter), to the last layer's
    completion.  Rates are KV bytes (2 * T * H * D * 2 per layer) per second;
    the restored caches are compared with the saved ones."""
    import types

    import torch

    from origami_amd.connector import KVConnectorRole, OrigamiConnector
    from origami_amd.metadata import (OrigamiConnectorMetadata, OrigamiRestoreRequest,
                                      OrigamiSaveRequest)
    from origami_amd.synthetic import fill_layer

    def connector(ns):
        cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
            kv_connector_extra_config={
                "origami_quantizer": "raw_byte_planes", "origami_lossless_cpu_backend": "zlib",
                "origami_store_uri": f"memory://{ns}", "origami_qat_threads": 16}))
        return OrigamiConnector(cfg, KVConnectorRole.WORKER)

    nblk = -(-T // bs)
    NB = nblk + nblk // 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    names = [f"model.layers.{i}.self_attn.attn" for i in range(layers)]
    src, dst = {}, {}
    for n in names:
        src[n] = torch.zeros((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev)
        fill_layer(src[n], torch.arange(NB, device=dev), gen)
        dst[n] = torch.zeros_like(src[n])
    src_ids = torch.randperm(NB, generator=gen, device=dev)[:nblk].tolist()
    dst_ids = torch.randperm(NB, generator=gen, device=dev)[:nblk].tolist()
    kv_bytes = layers * 2 * T * H * D * 2

    saver = connector("bench-connector")
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        "s": OrigamiSaveRequest(request_id="s", cache_key="bench", block_ids_per_group=(
            tuple(src_ids),), num_tokens=T)}))
    saver.start_load_kv(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()
    save_s = time.perf_counter() - t0
    payload = saver.store.get("bench")
    stored = sum(int(c.compressed.numel()) for lp in payload.layer_payloads.values()
                 for c in lp.chunks)

    loader = connector("bench-connector")  # same in-memory store namespace
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        "r": OrigamiRestoreRequest(request_id="r", cache_key="bench", block_ids_per_group=(
            tuple(dst_ids),), num_tokens=T)}))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    loader.start_load_kv(None)
    for n in names:
        loader.wait_for_layer_load(n)
    torch.cuda.synchronize()
    restore_s = time.perf_counter() - t0
    ok = all(torch.equal(dst[n][:, dst_ids].view(torch.int16), src[n][:, src_ids].view(torch.int16))
             for n in names[:2])
    return {
        "layers": layers, "tokens": T, "codec": "zlib level 1, 16 threads",
        "kv_bytes": kv_bytes, "stored_bytes": stored,
        "save_ms": round(save_s * 1e3, 2), "save_gbps": round(kv_bytes / save_s / 1e9, 3),
        "restore_ms": round(restore_s * 1e3, 2),
        "restore_gbps": round(kv_bytes / restore_s / 1e9, 3),
        "restore_ok": ok,
    }


def connector_batch_leg(dev, layers=4):
    """The Qwen2.5-7B batch (4 KV heads, head_dim 128, bf16, bs 16; 8
    requests of default_rng(2).integers(8192, 65537, 8) tokens saved as whole
    blocks, each table's first half from a shared prefix pool) restored
    through the connector's drop-in surface: one start_load_kv for the 8
    requests, wait_for_layer_load for each of `layers` layers.  The CPU codec
    is "raw" (a copy), so decompression does not hide the device work.  The
    kernel time per layer is what the worker's own event-timed metric rows
    (bitunpack_cuda) record for the restore launches of the layer, summed
    over its launches; `batched` restores each layer of the batch with one
    H2D and one launch, `per_request` with origami_batch_restores off (one
    launch per request and layer, as the reference's per-request threads).
    Each restored cache is checked against the saved source blocks."""
    import json as _json
    import tempfile
    import types

    import numpy as np
    import torch

    from origami_amd.connector import KVConnectorRole, OrigamiConnector
    from origami_amd.metadata import (OrigamiConnectorMetadata, OrigamiRestoreRequest,
                                      OrigamiSaveRequest)
    from origami_amd.synthetic import fill_layer

    H, D, bs = 4, 128, 16
    lengths = [int(T) for T in np.random.default_rng(2).integers(8192, 65537, 8)]
    nblks = [-(-T // bs) for T in lengths]
    shared = [T // 2 // bs for T in lengths]
    pool = max(shared)
    NB = pool + sum(n - k for n, k in zip(nblks, shared)) + 64
    rng = np.random.default_rng(2)

    def tables():
        perm = rng.permutation(NB)
        cur, ts = pool, []
        for n, k in zip(nblks, shared):
            ts.append([int(b) for b in np.concatenate([perm[:k], perm[cur:cur + n - k]])])
            cur += n - k
        return ts

    names = [f"model.layers.{i}.self_attn.attn" for i in range(layers)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    src = {}
    for n in names:
        src[n] = torch.zeros((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev)
        fill_layer(src[n], torch.arange(NB, device=dev), gen)
    src_t, dst_t = tables(), tables()
    mdir = tempfile.mkdtemp(prefix="origami-bench-")

    def connector(ns, batch, metrics=""):
        cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
            kv_connector_extra_config={
                "origami_quantizer": "raw_byte_planes", "origami_lossless_cpu_backend": "raw",
                "origami_store_uri": f"memory://{ns}", "origami_qat_threads": 16,
                "origami_metrics_dir": metrics, "origami_batch_restores": batch}))
        return OrigamiConnector(cfg, KVConnectorRole.WORKER)

    saver = connector("bench-batch", True)
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        f"s{i}": OrigamiSaveRequest(request_id=f"s{i}", cache_key=f"q{i}",
                                    block_ids_per_group=(tuple(t),), num_tokens=len(t) * bs)
        for i, t in enumerate(src_t)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()
    del saver

    out = {"layers": layers, "requests": len(lengths), "tokens": sum(lengths),
           "codec": "raw (copy)", "kv_heads": H, "head_dim": D}
    dst = {n: torch.zeros_like(src[n]) for n in names}
    reqs = {f"r{i}": OrigamiRestoreRequest(request_id=f"r{i}", cache_key=f"q{i}",
                                           block_ids_per_group=(tuple(t),),
                                           num_tokens=len(t) * bs)
            for i, t in enumerate(dst_t)}
    for label, batch in (("batched", True), ("per_request", False)):
        metrics = f"{mdir}/{label}"
        loader = connector("bench-batch", batch, metrics)
        loader.register_kv_caches(dst)
        worker = loader.connector_worker
        seen, res = 0, {}
        # the first pass builds the pipeline and its pinned staging; the
        # second is reported
        for _ in range(2):
            for n in names:
                dst[n].zero_()
            loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore=reqs))
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            loader.start_load_kv(None)
            for n in names:
                loader.wait_for_layer_load(n)
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            worker.flush_metrics()
            lines = open(f"{metrics}/origami_metrics.jsonl").read().splitlines()
            rows = [_json.loads(x) for x in lines[seen:]]
            seen = len(lines)
            per_layer = {}
            for r in rows:
                if r.get("type") == "bitunpack_cuda":
                    per_layer[r["layer_name"]] = per_layer.get(r["layer_name"], 0.0) + r["ms"]
            ok = all(torch.equal(dst[n][:, d].view(torch.int16), src[n][:, s_].view(torch.int16))
                     for n in names for s_, d in zip(src_t, dst_t))
            res = {"kernel_us_per_layer": round(1e3 * float(np.median(list(per_layer.values()))),
                                                 2),
                   "restore_wall_ms": round(wall * 1e3, 2), "restore_ok": bool(ok),
                   "launches_per_layer": sum(1 for r in rows if r.get("type") == "bitunpack_cuda")
                   // max(1, len(per_layer))}
        worker.shutdown()
        out[label] = res
    del src, dst
    torch.cuda.empty_cache()
    return out


def pipeline_leg(host, layout, T, dst_caches, dst_ids, dev, kernel_ms, layers=None):
    """Layer-wise restore from pinned host memory with the copy of layer L+1
    overlapped with the unpack+scatter of layer L, against the H2D copies
    alone.  "exposed" is the time the restore adds on top of the copies.
    Layer i reads host[i % len(host)] and restores into dst_caches[i % ...]
    through dst_ids[i % ...] (a ring, so a long model needs only a few
    buffers).  restore_ok: the last layer's cache equals a direct restore of
    its stream."""
    import torch

    from origami_amd.lossless import native_gpu
    from origami_amd.restore_pipeline import LayerRestorePipeline

    L = layers or len(host)
    nbytes = layout.stream_bytes
    last = (L - 1) % len(dst_caches)
    expect = torch.zeros_like(dst_caches[last])
    native_gpu.unpack_to_kv_cache(host[(L - 1) % len(host)].to(dev), layout, T, expect,
                                  dst_ids[last])
    for c in dst_caches:
        c.zero_()
    pipe = LayerRestorePipeline(dev, nbytes, num_lanes=2, host_staging=False)
    cur = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()

    def run(submit_layer):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(cur)
        pipe.begin(cur)
        for layer in range(L):
            submit_layer(layer)
        pipe.join(cur)
        end.record(cur)
        torch.cuda.synchronize()
        return start.elapsed_time(end)

    def copies_only():
        return run(lambda layer: pipe.copy_only(host[layer % len(host)], nbytes))

    def pipelined(compute=True):
        def one(layer):
            h = host[layer % len(host)]
            if compute:
                k = layer % len(dst_caches)
                pipe.restore_pinned(h, layout, T, dst_caches[k], dst_ids[k])
            else:
                pipe.submit(h, nbytes, lambda flat: None)
        return run(one)

    reps = 3
    copies_only()
    pipelined()
    pipelined(False)
    h2d = min(copies_only() for _ in range(reps))
    full = min(pipelined() for _ in range(reps))
    handoff = min(pipelined(False) for _ in range(reps))
    ok = bool(torch.equal(dst_caches[last], expect))
    return {
        "layers": L,
        "h2d_ms": round(h2d, 3),
        "h2d_gbps": round(L * nbytes / (h2d * 1e-3) / 1e9, 2),
        "pipelined_restore_ms": round(full, 3),
        # the same lanes with no restore: the lanes' copies overlap each
        # other, so this can come in under h2d_ms
        "pipelined_no_compute_ms": round(handoff, 3),
        # what the restore adds over the bare copies
        "exposed_ms": round(full - h2d, 3),
        "restore_compute_ms": round(L * kernel_ms, 3),
        # the share of the restore kernels' time the copies hide
        "restore_hidden_fraction": round(max(0.0, 1.0 - max(0.0, full - h2d) / (L * kernel_ms)),
                                         4),
        # hidden: the whole pipeline takes at most the bare copies plus two
        # unpacks (the trailing one and one of slack)
        "restore_hidden": bool(full - h2d <= 2 * kernel_ms),
        "restore_ok": ok,
        "source": (f"pinned host memory ({len(host)} buffers of {nbytes} B), 2 lanes (a stream "
                   "and a device slot each: H2D then restore)"),
    }


def pipeline_70b_leg(dev):
    """The Llama-3-70B geometry restored layer-wise from pinned host memory:
    80 layers of one 131072-token request (8 KV heads, head_dim 128, bf16,
    block size 16, 512 chunks of 1 MiB, permuted tables, seed 4), 512 MiB of
    stream per layer.  Four distinct streams and caches form the ring (2 GiB
    pinned, 2.5 GiB of caches), so the 40 GiB model needs no 40 GiB of host
    memory."""
    import torch

    from origami_amd.lossless import native_gpu
    from origami_amd.synthetic import fill_layer

    T, H, D, bs, L, ring = 131072, 8, 128, 16, 80, 4
    C = 2 * D
    nblk = T // bs
    NB = nblk + nblk // 4
    layout = _planner_layout(T, H, C)
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    src = torch.empty((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev)
    host, caches, ids = [], [], []
    for _ in range(ring):
        sid = torch.randperm(NB, generator=gen, device=dev)[:nblk].contiguous()
        fill_layer(src, sid, gen)
        h = torch.empty(layout.stream_bytes, dtype=torch.uint8, pin_memory=True)
        h.copy_(native_gpu.pack_from_kv_cache(src, sid, T, layout))
        host.append(h)
        caches.append(torch.zeros((2, NB, bs, H, D), dtype=torch.bfloat16, device=dev))
        ids.append(torch.randperm(NB, generator=gen, device=dev)[:nblk].contiguous())
    del src
    flat = host[0].to(dev)
    kernel_ms = _time_passes(
        lambda: native_gpu.unpack_to_kv_cache(flat, layout, T, caches[0], ids[0]), dev, 8)
    del flat
    torch.cuda.empty_cache()
    res = pipeline_leg(host, layout, T, caches, ids, dev, kernel_ms, layers=L)
    res["per_layer_restore_us"] = round(kernel_ms * 1e3, 2)
    del host, caches
    torch.cuda.empty_cache()
    return res


TRAFFIC_FILE = REPO / "profiles" / "rows_unpack_llama3_8b_32k.txt"


def committed_traffic(args):
    """HBM bytes per launch of the restore kernel from the committed PMC
    summary (size-resolved EA read and write requests of separate rocprofv3
    --pmc runs, not of this run), for the default workload."""
    default = (args.layers, args.tokens, args.heads, args.head_dim, args.block_size,
               args.bits) == (32, 32768, 8, 128, 16, 8)
    if not default or not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch rows_unpack_kernel<8, 2, false, false>:"):
            return int(line.split(":")[1].split()[0])
    return None


def _host_cpu_model() -> str:
    cpu_model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu_model


def _time_oracle_restore(flat, layout, specs, T, H, C, ids_np, cache, threads, warmup, reps):
    """Median seconds of the oracle's one-layer restore on `threads` host threads."""
    import numpy as np

    from oracle import oracle

    oracle.set_threads(threads)
    times = []
    for i in range(warmup + reps):
        t0 = time.perf_counter()
        oracle.restore_layer(flat, layout.offsets, layout.bits, specs, T, H, C, ids_np, cache)
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    return float(np.median(times))


def _time_index_copy(value, ids, cache, threads, warmup, reps):
    """Median seconds of torch's CPU index_copy_ of whole blocks along the
    block dimension (the scatter of the reference's raw-bytes restore path,
    benchmark_utils.py:434-444), on `threads` intra-op threads."""
    import numpy as np
    import torch

    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        times = []
        for i in range(warmup + reps):
            t0 = time.perf_counter()
            cache.index_copy_(1, ids, value)
            if i >= warmup:
                times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(saved)
    return float(np.median(times))


def _leg(name, layer_bytes, seconds, threads, warmup, reps, sample, **extra):
    return {"name": name, "value": round(layer_bytes / seconds / 1e9, 3), "unit": "GB/s",
            "ms_per_layer": round(seconds * 1e3, 2), "cores": threads, "warmup": warmup,
            "reps": reps, "sample": sample, **extra}


def cpu_baseline(stream, layout, specs, T, H, C, bs, NB, ids, restored_cache, layer_bytes,
                 reps, dev):
    """Host-core baselines for the restore of one layer.

    The headline (`value`) is the oracle's restore (unpack + paged scatter)
    of one layer of the workload on all host threads (at most 16).  `legs`
    adds the same restore on one thread, the 4096-token single-layer case
    (block table 0..255) on all threads and on one thread, and the scatter
    alone as the reference ships it for raw-byte payloads (torch CPU
    index_copy_ of whole blocks, no layout transform) at the workload's
    size.  Every oracle leg is checked against the GPU restore of the same
    stream."""
    import numpy as np
    import torch

    from origami_amd.layout import kv_symbol_layout
    from origami_amd.lossless import native_gpu
    from origami_amd.lossless.chunking import plan_head_channel_chunks
    from origami_amd.synthetic import fill_layer

    threads = min(16, os.cpu_count() or 1)
    flat = stream.cpu().numpy()
    ids_np = ids.cpu().numpy().astype(np.int64)
    gpu_cache = restored_cache.view(torch_u8()).cpu().numpy()
    cache = np.zeros((2, NB, bs, H, C), dtype=np.uint8)
    warm = 3
    med = _time_oracle_restore(flat, layout, specs, T, H, C, ids_np, cache, threads, warm, reps)
    ok = bool(np.array_equal(cache, gpu_cache))
    legs = [_leg("oracle restore, workload layer", layer_bytes, med, threads, warm, reps,
                 f"one {T}-token layer", matches_gpu=ok)]
    single_reps = 3
    cache[:] = 0
    med1 = _time_oracle_restore(flat, layout, specs, T, H, C, ids_np, cache, 1, 1, single_reps)
    legs.append(_leg("oracle restore, workload layer", layer_bytes, med1, 1, 1, single_reps,
                     f"one {T}-token layer", matches_gpu=bool(np.array_equal(cache, gpu_cache))))

    # the scatter alone, as shipped for raw-byte payloads
    nblk = ids_np.size
    value = torch.from_numpy(np.resize(flat, 2 * nblk * bs * H * C)).reshape(2, nblk, bs, H, C)
    tcache = torch.zeros((2, NB, bs, H, C), dtype=torch.uint8)
    tids = torch.from_numpy(ids_np)
    for th in (threads, 1):
        sec = _time_index_copy(value, tids, tcache, th, 3, 10)
        legs.append(_leg("raw-bytes scatter (index_copy_), workload layer", layer_bytes, sec, th,
                         3, 10, f"one {T}-token layer of whole blocks, no layout transform"))
    del value, tcache

    # the 4096-token single-layer case: block table 0..255, seed 0
    T1, bs1 = 4096, bs
    nblk1 = T1 // bs1
    plan1 = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T1,
                                     bytes_per_symbol=1, min_bytes=1 << 20, target_bytes=1 << 20,
                                     max_bytes=1 << 20)
    specs1 = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
               c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan1]
    layout1 = kv_symbol_layout(T1, H, C, 8, specs1)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    ids1 = torch.arange(nblk1, dtype=torch.int64, device=dev)
    src1 = torch.zeros((2, nblk1, bs1, H, C // 2), dtype=torch.bfloat16, device=dev)
    fill_layer(src1, ids1, gen)
    stream1 = native_gpu.pack_from_kv_cache(src1, ids1, T1, layout1)
    dst1 = torch.zeros_like(src1)
    native_gpu.unpack_to_kv_cache(stream1, layout1, T1, dst1, ids1)
    gpu1 = dst1.view(torch_u8()).cpu().numpy()
    flat1 = stream1.cpu().numpy()
    bytes1 = layout1.stream_bytes + 2 * nblk1 * bs1 * H * C + nblk1 * 8
    cache1 = np.zeros((2, nblk1, bs1, H, C), dtype=np.uint8)
    for th in (threads, 1):
        cache1[:] = 0
        sec = _time_oracle_restore(flat1, layout1, specs1, T1, H, C, ids1.cpu().numpy(), cache1,
                                   th, 3, 10)
        legs.append(_leg("oracle restore, 4096-token layer", bytes1, sec, th, 3, 10,
                         "one 4096-token layer, 8 heads, head_dim 128, bf16, block table 0..255",
                         matches_gpu=bool(np.array_equal(cache1, gpu1))))

    # context: the CPU codec (zlib level 1, raw deflate) over the 4096-token
    # layer's chunks, one thread
    from origami_amd.lossless.cpu_qat import CpuLosslessCodec

    codec = CpuLosslessCodec(backend="zlib")
    chunks = [stream1[int(a):int(b)].cpu() for a, b in zip(layout1.offsets[:-1],
                                                           layout1.offsets[1:])]
    t0 = time.perf_counter()
    comp = codec.compress_many(chunks)
    t_comp = time.perf_counter() - t0
    t0 = time.perf_counter()
    back = codec.decompress_many(comp, [c.numel() for c in chunks])
    t_dec = time.perf_counter() - t0
    zok = all(bool(torch.equal(a, b)) for a, b in zip(back, chunks))
    legs.append({"name": "zlib level 1 (context), 4096-token layer stream",
                 "compress_ms": round(t_comp * 1e3, 2), "decompress_ms": round(t_dec * 1e3, 2),
                 "ratio": round(layout1.stream_bytes / sum(c.numel() for c in comp), 3),
                 "round_trip_ok": zok, "sample": f"{len(chunks)} chunks of 1 MiB"})

    return {
        "value": legs[0]["value"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"one layer of the workload ({T} tokens, {layer_bytes} algorithmic bytes): "
                   f"unpack + paged scatter, OpenMP over chunks/blocks, {warm} warm-ups, "
                   f"median of {reps}"),
        "ms_per_layer": legs[0]["ms_per_layer"],
        "cpu_model": _host_cpu_model(),
        "host_cpus": os.cpu_count(),
        "cpus_usable": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
        "matches_gpu": all(leg.get("matches_gpu", True) for leg in legs),
        "legs": legs,
    }


def torch_u8():
    import torch

    return torch.uint8


if __name__ == "__main__":
    sys.exit(main())
