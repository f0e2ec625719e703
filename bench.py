"""Benchmark of the MI355X paged-KV data plane (one GPU).

Headline: paged decode attention over 28 layers at batch 256, lognormal contexts (median
2048, sigma 1.3, clipped to [256, 8192], about 90 GB of K/V resident in HBM).  One step =
for each of the 28 layers: append the new token's K/V into its slot (kernel 1, decode form)
and run paged GQA decode attention over the whole context (kernel 3).  ``value`` is the
algorithmic HBM bandwidth of the whole step: per layer sum(context) x 4096 B of K/V read,
plus Q read, O written and the appended K/V rows, divided by the timed step time.

Also measured in the same run (reported under ``kernels``): the 28-layer prefill scatter of
32 prompts U[128, 2048] and the block-table history gather, each on fragmented block tables (a
free list reordered by decode-style interleaved growth) and on near-sequential ones, the MFMA
chunked-prefill attention of 4 x 16384-token prompts in 2048-token chunks, and the KV block
records of 2048 blocks (pack / unpack in HBM, swap to pinned host memory and back); and (under ``e2e``)
the continuous-batching run of a random-init Qwen3-0.6B: 128 requests at 20 req/s, prompts
U[32, 1024], 128 output tokens, chunked prefill with a 2048-token budget (with mixed batching also
once with at most 1024 prompt tokens per mixed step).  The CPU baseline times the reference's torch
decode chain (the oracle) on the host cores on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only decode]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor datasheet
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
MFMA_FP64_PEAK_TFLOPS = 78.6    # MI355X dense fp64 matrix peak
MIXED_CHUNK_CAP = 1024  # prompt tokens per mixed step in the capped mixed-batching run
PCIE_PEAK_GBS = 64.0  # MI355X host link, PCIe 5.0 x16, one direction
METRIC = "paged decode-attn HBM GB/s (% peak) at B=256; e2e output tok/s Qwen3-0.6B"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
CALIB_LIBRARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mini_infra_qwen3_amd", "libmi_calib.so")
TRAFFIC_SOURCE = ("profiles/hbm_traffic.md: rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE (KiB per dispatch) of "
                  "this bench's single-kernel legs, scaled by the same counters over a copy of known size "
                  "(FETCH_SIZE x2.0, WRITE_SIZE x1.0)")


def profiled_traffic(kernel: str) -> int | None:
    """HBM bytes per launch of ``kernel`` from the committed counter summary (profiles/hbm_traffic.md,
    lines ``traffic <kernel> <bytes>``: rocprofv3 FETCH_SIZE and WRITE_SIZE per dispatch, scaled by
    the same counters' reading for a copy of known size); None if absent."""
    try:
        with open(os.path.join(PROFILES, "hbm_traffic.md")) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


class EventTimer:
    """HIP events on the current stream (the one every data-plane kernel is launched on)."""

    def __init__(self):
        self.pairs: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []

    def start(self):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.append((e, None))

    def stop(self):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs[-1] = (self.pairs[-1][0], e)

    def mean_ms(self) -> float:
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in self.pairs) / max(len(self.pairs), 1)


# --------------------------------------------------------------------------- decode (headline)
def bench_decode(steps: int, warmup: int, device: torch.device):
    from mini_infra_qwen3_amd import data_plane, workloads as wl

    t0 = time.perf_counter()
    w = wl.decode_at_scale(seed=0, device=device)
    torch.cuda.synchronize()
    log(f"decode workload ready in {time.perf_counter() - t0:.1f}s: batch {len(w.context_lens)}, "
        f"sum(ctx)={sum(w.context_lens)}, pool {w.num_blocks} blocks x 28 layers "
        f"({w.pools.numel() * 2 / 1e9:.1f} GB)")
    batch = len(w.context_lens)
    block_tables = w.block_tables.to(device)
    context_lens = torch.tensor(w.context_lens, dtype=torch.long, device=device)
    slots = w.slot_mapping.to(device)
    out = torch.empty((batch, wl.NUM_HEADS * wl.HEAD_DIM), dtype=torch.bfloat16, device=device)
    ws_bytes = data_plane.paged_decode_workspace_bytes(batch, block_tables.shape[1], wl.NUM_HEADS,
                                                       wl.HEAD_DIM, wl.BLOCK_SIZE, wl.NUM_KV_HEADS)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    keys = [w.pools[l, 0] for l in range(w.num_layers)]
    values = [w.pools[l, 1] for l in range(w.num_layers)]
    new_k = [w.new_key[l].unsqueeze(2) for l in range(w.num_layers)]
    new_v = [w.new_value[l].unsqueeze(2) for l in range(w.num_layers)]
    attn_timer = EventTimer()

    def step(timed: bool):
        for layer in range(w.num_layers):
            data_plane.reshape_and_cache([new_k[layer]], [new_v[layer]], slots, [keys[layer]], [values[layer]])
            if timed:
                attn_timer.start()
            data_plane.paged_decode_attention(w.query[layer], keys[layer], values[layer], block_tables,
                                              context_lens, wl.SCALE, out=out, workspace=workspace)
            if timed:
                attn_timer.stop()

    for _ in range(warmup):
        step(False)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = elapsed * 1000.0 / steps

    q_o_bytes = 2 * batch * wl.NUM_HEADS * wl.HEAD_DIM * 2
    append_bytes = 2 * batch * wl.KV_BYTES_PER_TOKEN_LAYER  # read + write of the new K/V rows
    attn_bytes_per_launch = w.kv_bytes_per_layer + q_o_bytes
    step_bytes = w.num_layers * (attn_bytes_per_launch + append_bytes)
    attn_ms = attn_timer.mean_ms()
    achieved = attn_bytes_per_launch / (attn_ms * 1e-3) / 1e9
    result = {
        "ms_per_step": ms_per_step,
        "value": step_bytes / (ms_per_step * 1e-3) / 1e9,
        "attn_launch_ms": attn_ms,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic("paged_decode_attention"),
            "traffic_source": TRAFFIC_SOURCE,
            "algorithmic_bytes_per_launch": attn_bytes_per_launch,
        },
        "workload": w,
    }
    # Spot-check the timed output of the last layer against its own inputs: finite values.
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("decode attention produced non-finite values")
    return result


def cpu_baseline_decode(w, device: torch.device, budget_s: float = 20.0) -> dict:
    """The reference's torch decode chain (oracle) on the host cores, one layer, bounded sample.

    Sample: the first sequences of the batch (in order) whose contexts sum to about 1/8 of the
    layer, gathered into a compact CPU pool; timed as gather + bias + repeat_interleave + bf16
    matmul + fp32 softmax, 1 warmup + repeats (median) within the time budget.
    """
    from mini_infra_qwen3_amd import workloads as wl
    from oracle import torch_ref

    torch.set_num_threads(cpu_threads())
    total = sum(w.context_lens)
    picked, acc = [], 0
    for b, n in enumerate(w.context_lens):
        picked.append(b)
        acc += n
        if acc >= total / 8:
            break
    blocks = [blk for b in picked for blk in w.tables[b]]
    index = torch.tensor(blocks, device=device)
    key_pool = torch.cat([torch.zeros(1, 16, 8, 128, dtype=torch.bfloat16), w.pools[0, 0][index].cpu()])
    value_pool = torch.cat([torch.zeros(1, 16, 8, 128, dtype=torch.bfloat16), w.pools[0, 1][index].cpu()])
    tables, k = [], 1
    for b in picked:
        tables.append(list(range(k, k + len(w.tables[b]))))
        k += len(w.tables[b])
    bt = wl.padded(tables)
    ctx = torch.tensor([w.context_lens[b] for b in picked])
    q = w.query[0][picked].cpu()
    sample_bytes = int(ctx.sum()) * wl.KV_BYTES_PER_TOKEN_LAYER
    times = []
    t_budget = time.perf_counter() + budget_s
    for i in range(6):
        t0 = time.perf_counter()
        torch_ref.paged_decode_attention(q, key_pool, value_pool, bt, ctx, wl.SCALE)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_budget and i >= 1:
            break
    timed = sorted(times[1:]) if len(times) > 1 else times
    median = timed[len(timed) // 2]
    return {
        "value": sample_bytes / median / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one layer, {len(picked)} of {len(w.context_lens)} sequences (sum ctx {int(ctx.sum())}), "
                   f"reference torch chain (gather+bias+repeat_interleave+bf16 matmul+fp32 softmax) on CPU, "
                   f"median of {len(timed)} after 1 warmup; {cpu_model()}"),
        "ms_per_layer_sample": median * 1000.0,
    }


def cpu_threads() -> int:
    """Host threads for the CPU baselines: OMP_NUM_THREADS when set (the process's share of the
    host), else every core."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def cpu_time(fn, budget_s: float, max_runs: int = 6) -> tuple[float, int]:
    """(median seconds of the timed runs, number of timed runs): 1 warm-up, then repeats within the
    time budget (at least one)."""
    fn()
    times = []
    t_budget = time.perf_counter() + budget_s
    while len(times) < max_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_budget:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline_decode_full(w, device: torch.device, slice_size: int = 32) -> dict:
    """The reference decode chain (oracle) over the whole batch of 256 on the host cores, one layer,
    as summed slices of ``slice_size`` sequences (each slice gathered from its own compact pool):
    the host-memory bound of one padded gather of all 256 rows (~17 GB) is avoided, the work is the
    full layer's."""
    from mini_infra_qwen3_amd import workloads as wl
    from oracle import torch_ref

    torch.set_num_threads(cpu_threads())
    total_s, runs = 0.0, []
    for lo in range(0, len(w.context_lens), slice_size):
        picked = list(range(lo, min(lo + slice_size, len(w.context_lens))))
        blocks = [blk for b in picked for blk in w.tables[b]]
        index = torch.tensor(blocks, device=device)
        key_pool = torch.cat([torch.zeros(1, 16, 8, 128, dtype=torch.bfloat16), w.pools[0, 0][index].cpu()])
        value_pool = torch.cat([torch.zeros(1, 16, 8, 128, dtype=torch.bfloat16), w.pools[0, 1][index].cpu()])
        tables, k = [], 1
        for b in picked:
            tables.append(list(range(k, k + len(w.tables[b]))))
            k += len(w.tables[b])
        bt, ctx, q = wl.padded(tables), torch.tensor([w.context_lens[b] for b in picked]), w.query[0][picked].cpu()
        sec, n = cpu_time(lambda: torch_ref.paged_decode_attention(q, key_pool, value_pool, bt, ctx, wl.SCALE), 6.0, 3)
        total_s += sec
        runs.append(n)
    nbytes = sum(w.context_lens) * wl.KV_BYTES_PER_TOKEN_LAYER
    return {"value": nbytes / total_s / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one layer, all 256 sequences as {len(runs)} slices of {slice_size} (sum of per-slice "
                      f"medians after 1 warm-up, {min(runs)}-{max(runs)} timed runs each), reference torch chain "
                      f"(gather + bias + repeat_interleave + bf16 matmul + fp32 softmax); {cpu_model()}",
            "ms_per_layer": total_s * 1000.0, "ms_per_28_layer_step": total_s * 28000.0}


# ------------------------------------------------------------------------------- scatter
def bench_scatter(steps: int, warmup: int, device: torch.device, layout: str = "token",
                  ceiling: float | None = None, cpu: bool = False, pattern_ceiling: float | None = None,
                  tables: str = "fragmented") -> dict:
    """The 28-layer prefill store of 32 prompts U[128, 2048] (40,636 tokens) into blocks from a
    churned ``FreeKVCacheBlockQueue`` (``tables``: ``fragmented`` or ``near_sequential``, the
    kinds of ``workloads.TABLE_KINDS``), one launch.  ``layout`` of the source ``[B, Hkv, L, D]`` per layer: ``token`` -- the
    memory of the HIP model's prefill K/V (``mi_qk_norm_rope`` writes ``[T, Hkv, D]`` rows, viewed
    as ``[B, Hkv, L, D]``), so a token's 2 KiB row is contiguous; ``head`` -- the reference's
    ``KVCache`` layout (contiguous ``[B, Hkv, L, D]``: a row is 8 pieces of 256 B, L x 256 B apart).
    ``ceiling``: the measured read+write copy rate the achieved rate is also read against;
    ``pattern_ceiling``: that of a copy whose destination 32 KiB units lie at scattered places.
    ``cpu``: time the oracle's ``write_prefill`` (the reference's index + index_copy_ chain) on the
    host cores over 4 of the 28 layers."""
    from mini_infra_qwen3_amd import workloads as wl
    from mini_infra_qwen3_amd.worker import KVCache, PagedKVCachePool

    w = wl.prefill_scatter(seed=0, device=device, tables=tables)
    sources = w.sources
    if layout == "token":
        sources = sources.transpose(-3, -2).contiguous().transpose(-3, -2)
    pool = PagedKVCachePool(wl.NUM_LAYERS, w.num_blocks, wl.BLOCK_SIZE, wl.NUM_KV_HEADS, wl.HEAD_DIM,
                            torch.bfloat16, device)
    cache = KVCache([(sources[l, 0], sources[l, 1]) for l in range(wl.NUM_LAYERS)])
    index = torch.from_numpy(w.index).to(device)
    timer = EventTimer()
    for _ in range(warmup):
        pool.write_prefill(cache, index[0], index[1], index[2])
    for _ in range(steps):
        timer.start()
        pool.write_prefill(cache, index[0], index[1], index[2])
        timer.stop()
    ms = timer.mean_ms()
    moved = 2 * w.num_tokens * wl.NUM_LAYERS * wl.KV_BYTES_PER_TOKEN_LAYER  # read + write
    gbs = moved / (ms * 1e-3) / 1e9
    source = "token-major (the model's K/V rows)" if layout == "token" else "head-major (the reference KVCache)"
    out = {"workload": f"prefill scatter, 28 layers, 32 prompts U[128,2048] ({w.num_tokens} tokens), "
                       f"{tables.replace('_', '-')} tables, {source} source",
           "tables": tables, "consecutive_block_fraction": round(wl.consecutive_fraction(w.tables), 4),
           "ms_per_launch": ms, "bytes_per_launch": moved, "achieved_GBps": gbs, "frac": gbs / HBM_PEAK_GBS,
           "frac_of_copy_ceiling": gbs / ceiling if ceiling else None,
           "frac_of_scattered_write_copy": gbs / pattern_ceiling if pattern_ceiling else None,
           "traffic": profiled_traffic("reshape_and_cache" if layout == "head" else "reshape_and_cache_token")}
    if cpu:
        from oracle import torch_ref

        torch.set_num_threads(cpu_threads())
        layers = 4
        cpu_pools = [(torch.zeros(w.num_blocks, 16, 8, 128, dtype=torch.bfloat16),
                      torch.zeros(w.num_blocks, 16, 8, 128, dtype=torch.bfloat16)) for _ in range(layers)]
        cpu_cache = [(w.sources[l, 0].cpu(), w.sources[l, 1].cpu()) for l in range(layers)]
        idx = torch.from_numpy(w.index)
        sec, n = cpu_time(lambda: torch_ref.write_prefill(cpu_pools, cpu_cache, idx[0], idx[1], idx[2]), 15.0)
        out["cpu_baseline"] = {
            "value": 2 * w.num_tokens * layers * wl.KV_BYTES_PER_TOKEN_LAYER / sec / 1e9, "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"4 of the 28 layers, all {w.num_tokens} tokens: the reference's write_prefill (advanced-index "
                      f"gather + index_copy_ per tensor per layer), median of {n} after 1 warm-up; {cpu_model()}"}
        del cpu_pools, cpu_cache
    del pool, cache, sources, w
    torch.cuda.empty_cache()
    return out


# -------------------------------------------------------------------------------- gather
def bench_gather(steps: int, warmup: int, device: torch.device, ceiling: float | None = None,
                 cpu: bool = False, pattern_ceiling: float | None = None, tables: str = "fragmented") -> dict:
    """The chunked-prefill history gather (the reference's ``gather_blocks``), 28 layers: every chunk c of the 4
    prompts gathers its 128 c history blocks, one launch per chunk; block tables of kind ``tables``
    (``fragmented`` or ``near_sequential``).  ``cpu``: the oracle's
    ``gather_blocks`` on the host cores for one of the 28 layers.  ``ceiling`` / ``pattern_ceiling``:
    the read+write copy rates (contiguous / from source 32 KiB units at scattered places) it is read against."""
    from mini_infra_qwen3_amd import workloads as wl
    from mini_infra_qwen3_amd.worker import PagedKVCachePool

    w = wl.chunked_prefill(seed=0, tables=tables)
    pool = PagedKVCachePool(wl.NUM_LAYERS, w.num_blocks, wl.BLOCK_SIZE, wl.NUM_KV_HEADS, wl.HEAD_DIM,
                            torch.bfloat16, device)
    pool.storage.view(torch.int16).random_(generator=torch.Generator(device=device).manual_seed(0))
    # each chunk c of each prompt gathers its 128 c history blocks, all layers in one launch
    chunk_tables = []
    for c in range(1, w.num_chunks):
        nb = c * w.chunk_len // wl.BLOCK_SIZE
        chunk_tables.append(torch.tensor([t[:nb] for t in w.tables], dtype=torch.long, device=device))
    timer = EventTimer()

    def run():
        for ids in chunk_tables:
            pool.gather_blocks(ids)

    for _ in range(warmup):
        run()
    for _ in range(steps):
        timer.start()
        run()
        timer.stop()
    ms = timer.mean_ms()
    moved = 2 * w.history_bytes_per_layer() * wl.NUM_LAYERS  # read history + write the gathered copy
    gbs = moved / (ms * 1e-3) / 1e9
    out = {"workload": f"history gather, 28 layers, 4 prompts x 16384 tokens in 2048-token chunks (7 launches), "
                       f"{tables.replace('_', '-')} tables",
           "tables": tables, "consecutive_block_fraction": round(wl.consecutive_fraction(w.tables), 4),
           "ms_per_prompt_set": ms, "bytes": moved, "achieved_GBps": gbs, "frac": gbs / HBM_PEAK_GBS,
           "frac_of_copy_ceiling": gbs / ceiling if ceiling else None,
           "frac_of_scattered_read_copy": gbs / pattern_ceiling if pattern_ceiling else None,
           "traffic_per_prompt_set": profiled_traffic("gather_blocks")}
    if cpu:
        from oracle import torch_ref

        torch.set_num_threads(cpu_threads())
        layer0 = [(pool.kv_pools[0][0].cpu(), pool.kv_pools[0][1].cpu())]
        tabs = [t.cpu() for t in chunk_tables]
        sec, n = cpu_time(lambda: [torch_ref.gather_blocks(layer0, t)[0][0].contiguous() for t in tabs], 15.0)
        out["cpu_baseline"] = {
            "value": 2 * w.history_bytes_per_layer() / sec / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"one of the 28 layers, all 7 chunk gathers of the 4 prompts: the reference's gather_blocks "
                      f"(pool[block_ids] per tensor), median of {n} after 1 warm-up; {cpu_model()}"}
        del layer0
    del pool
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------------------ device copy
def copy_ceiling(device: torch.device, nbytes: int = 2 << 30, reps: int = 5) -> dict:
    """What plain streaming traffic reaches on this device: the calibration kernels of
    libmi_calib.so (16-byte non-temporal accesses, with non-temporal or device-scope streaming
    stores, contiguous spans per workgroup) over 2 GiB
    buffers, for read + write (copy), read-only and write-only, best of the library's launch
    shapes, and for read + write copies whose destination (or source) 32 KiB units lie at scattered
    places, the write (read) pattern of the scatter (gather).  The read + write rate is the ceiling
    scatter, gather and the block records are read against, the read rate the one decode attention
    (a read stream) is."""
    lib = ctypes.CDLL(CALIB_LIBRARY)
    lib.calib_stream.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.c_int32, ctypes.c_void_p]
    lib.calib_stream.restype = ctypes.c_int32
    lib.calib_groups.argtypes = [ctypes.c_int64, ctypes.c_int32]
    lib.calib_groups.restype = ctypes.c_int64
    lib.calib_variant.argtypes = [ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32)]
    variants = lib.calib_num_variants()
    src = torch.empty(nbytes, dtype=torch.uint8, device=device).random_()
    dst = torch.empty_like(src)
    sink = torch.empty(max(lib.calib_groups(nbytes, v) for v in range(variants)), dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    result = {"workload": f"calibration streams over {nbytes >> 30} GiB buffers (libmi_calib.so)"}
    spans = []
    for v in range(variants):
        t, f, sp, st = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int32()
        lib.calib_variant(v, ctypes.byref(t), ctypes.byref(f), ctypes.byref(sp), ctypes.byref(st))
        spans.append(sp.value)
    # The scattered copies move whole 32 KiB units (pool blocks) to or from scattered places, with
    # workgroup spans of at most 32 KiB inside them.
    for shape, name, moved, max_span in ((0, "read_write", 2 * nbytes, None), (1, "read", nbytes, None),
                                         (2, "write", nbytes, None),
                                         (3, "scattered_write_copy", 2 * nbytes, 32 << 10),
                                         (4, "scattered_read_copy", 2 * nbytes, 32 << 10)):
        best = (0.0, None)
        for v in range(variants):
            if max_span is not None and spans[v] > max_span:
                continue
            def launch():
                rc = lib.calib_stream(shape, dst.data_ptr(), src.data_ptr(), sink.data_ptr(), nbytes, v, stream)
                if rc != 0:
                    raise RuntimeError(f"calib_stream({shape}, variant {v}) failed: {rc}")
            for _ in range(2):
                launch()
            timer = EventTimer()
            for _ in range(reps):
                timer.start()
                launch()
                timer.stop()
            gbs = moved / (timer.mean_ms() * 1e-3) / 1e9
            if gbs > best[0]:
                t, f, sp, st = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int32()
                lib.calib_variant(v, ctypes.byref(t), ctypes.byref(f), ctypes.byref(sp), ctypes.byref(st))
                best = (gbs, f"{t.value} lanes, {f.value} pieces in flight, {sp.value >> 10} KiB per workgroup"
                             + (", device-scope streaming stores" if st.value and shape != 1 else ""))
        result[f"{name}_GBps"] = round(best[0], 1)
        result[f"{name}_frac"] = round(best[0] / HBM_PEAK_GBS, 4)
        result[f"{name}_shape"] = best[1]
    del src, dst, sink
    torch.cuda.empty_cache()
    return result


def bench_copy(steps: int, device: torch.device, nbytes: int = 1 << 30) -> dict:
    """torch's device-to-device copy of a 1 GiB buffer (reads and writes exactly ``nbytes`` per
    launch; the calibration workload of the HBM traffic counters), and the calibration kernels'
    ceilings (``copy_ceiling``)."""
    src = torch.ones(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    timer = EventTimer()
    for _ in range(max(steps, 1)):
        timer.start()
        dst.copy_(src)
        timer.stop()
    ms = timer.mean_ms()
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return {"workload": "torch device copy, 1 GiB", "bytes_per_launch": 2 * nbytes, "ms_per_launch": ms,
            "achieved_GBps": gbs, "frac": gbs / HBM_PEAK_GBS, "ceiling": copy_ceiling(device)}


# ------------------------------------------------------------------------ KV block swap
def bench_swap(steps: int, warmup: int, device: torch.device, num_records: int = 2048) -> dict:
    """KV block records of the Qwen3-0.6B pool (28 layers, 1.75 MiB per block): pack 2048 randomly
    placed blocks into records and unpack them into other blocks (HBM: each moves 2 x 3.76 GB per
    launch), and the whole swap to pinned host memory and back (pack + DMA, DMA + unpack: PCIe)."""
    from mini_infra_qwen3_amd import workloads as wl
    from mini_infra_qwen3_amd.worker import HostSwapPool, PagedKVCachePool

    pool = PagedKVCachePool(wl.NUM_LAYERS, 2 * num_records + 1, wl.BLOCK_SIZE, wl.NUM_KV_HEADS, wl.HEAD_DIM,
                            torch.bfloat16, device)
    pool.storage.view(torch.int16).random_(generator=torch.Generator(device=device).manual_seed(0))
    perm = (torch.randperm(2 * num_records, generator=torch.Generator().manual_seed(1)) + 1).tolist()
    src, dst = perm[:num_records], perm[num_records:]
    src_t = torch.tensor(src, dtype=torch.long, device=device)
    dst_t = torch.tensor(dst, dtype=torch.long, device=device)
    record_bytes = pool.bytes_per_block
    records = pool.pack_blocks(src_t)
    res = {"workload": f"{num_records} blocks of a 28-layer Qwen3-0.6B pool ({record_bytes} B per block record), "
                       "random block ids"}
    for name, fn in (("pack", lambda: pool.pack_blocks(src_t)), ("unpack", lambda: pool.unpack_blocks(records, dst_t))):
        timer = EventTimer()
        for _ in range(warmup):
            fn()
        for _ in range(steps):
            timer.start()
            fn()
            timer.stop()
        ms = timer.mean_ms()
        gbs = 2 * num_records * record_bytes / (ms * 1e-3) / 1e9
        res[name] = {"ms_per_launch": ms, "bytes_per_launch": 2 * num_records * record_bytes, "achieved_GBps": gbs,
                     "frac": gbs / HBM_PEAK_GBS}
    del records
    swap = HostSwapPool(num_records, pool)
    for name in ("swap_out", "swap_in"):
        timer = EventTimer()
        for i in range(warmup + max(steps // 4, 2)):
            if i >= warmup:
                timer.start()
            if name == "swap_out":
                slots = swap.swap_out(pool, src)
            else:
                slots = swap.allocate(num_records)
                swap.swap_in(pool, slots, dst)
            if i >= warmup:
                timer.stop()
            if name == "swap_out":
                swap.free(slots)
        ms = timer.mean_ms()
        gbs = num_records * record_bytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": ms, "bytes": num_records * record_bytes, "achieved_GBps": gbs,
                     "frac_of_pcie": gbs / PCIE_PEAK_GBS}
    del swap, pool
    return res


# ------------------------------------------------------------------------- chunked prefill
def bench_prefill(steps: int, warmup: int, device: torch.device, cpu: bool = False) -> dict:
    """4 prompts x 16384 tokens, 2048-token chunks, one layer: 8 chunk steps, each one launch over the
    4 prompts (history 2048 c read from the pool through the block table, causal inside the chunk).
    ``cpu``: the oracle's chunked-prefill chain (gather + concat + mask + bf16 matmul + fp32
    softmax) on the host cores for one prompt's chunk 1 (2048 history tokens)."""
    from mini_infra_qwen3_amd import data_plane, workloads as wl

    w = wl.chunked_prefill(seed=0)
    gen = torch.Generator(device=device).manual_seed(3)
    pools = torch.randn((2, w.num_blocks, wl.BLOCK_SIZE, wl.NUM_KV_HEADS, wl.HEAD_DIM), generator=gen,
                        device=device).to(torch.bfloat16)
    L = w.chunk_len
    q = torch.randn((w.num_prompts, wl.NUM_HEADS, L, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn((w.num_prompts, wl.NUM_KV_HEADS, L, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn((w.num_prompts, wl.NUM_KV_HEADS, L, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    tables = torch.tensor(w.tables, dtype=torch.long, device=device)
    lens = torch.full((w.num_prompts,), L, dtype=torch.long, device=device)
    out = torch.empty((w.num_prompts, L, wl.NUM_HEADS * wl.HEAD_DIM), dtype=torch.bfloat16, device=device)
    steps_c = []
    for c in range(w.num_chunks):
        nb = c * L // wl.BLOCK_SIZE
        steps_c.append((tables[:, :nb], torch.full((w.num_prompts,), c * L, dtype=torch.long, device=device)))

    def layer():
        for hist, starts in steps_c:
            data_plane.chunked_prefill_attention(q, k, v, pools[0], pools[1], hist, starts, lens, wl.SCALE, out=out)

    timer = EventTimer()
    for _ in range(warmup):
        layer()
    for _ in range(steps):
        timer.start()
        layer()
        timer.stop()
    ms = timer.mean_ms()
    n = w.prompt_len
    flops = w.num_prompts * 2 * 2 * wl.NUM_HEADS * wl.HEAD_DIM * n * (n + 1) / 2  # QK^T and PV, causal pairs
    tflops = flops / (ms * 1e-3) / 1e12
    out = {"workload": "chunked prefill attention, 4 prompts x 16384 tokens, 2048-token chunks, one layer "
                       "(8 launches, history from the pool)",
           "ms_per_layer": ms, "tflop_per_layer": flops / 1e12, "achieved_TFLOPs": tflops,
           "peak_TFLOPs": MFMA_BF16_PEAK_TFLOPS, "frac": tflops / MFMA_BF16_PEAK_TFLOPS}
    if cpu:
        from oracle import torch_ref

        torch.set_num_threads(cpu_threads())
        c = 1
        hist = tables[:1, :c * L // wl.BLOCK_SIZE].cpu()
        kp, vp = pools[0].cpu(), pools[1].cpu()
        q1, k1, v1 = q[:1].cpu(), k[:1].cpu(), v[:1].cpu()
        sec, n = cpu_time(lambda: torch_ref.chunked_prefill_attention(q1, k1, v1, (kp, vp), hist, [c * L], [L],
                                                                      wl.SCALE), 20.0, 4)
        chunk_flops = 2 * 2 * wl.NUM_HEADS * wl.HEAD_DIM * (L * c * L + L * (L + 1) / 2)
        out["cpu_baseline"] = {
            "value": chunk_flops / sec / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one prompt's chunk {c} (2048 queries, 2048 history + causal chunk keys): the reference's "
                      f"gather + concat + mask + attend, median of {n} after 1 warm-up; {cpu_model()}",
            "ms_per_chunk": sec * 1000.0}
        del kp, vp
    del pools, q, k, v
    torch.cuda.empty_cache()
    return out


def bench_exact_prefill(steps: int, warmup: int, device: torch.device) -> dict:
    """Reference-numerics chunked prefill attention (the model's default: exact sums, fp64 matrix
    cores) on the heaviest chunk step the e2e workload makes: two 1024-token prompts (the longest it
    draws) in one 2048-token budget, no history, 16 query / 8 KV heads, one layer."""
    from mini_infra_qwen3_amd import data_plane, workloads as wl

    rows, n = 2, 1024
    gen = torch.Generator(device=device).manual_seed(4)
    q = torch.randn((rows, wl.NUM_HEADS, n, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn((rows, wl.NUM_KV_HEADS, n, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn((rows, wl.NUM_KV_HEADS, n, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    pools = torch.zeros((2, 1, wl.BLOCK_SIZE, wl.NUM_KV_HEADS, wl.HEAD_DIM), dtype=torch.bfloat16, device=device)
    hist = torch.zeros((rows, 0), dtype=torch.long, device=device)
    starts = torch.zeros((rows,), dtype=torch.long, device=device)
    lens = torch.full((rows,), n, dtype=torch.long, device=device)
    out = torch.empty((rows, n, wl.NUM_HEADS * wl.HEAD_DIM), dtype=torch.bfloat16, device=device)

    def layer():
        data_plane.chunked_prefill_attention(q, k, v, pools[0], pools[1], hist, starts, lens, wl.SCALE, out=out,
                                             exact=True)

    timer = EventTimer()
    for _ in range(warmup):
        layer()
    for _ in range(steps):
        timer.start()
        layer()
        timer.stop()
    ms = timer.mean_ms()
    flops = rows * 2 * 2 * wl.NUM_HEADS * wl.HEAD_DIM * n * (n + 1) / 2  # QK^T and PV, causal pairs
    tflops = flops / (ms * 1e-3) / 1e12
    del q, k, v, pools, out
    torch.cuda.empty_cache()
    return {"workload": "reference-numerics chunked prefill attention (exact sums, fp64 matrix cores), 2 prompts x "
                        "1024 tokens in one chunk, no history, one layer",
            "ms_per_layer": ms, "tflop_per_layer": flops / 1e12, "achieved_TFLOPs": tflops,
            "peak_TFLOPs": MFMA_FP64_PEAK_TFLOPS, "frac": tflops / MFMA_FP64_PEAK_TFLOPS, "dtype": "f64"}


# ------------------------------------------------------------------------ e2e continuous batching
def cpu_baseline_e2e(seed: int = 0, num_requests: int = 8, max_new_tokens: int = 64) -> dict:
    """The oracle's restatement of the reference schedule backend (the reference's torch model,
    runner and paged pool) on the host cores: the first requests of the continuous-batching workload with
    fewer output tokens, same loop, token budget and model.  Output tok/s over the loop's wall
    time (its busy time: no idle gaps, the loop runs back to back)."""
    from mini_infra_qwen3_amd.engine import run_scheduler
    from mini_infra_qwen3_amd.model import Qwen3ForCausalLM, init_random_, qwen3_0_6b
    from mini_infra_qwen3_amd.workloads import serving_requests
    from oracle import qwen3_ref

    torch.set_num_threads(cpu_threads())
    cfg = qwen3_0_6b()
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, seed=seed, std=0.02)
    ref = qwen3_ref.ReferenceQwen3(cfg, model.to(torch.bfloat16).state_dict(), "cpu")
    del model
    import dataclasses

    requests = [dataclasses.replace(r, max_new_tokens=max_new_tokens) for r in serving_requests(seed=seed)[:num_requests]]
    t0 = time.perf_counter()
    res = run_scheduler(qwen3_ref.ReferenceScheduleBackend(ref, requests, num_requests), requests,
                        token_budget=2048, eos_token_id=-1, stop_on_eos=False)
    wall = time.perf_counter() - t0
    return {"value": res.num_output_tokens / wall, "unit": "output tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"first {num_requests} requests of the workload (prompts {[r.prompt_len for r in requests]}), "
                      f"{max_new_tokens} greedy tokens each, the reference's torch model on the CPU (bf16), wall "
                      f"time of the loop; {cpu_model()}",
            "wall_s": wall}



def bench_e2e(device: torch.device, seed: int = 0, mixed: bool = False, exact: bool = True,
              mixed_chunk_tokens: int | None = None) -> dict:
    """Continuous batching with chunked prefill (token budget 2048, block 16, batch slots = number of
    requests) of a random-init Qwen3-0.6B (bf16, N(0, 0.02), tied embeddings): 128 requests, Poisson
    arrivals at 20 req/s, prompts U[32, 1024], 128 greedy tokens each, EOS disabled.  Output tok/s =
    output tokens x 1000 / busy_ms, busy_ms = sum over steps of (device-timed forward + host-timed
    cache management), on the logical clock the measured step times advance.  HIP graphs are
    captured when the backend is set up (``setup_s``, outside the timed run).
    ``exact`` (reference numerics, the configuration whose greedy tokens are identical to the
    oracle's): the exact attention kernels and the reference's GEMM calls; decode forwards replay
    a graph per batch size; prefill steps run eagerly at the chunks' own width; mixed steps run at
    their padded shape (width to a multiple of 128, decode rows to a power of two), replayed from
    a graph per shape.  ``exact=False``:
    the bandwidth kernels and fused GEMMs, decode graphs per padded (batch, blocks) bucket and
    prefill (and mixed) graphs per padded (rows, width) bucket.  ``mixed``: decode rows ride in
    the prefill steps (the mixed batching the reference plans) instead of the reference's
    alternating prefill / decode; ``mixed_chunk_tokens`` caps the prompt tokens of such a step
    (prefill-only steps keep the 2048-token budget), which bounds the decoding requests' gaps."""
    from mini_infra_qwen3_amd.core.scheduler import SchedulePhase
    from mini_infra_qwen3_amd.engine import PagedScheduleBackend, run_scheduler
    from mini_infra_qwen3_amd.model import Qwen3ForCausalLM, init_random_, qwen3_0_6b
    from mini_infra_qwen3_amd.workloads import serving_requests

    model = Qwen3ForCausalLM(qwen3_0_6b(), exact=exact)
    init_random_(model, seed=seed, std=0.02)
    model = model.to(device=device, dtype=torch.bfloat16).eval()

    def run(requests):
        t0 = time.perf_counter()
        backend = PagedScheduleBackend(model, requests, len(requests), decode_graphs=True, prefill_graphs=not exact,
                                       mixed_graphs=mixed, mixed_graph_tokens=mixed_chunk_tokens or 2048)
        setup_s = time.perf_counter() - t0
        return run_scheduler(backend, requests, token_budget=2048, eos_token_id=-1, stop_on_eos=False,
                             mixed_batching=mixed, mixed_chunk_tokens=mixed_chunk_tokens), setup_s

    run(serving_requests(seed=seed + 1, num_requests=8, max_new_tokens=8))  # warm-up: kernels, GEMM choices
    requests = serving_requests(seed=seed)
    res, setup_s = run(requests)
    decode = [e for e in res.events if e.phase is SchedulePhase.DECODE]
    prefill = [e for e in res.events if e.phase is SchedulePhase.PREFILL]
    mixed_steps = [e for e in res.events if e.phase is SchedulePhase.MIXED]
    out = {
        "metric": "e2e output tok/s Qwen3-0.6B (continuous batching, chunked prefill 2048, paged KV)",
        "numerics": "reference (exact sums; greedy tokens identical to the oracle)" if exact else "bandwidth kernels",
        "mixed_batching": mixed,
        "mixed_chunk_tokens": mixed_chunk_tokens,
        "output_tok_s": round(res.throughput_tok_s, 1),
        "wall_tok_s": round(res.wall_tok_s, 1),
        "busy_ms": round(res.busy_ms, 1),
        "model_ms": round(res.model_ms, 1),
        "cache_ms": round(res.cache_ms, 1),
        "wall_ms": round(res.wall_ms, 1),
        "makespan_ms": round(res.makespan_ms, 1),
        "output_tokens": res.num_output_tokens,
        "prompt_tokens": sum(r.prompt_len for r in requests),
        "decode_steps": len(decode),
        "prefill_steps": len(prefill),
        "decode_step_ms_mean": round(sum(e.step_ms for e in decode) / max(len(decode), 1), 3),
        "decode_cache_ms_mean": round(sum(e.cache_ms for e in decode) / max(len(decode), 1), 4),
        "prefill_cache_ms_mean": round(sum(e.cache_ms for e in prefill) / max(len(prefill), 1), 4),
        "decode_batch_mean": round(sum(len(e.request_ids) for e in decode) / max(len(decode), 1), 2),
        "prefill_step_ms_mean": round(sum(e.step_ms for e in prefill) / max(len(prefill), 1), 3),
        "mixed_steps": len(mixed_steps),
        "mixed_step_ms_mean": round(sum(e.step_ms for e in mixed_steps) / max(len(mixed_steps), 1), 3),
        "requests": len(requests),
        "arrival_rate_req_s": 20.0,
        "decode_graphs": "per batch size" if exact else "per padded (batch, blocks) bucket",
        "prefill_graphs": not exact,
        "mixed_graphs": mixed,
        "setup_s": round(setup_s, 2),
        "latency_ms": {k: round(v, 2) for k, v in res.latency_summary().items()},
        "_tokens": res.tokens,  # per request, for the token agreement; dropped from the JSON line
    }
    del model, res
    torch.cuda.empty_cache()
    return out


def token_agreement(reference: dict[int, list[int]], tokens: dict[int, list[int]], device: torch.device,
                    seed: int = 0) -> dict:
    """How many requests of a bandwidth-kernel run emit exactly the tokens of the reference-numerics
    run (whose tokens the GPU tests show identical to the oracle's; exact equality is the
    reference's own gate, src/mini_infra/bench/correctness.py:69-73), and for each other request its
    first divergence: the position, and the logit margin the reference-numerics model has there
    between its own token and the bandwidth run's, with the top-1 / top-2 margin beside it.  The
    logits are recomputed with one reference-numerics prefill over the prompt and the common prefix
    (the same weights); GEMM rows can round differently at another M, so a margin is a measure of
    how close to a tie the step was, not a bit-exact replay."""
    from mini_infra_qwen3_amd.model import Qwen3ForCausalLM, init_random_, qwen3_0_6b
    from mini_infra_qwen3_amd.workloads import serving_requests

    requests = serving_requests(seed=seed)
    model = Qwen3ForCausalLM(qwen3_0_6b(), exact=True)
    init_random_(model, seed=seed, std=0.02)
    model = model.to(device=device, dtype=torch.bfloat16).eval()
    identical, first, margins, top2, total_same = 0, [], [], [], 0
    with torch.inference_mode():
        for r in requests:
            ref, got = reference[r.request_idx], tokens[r.request_idx]
            total_same += sum(a == b for a, b in zip(ref, got))
            if ref == got:
                identical += 1
                continue
            d = next((i for i, (a, b) in enumerate(zip(ref, got)) if a != b), min(len(ref), len(got)))
            first.append(d)
            if d >= min(len(ref), len(got)):
                continue
            ids = torch.tensor([list(r.token_ids) + ref[:d]], dtype=torch.long, device=device)
            logits, _ = model(ids, last_logits_only=True)
            row = logits[0, -1].float()
            margins.append(float(row[ref[d]] - row[got[d]]))
            best = torch.topk(row, 2).values
            top2.append(float(best[0] - best[1]))
    del model
    torch.cuda.empty_cache()

    def spread(values):
        if not values:
            return None
        v = sorted(values)
        return {"min": round(v[0], 5), "median": round(v[len(v) // 2], 5), "max": round(v[-1], 5)}

    return {"requests": len(requests), "identical_requests": identical,
            "identical_tokens_frac": round(total_same / max(sum(len(t) for t in reference.values()), 1), 4),
            "first_divergence_position": spread(first),
            "margin_at_divergence": spread(margins), "top2_margin_at_divergence": spread(top2)}


def bench_decode_groups(steps: int, warmup: int, device) -> dict:
    """Decode attention (one launch + its merge) on the batch-256 workload's first layer for the
    GQA groups the library compiles: 8 KV heads, 8 G query heads (Qwen3-0.6B/1.7B: G = 2, 4B/8B:
    4, 14B: 5, 32B: 8).  The K/V bytes are the same for every G; only Q and O grow."""
    from mini_infra_qwen3_amd import data_plane, workloads as wl

    w = wl.decode_at_scale(seed=0, device=device, num_layers=1)
    tables = w.block_tables.to(device)
    ctx = torch.tensor(w.context_lens, dtype=torch.long, device=device)
    key_pool, value_pool = w.pools[0, 0], w.pools[0, 1]
    kv_bytes = sum(w.context_lens) * wl.KV_BYTES_PER_TOKEN_LAYER
    gen = torch.Generator(device=device).manual_seed(7)
    out = {"workload": f"decode attention, batch 256, sum(ctx)={sum(w.context_lens)}, 8 KV heads, one layer",
           "groups": {}}
    for group in (1, 2, 4, 5, 8):
        heads = wl.NUM_KV_HEADS * group
        query = torch.randn((len(w.context_lens), heads, wl.HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        res = torch.empty((len(w.context_lens), heads * wl.HEAD_DIM), dtype=torch.bfloat16, device=device)
        ws = torch.empty(max(data_plane.paged_decode_workspace_bytes(
            len(w.context_lens), tables.shape[1], heads, wl.HEAD_DIM, wl.BLOCK_SIZE, wl.NUM_KV_HEADS), 1),
            dtype=torch.uint8, device=device)
        run = lambda: data_plane.paged_decode_attention(query, key_pool, value_pool, tables, ctx, wl.SCALE,
                                                        out=res, workspace=ws)
        for _ in range(warmup):
            run()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(device)
        start.record()
        for _ in range(steps):
            run()
        end.record()
        torch.cuda.synchronize(device)
        ms = start.elapsed_time(end) / steps
        nbytes = kv_bytes + 2 * query.numel() * 2
        out["groups"][str(group)] = {"us_per_launch": round(ms * 1000, 1), "bytes": nbytes,
                                     "achieved_GBps": round(nbytes / ms / 1e6, 1),
                                     "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
    return out


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--only", choices=["decode", "decode-groups", "scatter", "scatter-sequential", "scatter-head",
                                           "gather", "gather-sequential", "prefill", "exact-prefill",
                                           "copy", "swap", "e2e", "e2e-mixed", "e2e-bandwidth", "e2e-mixed-bandwidth",
                                           "e2e-mixed-capped", "e2e-agreement", "all"],
                        default="all")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the multi-GPU sharding of this path "
              "is a design note, not a measured configuration.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    from mini_infra_qwen3_amd import _native

    _native.load()
    log(f"device {torch.cuda.get_device_name(device)}; library {_native.LIBRARY_PATH}")

    single = {
        "copy": lambda: bench_copy(args.steps, device),
        "scatter": lambda: bench_scatter(args.steps, args.warmup, device),
        "scatter-sequential": lambda: bench_scatter(args.steps, args.warmup, device, tables="near_sequential"),
        "scatter-head": lambda: bench_scatter(args.steps, args.warmup, device, layout="head"),
        "gather": lambda: bench_gather(args.steps, args.warmup, device),
        "gather-sequential": lambda: bench_gather(args.steps, args.warmup, device, tables="near_sequential"),
        "prefill": lambda: bench_prefill(args.steps, args.warmup, device),
        "exact-prefill": lambda: bench_exact_prefill(args.steps, args.warmup, device),
        "swap": lambda: bench_swap(args.steps, args.warmup, device),
        "decode-groups": lambda: bench_decode_groups(args.steps, args.warmup, device),
    }
    if args.only in single:  # one kernel alone (for counter runs)
        res = single[args.only]()
        log(f"{args.only}: {json.dumps(res)}")
        print(json.dumps(res), flush=True)
        return 0
    if args.only in ("e2e", "e2e-mixed", "e2e-bandwidth", "e2e-mixed-bandwidth", "e2e-mixed-capped"):
        res = bench_e2e(device, mixed=args.only.startswith("e2e-mixed"), exact=not args.only.endswith("bandwidth"),
                        mixed_chunk_tokens=MIXED_CHUNK_CAP if args.only == "e2e-mixed-capped" else None)
        res.pop("_tokens")
        log(f"e2e: {res['output_tok_s']:.1f} output tok/s (busy), {res['wall_tok_s']:.1f} tok/s (wall)")
        print(json.dumps(res), flush=True)
        return 0
    if args.only == "e2e-agreement":
        ref = bench_e2e(device)
        for key, mixed in (("e2e_bandwidth_kernels", False), ("e2e_mixed_batching", True)):
            bw = bench_e2e(device, mixed=mixed, exact=False)
            agreement = token_agreement(ref["_tokens"], bw["_tokens"], device)
            log(f"{key}: {json.dumps(agreement)}")
            print(json.dumps({key: agreement}), flush=True)
        return 0
    dec = bench_decode(args.steps, args.warmup, device)
    log(f"decode: {dec['ms_per_step']:.3f} ms/step, {dec['value']:.1f} GB/s; attention launch "
        f"{dec['attn_launch_ms']:.3f} ms = {dec['roofline']['achieved']:.1f} GB/s "
        f"({100 * dec['roofline']['frac']:.1f}% of peak)")
    w = dec.pop("workload")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_decode_full(w, device)
        log(f"cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads ({cpu['ms_per_layer']:.0f} ms per layer)")
    ctx_sum = sum(w.context_lens)
    num_blocks = w.num_blocks
    del w
    torch.cuda.empty_cache()

    kernels = {}
    if args.only == "all":
        want_cpu = not args.no_cpu_baseline
        kernels["device_copy"] = bench_copy(5, device)
        ceil = kernels["device_copy"]["ceiling"]
        log(f"device copy: {kernels['device_copy']['achieved_GBps']:.1f} GB/s; calibration streams: read+write "
            f"{ceil['read_write_GBps']:.0f}, read {ceil['read_GBps']:.0f}, write {ceil['write_GBps']:.0f} GB/s")
        log(f"scattered-block copies: destination {ceil['scattered_write_copy_GBps']:.0f}, source "
            f"{ceil['scattered_read_copy_GBps']:.0f} GB/s")
        for key, kind in (("scatter", "fragmented"), ("scatter_near_sequential_tables", "near_sequential")):
            kernels[key] = bench_scatter(max(args.steps, 10), 3, device, "token", ceil["read_write_GBps"],
                                         cpu=want_cpu and kind == "fragmented",
                                         pattern_ceiling=ceil["scattered_write_copy_GBps"], tables=kind)
            r = kernels[key]
            log(f"scatter, {kind} tables ({100 * r['consecutive_block_fraction']:.1f}% consecutive): "
                f"{r['achieved_GBps']:.1f} GB/s ({100 * r['frac']:.1f}% of peak, "
                f"{100 * r['frac_of_copy_ceiling']:.1f}% of the copy ceiling, "
                f"{100 * r['frac_of_scattered_write_copy']:.1f}% of the scattered-destination copy)")
        kernels["scatter_head_major_source"] = bench_scatter(max(args.steps, 10), 3, device, "head",
                                                             ceil["read_write_GBps"],
                                                             pattern_ceiling=ceil["scattered_write_copy_GBps"])
        log(f"scatter, head-major source: {kernels['scatter_head_major_source']['achieved_GBps']:.1f} GB/s")
        for key, kind in (("gather", "fragmented"), ("gather_near_sequential_tables", "near_sequential")):
            kernels[key] = bench_gather(max(args.steps // 2, 6), 2, device, ceil["read_write_GBps"],
                                        cpu=want_cpu and kind == "fragmented",
                                        pattern_ceiling=ceil["scattered_read_copy_GBps"], tables=kind)
            r = kernels[key]
            log(f"gather, {kind} tables ({100 * r['consecutive_block_fraction']:.1f}% consecutive): "
                f"{r['achieved_GBps']:.1f} GB/s ({100 * r['frac']:.1f}% of peak, "
                f"{100 * r['frac_of_copy_ceiling']:.1f}% of the copy ceiling, "
                f"{100 * r['frac_of_scattered_read_copy']:.1f}% of the scattered-source copy)")
        # 20 untimed layers (~90 ms): with 3, the first timed layers of a process ran ~5% slow.
        kernels["chunked_prefill"] = bench_prefill(max(args.steps // 2, 5), 20, device, cpu=want_cpu)
        log(f"chunked prefill: {kernels['chunked_prefill']['ms_per_layer']:.2f} ms/layer, "
            f"{kernels['chunked_prefill']['achieved_TFLOPs']:.1f} TFLOP/s")
        kernels["exact_prefill"] = bench_exact_prefill(max(args.steps // 2, 5), 3, device)
        log(f"exact prefill: {kernels['exact_prefill']['ms_per_layer'] * 1000:.0f} us/layer, "
            f"{kernels['exact_prefill']['achieved_TFLOPs']:.1f} TFLOP/s fp64")
        torch.cuda.empty_cache()
        kernels["kv_block_swap"] = bench_swap(max(args.steps // 4, 3), 1, device)
        sw = kernels["kv_block_swap"]
        log(f"kv block records: pack {sw['pack']['achieved_GBps']:.1f} GB/s, unpack "
            f"{sw['unpack']['achieved_GBps']:.1f} GB/s; swap out {sw['swap_out']['achieved_GBps']:.1f} GB/s, "
            f"swap in {sw['swap_in']['achieved_GBps']:.1f} GB/s")
        torch.cuda.empty_cache()
    e2e = e2e_mixed = e2e_mixed_exact = e2e_mixed_capped = e2e_bw = None
    if args.only == "all":
        e2e = bench_e2e(device)
        log(f"e2e: {e2e['output_tok_s']:.1f} output tok/s (busy), {e2e['wall_tok_s']:.1f} tok/s (wall)")
        e2e_bw = bench_e2e(device, exact=False)
        e2e_bw["token_agreement"] = token_agreement(e2e["_tokens"], e2e_bw["_tokens"], device)
        log(f"e2e bandwidth kernels: {e2e_bw['output_tok_s']:.1f} output tok/s (busy), ITL max "
            f"{e2e_bw['latency_ms']['itl_ms_max']:.2f} ms; {e2e_bw['token_agreement']['identical_requests']} of 128 "
            f"requests token-identical to reference numerics")
        e2e_mixed = bench_e2e(device, mixed=True, exact=False)
        e2e_mixed["token_agreement"] = token_agreement(e2e["_tokens"], e2e_mixed["_tokens"], device)
        log(f"e2e mixed batching (bandwidth kernels): {e2e_mixed['output_tok_s']:.1f} output tok/s (busy), ITL max "
            f"{e2e_mixed['latency_ms']['itl_ms_max']:.2f} ms; {e2e_mixed['token_agreement']['identical_requests']} "
            f"of 128 requests token-identical")
        e2e_mixed_exact = bench_e2e(device, mixed=True)
        e2e_mixed_exact["token_agreement"] = token_agreement(e2e["_tokens"], e2e_mixed_exact["_tokens"], device)
        log(f"e2e mixed batching (reference numerics): {e2e_mixed_exact['output_tok_s']:.1f} output tok/s (busy), "
            f"ITL max {e2e_mixed_exact['latency_ms']['itl_ms_max']:.2f} ms")
        e2e_mixed_capped = bench_e2e(device, mixed=True, mixed_chunk_tokens=MIXED_CHUNK_CAP)
        for r in (e2e, e2e_bw, e2e_mixed, e2e_mixed_exact, e2e_mixed_capped):
            r.pop("_tokens")
        log(f"e2e mixed batching (reference numerics, at most {MIXED_CHUNK_CAP} prompt tokens per mixed step): "
            f"{e2e_mixed_capped['output_tok_s']:.1f} output tok/s (busy), ITL max "
            f"{e2e_mixed_capped['latency_ms']['itl_ms_max']:.2f} ms, TTFT p95 "
            f"{e2e_mixed_capped['latency_ms']['ttft_ms_p95']:.2f} ms")
        if not args.no_cpu_baseline:
            e2e["cpu_baseline"] = cpu_baseline_e2e()
            log(f"e2e cpu baseline: {e2e['cpu_baseline']['value']:.2f} output tok/s")

    line = {
        "metric": METRIC,
        "value": round(dec["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "paged decode attention step over 28 layers (append + attention per layer), batch 256, "
                        "contexts lognormal median 2048 sigma 1.3 clipped [256,8192], 16q/8kv heads, head_dim 128, "
                        "block 16, randomly permuted blocks",
            "batch": 256,
            "sum_context_tokens": ctx_sum,
            "pool_blocks": num_blocks,
            "kv_bytes_per_step": ctx_sum * 4096 * 28,
            "pct_hbm_peak": round(100 * dec["value"] / HBM_PEAK_GBS, 2),
        },
        "roofline": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in dec["roofline"].items()},
        "read_ceiling_GBps": kernels.get("device_copy", {}).get("ceiling", {}).get("read_GBps"),
        "cpu_baseline": cpu,
        "kernels": kernels,
        "e2e": e2e,
        "e2e_mixed_batching": e2e_mixed,
        "e2e_mixed_batching_exact": e2e_mixed_exact,
        "e2e_mixed_batching_exact_chunk_cap": e2e_mixed_capped,
        "e2e_bandwidth_kernels": e2e_bw,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
