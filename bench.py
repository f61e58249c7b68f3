#!/usr/bin/env python3
"""Benchmark of the KV-cache hot path on one MI355X (BASELINE.json metric).

Workload (config 2): Qwen3-0.6B ragged batched decode over all 28 layers, fp16,
batch 32, context lengths U[128, 4096], 16-token pages in a 16384-page pool per
layer.  One step = for each of the 28 layers store_kv (one new token per sequence)
and paged decode attention, launched back to back on one stream through the C ABI
(no Python validation inside the timed region).  Layer 0's decode also writes the
step plan (the split of the batch's keys over the CUs, which every layer shares;
ifn_paged_decode_planning) and layers 1-27 read it (ifn_paged_decode_planned).

Reported:
  value            paged-decode attention HBM GB/s = algorithmic decode bytes / mean
                   decode kernel time over the 28 layers of the K timed steps; the
                   times come from HIP events recorded on the launch stream around
                   every launch
  plan_kernel_step the same step with the plan as a launch of its own first
                   (ifn_paged_decode_plan), for comparison
  kv_append_us_per_layer   the same events around every store_kv launch
  roofline         the decode kernel against 8 TB/s HBM (its own launches); traffic
                   (HBM bytes per launch from rocprofv3 FETCH_SIZE/WRITE_SIZE) is read
                   from the committed profile summary when it exists
  append_batched   the bandwidth-sized append (28 layers x 2048 tokens, one
                   launch) against 8 TB/s
  config1          the CPU-runnable case: one token's append + decode, µs per call
  page_size_sweep  config 2's planned decode over 16-, 32- and 64-token pages (same bytes)
  cpu_baseline     torch-CPU float32 SDPA (enable_gqa) over each row's gathered pages,
                   on all the host cores this process may use, on a bounded sample of
                   the same decode workload (value); the CPU oracle (plain C port of
                   the same algorithm, rows split over the same threads, and on one
                   thread) beside it as c_port
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged-decode attn HBM GB/s (% of peak) + KV-append µs/layer, Qwen3-0.6B B=32"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_config2_traffic.json")


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h: no cache writeback/invalidate on record


class HipEvents:
    """Thin ctypes access to hipEventCreateWithFlags/Record/ElapsedTime, cheap enough to bracket every
    launch.  The events are created with hipEventDisableSystemFence: a default event record performs a
    system-scope release (L2 writeback + invalidate) that lands inside the measured interval and slows
    the next kernel; these events only time work, and elapsed times are read after a device sync."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n: int) -> list:
        evs = []
        for _ in range(n):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreateWithFlags(ctypes.byref(e), HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            evs.append(e)
        return evs

    def elapsed_ms(self, a, b) -> float:
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, evs) -> None:
        for e in evs:
            self.hip.hipEventDestroy(e)


def _compact(pool_layer, table, lens, bs=16):
    import torch
    used = sorted({int(p) for b in range(table.shape[0]) for p in table[b, :-(-int(lens[b]) // bs)]})
    idx = torch.as_tensor(used, dtype=torch.long, device=pool_layer.device)
    sub = pool_layer.index_select(1, idx).cpu().numpy()
    remap = np.zeros(int(table.max()) + 1, np.int32)
    remap[np.asarray(used)] = np.arange(len(used), dtype=np.int32)
    t2 = np.zeros_like(table)
    for b in range(table.shape[0]):
        n = -(-int(lens[b]) // bs)
        t2[b, :n] = remap[table[b, :n]]
    return sub, t2


def run_cpu_baseline(w, pool_layer, q, seconds: float) -> dict:
    """The config-2 decode of one layer on the host cores, two ways, for about ``seconds`` in all.

    value: torch-CPU float32 scaled_dot_product_attention(enable_gqa=True) per row -- the contiguous
    SDPA of model.py:196-200 -- after gathering the row's pages (index_select) and upcasting them, on
    all the process's host threads (the attention a CPU host would run for this step).  c_port: the
    oracle (plain C port of the same algorithm) on all rows per pass, rows split over the same
    threads, then on one thread."""
    import torch
    import torch.nn.functional as F

    import oracle
    sub, t2 = _compact(pool_layer, w.block_tables, w.seq_lens)
    qn = q.cpu().numpy()
    tok = 2 * w.num_kv_heads * w.head_dim * 2
    row_bytes = [int(L) * tok + 2 * w.num_q_heads * w.head_dim * 2 for L in w.seq_lens]
    threads = oracle.host_threads()

    def timed(fn, budget):
        passes, t0 = 0, time.perf_counter()
        while True:
            fn()
            passes += 1
            if time.perf_counter() - t0 >= budget:
                return passes, time.perf_counter() - t0

    # torch-CPU SDPA over the gathered pages
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    sub_t = torch.from_numpy(sub)                       # [2, pages, 16, Hkv, D] fp16
    q_t = torch.from_numpy(qn).float()                  # [B, Hq, D]
    tables = [torch.from_numpy(np.ascontiguousarray(t2[b, :-(-int(L) // 16)]).astype(np.int64))
              for b, L in enumerate(w.seq_lens)]
    hkv, d = w.num_kv_heads, w.head_dim

    def sdpa_pass():
        for b, L in enumerate(w.seq_lens):
            L = int(L)
            kv = sub_t.index_select(1, tables[b]).reshape(2, -1, hkv, d)[:, :L].float()  # [2, L, Hkv, D]
            k, v = kv[0].transpose(0, 1)[None], kv[1].transpose(0, 1)[None]          # [1, Hkv, L, D]
            F.scaled_dot_product_attention(q_t[b][None, :, None, :], k, v, enable_gqa=True)

    with torch.inference_mode():
        passes_t, dt_t = timed(sdpa_pass, seconds / 2)
    torch.set_num_threads(prev_threads)
    bytes_t = passes_t * sum(row_bytes)

    # the C port
    passes, dt = timed(lambda: oracle.paged_attention_rows(qn, sub, t2, w.seq_lens, threads=threads), seconds / 3)
    nbytes = passes * sum(row_bytes)
    rows1, bytes1, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 6:
        b = rows1 % w.batch
        oracle.paged_attention(qn[b:b + 1], sub, t2[b:b + 1], w.seq_lens[b:b + 1])
        rows1 += 1
        bytes1 += row_bytes[b]
    dt1 = time.perf_counter() - t0
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return {"value": round(bytes_t / dt_t / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"torch {torch.__version__} CPU: per config-2 decode row of layer 0, index_select of its "
                      f"pages, fp32 upcast, scaled_dot_product_attention(enable_gqa=True); {passes_t} passes over "
                      f"all 32 rows ({bytes_t / 1e6:.1f} MB algorithmic) in {dt_t:.1f} s on {threads} threads",
            "c_port": {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": threads,
                       "sample": f"CPU oracle (oracle/ifn_oracle.c, scalar C) on all 32 rows, {passes} passes "
                                 f"({nbytes / 1e6:.1f} MB) in {dt:.1f} s, rows split over {threads} threads",
                       "single_thread_GB/s": round(bytes1 / dt1 / 1e9, 4)},
            "affinity_cores": affinity, "cpu_model": _cpu_model()}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_prefill(lib, hip, dev, g, stream) -> dict:
    """Config 3: 2048-token prompt as four 512-token chunks over 28 layers; per chunk-layer
    store_kv (512 tokens) then causal paged attention (MFMA).  Times every attention launch."""
    import torch
    from infurnace_amd import workloads
    w = workloads.config3()
    L, hq, hkv, d, C = w.num_layers, w.num_q_heads, w.num_kv_heads, w.head_dim, w.chunk
    pool = torch.empty((L, 2, w.num_pages, 16, hkv, d), dtype=torch.float16, device=dev).normal_(generator=g)
    q = torch.randn((L, 4, C, hq, d), generator=g, device=dev, dtype=torch.float16)
    k = torch.randn((L, 4, C, hkv, d), generator=g, device=dev, dtype=torch.float16)
    v = torch.randn((L, 4, C, hkv, d), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty((C, hq, d), dtype=torch.float16, device=dev)
    table = torch.from_numpy(w.block_table).to(dev)
    pos = np.arange(w.prompt_len)
    slots = torch.from_numpy((w.block_table.astype(np.int64)[pos // 16] * 16 + pos % 16).astype(np.int32)).to(dev)
    ws_bytes = max(lib.ifn_paged_prefill_workspace_bytes(C, c * C, hq, hkv, d, 16) for c in range(4))
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    lb = pool[0].numel() * 2
    scale = 1.0 / np.sqrt(d)

    def one_pass(evs=None):
        j = 0
        for layer in range(L):
            for c in range(4):
                if evs is not None:
                    hip.hip.hipEventRecord(evs[3 * j], stream)
                rc = lib.ifn_store_kv(pool.data_ptr() + layer * lb, w.num_pages, slots.data_ptr() + 4 * c * C, None,
                                      k[layer, c].data_ptr(), v[layer, c].data_ptr(), C, hkv, d, 16, stream)
                if evs is not None:
                    hip.hip.hipEventRecord(evs[3 * j + 1], stream)
                rc |= lib.ifn_paged_prefill(out.data_ptr(), q[layer, c].data_ptr(), pool.data_ptr() + layer * lb,
                                            w.num_pages, table.data_ptr(), w.block_table.shape[0], c * C, C, hq, hkv,
                                            d, 16, scale, ws.data_ptr(), ws_bytes, stream)
                if evs is not None:
                    hip.hip.hipEventRecord(evs[3 * j + 2], stream)
                if rc:
                    raise RuntimeError(f"prefill launch failed: {rc}")
                j += 1

    def fused_pass(evs=None):  # ifn_paged_prefill_append: the store and the attention in one launch
        j = 0
        for layer in range(L):
            for c in range(4):
                if evs is not None:
                    hip.hip.hipEventRecord(evs[2 * j], stream)
                rc = lib.ifn_paged_prefill_append(out.data_ptr(), q[layer, c].data_ptr(), pool.data_ptr() + layer * lb,
                                                  w.num_pages, table.data_ptr(), w.block_table.shape[0], c * C, C,
                                                  k[layer, c].data_ptr(), v[layer, c].data_ptr(), hq, hkv, d, 16,
                                                  scale, ws.data_ptr(), ws_bytes, stream)
                if evs is not None:
                    hip.hip.hipEventRecord(evs[2 * j + 1], stream)
                if rc:
                    raise RuntimeError(f"fused prefill launch failed: {rc}")
                j += 1

    one_pass()
    torch.cuda.synchronize()
    evs = hip.create(3 * L * 4)
    one_pass(evs)
    torch.cuda.synchronize()
    ms = np.asarray([hip.elapsed_ms(evs[3 * j + 1], evs[3 * j + 2]) for j in range(L * 4)]).reshape(L, 4)
    st_ms = np.asarray([hip.elapsed_ms(evs[3 * j], evs[3 * j + 1]) for j in range(L * 4)]).reshape(L, 4)
    hip.destroy(evs)
    fused_pass()
    torch.cuda.synchronize()
    fevs = hip.create(2 * L * 4)
    fused_pass(fevs)
    torch.cuda.synchronize()
    fms = np.asarray([hip.elapsed_ms(fevs[2 * j], fevs[2 * j + 1]) for j in range(L * 4)]).reshape(L, 4)
    hip.destroy(fevs)
    flops = np.asarray([w.chunk_flops(c) for c in range(4)], np.float64)
    per_chunk_us = ms.mean(0) * 1e3
    tflops = float(flops.sum() * L / (ms.sum() / 1e3) / 1e12)
    return {"workload": w.name + ", 28 layers, store_kv + causal paged attention per chunk-layer",
            "attn_us_per_chunk_layer": [round(float(x), 2) for x in per_chunk_us],
            "attn_us_per_layer": round(float(ms.sum(1).mean() * 1e3), 2),
            "gflop_per_layer": round(float(flops.sum() / 1e9), 3),
            "TFLOP/s": round(tflops, 2), "mfma_peak_TFLOP/s": MFMA_F16_PEAK_TFLOPS,
            "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "store_us_per_chunk_layer": round(float(st_ms.mean() * 1e3), 2),
            "fused_us_per_chunk_layer": [round(float(x), 2) for x in fms.mean(0) * 1e3],
            "fused_us_per_layer": round(float(fms.sum(1).mean() * 1e3), 2),
            "two_launch_us_per_layer": round(float((ms + st_ms).sum(1).mean() * 1e3), 2)}


def run_prefill_prep(lib, hip, dev, g, stream) -> dict:
    """Config 3 from fp32 projections: per chunk-layer, the pre-append (q/k RMSNorm + rotary + fp16
    cast + append) and the causal attention, as two launches (ifn_qk_norm_rope_append then
    ifn_paged_prefill) and as one (ifn_paged_prefill_prep_append); HIP events around each
    chunk-layer's launches."""
    import torch
    from infurnace_amd import workloads
    from infurnace_amd.kernels import rope_table
    w = workloads.config3()
    L, hq, hkv, d, C = w.num_layers, w.num_q_heads, w.num_kv_heads, w.head_dim, w.chunk
    pool = torch.zeros((L, 2, w.num_pages, 16, hkv, d), dtype=torch.float16, device=dev)
    q = torch.randn((L, 4, C, hq, d), generator=g, device=dev)
    k = torch.randn((L, 4, C, hkv, d), generator=g, device=dev)
    v = torch.randn((L, 4, C, hkv, d), generator=g, device=dev)
    wt = 1 + 0.1 * torch.randn(d, generator=g, device=dev)
    rope = rope_table(w.prompt_len, d, 1e6, device=dev)
    table = torch.from_numpy(w.block_table).to(dev)
    pos = np.arange(w.prompt_len)
    positions = torch.from_numpy(pos.astype(np.int32)).to(dev)
    slots = torch.from_numpy((w.block_table.astype(np.int64)[pos // 16] * 16 + pos % 16).astype(np.int32)).to(dev)
    q16 = torch.empty((C, hq, d), dtype=torch.float16, device=dev)
    out = torch.empty((C, hq, d), dtype=torch.float16, device=dev)
    ws_bytes = max(lib.ifn_paged_prefill_workspace_bytes(C, c * C, hq, hkv, d, 16) for c in range(4))
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    lb = pool[0].numel() * 2
    scale = 1.0 / np.sqrt(d)

    def two(layer, c):
        rc = lib.ifn_qk_norm_rope_append(q16.data_ptr(), q[layer, c].data_ptr(), k[layer, c].data_ptr(),
                                         v[layer, c].data_ptr(), wt.data_ptr(), wt.data_ptr(), rope.data_ptr(),
                                         rope.shape[0], positions.data_ptr() + 4 * c * C, slots.data_ptr() + 4 * c * C,
                                         None, pool.data_ptr() + layer * lb, w.num_pages, C, hq, hkv, d, 16, 1e-6,
                                         stream)
        rc |= lib.ifn_paged_prefill(out.data_ptr(), q16.data_ptr(), pool.data_ptr() + layer * lb, w.num_pages,
                                    table.data_ptr(), w.block_table.shape[0], c * C, C, hq, hkv, d, 16, scale,
                                    ws.data_ptr(), ws_bytes, stream)
        if rc:
            raise RuntimeError(f"two-launch prefill chunk failed: {rc}")

    def one(layer, c):
        rc = lib.ifn_paged_prefill_prep_append(out.data_ptr(), q[layer, c].data_ptr(), k[layer, c].data_ptr(),
                                               v[layer, c].data_ptr(), wt.data_ptr(), wt.data_ptr(), rope.data_ptr(),
                                               rope.shape[0], pool.data_ptr() + layer * lb, w.num_pages,
                                               table.data_ptr(), w.block_table.shape[0], c * C, C, hq, hkv, d, 16,
                                               1e-6, scale, ws.data_ptr(), ws_bytes, stream)
        if rc:
            raise RuntimeError(f"fused prefill chunk failed: {rc}")

    def timed(fn):
        for layer in range(L):
            for c in range(4):
                fn(layer, c)
        torch.cuda.synchronize()
        evs = hip.create(2 * L * 4)
        for layer in range(L):
            for c in range(4):
                j = layer * 4 + c
                hip.hip.hipEventRecord(evs[2 * j], stream)
                fn(layer, c)
                hip.hip.hipEventRecord(evs[2 * j + 1], stream)
        torch.cuda.synchronize()
        ms = np.asarray([hip.elapsed_ms(evs[2 * j], evs[2 * j + 1]) for j in range(L * 4)]).reshape(L, 4)
        hip.destroy(evs)
        return ms

    ms2 = timed(two)
    ms1 = timed(one)
    return {"prep_workload": "config 3 from fp32 projections: q/k RMSNorm + rotary + fp16 cast + append, then "
                             "causal attention, per chunk-layer",
            "prep_entry": "ifn_paged_prefill_prep_append (one launch per chunk-layer)",
            "prep_fused_us_per_chunk_layer": [round(float(x), 2) for x in ms1.mean(0) * 1e3],
            "prep_fused_us_per_layer": round(float(ms1.sum(1).mean() * 1e3), 2),
            "prep_two_launch_us_per_chunk_layer": [round(float(x), 2) for x in ms2.mean(0) * 1e3],
            "prep_two_launch_us_per_layer": round(float(ms2.sum(1).mean() * 1e3), 2)}


def run_pre_append(lib, hip, dev, g, stream) -> dict:
    """Fused pre-append (q/k RMSNorm + rotary + fp16 cast + slot append) on config-3 chunks:
    512 tokens per launch, 28 layers with distinct inputs, HIP events around every launch."""
    import torch
    from infurnace_amd import workloads
    from infurnace_amd.kernels import rope_table
    w = workloads.config3()
    L, hq, hkv, d, T = w.num_layers, w.num_q_heads, w.num_kv_heads, w.head_dim, w.chunk
    pool = torch.zeros((L, 2, w.num_pages, 16, hkv, d), dtype=torch.float16, device=dev)
    q = torch.randn((L, T, hq, d), generator=g, device=dev)
    k = torch.randn((L, T, hkv, d), generator=g, device=dev)
    v = torch.randn((L, T, hkv, d), generator=g, device=dev)
    qw = torch.ones(d, device=dev)
    rope = rope_table(w.prompt_len, d, 1e6, device=dev)
    pos = torch.arange(T, dtype=torch.int32, device=dev) + 3 * T
    slots = torch.from_numpy((w.block_table.astype(np.int64)[(np.arange(T) + 3 * T) // 16] * 16
                              + (np.arange(T) + 3 * T) % 16).astype(np.int32)).to(dev)
    q_out = torch.empty((T, hq, d), dtype=torch.float16, device=dev)
    lb = pool[0].numel() * 2

    def one(layer):
        rc = lib.ifn_qk_norm_rope_append(q_out.data_ptr(), q[layer].data_ptr(), k[layer].data_ptr(), v[layer].data_ptr(),
                                         qw.data_ptr(), qw.data_ptr(), rope.data_ptr(), rope.shape[0], pos.data_ptr(),
                                         slots.data_ptr(), None, pool.data_ptr() + layer * lb, w.num_pages, T, hq, hkv,
                                         d, 16, 1e-6, stream)
        if rc:
            raise RuntimeError(f"pre-append launch failed: {rc}")

    for layer in range(L):
        one(layer)
    torch.cuda.synchronize()
    reps = 5
    evs = hip.create(2 * L * reps)
    for r in range(reps):
        for layer in range(L):
            hip.hip.hipEventRecord(evs[2 * (r * L + layer)], stream)
            one(layer)
            hip.hip.hipEventRecord(evs[2 * (r * L + layer) + 1], stream)
    torch.cuda.synchronize()
    us = float(np.mean([hip.elapsed_ms(evs[2 * j], evs[2 * j + 1]) for j in range(L * reps)])) * 1e3
    hip.destroy(evs)
    rows = T * (hq + 2 * hkv)
    nbytes = rows * d * 4 + rows * d * 2 + T * d * 4 + 2 * d * 4 + 2 * T * 4  # fp32 in, fp16 out, rope rows
    gbps = nbytes / (us / 1e6) / 1e9
    return {"workload": "config-3 chunk: 512 tokens x (16 q + 8 k + 8 v heads) x 128, 28 layers",
            "us_per_launch": round(us, 2), "bytes": nbytes, "GB/s": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4)}


def run_prep_step(lib, hip, dev, g, stream, w, pool, plan, plan_bytes, ws, ws_bytes, steps: int) -> dict:
    """Config 2's decode step from fp32 projections: per layer either the pre-append
    (ifn_qk_norm_rope_append, 32 tokens) then the planned decode, or both in one launch
    (ifn_paged_decode_prep_append).  Same plan, pool and workspace as the headline step; HIP events
    around every launch."""
    import torch
    from infurnace_amd.kernels import rope_table
    L, B, hq, hkv, d, P = w.num_layers, w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_pages
    q32 = torch.randn((L, B, hq, d), generator=g, device=dev)
    k32 = torch.randn((L, B, hkv, d), generator=g, device=dev)
    v32 = torch.randn((L, B, hkv, d), generator=g, device=dev)
    nw = torch.ones(d, device=dev) + 0.1 * torch.randn(d, generator=g, device=dev)
    max_len = int(w.seq_lens.max())
    rope = rope_table(max_len, d, 1e6, device=dev)
    pos = torch.from_numpy((w.seq_lens - 1).astype(np.int32)).to(dev)
    bt = torch.from_numpy(w.block_tables).to(dev)
    sl = torch.from_numpy(w.seq_lens).to(dev)
    slots = torch.from_numpy(w.append_slots).to(dev)
    q16 = torch.empty((B, hq, d), dtype=torch.float16, device=dev)
    out = torch.empty((B, hq, d), dtype=torch.float16, device=dev)
    lb = pool[0].numel() * 2
    scale = 1.0 / np.sqrt(d)

    def two(i):
        rc = lib.ifn_qk_norm_rope_append(q16.data_ptr(), q32[i].data_ptr(), k32[i].data_ptr(), v32[i].data_ptr(),
                                         nw.data_ptr(), nw.data_ptr(), rope.data_ptr(), max_len, pos.data_ptr(),
                                         slots.data_ptr(), None, pool.data_ptr() + i * lb, P, B, hq, hkv, d, 16, 1e-6,
                                         stream)
        return rc | lib.ifn_paged_decode_planned(out.data_ptr(), q16.data_ptr(), pool.data_ptr() + i * lb, P,
                                                 bt.data_ptr(), w.max_pages, sl.data_ptr(), None, B, hq, hkv, d, 16,
                                                 max_len, scale, plan.data_ptr(), plan_bytes, ws.data_ptr(), ws_bytes,
                                                 stream)

    def one(i):
        return lib.ifn_paged_decode_prep_append(out.data_ptr(), q32[i].data_ptr(), k32[i].data_ptr(),
                                                v32[i].data_ptr(), nw.data_ptr(), nw.data_ptr(), rope.data_ptr(),
                                                max_len, pos.data_ptr(), slots.data_ptr(), pool.data_ptr() + i * lb, P,
                                                bt.data_ptr(), w.max_pages, sl.data_ptr(), None, B, hq, hkv, d, 16,
                                                max_len, scale, 1e-6, plan.data_ptr(), plan_bytes, ws.data_ptr(),
                                                ws_bytes, stream)

    res = {}
    for name, fn in (("two_launch", two), ("fused", one)):
        for i in range(L):
            if fn(i):
                raise RuntimeError(f"prep step ({name}) launch failed")
        torch.cuda.synchronize()
        evs = hip.create(2 * L * steps)
        for s_ in range(steps):
            for i in range(L):
                hip.hip.hipEventRecord(evs[2 * (s_ * L + i)], stream)
                fn(i)
                hip.hip.hipEventRecord(evs[2 * (s_ * L + i) + 1], stream)
        torch.cuda.synchronize()
        res[name] = float(np.mean([hip.elapsed_ms(evs[2 * j], evs[2 * j + 1]) for j in range(L * steps)])) * 1e3
        hip.destroy(evs)
    return {"workload": "config 2 decode step from fp32 projections: q/k RMSNorm + rotary + fp16 cast + append, "
                        "then planned decode, per layer",
            "entry": "ifn_paged_decode_prep_append (one launch per layer, after the step plan)",
            "us_per_layer": round(res["fused"], 3), "two_launch_us_per_layer": round(res["two_launch"], 3),
            "layers": L, "steps": steps}


def run_decode_config(lib, hip, dev, g, stream, w, layers: int, reps: int) -> dict:
    """Decode leg for a second or third workload (configs 4 and 5): `layers` distinct layer pools,
    store_kv (one token per row) then decode per layer; HIP events around every decode launch.
    For a table with shared pages the roofline counts each physical page once (`unique`); the
    logical K/V a launch attends is reported beside it.  Such a workload is timed through the
    shared-prefix entry point (prefix pass + decode over private pages, both inside the events),
    through the plain decode with cached page loads (the same entry with no shared pages: the path
    for rows that share pages outside a common leading run) and through ifn_paged_decode, whose
    streaming page loads re-read shared pages from HBM."""
    import torch
    B, hq, hkv, d, P = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_pages
    pool = torch.empty((layers, 2, P, 16, hkv, d), dtype=torch.float16, device=dev)
    for layer in range(layers):
        pool[layer].normal_(generator=g)
    q = torch.randn((layers, B, hq, d), generator=g, device=dev, dtype=torch.float16)
    nk = torch.randn((layers, B, hkv, d), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty((B, hq, d), dtype=torch.float16, device=dev)
    bt = torch.from_numpy(w.block_tables).to(dev)
    sl = torch.from_numpy(w.seq_lens).to(dev)
    slots = torch.from_numpy(w.append_slots).to(dev)
    max_len = int(w.seq_lens.max())
    sp = int(w.shared_prefix_pages or 0)
    prefix = torch.from_numpy(np.ascontiguousarray(w.block_tables[0, :sp])).to(dev) if sp else None
    ws_bytes = max(lib.ifn_paged_decode_workspace_bytes(B, hq, hkv, d, 16, max_len),
                   lib.ifn_paged_decode_shared_prefix_workspace_bytes(B, hq, hkv, d, 16, sp) if sp else 0)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    lb = pool[0].numel() * 2
    scale = 1.0 / np.sqrt(d)

    def one(layer, mode, evs=None, j=0):
        rc = lib.ifn_store_kv(pool.data_ptr() + layer * lb, P, slots.data_ptr(), None, nk[layer].data_ptr(),
                              nk[layer].data_ptr(), B, hkv, d, 16, stream)
        if evs is not None:
            hip.hip.hipEventRecord(evs[2 * j], stream)
        if mode in ("prefix", "cached"):
            n_sp = sp if mode == "prefix" else 0
            rc |= lib.ifn_paged_decode_shared_prefix(
                out.data_ptr(), q[layer].data_ptr(), pool.data_ptr() + layer * lb, P,
                prefix.data_ptr() if n_sp else None, n_sp, bt.data_ptr(), w.max_pages, sl.data_ptr(), None, B, hq,
                hkv, d, 16, max_len, scale, ws.data_ptr(), ws_bytes, stream)
        else:
            rc |= lib.ifn_paged_decode(out.data_ptr(), q[layer].data_ptr(), pool.data_ptr() + layer * lb, P,
                                       bt.data_ptr(), w.max_pages, sl.data_ptr(), None, B, hq, hkv, d, 16, max_len,
                                       scale, ws.data_ptr(), ws_bytes, stream)
        if evs is not None:
            hip.hip.hipEventRecord(evs[2 * j + 1], stream)
        if rc:
            raise RuntimeError(f"{w.name}: launch failed: {rc}")

    def timed(mode: str) -> float:
        for layer in range(layers):
            one(layer, mode)
        torch.cuda.synchronize()
        n = layers * reps
        evs = hip.create(2 * n)
        for r in range(reps):
            for layer in range(layers):
                one(layer, mode, evs, r * layers + layer)
        torch.cuda.synchronize()
        us = float(np.mean([hip.elapsed_ms(evs[2 * j], evs[2 * j + 1]) for j in range(n)])) * 1e3
        hip.destroy(evs)
        return us

    us = timed("prefix" if sp else "stream")
    us_cached = timed("cached") if sp else None
    us_stream = timed("stream") if sp else us
    del pool
    uniq = w.decode_bytes(unique=True)
    logical = w.decode_bytes()
    gbps = uniq / (us / 1e6) / 1e9
    res = {"workload": w.name, "layers_timed": layers, "reps": reps,
           "entry": "ifn_paged_decode_shared_prefix" if sp else "ifn_paged_decode",
           "decode_us_per_layer": round(us, 2), "bytes_per_layer": uniq, "GB/s": round(gbps, 1),
           "frac": round(gbps / HBM_PEAK_GBPS, 4), "logical_bytes_per_layer": logical,
           "effective_GB/s": round(logical / (us / 1e6) / 1e9, 1)}
    if sp:
        res["plain_decode_us_per_layer"] = round(us_cached, 2)  # cached page loads
        res["plain_stream_decode_us_per_layer"] = round(us_stream, 2)
    return res


def run_page_size_sweep(lib, hip, dev, g, stream, layers: int = 8, reps: int = 10) -> dict:
    """The page-size choice (docs/roadmap.md:327): config 2's lengths and query shapes over pools of
    the same bytes per layer (16384 x 16, 8192 x 32, 4096 x 64 tokens), each row's pages consecutive
    ids of one seeded permutation; planned decode, HIP events around every launch, `layers` distinct
    layer pools so that launches read cold HBM."""
    import torch
    w = workloads_mod().config2()
    B, hq, hkv, d = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim
    lens = w.seq_lens.astype(np.int32)
    max_len = int(lens.max())
    scale = 1.0 / np.sqrt(d)
    sl = torch.from_numpy(lens).to(dev)
    q = torch.randn((layers, B, hq, d), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty((B, hq, d), dtype=torch.float16, device=dev)
    res = {"workload": "config 2 lengths (B=32, U[128,4096]), 1 GiB of K/V per layer at every page size, planned decode",
           "layers_timed": layers, "reps": reps, "us_per_layer": {}}
    for bs in (16, 32, 64):
        P = 16384 * 16 // bs
        rng = np.random.default_rng(w.seed)
        perm = rng.permutation(P).astype(np.int32)
        pages = -(-lens // bs)
        table = np.zeros((B, int(-(-max_len // bs))), np.int32)
        off = 0
        for b in range(B):
            table[b, :pages[b]] = perm[off:off + pages[b]]
            off += int(pages[b])
        bt = torch.from_numpy(table).to(dev)
        max_pages = table.shape[1]
        pool = torch.empty((layers, 2, P, bs, hkv, d), dtype=torch.float16, device=dev)
        for layer in range(layers):
            pool[layer].normal_(generator=g)
        lb = pool[0].numel() * 2
        ws_bytes = lib.ifn_paged_decode_workspace_bytes(B, hq, hkv, d, bs, max_len)
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
        pb = lib.ifn_paged_decode_plan_bytes(B, hq, hkv, d, bs, max_pages, max_len)
        plan = torch.zeros(max(pb, 256), dtype=torch.uint8, device=dev)
        if lib.ifn_paged_decode_plan(plan.data_ptr(), pb, bt.data_ptr(), max_pages, sl.data_ptr(), None, None, P, B, hq,
                                     hkv, d, bs, max_len, stream):
            raise RuntimeError(f"page size {bs}: plan failed")

        def one(layer, evs=None, j=0):
            if evs is not None:
                hip.hip.hipEventRecord(evs[2 * j], stream)
            rc = lib.ifn_paged_decode_planned(out.data_ptr(), q[layer].data_ptr(), pool.data_ptr() + layer * lb, P,
                                              bt.data_ptr(), max_pages, sl.data_ptr(), None, B, hq, hkv, d, bs,
                                              max_len, scale, plan.data_ptr(), pb, ws.data_ptr(), ws_bytes, stream)
            if evs is not None:
                hip.hip.hipEventRecord(evs[2 * j + 1], stream)
            if rc:
                raise RuntimeError(f"page size {bs}: decode failed: {rc}")

        for layer in range(layers):
            one(layer)
        torch.cuda.synchronize()
        n = layers * reps
        evs = hip.create(2 * n)
        for r in range(reps):
            for layer in range(layers):
                one(layer, evs, r * layers + layer)
        torch.cuda.synchronize()
        us = float(np.mean([hip.elapsed_ms(evs[2 * j], evs[2 * j + 1]) for j in range(n)])) * 1e3
        hip.destroy(evs)
        res["us_per_layer"][str(bs)] = round(us, 2)
        del pool
        torch.cuda.empty_cache()
    return res


def run_config1(lib, hip, dev, stream, reps: int = 200) -> dict:
    """Config 1 (the CPU-runnable case): one token's append at position 511 and single-row decode over
    512 tokens, timed as two launches (ifn_store_kv + ifn_paged_decode), as one fused launch
    (ifn_paged_decode_append) and as one fused launch with the step plan (the plan's own launch
    timed beside it and charged per layer of a 28-layer step); µs per call from HIP events, median
    over ``reps`` calls."""
    import torch
    c = workloads_mod().config1()
    pool = torch.from_numpy(c["pool"]).to(dev)
    P = pool.shape[1]
    bt = torch.from_numpy(c["block_tables"]).to(dev)
    sl = torch.from_numpy(c["seq_lens"]).to(dev)
    slots = torch.from_numpy(c["slot_mapping"]).to(dev)
    q, k, v = (torch.from_numpy(c[n]).to(dev) for n in ("q", "new_k", "new_v"))
    out = torch.empty_like(q)
    ws_bytes = lib.ifn_paged_decode_workspace_bytes(1, 16, 8, 128, 16, 512)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    scale = float(c["scale"])

    def two():
        rc = lib.ifn_store_kv(pool.data_ptr(), P, slots.data_ptr(), None, k.data_ptr(), v.data_ptr(), 1, 8, 128, 16,
                              stream)
        return rc | lib.ifn_paged_decode(out.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), 32,
                                         sl.data_ptr(), None, 1, 16, 8, 128, 16, 512, scale, ws.data_ptr(), ws_bytes,
                                         stream)

    def fused():
        return lib.ifn_paged_decode_append(out.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), 32,
                                           sl.data_ptr(), None, slots.data_ptr(), k.data_ptr(), v.data_ptr(), 1, 16,
                                           8, 128, 16, 512, scale, ws.data_ptr(), ws_bytes, stream)

    # the step plan of a one-row decode step (built once per step, shared by its layers)
    plan_bytes = lib.ifn_paged_decode_plan_bytes(1, 16, 8, 128, 16, 32, 512)
    plan = torch.zeros(plan_bytes, dtype=torch.uint8, device=dev)

    def mkplan():
        return lib.ifn_paged_decode_plan(plan.data_ptr(), plan_bytes, bt.data_ptr(), 32, sl.data_ptr(), None,
                                         slots.data_ptr(), P, 1, 16, 8, 128, 16, 512, stream)

    def fused_planned():
        return lib.ifn_paged_decode_append_planned(out.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), 32,
                                                   sl.data_ptr(), None, slots.data_ptr(), k.data_ptr(), v.data_ptr(), 1,
                                                   16, 8, 128, 16, 512, scale, plan.data_ptr(), plan_bytes,
                                                   ws.data_ptr(), ws_bytes, stream)

    plan2 = torch.zeros(plan_bytes, dtype=torch.uint8, device=dev)

    def fused_planning():  # the step's first layer: decodes unplanned and writes the plan
        return lib.ifn_paged_decode_append_planning(out.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(),
                                                    32, sl.data_ptr(), None, slots.data_ptr(), k.data_ptr(),
                                                    v.data_ptr(), 1, 16, 8, 128, 16, 512, scale, plan2.data_ptr(),
                                                    plan_bytes, ws.data_ptr(), ws_bytes, stream)

    if mkplan():
        raise RuntimeError("config 1: plan launch failed")
    res = {"workload": "config 1: B=1, context 512, 64-page pool, one layer (append at 511 + decode)"}
    for name, fn in (("two_launch", two), ("fused", fused), ("fused_planned", fused_planned), ("plan", mkplan),
                     ("fused_planning", fused_planning)):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        evs = hip.create(2 * reps)
        t0 = time.perf_counter()
        for r in range(reps):
            hip.hip.hipEventRecord(evs[2 * r], stream)
            rc = fn()
            hip.hip.hipEventRecord(evs[2 * r + 1], stream)
            if rc:
                raise RuntimeError(f"config 1 {name}: launch failed: {rc}")
        torch.cuda.synchronize()
        wall_us = (time.perf_counter() - t0) / reps * 1e6
        res[f"{name}_us"] = round(float(np.median([hip.elapsed_ms(evs[2 * r], evs[2 * r + 1])
                                                   for r in range(reps)])) * 1e3, 2)
        res[f"{name}_host_us_per_call"] = round(wall_us, 2)  # launch rate through ctypes, back to back
        hip.destroy(evs)
    # a 28-layer step of the planned fused form: one plan, then 28 launches; or the first layer writing the
    # plan and 27 planned
    res["fused_planned_us_per_layer_with_plan"] = round(res["fused_planned_us"] + res["plan_us"] / 28, 2)
    res["fused_step_us_per_layer"] = round((res["fused_planning_us"] + 27 * res["fused_planned_us"]) / 28, 2)
    return res


def workloads_mod():
    from infurnace_amd import workloads
    return workloads


def run_config5_churn(lib, hip, dev, g, stream, steps: int) -> dict:
    """Config 5 as serving runs it: each step first churns 10% of the private pages (KVManager.replace_blocks
    frees them and takes fresh ones), uploads the new block tables, rewrites the fresh pages of all 36 layers
    (one ifn_store_kv_layers launch over their 16 slots each), then for each layer appends one token per row
    (ifn_store_kv) and decodes through the shared-prefix entry point.

    The pages come from a BlockPool handing out ids in the workload's seeded order, so the first step's
    tables are the workload's own.  Decode µs per layer (HIP events around every decode launch) and whole
    step ms (host clock, churn bookkeeping included) are reported separately."""
    import torch
    from infurnace_amd.cache import BlockPool, KVManager
    w = workloads_mod().config5()
    L, B, hq, hkv, d, P = w.num_layers, w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_pages
    sp = w.shared_prefix_pages
    perm = np.concatenate([w.block_tables[0, :sp], w.block_tables[:, sp:].reshape(-1), w.extra["free_ids"]])
    bpool = BlockPool(P, 16, reserve_dummy=False, order=perm)
    mgr = KVManager(bpool, max_pages_per_seq=w.max_pages)
    prefix = bpool.allocate(sp)
    for b in range(B):
        mgr.add_sequence(b, prefix_blocks=prefix, prefix_len=sp * 16)
        mgr.append(b, int(w.seq_lens[b]) - sp * 16)
    rows = list(range(B))
    table = mgr.block_tables(rows, max_pages=w.max_pages)
    assert np.array_equal(table, w.block_tables), "config 5: the pool's order does not reproduce the tables"

    pool = torch.empty((L, 2, P, 16, hkv, d), dtype=torch.float16, device=dev)
    for layer in range(L):
        pool[layer].normal_(generator=g)
    q = torch.randn((L, B, hq, d), generator=g, device=dev, dtype=torch.float16)
    nk = torch.randn((L, B, hkv, d), generator=g, device=dev, dtype=torch.float16)
    n_fresh = max(len(c) for c in w.extra["churn"])
    rk = torch.randn((L, n_fresh * 16, hkv, d), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty((B, hq, d), dtype=torch.float16, device=dev)
    bt = torch.from_numpy(table).to(dev)
    sl = torch.from_numpy(w.seq_lens).to(dev)
    slots = torch.empty(B, dtype=torch.int32, device=dev)
    fresh_slots = torch.empty(n_fresh * 16, dtype=torch.int32, device=dev)
    prefix_d = torch.as_tensor(np.asarray(prefix, np.int32), device=dev)
    max_len = int(w.seq_lens.max())
    ws_bytes = lib.ifn_paged_decode_shared_prefix_workspace_bytes(B, hq, hkv, d, 16, sp)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    lb = pool[0].numel() * 2
    scale = 1.0 / np.sqrt(d)
    pos = w.seq_lens.astype(np.int64) - 1

    def step(s_, evs=None, base=0):
        # churn: free 10% of the private pages and take fresh ones (host bookkeeping)
        ch = w.extra["churn"][s_ % len(w.extra["churn"])]
        fresh = []
        for b in np.unique(ch[:, 0]):
            fresh += mgr.replace_blocks(int(b), ch[ch[:, 0] == b, 1].tolist())
        tab = mgr.block_tables(rows, max_pages=w.max_pages)
        app = (tab[np.arange(B), pos // 16].astype(np.int64) * 16 + pos % 16).astype(np.int32)
        fs = (np.repeat(np.asarray(fresh, np.int64) * 16, 16) + np.tile(np.arange(16), len(fresh))).astype(np.int32)
        # uploads on the launch stream (pinned staging keeps them asynchronous and stream-ordered)
        bt.copy_(torch.from_numpy(tab).pin_memory(), non_blocking=True)
        slots.copy_(torch.from_numpy(app).pin_memory(), non_blocking=True)
        fresh_slots[:len(fs)].copy_(torch.from_numpy(fs).pin_memory(), non_blocking=True)
        # rewrite the fresh pages of every layer: one launch, 16 slots per page
        rc = lib.ifn_store_kv_layers(pool.data_ptr(), L, P, fresh_slots.data_ptr(), None, rk.data_ptr(),
                                     rk.data_ptr(), len(fs), hkv, d, 16, stream)
        for layer in range(L):
            rc |= lib.ifn_store_kv(pool.data_ptr() + layer * lb, P, slots.data_ptr(), None, nk[layer].data_ptr(),
                                   nk[layer].data_ptr(), B, hkv, d, 16, stream)
            if evs is not None:
                hip.hip.hipEventRecord(evs[base + 2 * layer], stream)
            rc |= lib.ifn_paged_decode_shared_prefix(
                out.data_ptr(), q[layer].data_ptr(), pool.data_ptr() + layer * lb, P, prefix_d.data_ptr(), sp,
                bt.data_ptr(), w.max_pages, sl.data_ptr(), None, B, hq, hkv, d, 16, max_len, scale, ws.data_ptr(),
                ws_bytes, stream)
            if evs is not None:
                hip.hip.hipEventRecord(evs[base + 2 * layer + 1], stream)
        if rc:
            raise RuntimeError(f"config 5 step {s_}: launch failed: {rc}")
        return len(fresh)

    step(0)
    torch.cuda.synchronize()
    evs = hip.create(2 * L * steps)
    t0 = time.perf_counter()
    churned = [step(1 + s_, evs, 2 * L * s_) for s_ in range(steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us = float(np.mean([hip.elapsed_ms(evs[2 * j], evs[2 * j + 1]) for j in range(L * steps)])) * 1e3
    hip.destroy(evs)
    bpool.check_invariants()
    # the roofline counts each physical page once, for the tables the timed steps used
    w_now = workloads_mod().DecodeWorkload(w.name, L, hq, hkv, d, P, w.seq_lens,
                                           mgr.block_tables(rows, max_pages=w.max_pages), w.seed,
                                           shared_prefix_pages=sp)
    uniq = w_now.decode_bytes(unique=True)
    logical = w_now.decode_bytes()
    del pool, rk
    gbps = uniq / (us / 1e6) / 1e9
    return {"workload": w.name + ", 36 layers, 10% private-page churn per step", "steps_timed": steps,
            "entry": "ifn_paged_decode_shared_prefix", "pages_churned_per_step": int(np.mean(churned)),
            "decode_us_per_layer": round(us, 2), "bytes_per_layer": uniq, "GB/s": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "logical_bytes_per_layer": logical,
            "effective_GB/s": round(logical / (us / 1e6) / 1e9, 1),
            "ms_per_step": round(wall / steps * 1e3, 3),
            "step": "churn (replace_blocks) + table upload + fresh-page rewrite (store_kv_layers) + 36 x "
                    "(store_kv + shared-prefix decode)"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-3 chunked-prefill leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the config-4 and config-5 decode legs")
    ap.add_argument("--profile-pass", action="store_true",
                    help="short run for rocprofv3 counter passes: no CPU baseline, no prefill leg, plus one "
                         "1 GiB elementwise copy (torch.neg) whose FETCH/WRITE counters calibrate HBM bytes")
    ap.add_argument("--config5-only", action="store_true",
                    help="counter runs of the shared-prefix path: only the config-5 legs (with churn, then "
                         "without) and the 1 GiB calibration copy; prints their JSON object")
    args = ap.parse_args()
    if args.profile_pass:
        args.no_cpu_baseline = True
        args.no_prefill = True
        args.no_extra = True
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the hot path shards by sequence "
              "with no exchange, so N GPUs run N independent copies of this benchmark.", file=sys.stderr)
        return 2

    import torch
    from infurnace_amd import _capi, workloads

    lib = _capi.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.config5_only:
        hip5 = HipEvents()
        stream5 = torch.cuda.current_stream(dev).cuda_stream
        g5 = torch.Generator(device=dev).manual_seed(workloads.config5().seed)
        res = run_config5_churn(lib, hip5, dev, g5, stream5, steps=2)
        torch.cuda.empty_cache()
        res["no_churn"] = run_decode_config(lib, hip5, dev, g5, stream5, workloads.config5(), layers=36, reps=1)
        torch.cuda.empty_cache()
        src = torch.empty(1 << 29, dtype=torch.float16, device=dev).normal_(generator=g5)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)  # reads 1 GiB, writes 1 GiB: the counters' calibration kernel
        torch.cuda.synchronize()
        print(json.dumps({"config5": res}), flush=True)
        return 0
    w = workloads.config2()
    L, B, hq, hkv, d, P = w.num_layers, w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_pages
    g = torch.Generator(device=dev).manual_seed(w.seed)
    print(f"[bench] allocating {L}x{P}-page pool ({L * P * 65536 / 2**30:.1f} GiB)", file=sys.stderr, flush=True)
    pool = torch.empty((L, 2, P, 16, hkv, d), dtype=torch.float16, device=dev)
    for layer in range(L):
        pool[layer].normal_(generator=g)
    q = torch.randn((L, B, hq, d), generator=g, device=dev, dtype=torch.float16)
    nk = torch.randn((L, B, hkv, d), generator=g, device=dev, dtype=torch.float16)
    nv = torch.randn((L, B, hkv, d), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty((L, B, hq, d), dtype=torch.float16, device=dev)
    bt = torch.from_numpy(w.block_tables).to(dev)
    sl = torch.from_numpy(w.seq_lens).to(dev)
    slots = torch.from_numpy(w.append_slots).to(dev)
    max_len = int(w.seq_lens.max())
    ws_bytes = lib.ifn_paged_decode_workspace_bytes(B, hq, hkv, d, 16, max_len)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    scale = 1.0 / np.sqrt(d)

    layer_bytes = pool[0].numel() * 2
    # the step plan: the split of the batch's keys over the CUs, shared by every layer of the step
    plan_bytes = lib.ifn_paged_decode_plan_bytes(B, hq, hkv, d, 16, w.max_pages, max_len)
    plan = torch.zeros(max(plan_bytes, 256), dtype=torch.uint8, device=dev)
    plan_args = (plan.data_ptr(), plan_bytes, bt.data_ptr(), w.max_pages, sl.data_ptr(), None, slots.data_ptr(), P,
                 B, hq, hkv, d, 16, max_len, stream)
    store_args = [(pool.data_ptr() + i * layer_bytes, P, slots.data_ptr(), None, nk[i].data_ptr(), nv[i].data_ptr(),
                   B, hkv, d, 16, stream) for i in range(L)]
    dec_args = [(out[i].data_ptr(), q[i].data_ptr(), pool.data_ptr() + i * layer_bytes, P, bt.data_ptr(),
                 w.max_pages, sl.data_ptr(), None, B, hq, hkv, d, 16, max_len, scale, plan.data_ptr(), plan_bytes,
                 ws.data_ptr(), ws_bytes, stream) for i in range(L)]
    plan_fn, store_fn, dec_fn = lib.ifn_paged_decode_plan, lib.ifn_store_kv, lib.ifn_paged_decode_planned
    planning_fn = lib.ifn_paged_decode_planning  # layer 0: decodes unplanned and writes the step's plan
    hip = HipEvents()
    E = 3 * L  # events per step: store_kv and decode per layer

    def step(evs=None, base=0):
        for i in range(L):
            b = base + 3 * i
            if evs is not None:
                hip.hip.hipEventRecord(evs[b], stream)
            rc = store_fn(*store_args[i])
            if evs is not None:
                hip.hip.hipEventRecord(evs[b + 1], stream)
            rc |= (planning_fn if i == 0 else dec_fn)(*dec_args[i])
            if evs is not None:
                hip.hip.hipEventRecord(evs[b + 2], stream)
            if rc:
                raise RuntimeError(f"launch failed in layer {i}: {_capi.status_string(rc)}")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    K = args.steps
    evs = hip.create(E * K)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s_ in range(K):
        step(evs, E * s_)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dec_ms = [hip.elapsed_ms(evs[E * s_ + 3 * i + 1], evs[E * s_ + 3 * i + 2]) for s_ in range(K) for i in range(L)]
    app_ms = [hip.elapsed_ms(evs[E * s_ + 3 * i], evs[E * s_ + 3 * i + 1]) for s_ in range(K) for i in range(L)]
    hip.destroy(evs)
    print(f"[bench] timed {K} steps x {L} layers in {wall:.3f} s", file=sys.stderr, flush=True)

    # The same step with the plan as its own launch (ifn_paged_decode_plan, then 28 planned decodes), for
    # comparison: the plan launch's time, and the planned layers'.
    PE = 2 + 2 * L

    def plan_step(evs=None, base=0):
        if evs is not None:
            hip.hip.hipEventRecord(evs[base], stream)
        rc = plan_fn(*plan_args)
        if evs is not None:
            hip.hip.hipEventRecord(evs[base + 1], stream)
        for i in range(L):
            rc |= store_fn(*store_args[i])
            if evs is not None:
                hip.hip.hipEventRecord(evs[base + 2 + 2 * i], stream)
            rc |= dec_fn(*dec_args[i])
            if evs is not None:
                hip.hip.hipEventRecord(evs[base + 3 + 2 * i], stream)
            if rc:
                raise RuntimeError(f"launch failed in layer {i}: {_capi.status_string(rc)}")

    plan_step()
    torch.cuda.synchronize()
    pevs = hip.create(PE * K)
    for s_ in range(K):
        plan_step(pevs, PE * s_)
    torch.cuda.synchronize()
    plan_ms = [hip.elapsed_ms(pevs[PE * s_], pevs[PE * s_ + 1]) for s_ in range(K)]
    planned_ms = [hip.elapsed_ms(pevs[PE * s_ + 2 + 2 * i], pevs[PE * s_ + 3 + 2 * i]) for s_ in range(K)
                  for i in range(L)]
    hip.destroy(pevs)

    # The same decode launches without a plan (each launch splits the batch itself), for comparison.
    unplanned_args = [a[:15] + a[17:] for a in dec_args]
    uevs = hip.create(2 * L * 2)
    for r in range(2):
        for i in range(L):
            hip.hip.hipEventRecord(uevs[2 * (r * L + i)], stream)
            rc = lib.ifn_paged_decode(*unplanned_args[i])
            hip.hip.hipEventRecord(uevs[2 * (r * L + i) + 1], stream)
            if rc:
                raise RuntimeError(_capi.status_string(rc))
    torch.cuda.synchronize()
    unplanned_us = float(np.mean([hip.elapsed_ms(uevs[2 * j], uevs[2 * j + 1]) for j in range(L, 2 * L)])) * 1e3
    hip.destroy(uevs)

    # The same step with the append fused into the decode launch (ifn_paged_decode_append_planned): one
    # launch per layer after the plan, same output and pool bytes.
    fused_args = [(out[i].data_ptr(), q[i].data_ptr(), pool.data_ptr() + i * layer_bytes, P, bt.data_ptr(),
                   w.max_pages, sl.data_ptr(), None, slots.data_ptr(), nk[i].data_ptr(), nv[i].data_ptr(), B, hq,
                   hkv, d, 16, max_len, scale, plan.data_ptr(), plan_bytes, ws.data_ptr(), ws_bytes, stream)
                  for i in range(L)]
    fused_fn, fused_planning_fn = lib.ifn_paged_decode_append_planned, lib.ifn_paged_decode_append_planning
    EF = 2 * L

    def fused_step(evs=None, base=0):
        rc = 0
        for i in range(L):
            if evs is not None:
                hip.hip.hipEventRecord(evs[base + 2 * i], stream)
            rc |= (fused_planning_fn if i == 0 else fused_fn)(*fused_args[i])
            if evs is not None:
                hip.hip.hipEventRecord(evs[base + 1 + 2 * i], stream)
            if rc:
                raise RuntimeError(f"fused launch failed in layer {i}: {_capi.status_string(rc)}")

    for _ in range(args.warmup):
        fused_step()
    torch.cuda.synchronize()
    fevs = hip.create(EF * K)
    t0 = time.perf_counter()
    for s_ in range(K):
        fused_step(fevs, EF * s_)
    torch.cuda.synchronize()
    fused_wall = time.perf_counter() - t0
    fused_ms = [hip.elapsed_ms(fevs[EF * s_ + 2 * i], fevs[EF * s_ + 1 + 2 * i]) for s_ in range(K) for i in range(L)]
    hip.destroy(fevs)
    prep_step = run_prep_step(lib, hip, dev, g, stream, w, pool, plan, plan_bytes, ws, ws_bytes, steps=4)

    dec_bytes = w.decode_bytes()
    dec_s = float(np.mean(dec_ms)) / 1e3            # the decode kernel, per launch (layer 0 writes the plan)
    plan_s = float(np.mean(plan_ms)) / 1e3          # the plan as its own launch, once per step (comparison)
    planned_s = float(np.mean(planned_ms)) / 1e3    # a planned layer after that plan launch (comparison)
    layer_s = dec_s                                 # the step has no other decode work
    gbps = dec_bytes / layer_s / 1e9
    kernel_gbps = dec_bytes / dec_s / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        try:
            traffic = json.load(open(TRAFFIC_FILE)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    # bandwidth-sized append: 28 layers x 2048 tokens in one launch (config 3 prompt)
    w3 = workloads.config3()
    del out
    T3 = w3.prompt_len
    pool3 = torch.empty((L, 2, w3.num_pages, 16, hkv, d), dtype=torch.float16, device=dev)
    k3 = torch.randn((L, T3, hkv, d), generator=g, device=dev, dtype=torch.float16)
    v3 = torch.randn((L, T3, hkv, d), generator=g, device=dev, dtype=torch.float16)
    slots3 = torch.from_numpy((w3.block_table.astype(np.int64)[np.arange(T3) // 16] * 16
                               + np.arange(T3) % 16).astype(np.int32)).to(dev)
    a_args = (pool3.data_ptr(), L, w3.num_pages, slots3.data_ptr(), None, k3.data_ptr(), v3.data_ptr(), T3, hkv, d,
              16, stream)
    for _ in range(3):
        lib.ifn_store_kv_layers(*a_args)
    reps = 20
    aev = hip.create(2 * reps)
    torch.cuda.synchronize()
    for r in range(reps):
        hip.hip.hipEventRecord(aev[2 * r], stream)
        rc = lib.ifn_store_kv_layers(*a_args)
        hip.hip.hipEventRecord(aev[2 * r + 1], stream)
        if rc:
            raise RuntimeError(_capi.status_string(rc))
    torch.cuda.synchronize()
    a_ms = float(np.median([hip.elapsed_ms(aev[2 * r], aev[2 * r + 1]) for r in range(reps)]))
    hip.destroy(aev)
    a_bytes = L * T3 * (2 * 2 * hkv * d * 2 + 4)
    a_gbps = a_bytes / (a_ms / 1e3) / 1e9
    del pool3, k3, v3

    prefill = None
    pre_append = None
    if not args.no_prefill:
        prefill = run_prefill(lib, hip, dev, g, stream)
        prefill.update(run_prefill_prep(lib, hip, dev, g, stream))
        pre_append = run_pre_append(lib, hip, dev, g, stream)

    extra = {}
    if not args.no_extra:
        cpu_pool = pool[0].cpu() if not args.no_cpu_baseline else None  # the CPU leg reads layer 0
        del pool
        torch.cuda.empty_cache()
        print("[bench] config 4 (8.6 GB per layer) ...", file=sys.stderr, flush=True)
        extra["config4"] = run_decode_config(lib, hip, dev, g, stream, workloads.config4(), layers=1, reps=10)
        torch.cuda.empty_cache()
        print("[bench] config 5 (Qwen3-8B shapes, shared prefix, page churn) ...", file=sys.stderr, flush=True)
        extra["config5"] = run_config5_churn(lib, hip, dev, g, stream, steps=4)
        torch.cuda.empty_cache()
        extra["config5"]["no_churn"] = run_decode_config(lib, hip, dev, g, stream, workloads.config5(), layers=36,
                                                         reps=3)
        torch.cuda.empty_cache()
        print("[bench] page-size sweep (16/32/64-token pages) ...", file=sys.stderr, flush=True)
        extra["page_size_sweep"] = run_page_size_sweep(lib, hip, dev, g, stream)
        torch.cuda.empty_cache()
    else:
        cpu_pool = pool[0]
    config1 = run_config1(lib, hip, dev, stream)

    if args.profile_pass:
        src = torch.empty(1 << 29, dtype=torch.float16, device=dev).normal_(generator=g)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)  # reads 1 GiB, writes 1 GiB: the counters' calibration kernel
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline ...", file=sys.stderr, flush=True)
        cpu = run_cpu_baseline(w, cpu_pool, q[0], args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(wall / K * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) fp16 pool/queries; numpy PCG64 lengths and page permutations)",
        "config": {"workload": w.name + ", 28 layers, store_kv + paged decode per layer",
                   "batch": B, "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d, "block_size": 16,
                   "pages_per_layer": P, "context_tokens": int(w.seq_lens.sum()), "layers": L, "seed": w.seed},
        "decode_frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "decode_us_per_layer": round(dec_s * 1e6, 3),
        "planning_layer_us": round(float(np.mean(dec_ms[::L])) * 1e3, 3),
        "plan_kernel_step": {"plan_us_per_step": round(plan_s * 1e6, 3),
                             "planned_decode_us_per_layer": round(planned_s * 1e6, 3),
                             "us_per_layer_with_plan": round((planned_s + plan_s / L) * 1e6, 3)},
        "decode_kernel_GB/s": round(kernel_gbps, 2),
        "unplanned_decode_us_per_layer": round(unplanned_us, 3),
        "decode_bytes_per_layer": dec_bytes,
        "kv_append_us_per_layer": round(float(np.mean(app_ms)) * 1e3, 3),
        "fused_step": {"entry": "ifn_paged_decode_append_planning (layer 0: writes the step plan), then "
                                "ifn_paged_decode_append_planned (store_kv + paged decode in one launch per layer)",
                       "us_per_layer": round(float(np.mean(fused_ms)) * 1e3, 3),
                       "two_launch_us_per_layer": round((float(np.mean(app_ms)) + float(np.mean(dec_ms))) * 1e3, 3),
                       # what the append adds to a decode launch when fused into it
                       "append_marginal_us_per_layer": round((float(np.mean(fused_ms)) - float(np.mean(dec_ms))) * 1e3,
                                                             3),
                       "ms_per_step": round(fused_wall / K * 1e3, 4)},
        "roofline": {"bound": "hbm", "kernel": "decode_rows_kernel", "achieved": round(kernel_gbps, 2),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(kernel_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic},
        "prep_step": prep_step,
        "append_batched": {"workload": "store_kv_layers, 28 layers x 2048 tokens (config 3 prompt), one launch",
                           "us": round(a_ms * 1e3, 2), "bytes": a_bytes, "GB/s": round(a_gbps, 2),
                           "frac": round(a_gbps / HBM_PEAK_GBPS, 4)},
        "prefill": prefill,
        "pre_append": pre_append,
        "config1": config1,
        "config4": extra.get("config4"),
        "config5": extra.get("config5"),
        "page_size_sweep": extra.get("page_size_sweep"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
