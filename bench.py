#!/usr/bin/env python3
"""Benchmark of the paged KV-cache hot path on one MI355X.

Default workload ("Llama-3-8B-shaped decode step"):
64 sequences, 32 layers, 32 query / 8 KV heads (GQA 4), head_dim 128, f16 KV,
block 16, context lengths uniform in [128, 4096] (seed 0), block tables
scattered over the pool by a seeded permutation. One step = for every layer,
append 1 token per sequence through the slot mapping, then paged decode
attention over the grown context. Q/K/V ~ N(0,1) (synthetic; no checkpoint).

Printed JSON line: value = decode-attention algorithmic HBM bytes per step /
wall time per step (whole step, appends included). roofline.achieved uses the
attention launches alone, timed with HIP events on the launch stream.
cpu_baseline times the oracle's AVX2 restatement of the reference loop on this
host, on one full layer of the same pool (a bounded sample).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, os.cpu_count())")
    return ap.parse_args()


def attn_bytes(ctx, hq, hkv, d, elem_bytes):
    """Algorithmic HBM bytes of decode attention for one (sequence, layer):
    K+V once per KV head (GQA shares tiles), q and out in f32, block table, ctx_len."""
    ctx = np.asarray(ctx, dtype=np.int64)
    return int((ctx * hkv * d * 2 * elem_bytes + hq * d * 4 * 2 + ((ctx + 15) // 16) * 4 + 4).sum())


def append_bytes(n_tokens, hkv, d, elem_bytes):
    """Per token per layer: f32 K/V read, stored K/V written, 8-byte slot."""
    return int(n_tokens * (2 * hkv * d * 4 + 2 * hkv * d * elem_bytes + 8))


def read_traffic(path):
    """HBM bytes per attention call from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (the line `hbm_bytes_per_launch: N`), or None when it is absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding of the path is design-only, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    import ferrum_amd as fa
    from ferrum_amd import _lib

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    lib = _lib.load()

    n_seqs, L, hq, hkv, d, bs = 64, 32, 32, 8, 128, 16
    K, W = args.steps, args.warmup
    rng = np.random.default_rng(args.seed)
    ctx0 = rng.integers(128, 4097, n_seqs).astype(np.int64)
    max_ctx_final = ctx0 + W + K
    nblk_seq = (max_ctx_final + bs - 1) // bs
    num_blocks = int(nblk_seq.sum()) + 64

    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=num_blocks, block_size=bs,
                                         kv_dtype=fa.DTYPE_F16))
    ids = pool.alloc_blocks(int(nblk_seq.sum()))
    ids = ids[rng.permutation(ids.size)]  # scatter every table over the pool
    max_blocks = int(nblk_seq.max())
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    off = 0
    for s in range(n_seqs):
        tables[s, : nblk_seq[s]] = ids[off: off + nblk_seq[s]]
        off += nblk_seq[s]
    tables_d = torch.from_numpy(tables).to(dev)

    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    # Initial context: bulk append of every sequence's prefix into every layer
    # (also the bulk-append throughput measurement).
    pos = np.concatenate([np.arange(c) for c in ctx0])
    seq_of = np.repeat(np.arange(n_seqs), ctx0)
    slots_fill = tables[seq_of, pos // bs].astype(np.int64) * bs + pos % bs
    slots_fill_d = torch.from_numpy(slots_fill).to(dev)
    n_fill = slots_fill.size
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ev_fill = []
    for layer in range(L):
        kf = torch.randn((n_fill, hkv, d), generator=gen, device=dev)
        vf = torch.randn((n_fill, hkv, d), generator=gen, device=dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        pool.append(layer, kf, vf, slots_fill_d)
        e1.record(stream)
        ev_fill.append((e0, e1))
        del kf, vf
    torch.cuda.synchronize()
    fill_ms = [a.elapsed_time(b) for a, b in ev_fill]
    bulk_append_ms = float(np.median(fill_ms[1:])) if len(fill_ms) > 1 else fill_ms[0]

    # Per-step inputs, resident in HBM before timing.
    n_steps = W + K
    q = torch.randn((L, n_seqs, hq, d), generator=gen, device=dev)
    out = torch.empty((L, n_seqs, hq, d), device=dev)
    knew = torch.randn((L, n_seqs, hkv, d), generator=gen, device=dev)
    vnew = torch.randn((L, n_seqs, hkv, d), generator=gen, device=dev)
    slots_step = np.zeros((n_steps, n_seqs), np.int64)
    ctx_step = np.zeros((n_steps, n_seqs), np.int32)
    for t in range(n_steps):
        p = ctx0 + t
        slots_step[t] = tables[np.arange(n_seqs), p // bs].astype(np.int64) * bs + p % bs
        ctx_step[t] = p + 1
    slots_step_d = torch.from_numpy(slots_step).to(dev)
    ctx_step_d = torch.from_numpy(ctx_step).to(dev)
    max_ctx = int(ctx_step.max())
    ws_bytes = pool.attention_workspace_bytes(hq, n_seqs, max_ctx)
    ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    scale = fa.default_scale(d)

    h = ctypes.c_void_p(pool.handle)
    qp = [q[l].data_ptr() for l in range(L)]
    op = [out[l].data_ptr() for l in range(L)]
    kp = [knew[l].data_ptr() for l in range(L)]
    vp = [vnew[l].data_ptr() for l in range(L)]
    tp = tables_d.data_ptr()

    def step(t, events=None):
        sl = slots_step_d[t].data_ptr()
        cl = ctx_step_d[t].data_ptr()
        for l in range(L):
            rc = lib.fkv_append(h, l, kp[l], vp[l], sl, n_seqs, sp)
            if rc:
                fa.errors.check(rc)
            if events is not None:
                events[l][0].record(stream)
            rc = lib.fkv_decode_attention(h, l, hq, qp[l], op[l], tp, max_blocks, cl, n_seqs,
                                          max_ctx, scale, ws.data_ptr(), ws_bytes, sp)
            if events is not None:
                events[l][1].record(stream)
            if rc:
                fa.errors.check(rc)

    for t in range(W):
        step(t)
    torch.cuda.synchronize()

    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(L)] for _ in range(K)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        step(W + i, ev[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    assert pool.take_fault_flags() == 0

    attn_ms = np.array([[a.elapsed_time(b) for a, b in ev[i]] for i in range(K)])
    per_step_attn_bytes = [attn_bytes(ctx_step[W + i], hq, hkv, d, 2) * L for i in range(K)]
    total_attn_bytes = float(sum(per_step_attn_bytes))
    ms_per_step = wall * 1e3 / K
    value = total_attn_bytes / wall / 1e9
    launch_bytes = total_attn_bytes / (K * L)
    launch_ms = float(attn_ms.mean())
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    append_tok_s = n_seqs * K / wall  # tokens appended into all L layers per second

    # Calibration: plain device copy of 4 GiB (reported alongside; not the peak).
    nbytes = 4 << 30
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    fa.device_copy(b, a, nbytes)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(5):
        fa.device_copy(b, a, nbytes)
    c1.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 2 * nbytes * 5 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del a, b

    traffic = read_traffic(os.path.join(ROOT, "profiles", "decode_attention_llama3_8b_c2_hbm_traffic.md"))

    result = {
        "metric": "paged decode-attn HBM GB/s (% of peak) + KV append tokens/s, 1xMI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic N(0,1) Q/K/V, seeded; random-permutation block tables",
        "config": {
            "workload": "llama3-8b decode step (BASELINE configs[1])",
            "n_seqs": n_seqs, "n_layers": L, "n_heads": hq, "n_kv_heads": hkv,
            "head_dim": d, "block_size": bs, "kv_dtype": "f16", "accumulate": "f32",
            "ctx": "uniform[128,4096] seed %d" % args.seed,
            "mean_ctx": float(ctx_step[W:].mean()),
            "parallelism": "single GPU",
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "append_tokens_per_s": round(append_tok_s, 1),
        "append_token_layers_per_s": round(append_tok_s * L, 1),
        "bulk_append": {
            "tokens_per_launch": int(n_fill),
            "ms_per_launch": round(bulk_append_ms, 4),
            "token_layers_per_s": round(n_fill / (bulk_append_ms * 1e-3), 1),
            "gbs": round(append_bytes(n_fill, hkv, d, 2) / (bulk_append_ms * 1e-3) / 1e9, 2),
        },
        "device_copy_gbs": round(copy_gbs, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "fkv_decode_attention (attn_split_kernel + attn_combine_kernel)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(launch_bytes),
            "ms_per_launch": round(launch_ms, 5),
        },
        "cpu_baseline": None,
    }

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(pool, tables, ctx_step[W + K - 1], q, out,
                                              L - 1, hq, hkv, d, bs, args)
    print(json.dumps(result), flush=True)


def cpu_baseline(pool, tables, ctx, q, out, layer, hq, hkv, d, bs, args):
    """Oracle AVX2 restatement of the reference attention loop on one full layer
    of the same pool (copied to host), at 1 thread and at `threads` threads.
    Also counts GPU outputs outside tolerance on that layer."""
    from oracle import ref
    import ferrum_amd as fa

    n_seqs = tables.shape[0]
    nb = (ctx + bs - 1) // bs
    used = [int(b) for s in range(n_seqs) for b in tables[s, : nb[s]]]
    remap = {b: i for i, b in enumerate(used)}
    lay = ref.Layout(1, hkv, d, bs, len(used), dtype=1)
    region = lay.block_bytes
    image = np.empty(lay.pool_bytes, np.uint8)
    for b, i in remap.items():
        src = b * pool.block_bytes + layer * region
        image[i * region:(i + 1) * region] = pool.read(src, region)
    tab = np.zeros_like(tables)
    for s in range(n_seqs):
        tab[s, : nb[s]] = [remap[int(b)] for b in tables[s, : nb[s]]]
    qh = q[layer].cpu().numpy()
    gpu_out = out[layer].cpu().numpy()
    scale = fa.default_scale(d)
    if not ref.avx2_available():
        return None
    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    bytes_layer = attn_bytes(ctx, hq, hkv, d, 2)
    t0 = time.perf_counter()
    o1 = ref.avx2_attention(lay, image, 0, qh, tab, ctx.astype(np.int32), scale, 1)
    t1 = time.perf_counter() - t0
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        on = ref.avx2_attention(lay, image, 0, qh, tab, ctx.astype(np.int32), scale, threads)
    tn = (time.perf_counter() - t0) / reps
    err = np.abs(gpu_out.astype(np.float64) - o1)
    bad = int((err > 2e-3 + 1e-2 * np.abs(o1)).sum())
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    assert np.array_equal(o1, on)
    return {
        "value": round(bytes_layer / tn / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"1 of 32 layers (all {n_seqs} seqs, {int(ctx.sum())} tokens, "
                   f"{bytes_layer / 1e6:.1f} MB algorithmic), AVX2 restatement of "
                   "llama.rs:220-247 (per query head, no GQA reuse); "
                   f"{reps} reps at {threads} threads"),
        "value_1thread": round(bytes_layer / t1 / 1e9, 3),
        "seconds_1thread": round(t1, 3),
        "seconds_threads": round(tn, 3),
        "cpu_model": model,
        "host_cpus": os.cpu_count(),
        "gpu_vs_cpu_out_of_tolerance": bad,
        "gpu_vs_cpu_max_abs_err": float(err.max()),
    }


if __name__ == "__main__":
    main()
