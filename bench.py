#!/usr/bin/env python3
"""Benchmark of the paged KV-cache hot path on one MI355X.

Default workload ("Llama-3-8B-shaped decode step"):
64 sequences, 32 layers, 32 query / 8 KV heads (GQA 4), head_dim 128, f16 KV,
block 16, context lengths uniform in [128, 4096] (seed 0), block tables scattered
over the pool by a seeded permutation. One step = for every layer, one
fkv_append_decode_attention call: append the new token of every sequence through
its block table, then paged decode attention over the grown context (the per-layer
KV work of Llama::forward_one_token, crates/model/src/llama.rs:218-247). Q/K/V ~
N(0,1), synthetic (no checkpoint).

--workload picks another BASELINE config (c1 TinyLlama prefill + 64 decode steps,
c3 continuous batching with chunked prefill in a fragmented 60%-of-HBM pool, c4
Q8_0 KV, c5 70B long context plus copy_blocks and swap), q8gemv, the decode layer's
Q8_0 weight projections (fkv_gemm_q8_0 over Llama-3-8B's 32 layers), gguf, the
GGUF open + weight upload to HBM, or layer, the attention half of the decode layer
GPU-resident (q/k/v projections, RoPE + append + attention, attn_output, C2's batch),
or gather, the block-table gather (fkv_gather_tables) on C2's shapes; each prints its
own line. The default run adds `configs` to its line: compact results of c1, c3, c4
(with the exact Q8_0 instance measured), c5 (with copy_blocks and swap) and gather
(F16 and Q8_0), run after the headline in the same process (--no-configs skips them).

Printed JSON line: value = algorithmic HBM bytes of the step's calls (attention +
append) / wall time per step, timed over K steps bracketed by synchronisation.
roofline.achieved = the same bytes per call / the average call duration from HIP
events on the launch stream around the timed region (every launch in it belongs
to the measured call). cpu_baseline times the oracle's AVX2 restatement of the
reference loop on host cores, on a bounded sample of the same pool.
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

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
METRIC = "paged decode-attn HBM GB/s (% of peak) + KV append tokens/s, 1xMI355X"


def cpu_timed(fn, min_seconds, min_reps=1):
    """Seconds per call of fn, repeated until min_seconds have passed (at least min_reps
    calls), and the number of calls."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if reps >= min_reps and el >= min_seconds:
            return el / reps, reps

def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--workload", default="c2",
                    choices=["c1", "c2", "c3", "c4", "c5", "q8gemv", "gguf", "layer", "gather"])
    ap.add_argument("--gguf-layers", type=int, default=4,
                    help="gguf: Llama-3-8B layers in the synthetic file (232 MB of Q8_0 each)")
    ap.add_argument("--gguf-threads", type=int, default=0, help="gguf: host threads (0 = 4, fewer on fewer CPUs)")
    ap.add_argument("--gguf-chunk-mib", type=int, default=0, help="gguf: staging chunk (0 = 8 MiB)")
    ap.add_argument("--tokens", type=int, default=1,
                    help="q8gemv: activation rows a call (1 = Kernels::gemv, more = gemm)")
    ap.add_argument("--gemv-fused", action="store_true",
                    help="q8gemv: q/k/v and gate/up each in one fkv_gemm_q8_0_multi launch")
    ap.add_argument("--gemm-batched", action="store_true",
                    help="q8gemv: the same groups through fkv_gemm_q8_0_batched (the matrix "
                         "cores from 8 tokens)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="default run: skip the other configs' summary after the headline")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, os.cpu_count())")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline budget: a third at 1 thread, the rest at --cpu-threads")
    ap.add_argument("--rope-dim", type=int, default=0,
                    help="> 0: time fkv_rope_append_decode_attention (q and k before RoPE)")
    ap.add_argument("--rope-theta", type=float, default=500000.0)
    ap.add_argument("--kv-dtype", default="f16", choices=["f16", "f32", "q8_0"],
                    help="c2: KV storage (f32 runs the VALU attention kernel); c3, gather: f16 "
                         "(BASELINE's) or q8_0")
    ap.add_argument("--attn-engine", default="mfma", choices=["mfma", "valu"],
                    help="F16 decode arithmetic: matrix cores (default) or the VALU partition "
                         "kernel (fkv_set_tuning FKV_TUNE_ATTN_ENGINE), to measure the choice")
    ap.add_argument("--n-heads", type=int, default=32,
                    help="c2: query heads over the 8 KV heads (64: GQA group 8)")
    ap.add_argument("--c3-decode-wgs-per-cu", type=int, default=-1, choices=[-1, 0, 2, 3],
                    help="c3: cap the decode call at this many workgroups a CU "
                         "(FKV_TUNE_ATTN_WGS_PER_CU; 0: no cap) so the prefill stream runs "
                         "beside it; -1: 2 for f16 KV, none for q8_0 (measured)")
    ap.add_argument("--c3-streams", type=int, default=2, choices=[1, 2],
                    help="c3: 2 (default) issues each layer's chunk append + prefill attention on "
                         "a second stream beside its decode call (independent sequences); 1 "
                         "serialises them on one stream")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# Algorithmic bytes
# ---------------------------------------------------------------------------

def elem_bytes(dtype):
    """Stored bytes per K/V value: f16 2, f32 4, Q8_0 34/32 (32 int8 + one f16 scale)."""
    return {0: 4.0, 1: 2.0, 8: 34.0 / 32.0}[dtype]


def attn_bytes(ctx, hq, hkv, d, e):
    """Decode attention for one (sequence, layer): K+V once per KV head (GQA shares
    tiles), q and out in f32, the block-table entries, ctx_len."""
    ctx = np.asarray(ctx, dtype=np.int64)
    return float((ctx * hkv * d * 2 * e + hq * d * 4 * 2 + ((ctx + 15) // 16) * 4 + 4).sum())


def append_bytes(n_tokens, hkv, d, e, slot_bytes=8):
    """Per token per layer: f32 K/V read, stored K/V written, the slot (8 bytes
    for a slot mapping; 0 when the slot comes from the block table already counted)."""
    return float(n_tokens * (2 * hkv * d * 4 + 2 * hkv * d * e + slot_bytes))


# ---------------------------------------------------------------------------
# Setup helpers
# ---------------------------------------------------------------------------

def make_tables(pool, nblk_seq, rng, fragment_cycles=0):
    """Block tables from the pool's allocator. With fragment_cycles, the free list is
    first churned by seeded alloc/free cycles of 1..64 blocks, so tables come out
    scattered the way a long-running server leaves them; otherwise the allocated ids
    are permuted."""
    if fragment_cycles:
        held = []
        for _ in range(fragment_cycles):
            if held and (rng.random() < 0.5 or pool.free_block_count() < 64):
                pool.free_blocks(held.pop(int(rng.integers(len(held)))))
            else:
                held.append(pool.alloc_blocks(int(rng.integers(1, 65))))
        for h in held:
            pool.free_blocks(h)
        ids = pool.alloc_blocks(int(nblk_seq.sum()))
    else:
        ids = pool.alloc_blocks(int(nblk_seq.sum()))
        ids = ids[rng.permutation(ids.size)]
    tables = np.zeros((len(nblk_seq), max(1, int(nblk_seq.max()))), np.int32)
    off = 0
    for s, n in enumerate(nblk_seq):
        tables[s, :n] = ids[off: off + n]
        off += n
    return tables


def slots_of(tables, seqs, pos, bs=16):
    return tables[seqs, pos // bs].astype(np.int64) * bs + pos % bs


def fill_context(torch, pool, layers, tables, ctx, hkv, d, gen, dev, outlier_frac=0.0,
                 chunk=1 << 18, timer=None):
    """Append N(0,1) K/V (optionally with a fraction of +-20 outliers) for positions
    0 .. ctx[s]-1 of every sequence into every layer, in launches of `chunk` tokens.
    With `timer`, the HIP-event time of every full-size launch (or of the single launch
    of a smaller fill) goes to it; returns the tokens of one timed launch."""
    ctx = np.asarray(ctx, np.int64)
    seq_of = np.repeat(np.arange(ctx.size), ctx)
    pos = np.concatenate([np.arange(c) for c in ctx]) if ctx.sum() else np.zeros(0, np.int64)
    slots_all = torch.from_numpy(slots_of(tables, seq_of, pos)).to(dev)
    n = slots_all.numel()
    times = []
    for layer in layers:
        for a in range(0, n, chunk):
            b = min(n, a + chunk)
            k = torch.randn((b - a, hkv, d), generator=gen, device=dev)
            v = torch.randn((b - a, hkv, d), generator=gen, device=dev)
            if outlier_frac:
                for x in (k, v):
                    m = torch.rand(x.shape, generator=gen, device=dev) < outlier_frac
                    sgn = torch.where(torch.rand(x.shape, generator=gen, device=dev) < 0.5, -20.0, 20.0)
                    x[m] = sgn[m]
            e0 = e1 = None
            if timer is not None and (b - a == chunk or (a == 0 and b == n)):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
            pool.append(layer, k, v, slots_all[a:b])
            if e0 is not None:
                e1.record()
                times.append((e0, e1))
            del k, v
    torch.cuda.synchronize()
    if timer is not None and times:
        timer.extend(a.elapsed_time(b) for a, b in times)
    return min(n, chunk)  # tokens of each timed launch


def calibrate_copy(torch, fa, dev, nbytes=4 << 30):
    """Plain 16-byte device copy (reported alongside; not the peak)."""
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    fa.device_copy(b, a, nbytes)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(5):
        fa.device_copy(b, a, nbytes)
    c1.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * 5 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del a, b
    return gbs


def read_traffic(path):
    """HBM bytes per call from a committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (the line `hbm_bytes_per_launch: N`), or None when it is absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


# ---------------------------------------------------------------------------
# Decode steps
# ---------------------------------------------------------------------------

class DecodeLoop:
    """Per-layer fused decode calls over K timed steps (plus W warm-up steps).
    ctx_step[t] holds every sequence's context after step t's append."""

    def __init__(self, torch, fa, lib, pool, L, n_seqs, hq, hkv, d, tables, ctx0, n_steps, gen,
                 dev, seqs=None, rope=(0, 0.0)):
        self.torch, self.fa, self.lib, self.pool, self.L = torch, fa, lib, pool, L
        self.n_seqs, self.hq, self.hkv, self.d = n_seqs, hq, hkv, d
        self.q = torch.randn((L, n_seqs, hq, d), generator=gen, device=dev)
        self.out = torch.empty((L, n_seqs, hq, d), device=dev)
        self.knew = torch.randn((L, n_seqs, hkv, d), generator=gen, device=dev)
        self.vnew = torch.randn((L, n_seqs, hkv, d), generator=gen, device=dev)
        self.ctx_step = np.stack([ctx0 + t + 1 for t in range(n_steps)]).astype(np.int32)
        self.ctx_step_d = torch.from_numpy(self.ctx_step).to(dev)
        self.tables = tables
        self.tables_d = torch.from_numpy(tables).to(dev)
        self.max_blocks = tables.shape[1]
        self.max_ctx = int(self.ctx_step.max())
        self.rope_dim, self.rope_theta = int(rope[0]), float(rope[1])
        n = ctypes.c_uint64()
        size_fn = (lib.fkv_rope_append_decode_attention_workspace_size if self.rope_dim
                   else lib.fkv_append_decode_attention_workspace_size)
        fa.errors.check(size_fn(ctypes.c_void_p(pool.handle), hq, n_seqs, self.max_ctx,
                                ctypes.byref(n)))
        self.ws_bytes = n.value
        self.ws = torch.zeros(max(self.ws_bytes, 16), dtype=torch.uint8, device=dev)
        self.scale = fa.default_scale(d)
        self.h = ctypes.c_void_p(pool.handle)
        self.ptrs = [(self.q[l].data_ptr(), self.out[l].data_ptr(), self.knew[l].data_ptr(),
                      self.vnew[l].data_ptr()) for l in range(L)]

    def step(self, t, sp):
        cl = self.ctx_step_d[t].data_ptr()
        tp = self.tables_d.data_ptr()
        for l in range(self.L):
            qp, op, kp, vp = self.ptrs[l]
            if self.rope_dim:
                rc = self.lib.fkv_rope_append_decode_attention(
                    self.h, l, self.hq, self.rope_dim, self.rope_theta, kp, vp, qp, op, tp,
                    self.max_blocks, cl, self.n_seqs, self.max_ctx, self.scale,
                    self.ws.data_ptr(), self.ws_bytes, sp)
            else:
                rc = self.lib.fkv_append_decode_attention(
                    self.h, l, self.hq, kp, vp, qp, op, tp, self.max_blocks, cl, self.n_seqs,
                    self.max_ctx, self.scale, self.ws.data_ptr(), self.ws_bytes, sp)
            if rc:
                self.fa.errors.check(rc)

    def run(self, W, K):
        torch = self.torch
        stream = torch.cuda.current_stream()
        sp = stream.cuda_stream
        for t in range(W):
            self.step(t, sp)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(K):
            self.step(W + i, sp)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        assert self.pool.take_fault_flags() == 0
        return wall, e0.elapsed_time(e1)


def decode_result(args, dl, W, K, wall, region_ms, e, workload, extra_cfg, kernel_name, traffic):
    L, hq, hkv, d = dl.L, dl.hq, dl.hkv, dl.d
    per_step = [attn_bytes(dl.ctx_step[W + i], hq, hkv, d, e) * L for i in range(K)]
    app_step = append_bytes(dl.n_seqs, hkv, d, e, slot_bytes=0) * L
    total = float(sum(per_step)) + app_step * K
    value = total / wall / 1e9
    call_bytes = total / (K * L)
    call_ms = region_ms / (K * L)
    achieved = call_bytes / (call_ms * 1e-3) / 1e9
    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {0: "f32", 1: "f16", 8: "q8_0"}[dl.pool.config.kv_dtype],
        "data": "synthetic N(0,1) Q/K/V, seeded; scattered block tables",
        "config": dict({"workload": workload, "n_seqs": dl.n_seqs, "n_layers": L,
                        "n_heads": hq, "n_kv_heads": hkv, "head_dim": d, "block_size": 16,
                        "accumulate": "f32", "mean_ctx": float(dl.ctx_step[W:W + K].mean()),
                        "parallelism": "single GPU"}, **extra_cfg),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "append_tokens_per_s": round(dl.n_seqs * K / wall, 1),
        "append_token_layers_per_s": round(dl.n_seqs * K * L / wall, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name,
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(call_bytes),
            "ms_per_launch": round(call_ms, 5),
        },
        "cpu_baseline": None,
    }


# ---------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------

def cpu_baseline(args, pool, tables, ctx, q_layer, out_layer, layer, hq, hkv, d, dtype,
                 seqs=None):
    """The oracle's AVX2 restatement of the reference attention loop (llama.rs:220-247:
    per query head, no GQA reuse) on one layer of the same pool, copied to the host,
    at 1 thread and at `threads` threads; `seqs` bounds the sample. Also counts GPU
    outputs outside the attention tolerance on that sample."""
    from oracle import ref
    import ferrum_amd as fa

    if not ref.avx2_available():
        return None
    bs = 16
    seqs = np.arange(tables.shape[0]) if seqs is None else np.asarray(seqs)
    ctx = np.asarray(ctx, np.int64)[seqs]
    nb = (ctx + bs - 1) // bs
    used = [int(b) for s, n in zip(seqs, nb) for b in tables[s, :n]]
    remap = {b: i for i, b in enumerate(used)}
    lay = ref.Layout(1, hkv, d, bs, len(used), dtype=dtype)
    region = lay.block_bytes
    image = np.empty(lay.pool_bytes, np.uint8)
    for b, i in remap.items():
        image[i * region:(i + 1) * region] = pool.read(b * pool.block_bytes + layer * region, region)
    tab = np.zeros((len(seqs), max(1, int(nb.max()))), np.int32)
    for j, (s, n) in enumerate(zip(seqs, nb)):
        tab[j, :n] = [remap[int(b)] for b in tables[s, :n]]
    qh = np.ascontiguousarray(q_layer[seqs])
    if args.rope_dim:  # the step attended with q rotated at position ctx - 1
        for j, c in enumerate(ctx):
            qh[j] = ref.rope(qh[j], args.rope_dim, int(c) - 1 if c > 0 else 0, args.rope_theta)
    gpu_out = out_layer[seqs]
    scale = fa.default_scale(d)
    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    e = elem_bytes(dtype)
    nbytes = attn_bytes(ctx, hq, hkv, d, e)
    ctx32 = ctx.astype(np.int32)
    o1 = ref.avx2_attention(lay, image, 0, qh, tab, ctx32, scale, 1)
    t1, reps1 = cpu_timed(lambda: ref.avx2_attention(lay, image, 0, qh, tab, ctx32, scale, 1),
                          args.cpu_seconds / 3)
    on = ref.avx2_attention(lay, image, 0, qh, tab, ctx32, scale, threads)
    tn, reps = cpu_timed(lambda: ref.avx2_attention(lay, image, 0, qh, tab, ctx32, scale, threads),
                         args.cpu_seconds * 2 / 3)
    assert np.array_equal(o1, on)
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
    return {
        "value": round(nbytes / tn / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"layer {layer}, {len(seqs)} seqs ({int(ctx.sum())} tokens, "
                   f"{nbytes / 1e6:.1f} MB algorithmic): AVX2 restatement of llama.rs:220-247 "
                   f"(per query head, no GQA reuse); {reps1} reps at 1 thread, {reps} reps at "
                   f"{threads} threads"),
        "value_1thread": round(nbytes / t1 / 1e9, 3),
        "seconds_1thread": round(t1, 3),
        "seconds_threads": round(tn, 3),
        "cpu_model": model,
        "host_cpus": os.cpu_count(),
        "gpu_vs_cpu_out_of_tolerance": bad,
        "gpu_vs_cpu_max_abs_err": float(np.nanmax(err)) if err.size else 0.0,
    }


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------

def decode_workload(args, torch, fa, lib, dev, *, name, L, n_seqs, hq, hkv, d, dtype, ctx0,
                    num_blocks, fragment_cycles=0, outlier_frac=0.0, extra_cfg=None,
                    cpu_seqs=None, num_host_blocks=0):
    """Common decode leg: pool, tables, context fill (bulk append measured), K timed
    fused steps. Returns (result dict, pool, DecodeLoop) for workload-specific extras."""
    K, W = args.steps, args.warmup
    rng = np.random.default_rng(args.seed)
    nblk_seq = (ctx0 + W + K + 15) // 16
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=num_blocks, block_size=16, kv_dtype=dtype,
                                         num_host_blocks=num_host_blocks))
    tables = make_tables(pool, nblk_seq, rng, fragment_cycles)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    fill_ms = []
    n_fill = fill_context(torch, pool, range(L), tables, ctx0, hkv, d, gen, dev,
                          outlier_frac=outlier_frac, timer=fill_ms)
    dl = DecodeLoop(torch, fa, lib, pool, L, n_seqs, hq, hkv, d, tables, ctx0, W + K, gen, dev,
                    rope=(args.rope_dim, args.rope_theta))
    wall, region_ms = dl.run(W, K)
    if args.rope_dim:
        extra_cfg = dict(extra_cfg or {}, rope_dim=args.rope_dim, rope_theta=args.rope_theta)
    e = elem_bytes(dtype)
    kname = {1: "fkv_append_decode_attention (attn_mfma_kernel + attn_combine_kernel)",
             8: "fkv_append_decode_attention (attn_mfma_kernel<q8_0>, its exact instance "
                "(exits at once unless the pool holds a scale >= 512), attn_combine_kernel)",
             0: "fkv_append_decode_attention (tail slots + append_f32_kernel + "
                "attn_partition_kernel + attn_combine_kernel)"}[dtype]
    res = decode_result(args, dl, W, K, wall, region_ms, e, name, dict(extra_cfg or {}), kname,
                        None)
    if fill_ms:
        ms = float(np.median(fill_ms))
        res["bulk_append"] = {
            "tokens_per_launch": int(n_fill), "ms_per_launch": round(ms, 4),
            "token_layers_per_s": round(n_fill / (ms * 1e-3), 1),
            "gbs": round(append_bytes(n_fill, hkv, d, e) / (ms * 1e-3) / 1e9, 2)}
    if not args.no_cpu:
        t_last = W + K - 1
        res["cpu_baseline"] = cpu_baseline(args, pool, tables, dl.ctx_step[t_last],
                                           dl.q[L - 1].cpu().numpy(), dl.out[L - 1].cpu().numpy(),
                                           L - 1, hq, hkv, d, dtype, seqs=cpu_seqs)
    return res, pool, dl


def run_c2(args, torch, fa, lib, dev):
    rng = np.random.default_rng(args.seed)
    n_seqs = 64
    ctx0 = rng.integers(128, 4097, n_seqs).astype(np.int64)
    nb = int(((ctx0 + args.warmup + args.steps + 15) // 16).sum()) + 64
    dtype = {"f16": 1, "f32": 0, "q8_0": 8}[args.kv_dtype]
    variant = args.kv_dtype != "f16" or args.n_heads != 32
    name = "llama3-8b decode step (BASELINE configs[1])"
    if variant:  # a counter-study variant of the config, not the headline line
        name += f", variant: {args.kv_dtype} KV, {args.n_heads} query heads"
    res, pool, dl = decode_workload(
        args, torch, fa, lib, dev, name=name, L=32, n_seqs=n_seqs, hq=args.n_heads, hkv=8,
        d=128, dtype=dtype, ctx0=ctx0, num_blocks=nb,
        extra_cfg={"kv_dtype": args.kv_dtype, "ctx": f"uniform[128,4096] seed {args.seed}"})
    if not variant:
        res["roofline"]["traffic"] = read_traffic(
            os.path.join(ROOT, "profiles", "decode_attention_llama3_8b_c2_hbm_traffic.md"))
    res["device_copy_gbs"] = round(calibrate_copy(torch, fa, dev), 1)
    return res


def run_c4(args, torch, fa, lib, dev):
    n_seqs, ctx = 128, 8192
    ctx0 = np.full(n_seqs, ctx - args.warmup - args.steps, np.int64)
    nb = int(((ctx0 + args.warmup + args.steps + 15) // 16).sum()) + 64
    res, pool, dl = decode_workload(
        args, torch, fa, lib, dev, name="llama3-8b q8_0 kv, 128 x 8192 (BASELINE configs[3])",
        L=32, n_seqs=n_seqs, hq=32, hkv=8, d=128, dtype=8, ctx0=ctx0, num_blocks=nb,
        outlier_frac=0.01, extra_cfg={"kv_dtype": "q8_0", "outliers": "1% at +-20"},
        cpu_seqs=np.arange(8))
    res["exact_instance"] = exact_instance_leg(torch, pool, dl, args.steps, ctx)
    return res


def exact_instance_leg(torch, pool, dl, K, ctx):
    """The same fused decode calls after one token of every 4096-token context split of
    every sequence was appended (layer 0) with a V value of 1e6: a Q8_0 scale of ~7,874
    marks that block, so every workgroup of every call runs the exact instance (f32
    scales, int8 operands) instead of the binary16 one. Same algorithmic bytes."""
    dev = dl.q.device
    pos = np.arange(0, ctx, 4096)
    seqs = np.repeat(np.arange(dl.n_seqs), pos.size)
    slots = slots_of(dl.tables, seqs, np.tile(pos, dl.n_seqs))
    k = torch.zeros((slots.size, dl.hkv, dl.d), device=dev)
    v = torch.zeros_like(k)
    v[:, :, 0] = 1e6
    pool.append(0, k, v, torch.from_numpy(slots).to(dev))
    torch.cuda.synchronize()
    marked = pool.marked_blocks()
    wall, region_ms = dl.run(0, K)
    e = elem_bytes(8)
    call_bytes = sum(attn_bytes(dl.ctx_step[i], dl.hq, dl.hkv, dl.d, e)
                     + append_bytes(dl.n_seqs, dl.hkv, dl.d, e, slot_bytes=0)
                     for i in range(K)) / K
    call_ms = region_ms / (K * dl.L)
    gbs = call_bytes / (call_ms * 1e-3) / 1e9
    return {"marked_blocks": int(marked), "us_per_call": round(call_ms * 1e3, 2),
            "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "attn_mfma_kernel<q8_0, exact> (qk_block_q8x / pv_block_q8x)"}


def run_c5(args, torch, fa, lib, dev):
    """131,072-token decode on 70B-shaped KV, then copy_blocks of 20,000 (src, dst)
    pairs (CoW fork) and a swap of 20% of the context's blocks out and back in."""
    ctx = 131072
    K, W = args.steps, args.warmup
    ctx0 = np.array([ctx - W - K], np.int64)
    ctx_blocks = (ctx + 15) // 16
    n_pairs = 20000
    n_swap = ctx_blocks // 5
    nb = ctx_blocks + n_pairs + 64
    res, pool, dl = decode_workload(
        args, torch, fa, lib, dev, name="llama3-70b long context 1 x 131072 (BASELINE configs[4])",
        L=80, n_seqs=1, hq=64, hkv=8, d=128, dtype=1, ctx0=ctx0, num_blocks=nb,
        extra_cfg={"kv_dtype": "f16", "ctx": ctx}, cpu_seqs=None, num_host_blocks=n_swap)
    # copy_blocks: sources among the context's blocks, destinations distinct free blocks
    rng = np.random.default_rng(args.seed + 1)
    used = dl.tables[0, :ctx_blocks]
    dst = pool.alloc_blocks(n_pairs)
    src = used[rng.integers(0, ctx_blocks, n_pairs)]
    pairs = np.stack([src, dst], 1).astype(np.int64)
    pairs_d = torch.from_numpy(pairs).to(dev)
    pool.copy_blocks(pairs_d)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    reps = 3
    for _ in range(reps):
        pool.copy_blocks(pairs_d)
    e1.record()
    torch.cuda.synchronize()
    cms = e0.elapsed_time(e1) / reps
    cbytes = 2.0 * n_pairs * pool.block_bytes
    for j in rng.integers(0, n_pairs, 4):  # spot check: dst bytes == src bytes
        a = pool.read(int(src[j]) * pool.block_bytes, pool.block_bytes)
        b = pool.read(int(dst[j]) * pool.block_bytes, pool.block_bytes)
        assert np.array_equal(a, b), "copy_blocks mismatch"
    res["copy_blocks"] = {"pairs": n_pairs, "bytes_per_block": pool.block_bytes,
                          "ms": round(cms, 3), "gbs": round(cbytes / (cms * 1e-3) / 1e9, 1),
                          "pct_of_hbm_peak": round(100 * cbytes / (cms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
    pool.free_blocks(dst)
    res["swap"] = swap_leg(torch, fa, pool, used, n_swap, rng)
    return res


def swap_leg(torch, fa, pool, used, n_swap, rng):
    """Swap n_swap of the context's blocks out to a second pool's pinned host
    storage and back; byte-identical round trip checked on a sample."""
    sel = np.sort(rng.choice(used, n_swap, replace=False)).astype(np.int64)
    host_pool = pool  # pinned host storage belongs to the pool that swaps
    pairs_out = np.stack([sel, np.arange(n_swap)], 1)
    pairs_in = np.stack([np.arange(n_swap), sel], 1)
    check = sel[rng.integers(0, n_swap, 4)]
    before = [pool.read(int(b) * pool.block_bytes, pool.block_bytes) for b in check]
    s = torch.cuda.current_stream()
    e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    e0.record(s)
    host_pool.swap_out(pairs_out)
    e1.record(s)
    pool.fill(0xA5)  # clobber device copies (the whole pool) before swapping back
    s2 = torch.cuda.Event(enable_timing=True)
    s2.record(s)
    host_pool.swap_in(pairs_in)
    e2.record(s)
    torch.cuda.synchronize()
    out_ms, in_ms = e0.elapsed_time(e1), s2.elapsed_time(e2)
    after = [pool.read(int(b) * pool.block_bytes, pool.block_bytes) for b in check]
    assert all(np.array_equal(a, b) for a, b in zip(before, after)), "swap round trip mismatch"
    nbytes = float(n_swap * pool.block_bytes)
    return {"blocks": int(n_swap), "bytes": int(nbytes), "out_ms": round(out_ms, 2),
            "in_ms": round(in_ms, 2), "out_gbs": round(nbytes / (out_ms * 1e-3) / 1e9, 2),
            "in_gbs": round(nbytes / (in_ms * 1e-3) / 1e9, 2), "bound": "host link (PCIe)"}


def run_c3(args, torch, fa, lib, dev):
    """Continuous batching: 256 decode sequences with log-normal contexts (median
    2048, sigma 1.0, cap 32768) and 4 chunked-prefill sequences appending 512 tokens
    each, in one pool sized to ~60% of 288 GB and fragmented by 10,000 seeded
    alloc/free cycles. Step per layer: fused decode call for the 256 sequences, the
    prefill chunk's append, then chunked-prefill attention for the 4 sequences."""
    K, W = args.steps, args.warmup
    rng = np.random.default_rng(args.seed)
    L, hq, hkv, d = 32, 32, 8, 128
    n_dec, n_pre, chunk = 256, 4, 512
    ctx_dec = np.minimum(np.round(np.exp(rng.normal(np.log(2048), 1.0, n_dec))), 32768 - W - K)
    ctx_dec = np.maximum(ctx_dec, 1).astype(np.int64)
    pre_prior = np.array([0, 512, 1024, 1536], np.int64)  # chunked prefill in progress
    if args.kv_dtype not in ("f16", "q8_0"):
        raise SystemExit("c3: --kv-dtype f16 or q8_0")
    dtype = {"f16": 1, "q8_0": 8}[args.kv_dtype]
    block_bytes = int(L * 2 * hkv * 16 * d * elem_bytes(dtype))
    num_blocks = int(0.6 * 288e9 // block_bytes)
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=num_blocks, block_size=16, kv_dtype=dtype))
    nblk = np.concatenate([(ctx_dec + W + K + 15) // 16, (pre_prior + chunk * (W + K) + 15) // 16])
    tables = make_tables(pool, nblk, rng, fragment_cycles=10000)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    fill_context(torch, pool, range(L), tables, np.concatenate([ctx_dec, pre_prior]), hkv, d,
                 gen, dev)
    dl = DecodeLoop(torch, fa, lib, pool, L, n_dec, hq, hkv, d, tables[:n_dec], ctx_dec, W + K,
                    gen, dev, rope=(args.rope_dim, args.rope_theta))
    # prefill inputs: chunk t of sequence p covers positions prior + t*chunk .. +chunk-1
    tab_pre = torch.from_numpy(np.ascontiguousarray(tables[n_dec:])).to(dev)
    kp = torch.randn((L, n_pre * chunk, hkv, d), generator=gen, device=dev)
    vp = torch.randn((L, n_pre * chunk, hkv, d), generator=gen, device=dev)
    qp = torch.randn((L, n_pre * chunk, hq, d), generator=gen, device=dev)
    op = torch.empty_like(qp)
    pre_slots, pre_ctx = [], []
    for t in range(W + K):
        start = pre_prior + t * chunk
        seqs = np.repeat(np.arange(n_pre), chunk)
        pos = np.concatenate([np.arange(s, s + chunk) for s in start])
        pre_slots.append(torch.from_numpy(slots_of(tables[n_dec:], seqs, pos)).to(dev))
        pre_ctx.append(torch.from_numpy((start + chunk).astype(np.int32)).to(dev))
    q_lens = torch.full((n_pre,), chunk, dtype=torch.int32, device=dev)
    q_offs = torch.arange(0, n_pre * chunk, chunk, dtype=torch.int64, device=dev)
    max_pre_ctx = int(pre_prior.max() + chunk * (W + K))
    h = ctypes.c_void_p(pool.handle)
    scale = fa.default_scale(d)
    pre_ws_bytes = pool.prefill_workspace_bytes(hq, n_pre, chunk, max_pre_ctx)
    pre_ws = torch.empty(max(pre_ws_bytes, 1), dtype=torch.uint8, device=dev)

    def prefill(t, l, sp):
        fa.errors.check(lib.fkv_prefill_attention(
            h, l, hq, qp[l].data_ptr(), op[l].data_ptr(), tab_pre.data_ptr(),
            tab_pre.shape[1], pre_ctx[t].data_ptr(), q_lens.data_ptr(), q_offs.data_ptr(),
            n_pre, chunk, max_pre_ctx, scale, pre_ws.data_ptr() if pre_ws_bytes else None,
            pre_ws_bytes, sp))

    # --c3-streams 2: a layer's prefill chunk (append, then prefill attention) goes to a
    # second stream of default priority; the decode sequences and the prefill sequences
    # share no block, so the two streams need no ordering inside the step
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    stream_b = torch.cuda.Stream() if args.c3_streams == 2 else stream
    spb = stream_b.cuda_stream

    def step(t, sp):
        cl = dl.ctx_step_d[t].data_ptr()
        for l in range(L):
            q_, o_, k_, v_ = dl.ptrs[l]
            fa.errors.check(lib.fkv_append_decode_attention(
                h, l, hq, k_, v_, q_, o_, dl.tables_d.data_ptr(), dl.max_blocks, cl, n_dec,
                dl.max_ctx, scale, dl.ws.data_ptr(), dl.ws_bytes, sp))
            fa.errors.check(lib.fkv_append(h, l, kp[l].data_ptr(), vp[l].data_ptr(),
                                           pre_slots[t].data_ptr(), n_pre * chunk, spb))
            prefill(t, l, spb)

    # The cap leaves room on each CU for the prefill stream (one stream has nothing to run
    # beside the decode call). Measured on the mixed step: f16 KV 4,500 -> 4,875 GB/s with
    # 2 decode workgroups a CU; q8_0 KV 3,249 -> 3,055 (its prefill, with the staging pass,
    # is the larger share of the step), so q8_0 runs uncapped by default.
    cap = args.c3_decode_wgs_per_cu
    if cap < 0:
        cap = 2 if dtype == 1 else 0
    if stream_b is stream:
        cap = 0
    fa.set_tuning(fa.TUNE_ATTN_WGS_PER_CU, cap)
    try:  # the knob is process-wide: the later legs run uncapped whatever happens here
        for t in range(W):
            step(t, sp)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        stream_b.wait_event(e0)
        for i in range(K):
            step(W + i, sp)
        if stream_b is not stream:  # the timed region ends when both streams have drained
            done_b = torch.cuda.Event()
            done_b.record(stream_b)
            stream.wait_event(done_b)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    finally:
        fa.set_tuning(fa.TUNE_ATTN_WGS_PER_CU, 0)
    assert pool.take_fault_flags() == 0
    # chunked-prefill attention alone over the timed steps' chunks (it reads the pool
    # only, so the calls can run again): 4 * D * Hq flops per (query, key) pair
    p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    p0.record(stream)
    for i in range(K):
        for l in range(L):
            prefill(W + i, l, sp)
    p1.record(stream)
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == 0
    pre_us = p0.elapsed_time(p1) * 1e3 / (K * L)
    pairs = sum(int((pre_prior + (W + i) * chunk).sum()) * chunk + n_pre * chunk * (chunk + 1) // 2
                for i in range(K)) / K
    pre_flop = 4.0 * d * hq * pairs
    # The leak-safe instance: the same calls after position 0 of every prefill sequence
    # (layer 0) was given a NaN V, which marks its first block, a block every workgroup
    # of the sequence reads, so every workgroup runs the leak-safe instance. (The NaN
    # reaches every query; the timing is the instance's, on the same bytes.)
    if dtype == 1:
        nan_slots = slots_of(tables[n_dec:], np.arange(n_pre), np.zeros(n_pre, np.int64))
        kn = torch.zeros((n_pre, hkv, d), device=dev)
        vn = torch.full((n_pre, hkv, d), float("nan"), device=dev)
        pool.append(0, kn, vn, torch.from_numpy(nan_slots).to(dev))
        torch.cuda.synchronize()
        p2, p3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p2.record(stream)
        for i in range(K):
            for l in range(L):
                prefill(W + i, l, sp)
        p3.record(stream)
        torch.cuda.synchronize()
        assert pool.take_fault_flags() == 0
        safe_us = p2.elapsed_time(p3) * 1e3 / (K * L)
        leak_safe = {"us_per_call": round(safe_us, 2),
                     "tflops": round(pre_flop / (safe_us * 1e-6) / 1e12, 1),
                     "marked_blocks": int(pool.marked_blocks()),
                     "kernel": "attn_prefill_kernel<f16, leak-safe>"}
    else:
        leak_safe = None
    # decode-only rate from a separate region of back-to-back fused decode calls
    dw, dms = dl.run(0, K)
    e = elem_bytes(dtype)
    dec_bytes = [attn_bytes(dl.ctx_step[W + i], hq, hkv, d, e) * L for i in range(K)]
    pre_attn = sum(attn_bytes_prefill(pre_prior + (W + i) * chunk + chunk, chunk, hq, hkv, d, e)
                   for i in range(K)) * L
    app = (append_bytes(n_dec, hkv, d, e, 0) + append_bytes(n_pre * chunk, hkv, d, e)) * L * K
    total = float(sum(dec_bytes)) + pre_attn + app
    res = decode_result(args, dl, 0, K, dw, dms, e, "llama3-8b continuous batching "
                        "(BASELINE configs[2])",
                        {"kv_dtype": args.kv_dtype, "ctx": "log-normal median 2048 sigma 1.0 cap 32768",
                         "prefill": f"{n_pre} x {chunk}-token chunks",
                         "streams": args.c3_streams,
                         "decode_wgs_per_cu": cap or None,
                         "pool_blocks": num_blocks, "pool_gb": round(pool.pool_bytes / 1e9, 1),
                         "fragmented_by": "10000 seeded alloc/free cycles"},
                        "fkv_append_decode_attention (attn_mfma_kernel + attn_combine_kernel)",
                        None)
    # the headline value of this leg is the whole mixed step
    res["value"] = round(total / wall / 1e9, 2)
    res["ms_per_step"] = round(wall * 1e3 / K, 4)
    res["pct_of_hbm_peak"] = round(100 * res["value"] / HBM_PEAK_GBS, 2)
    res["decode_only_ms_per_step"] = round(dw * 1e3 / K, 4)
    res["append_tokens_per_s"] = round((n_dec + n_pre * chunk) * K / wall, 1)
    res["prefill_attention"] = {
        "kernel": "attn_prefill_kernel (+ attn_prefill_combine_kernel for split key ranges)",
        "us_per_call": round(pre_us, 2), "gflop_per_call": round(pre_flop / 1e9, 3),
        "tflops": round(pre_flop / (pre_us * 1e-6) / 1e12, 1),
        "flop_count": "4 * head_dim * n_heads per (query, key) pair",
        "pct_of_mfma_peak": round(100 * pre_flop / (pre_us * 1e-6) / 2.5e15, 2),
        "workspace_bytes": int(pre_ws_bytes), "leak_safe_instance": leak_safe}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args, pool, dl.tables, dl.ctx_step[K - 1],
                                           dl.q[L - 1].cpu().numpy(), dl.out[L - 1].cpu().numpy(),
                                           L - 1, hq, hkv, d, 1, seqs=np.arange(16))
    return res


def gather_bytes(ctx, hkv, d, e, out_e):
    """fkv_gather_tables of one layer: K+V of every position read once (e bytes a
    value), written as out_e bytes a value, the block-table entries, ctx_lens and the
    output offsets."""
    ctx = np.asarray(ctx, np.int64)
    n = float(ctx.sum())
    return n * hkv * d * 2 * e + n * hkv * d * 2 * out_e + float(((ctx + 15) // 16).sum()) * 4 + \
        ctx.size * 12


def run_gather(args, torch, fa, lib, dev):
    """Block-table gather (the paged KvPool::k / v, crates/kvcache/src/pool.rs:174-204) on
    C2's shapes: 64 sequences with contexts U[128, 4096] (seed), 32 layers, 8 KV heads,
    head_dim 128, F16 (default) or Q8_0 storage. One step = fkv_gather_tables of every
    layer's K and V for every sequence into one contiguous output, in the raw storage
    format (the headline) and decoded to f32."""
    K, W = args.steps, args.warmup
    rng = np.random.default_rng(args.seed)
    L, hkv, d, n_seqs = 32, 8, 128, 64
    dtype = {"f16": 1, "q8_0": 8}.get(args.kv_dtype)
    if dtype is None:
        raise SystemExit("gather: --kv-dtype f16 or q8_0")
    ctx = rng.integers(128, 4097, n_seqs).astype(np.int64)
    nblk_seq = (ctx + 15) // 16
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=int(nblk_seq.sum()) + 64, block_size=16,
                                         kv_dtype=dtype))
    tables = make_tables(pool, nblk_seq, rng)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    fill_context(torch, pool, range(L), tables, ctx, hkv, d, gen, dev)
    e = elem_bytes(dtype)
    n_tok = int(ctx.sum())
    tables_d = torch.from_numpy(tables).to(dev)
    ctx_d = torch.from_numpy(ctx.astype(np.int32)).to(dev)
    offs = np.zeros(n_seqs, np.int64)
    offs[1:] = np.cumsum(ctx[:-1])
    offs_d = torch.from_numpy(offs).to(dev)
    h = ctypes.c_void_p(pool.handle)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    legs = {}
    for fmt, name in ((1, "raw"), (0, "f32")):
        row = (d * 2 if dtype == 1 else d // 32 * 34) if fmt == 1 else d * 4
        out_e = row / d
        ok = torch.empty((n_tok, hkv, row), dtype=torch.uint8, device=dev)
        ov = torch.empty_like(ok)

        def step():
            for l in range(L):
                rc = lib.fkv_gather_tables(h, l, tables_d.data_ptr(), tables.shape[1],
                                           ctx_d.data_ptr(), offs_d.data_ptr(), n_seqs,
                                           int(ctx.max()), fmt, ok.data_ptr(), ov.data_ptr(), sp)
                if rc:
                    fa.errors.check(rc)
        for _ in range(W):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(K):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        assert pool.take_fault_flags() == 0
        call_bytes = gather_bytes(ctx, hkv, d, e, out_e)
        call_ms = e0.elapsed_time(e1) / (K * L)
        legs[name] = {"gbs": round(call_bytes * K * L / wall / 1e9, 2),
                      "kernel_gbs": round(call_bytes / (call_ms * 1e-3) / 1e9, 2),
                      "us_per_call": round(call_ms * 1e3, 2),
                      "bytes_per_call": int(call_bytes), "ms_per_step": round(wall * 1e3 / K, 4)}
        if name == "raw":
            last = (ok, ov)
        else:
            del ok, ov
    copy_gbs = calibrate_copy(torch, fa, dev)
    raw = legs["raw"]
    res = {
        "metric": METRIC + " [gather leg: block-table gather GB/s]",
        "value": raw["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": raw["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": {1: "f16", 8: "q8_0"}[dtype],
        "data": "synthetic N(0,1) K/V, seeded; scattered block tables",
        "config": {"workload": "block-table gather, C2 shapes (BASELINE configs[1])",
                   "n_seqs": n_seqs, "n_layers": L, "n_kv_heads": hkv, "head_dim": d,
                   "block_size": 16, "tokens": n_tok, "kv_dtype": args.kv_dtype,
                   "format": "raw storage (f32 decode in `f32`)", "parallelism": "single GPU"},
        "pct_of_hbm_peak": round(100 * raw["gbs"] / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "kernel": "gather_tables_tile_kernel (raw)",
                     "achieved": raw["kernel_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(raw["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(os.path.join(
                         ROOT, "profiles", f"gather_{args.kv_dtype}_llama3_8b_c2_kernel_stats_and_traffic.md")),
                     "bytes_per_launch": raw["bytes_per_call"],
                     "ms_per_launch": round(raw["us_per_call"] * 1e-3, 5)},
        "f32": legs["f32"], "device_copy_gbs": round(copy_gbs, 1),
        "raw_vs_device_copy": round(raw["kernel_gbs"] / copy_gbs, 3),
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        res["cpu_baseline"] = gather_cpu_baseline(args, pool, tables, ctx, L - 1, hkv, d, dtype,
                                                  last, offs)
    return res


def gather_cpu_baseline(args, pool, tables, ctx, layer, hkv, d, dtype, gpu_out, offs):
    """The oracle's restatement of the gather (fo_gather_tables: KvPool::k / v per
    position, decoded to f32) on layer `layer` of 16 sequences, one thread; also counts
    GPU raw-format bytes that differ from the oracle's on the same sample."""
    from oracle import ref
    seqs = np.arange(16)
    bs = 16
    c = np.asarray(ctx, np.int64)[seqs]
    nb = (c + bs - 1) // bs
    used = [int(b) for s, n in zip(seqs, nb) for b in tables[s, :n]]
    remap = {b: i for i, b in enumerate(used)}
    lay = ref.Layout(1, hkv, d, bs, len(used), dtype=dtype)
    region = lay.block_bytes
    image = np.empty(lay.pool_bytes, np.uint8)
    for b, i in remap.items():
        image[i * region:(i + 1) * region] = pool.read(b * pool.block_bytes + layer * region, region)
    tab = np.zeros((len(seqs), int(nb.max())), np.int32)
    for j, (s, n) in enumerate(zip(seqs, nb)):
        tab[j, :n] = [remap[int(b)] for b in tables[s, :n]]
    c32 = c.astype(np.int32)
    t1, reps = cpu_timed(lambda: ref.gather_tables(lay, image, 0, tab, c32, 0), args.cpu_seconds / 2)
    wk, wv, _ = ref.gather_tables(lay, image, 0, tab, c32, 1)
    # the GPU's raw output of the last layer for these sequences (rows offs[s] ..)
    gk = gpu_out[0][: int(c.sum())].cpu().numpy().reshape(-1)
    gv = gpu_out[1][: int(c.sum())].cpu().numpy().reshape(-1)
    bad = int((gk != wk.reshape(-1)).sum() + (gv != wv.reshape(-1)).sum())
    nbytes = gather_bytes(c, hkv, d, elem_bytes(dtype), 4.0)
    return {"value": round(nbytes / t1 / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"layer {layer}, {len(seqs)} seqs ({int(c.sum())} tokens): the oracle's "
                       f"fo_gather_tables (KvPool::k/v per position decoded to f32, "
                       f"pool.rs:174-204), {reps} reps at 1 thread"),
            "gpu_vs_cpu_raw_bytes_differing": bad}


def attn_bytes_prefill(ctx_end, q_len, hq, hkv, d, e=2.0):
    """Chunked prefill of q_len queries ending at ctx_end per sequence: K/V of the
    whole context once per KV head (e bytes a value), q and out in f32."""
    ctx_end = np.asarray(ctx_end, np.int64)
    return float((ctx_end * hkv * d * 2 * e + q_len * hq * d * 8 + ((ctx_end + 15) // 16) * 4).sum())


def run_c1(args, torch, fa, lib, dev):
    """TinyLlama-shaped: 1 sequence, 22 layers, 32/4 heads, D = 64, 256-block pool with
    the table a seeded permutation; a 512-token prefill append, then 64 decode steps."""
    rng = np.random.default_rng(args.seed)
    L, hq, hkv, d = 22, 32, 4, 64
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d, num_blocks=256,
                                         block_size=16, kv_dtype=1))
    perm = rng.permutation(256).astype(np.int32)
    tables = perm[None, : (512 + 64 + 15) // 16].copy()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    fill_ms = []
    fill_context(torch, pool, range(L), tables, np.array([512]), hkv, d, gen, dev, timer=fill_ms)
    K = 64
    dl = DecodeLoop(torch, fa, lib, pool, L, 1, hq, hkv, d, tables, np.array([512]), K, gen, dev,
                    rope=(args.rope_dim, args.rope_theta))
    wall, region_ms = dl.run(0, K)
    res = decode_result(args, dl, 0, K, wall, region_ms, 2.0, "tinyllama prefill 512 + 64 "
                        "decode steps (BASELINE configs[0])", {"kv_dtype": "f16"},
                        "fkv_append_decode_attention (attn_mfma_kernel + attn_combine_kernel)",
                        None)
    res["bulk_append"] = {"tokens_per_launch": 512, "ms_per_launch": round(float(np.median(fill_ms)), 4)}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args, pool, tables, dl.ctx_step[K - 1],
                                           dl.q[L - 1].cpu().numpy(), dl.out[L - 1].cpu().numpy(),
                                           L - 1, hq, hkv, d, 1)
    return res


# Llama-3-8B projection shapes (rows, cols) of one layer, in forward_one_token's order
# (crates/model/src/llama.rs:185-205 attn_q/k/v, :249-255 attn_output, then the FFN).
LLAMA3_8B_PROJ = [("attn_q", 4096, 4096), ("attn_k", 1024, 4096), ("attn_v", 1024, 4096),
                  ("attn_output", 4096, 4096), ("ffn_gate", 14336, 4096),
                  ("ffn_up", 14336, 4096), ("ffn_down", 4096, 14336)]


def q8_weights(torch, rows, cols, gen, dev):
    """Synthetic Q8_0 tensor bytes: random int8 quants, binary16 scales of random sign
    and mantissa in [2^-10, 2^-6) (the range of trained Llama Q8_0 weight scales)."""
    nb = rows * (cols // 32)
    w = torch.randint(-128, 128, (nb * 34,), dtype=torch.int8, device=dev, generator=gen)
    w = w.view(torch.uint8)
    sc = torch.randint(0x1400, 0x2400, (nb,), dtype=torch.int32, device=dev, generator=gen)
    sc |= torch.randint(0, 2, (nb,), dtype=torch.int32, device=dev, generator=gen) << 15
    blk = w.view(nb, 34)
    blk[:, 0] = (sc & 0xFF).to(torch.uint8)
    blk[:, 1] = ((sc >> 8) & 0xFF).to(torch.uint8)
    return w


def run_q8gemv(args, torch, fa, lib, dev):
    """The decode layer's projections with Q8_0 weights: one step = Kernels::gemv of
    attn_q/k/v/output and ffn_gate/up/down for each of Llama-3-8B's 32 layers (one token;
    --tokens n: Kernels::gemm of n tokens), distinct synthetic weights per layer (7.4 GB,
    so no launch reads weights another left in a cache). value = weight + activation +
    output bytes a step / wall time a step."""
    from oracle import ref

    L, T = 32, max(1, args.tokens)
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    xs = {c: torch.randn(T, c, device=dev, generator=gen) for c in (4096, 14336)}
    ys = {r: torch.empty(T, r, device=dev) for r in (1024, 4096, 14336)}
    ys_of = {name: torch.empty(T, rows, device=dev) for name, rows, _ in LLAMA3_8B_PROJ}
    calls, weights = [], []
    step_bytes = 0.0
    fused = args.gemv_fused or args.gemm_batched
    groups = ([["attn_q", "attn_k", "attn_v"], ["attn_output"], ["ffn_gate", "ffn_up"],
               ["ffn_down"]] if fused else [[n] for n, _, _ in LLAMA3_8B_PROJ])
    gws = None
    if args.gemm_batched:  # one workspace for every call (they are stream-ordered)
        need = max(fa.gemm_q8_0_batched_workspace_bytes(c, T) for c in (4096, 14336))
        gws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    shape = {n: (r, c) for n, r, c in LLAMA3_8B_PROJ}
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    keep = []  # ctypes arrays of the multi calls
    for _ in range(L):
        layer_w = {}
        for name, rows, cols in LLAMA3_8B_PROJ:
            w = q8_weights(torch, rows, cols, gen, dev)
            weights.append((name, rows, cols, w))
            layer_w[name] = w
            step_bytes += w.numel() + T * cols * 4 + T * rows * 4
        for g in groups:
            cols = shape[g[0]][1]
            if args.gemm_batched:
                n = len(g)
                arr_p, arr_u = ctypes.c_void_p * n, ctypes.c_uint64 * n
                a = (arr_p(*[layer_w[m].data_ptr() for m in g]),
                     arr_u(*[layer_w[m].numel() for m in g]), arr_u(*[shape[m][0] for m in g]),
                     arr_p(*[ys_of[m].data_ptr() for m in g]),
                     arr_u(*[T * shape[m][0] for m in g]))
                keep.append(a)
                calls.append((lib.fkv_gemm_q8_0_batched,
                              (n, a[0], a[1], a[2], cols, xs[cols].data_ptr(), T * cols, T, a[3],
                               a[4], gws.data_ptr(), gws.numel(), sp)))
            elif len(g) == 1:
                r = shape[g[0]][0]
                w = layer_w[g[0]]
                calls.append((lib.fkv_gemm_q8_0, (w.data_ptr(), w.numel(), r, cols,
                                                  xs[cols].data_ptr(), T * cols, T,
                                                  ys_of[g[0]].data_ptr(), T * r, sp)))
            else:
                n = len(g)
                arr_p, arr_u = ctypes.c_void_p * n, ctypes.c_uint64 * n
                a = (arr_p(*[layer_w[m].data_ptr() for m in g]),
                     arr_u(*[layer_w[m].numel() for m in g]), arr_u(*[shape[m][0] for m in g]),
                     arr_p(*[ys_of[m].data_ptr() for m in g]),
                     arr_u(*[T * shape[m][0] for m in g]))
                keep.append(a)
                calls.append((lib.fkv_gemm_q8_0_multi, (n, a[0], a[1], a[2], cols,
                                                        xs[cols].data_ptr(), T * cols, T, a[3],
                                                        a[4], sp)))
    torch.cuda.synchronize()

    def step():
        for f, c in calls:
            if f(*c) != 0:
                raise RuntimeError(lib.fkv_last_error().decode())

    W, K = args.warmup, args.steps
    for _ in range(W):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    region_ms = e0.elapsed_time(e1)
    n_launch = K * len(calls)
    value = step_bytes * K / wall / 1e9
    achieved = step_bytes / len(calls) / (region_ms * 1e-3 / n_launch) / 1e9
    kname = "gemv_q8_kernel<%d>" % (4 if T >= 3 else T)
    if args.gemm_batched and T >= 8:
        kname = "q8_act_kernel + gemm_q8_mfma_kernel (fkv_gemm_q8_0_batched)"
    res = {
        "metric": "Q8_0 weight GEMV HBM GB/s (Llama-3-8B decode projections), 1xMI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 x q8_0 -> i32, f32 accumulate",
        "data": "synthetic: random int8 quants, f16 scales in [2^-10, 2^-6); x ~ N(0,1)",
        "config": {"workload": "q8gemv", "model_shapes": "Llama-3-8B", "n_layers": L,
                   "tokens": T, "calls_per_step": len(calls),
                   "fused": "q/k/v and gate/up one launch each" if fused else "none",
                   "batched_gemm": bool(args.gemm_batched),
                   "weight_bytes_per_step": int(sum(w[3].numel() for w in weights)),
                   "parallelism": "single GPU"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": kname,
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(os.path.join(ROOT, "profiles",
                                                 "q8_gemv_llama3_8b_decode_kernel_stats.md"))
            if T == 1 and not fused else None,
            "bytes_per_launch": int(step_bytes / len(calls)),
            "ms_per_launch": round(region_ms / n_launch, 5),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        # the oracle's restatement of scalar.rs:191-204 + q8_dot.rs on layer 0's seven
        # matrices, on host cores; the GPU's outputs for the same inputs must equal it
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        x_h = {c: xs[c].cpu().numpy() for c in xs}
        mats = [(r, c, wd, wd.cpu().numpy()) for _, r, c, wd in weights[:len(LLAMA3_8B_PROJ)]]
        nbytes = sum(w.size + T * c * 4 + T * r * 4 for r, c, _, w in mats)
        mism = 0
        for r, c, wd, w in mats:
            y = torch.empty(T, r, device=dev)
            if lib.fkv_gemm_q8_0(wd.data_ptr(), w.size, r, c, xs[c].data_ptr(), T * c, T,
                                 y.data_ptr(), T * r, sp):
                raise RuntimeError(lib.fkv_last_error().decode())
            torch.cuda.synchronize()
            want = ref.q8_gemm(w, r, c, x_h[c], threads)
            mism += int((y.cpu().numpy().view(np.uint32) != want.view(np.uint32)).sum())
        def cpu_pass(nthr):
            for r, c, _, w in mats:
                ref.q8_gemm(w, r, c, x_h[c], nthr)
        t1, reps1 = cpu_timed(lambda: cpu_pass(1), args.cpu_seconds / 3)
        tn, reps = cpu_timed(lambda: cpu_pass(threads), args.cpu_seconds * 2 / 3)
        res["cpu_baseline"] = {
            "value": round(nbytes / tn / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": (f"layer 0's 7 projections ({nbytes / 1e6:.1f} MB), {T} token(s): the "
                       f"oracle's restatement of q8_dot.rs:35-109 / scalar.rs:191-204, "
                       f"{reps1} reps at 1 thread, {reps} reps at {threads} threads"),
            "value_1thread": round(nbytes / t1 / 1e9, 3),
            "seconds_1thread": round(t1, 3),
            "seconds_threads": round(tn, 3),
            "gpu_vs_cpu_bit_mismatches": mism,
        }
    return res


def run_layer(args, torch, fa, lib, dev):
    """The attention half of Llama-3-8B's decode layer, GPU-resident (DecodeAttentionLayer,
    llama.rs:185-255): per layer, q/k/v from the normed rows (one fkv_gemm_q8_0_batched
    call), RoPE + KV append + decode attention (fkv_rope_append_decode_attention), and
    attn_output (fkv_gemm_q8_0_batched), for C2's batch: 64 sequences, contexts uniform in
    [128, 4096], 32 layers with distinct synthetic Q8_0 weights (44.6 MB a layer), f16 KV.
    value = algorithmic bytes a step (weights, KV read and appended, activations) / wall
    time a step."""
    from oracle import ref

    K, W = args.steps, args.warmup
    rng = np.random.default_rng(args.seed)
    L, hq, hkv, d, n_embd, n_seqs = 32, 32, 8, 128, 4096, 64
    rope_dim, theta = 128, 500000.0
    ctx0 = rng.integers(128, 4097, n_seqs).astype(np.int64)
    nblk_seq = (ctx0 + W + K + 15) // 16
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=int(nblk_seq.sum()) + 64, block_size=16,
                                         kv_dtype=1))
    tables = make_tables(pool, nblk_seq, rng)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    fill_context(torch, pool, range(L), tables, ctx0, hkv, d, gen, dev)
    ctx_step = np.stack([ctx0 + t + 1 for t in range(W + K)]).astype(np.int32)
    ctx_d = torch.from_numpy(ctx_step).to(dev)
    tab_d = torch.from_numpy(tables).to(dev)
    max_ctx = int(ctx_step.max())
    shapes = [(hq * d, n_embd), (hkv * d, n_embd), (hkv * d, n_embd), (n_embd, hq * d)]
    layers, w_bytes = [], 0
    for l in range(L):
        w = [q8_weights(torch, r, c, gen, dev) for r, c in shapes]
        w_bytes += sum(x.numel() for x in w)
        layers.append(fa.DecodeAttentionLayer(pool, l, *w, hq, n_embd, rope_dim, theta,
                                              max_seqs=n_seqs, max_ctx_len=max_ctx))
    x = torch.randn((L, n_seqs, n_embd), generator=gen, device=dev)
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream()

    def step(t):
        for l in range(L):
            layers[l].forward(x[l], tab_d, ctx_d[t], max_ctx, y[l], stream=stream)

    for t in range(W):
        step(t)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(K):
        step(W + i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    region_ms = e0.elapsed_time(e1)
    assert pool.take_fault_flags() == 0
    # activations: x read, q/k/v written and read, attention rows written and read, y written
    act = n_seqs * 4 * (n_embd + 2 * (hq + 2 * hkv) * d + 2 * hq * d + n_embd)
    kv = [attn_bytes(ctx_step[W + i], hq, hkv, d, 2.0) + append_bytes(n_seqs, hkv, d, 2.0, 0)
          for i in range(K)]
    step_bytes = [float(k) * L + w_bytes + act * L for k in kv]
    value = sum(step_bytes) / wall / 1e9
    res = {
        "metric": METRIC + " (decode layer leg: attention half of the layer)",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16",
        "data": "synthetic: N(0,1) normed rows and K/V, random Q8_0 weights, seeded",
        "config": {"workload": "llama3-8b decode layer, attention half (q/k/v gemm, RoPE + "
                               "append + attention, attn_output gemm), C2 batch",
                   "n_seqs": n_seqs, "n_layers": L, "n_heads": hq, "n_kv_heads": hkv,
                   "head_dim": d, "n_embd": n_embd, "weights": "q8_0", "kv_dtype": "f16",
                   "rope_dim": rope_dim, "rope_theta": theta,
                   "mean_ctx": float(ctx_step[W:W + K].mean()), "parallelism": "single GPU"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(n_seqs * K / wall, 1),
        "us_per_layer": round(region_ms * 1e3 / (K * L), 2),
        "bytes_per_step": {"weights": int(w_bytes), "kv": int(np.mean(kv) * L),
                           "activations": int(act * L)},
        "roofline": {"bound": "hbm", "kernel": "whole layer (q8_act_kernel + "
                     "gemm_q8_mfma_kernel, attn_mfma_kernel + attn_combine_kernel, "
                     "q8_act_kernel + gemm_q8_mfma_kernel)",
                     "achieved": round(sum(step_bytes) / K / (region_ms * 1e-3 / K) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(sum(step_bytes) / (region_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        res["cpu_baseline"] = layer_cpu_baseline(args, torch, fa, pool, layers[L - 1], x[L - 1],
                                                 tables, ctx_step[W + K - 1], shapes)
    return res


def layer_cpu_baseline(args, torch, fa, pool, lay, x, tables, ctx, shapes):
    """The oracle chain of the same layer (fo_q8_gemm for q/k/v, fo_rope, the AVX2
    attention restatement, fo_q8_gemm for attn_output) on a bounded sample of the batch,
    at 16 threads (GEMMs and attention), in the leg's unit."""
    from oracle import ref
    if not ref.avx2_available():
        return None
    hq, hkv, d, n_embd = lay.n_heads, lay.hkv, lay.d, lay.n_embd
    seqs = np.arange(4)
    ctx = np.asarray(ctx, np.int64)[seqs]
    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    w = [t.cpu().numpy() for t in (lay.wq, lay.wk, lay.wv, lay.wo)]
    xs = x[seqs].cpu().numpy()
    bs = 16
    nb = (ctx + bs - 1) // bs
    used = [int(b) for s, n in zip(seqs, nb) for b in tables[s, :n]]
    remap = {b: i for i, b in enumerate(used)}
    lay1 = ref.Layout(1, hkv, d, bs, len(used), dtype=1)
    region = lay1.block_bytes
    image = np.empty(lay1.pool_bytes, np.uint8)
    for b, i in remap.items():
        image[i * region:(i + 1) * region] = pool.read(b * pool.block_bytes + lay.layer * region,
                                                       region)
    tab = np.zeros((len(seqs), int(nb.max())), np.int32)
    for j, (s, n) in enumerate(zip(seqs, nb)):
        tab[j, :n] = [remap[int(b)] for b in tables[s, :n]]
    scale = fa.default_scale(d)
    ctx32 = ctx.astype(np.int32)

    def chain():
        q = ref.q8_gemm(w[0], shapes[0][0], n_embd, xs, threads).reshape(len(seqs), hq, d)
        k = ref.q8_gemm(w[1], shapes[1][0], n_embd, xs, threads).reshape(len(seqs), hkv, d)
        ref.q8_gemm(w[2], shapes[2][0], n_embd, xs, threads)
        qr, _ = ref.rope_step(q, k, ctx32, lay.rope_dim, lay.theta)
        o = ref.avx2_attention(lay1, image, 0, qr, tab, ctx32, scale, threads)
        return ref.q8_gemm(w[3], n_embd, hq * d, o.reshape(len(seqs), hq * d), threads)

    sec, reps = cpu_timed(chain, args.cpu_seconds)
    wb = sum(a.size for a in w)
    nbytes = wb + attn_bytes(ctx, hq, hkv, d, 2.0)
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"layer {lay.layer}, {len(seqs)} of the batch's sequences "
                       f"({int(ctx.sum())} tokens): the oracle chain fo_q8_gemm x3, fo_rope, "
                       f"AVX2 attention, fo_q8_gemm; {reps} reps at {threads} threads "
                       "(the K/V append is not timed)"),
            "seconds_per_chain": round(sec, 4)}


def run_gguf(args, torch, fa, lib, dev):
    """gguf::load + weight upload to HBM: a synthetic Llama-3-8B-shaped Q8_0 GGUF
    (--gguf-layers layers of the 7 projections, alignment 32) is written to a temporary
    file, then opened (mmap + decode) and its data section uploaded to HBM through pinned
    staging; K timed repeats after W warm-ups (the file stays in the page cache, as a
    server restarting on the same model finds it). value = data-section bytes / time of
    open + upload. The plain pinned host-to-device copy of the same size is measured
    beside it as the link's ceiling."""
    import tempfile
    from tests import gguf_build as gb

    rng = np.random.default_rng(args.seed)
    tensors, cursor = [], 0
    one = {}
    for name, rows, cols in LLAMA3_8B_PROJ:  # random bytes a matrix, reused across layers
        nb = rows * cols // 32
        blk = rng.integers(0, 256, (nb, 34), dtype=np.uint8)
        blk[:, 1] = rng.integers(0x14, 0x24, nb, dtype=np.uint8)
        one[name] = blk.reshape(-1)
    for layer in range(args.gguf_layers):
        for name, rows, cols in LLAMA3_8B_PROJ:
            off = gb.align_up(cursor, 32)
            tensors.append((f"blk.{layer}.{name}.weight", [cols, rows], 8, off, one[name]))
            cursor = off + one[name].size
    head = gb.build(3, [("general.architecture", gb.Str("llama")),
                        ("llama.block_count", gb.U32(args.gguf_layers))],
                    [(n, d, g, o, b"") for n, d, g, o, _ in tensors], 32)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(head)
            for n, d, g, o, data in tensors:
                f.seek(len(head) + o)
                f.write(data.tobytes())
        with fa.GgufFile(path) as g:
            nbytes = g.data_bytes
        dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)

        def once():
            with fa.GgufFile(path) as g:
                g.upload(dst, chunk_bytes=args.gguf_chunk_mib << 20, threads=args.gguf_threads)

        for _ in range(args.warmup):
            once()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            once()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
        # correctness of the last upload: every tensor's bytes in HBM are the file's
        check = dst.cpu().numpy()
        with fa.GgufFile(path) as g:
            bad = sum(int(not np.array_equal(check[t.data_offset:t.data_offset + t.nbytes],
                                             one[t.name.split(".")[2]]))
                      for t in g.tensors)
        # the link's ceiling: one pinned buffer of the same size, copied to the device
        pinned = torch.empty(nbytes, dtype=torch.uint8).pin_memory()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            dst.copy_(pinned, non_blocking=True)
        torch.cuda.synchronize()
        link = (time.perf_counter() - t0) / 3
    finally:
        os.unlink(path)
    return {
        "metric": "GGUF open + weight upload to HBM GB/s, 1xMI355X",
        "value": round(nbytes / wall / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bytes (Q8_0 tensors copied as stored)",
        "data": "synthetic Llama-3-8B-shaped Q8_0 GGUF in the page cache",
        "config": {"workload": "gguf", "layers": args.gguf_layers, "tensors": len(tensors),
                   "data_bytes": int(nbytes), "chunk_bytes": (args.gguf_chunk_mib or 8) << 20,
                   "host_threads": args.gguf_threads or min(len(os.sched_getaffinity(0)), 4),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "pcie", "achieved": round(nbytes / wall / 1e9, 2),
                     "peak": round(nbytes / link / 1e9, 2), "unit": "GB/s",
                     "frac": round(link / wall, 4), "traffic": None,
                     "peak_is": "pinned host-to-device copy of the same size, measured"},
        "tensors_differing_after_upload": bad,
        "cpu_baseline": None,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "sharding the path over several GPUs is a design, not built here", file=sys.stderr)
        sys.exit(2)

    import torch

    import ferrum_amd as fa
    from ferrum_amd import _lib

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    lib = _lib.load()
    if args.attn_engine == "valu":
        fa.set_tuning(fa.TUNE_ATTN_ENGINE, 1)
    run = {"c1": run_c1, "c2": run_c2, "c3": run_c3, "c4": run_c4, "c5": run_c5,
           "q8gemv": run_q8gemv, "gguf": run_gguf, "layer": run_layer,
           "gather": run_gather}[args.workload]
    result = run(args, torch, fa, lib, dev)
    if args.attn_engine == "valu":
        # a measurement of the alternative engine: the committed traffic figure belongs
        # to the matrix-core kernel
        result["attn_engine"] = "valu (attn_partition_kernel on F16 storage)"
        if isinstance(result.get("roofline"), dict):
            result["roofline"]["traffic"] = None
    if (args.workload == "c2" and args.kv_dtype == "f16" and args.n_heads == 32
            and not args.rope_dim and not args.no_configs and args.attn_engine == "mfma"):
        result["configs"] = other_configs(args, torch, fa, lib, dev)
    print(json.dumps(result), flush=True)


def other_configs(args, torch, fa, lib, dev):
    """Compact results of the other BASELINE configs and the gather leg, run after the
    headline in the same process (no CPU baselines; each leg's pool is released before
    the next). A leg that fails records its error instead of hiding the headline."""
    import copy
    import gc

    def pct(v):
        return round(100 * v / HBM_PEAK_GBS, 2)

    def c1(r):
        return {"value_gbs": r["value"], "pct_of_hbm_peak": pct(r["value"]),
                "us_per_call": round(r["roofline"]["ms_per_launch"] * 1e3, 2),
                "frac": r["roofline"]["frac"], "note": "latency-bound: 0.58 MB a call"}

    def c3(r):
        p = r["prefill_attention"]
        return {"value_gbs": r["value"], "pct_of_hbm_peak": r["pct_of_hbm_peak"],
                "ms_per_step": r["ms_per_step"], "decode_only_ms_per_step": r["decode_only_ms_per_step"],
                "decode_frac": r["roofline"]["frac"], "prefill_us_per_call": p["us_per_call"],
                "prefill_tflops": p["tflops"], "prefill_pct_of_mfma_peak": p["pct_of_mfma_peak"],
                "prefill_leak_safe": p["leak_safe_instance"],
                "streams": r["config"].get("streams", 1),
                "decode_wgs_per_cu": r["config"].get("decode_wgs_per_cu")}

    def c4(r):
        return {"value_gbs": r["value"], "pct_of_hbm_peak": r["pct_of_hbm_peak"],
                "ms_per_step": r["ms_per_step"], "frac": r["roofline"]["frac"],
                "exact_instance": r["exact_instance"]}

    def c5(r):
        return {"value_gbs": r["value"], "pct_of_hbm_peak": r["pct_of_hbm_peak"],
                "ms_per_step": r["ms_per_step"], "frac": r["roofline"]["frac"],
                "copy_blocks_gbs": r["copy_blocks"]["gbs"],
                "copy_blocks_pct_of_hbm_peak": r["copy_blocks"]["pct_of_hbm_peak"],
                "swap_out_gbs": r["swap"]["out_gbs"], "swap_in_gbs": r["swap"]["in_gbs"]}

    def gather(r):
        return {"raw_gbs": r["value"], "raw_kernel_gbs": r["roofline"]["achieved"],
                "frac": r["roofline"]["frac"], "raw_vs_device_copy": r["raw_vs_device_copy"],
                "f32_kernel_gbs": r["f32"]["kernel_gbs"], "device_copy_gbs": r["device_copy_gbs"]}

    legs = [("c1", run_c1, "f16", c1), ("c4", run_c4, "q8_0", c4), ("c5", run_c5, "f16", c5),
            ("c3", run_c3, "f16", c3), ("gather_f16", run_gather, "f16", gather),
            ("gather_q8_0", run_gather, "q8_0", gather)]
    out = {}
    for name, fn, kv, pick in legs:
        a = copy.copy(args)
        a.no_cpu, a.kv_dtype = True, kv
        t0 = time.perf_counter()
        try:
            out[name] = pick(fn(a, torch, fa, lib, dev))
        except Exception as ex:  # recorded in the line; the headline still prints
            out[name] = {"error": f"{type(ex).__name__}: {ex}"[:400]}
        out[name]["leg_seconds"] = round(time.perf_counter() - t0, 1)
        gc.collect()
        torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    main()
