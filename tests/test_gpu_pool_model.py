"""GPU parity: the paged pool against a model, one random operation at a time.

A seeded sequence of appends (through random slot mappings, some rows holding a value
that marks its block: a Q8_0 scale past 512, an infinite F16 V), copy_blocks (distinct
destinations that are not sources), swap_out / swap_in through the pinned host blocks,
fill(0), and slot and block-table gathers, applied to the device pool and to the oracle's
image (pool.rs:122-153 append, :174-204 reads; copy and swap move whole blocks). After
every operation the device image equals the oracle's byte for byte, the marked-block count
equals the model's (marks travel with copies and swaps; fill(0) clears them), and every
gather equals the oracle's, bit for bit.
"""
import numpy as np
import pytest

from tests.helpers import make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu

NB, NHOST, B = 24, 8, 16


@pytest.mark.parametrize("dtype,rounding", [(1, 0), (1, 1), (8, 0), (0, 0)])
def test_random_operations_match_the_model(dtype, rounding):
    import torch
    from oracle import ref
    rng = np.random.default_rng(5000 + 10 * dtype + rounding)
    layers, hkv, d = 2, 2, 64
    pool, layout = make_pools(layers, hkv, d, NB, dtype=dtype, rounding=rounding,
                              num_host_blocks=NHOST)
    pool.fill(0)
    image = ref.new_pool(layout)
    bb = pool.block_bytes
    host = {}                  # host block -> bytes
    marked, host_marked = set(), set()
    for step in range(60):
        op = rng.choice(["append", "append", "copy", "swap_out", "swap_in", "gather", "fill"],
                        p=[0.3, 0.1, 0.15, 0.12, 0.12, 0.16, 0.05])
        if op == "append":
            layer = int(rng.integers(0, layers))
            n = int(rng.integers(1, 41))
            slots = rng.choice(NB * B, n, replace=False).astype(np.int64)
            k = rng.standard_normal((n, hkv, d)).astype(np.float32)
            v = rng.standard_normal((n, hkv, d)).astype(np.float32)
            if dtype in (1, 8) and rng.random() < 0.3:  # a value that marks its block
                t = int(rng.integers(0, n))
                v[t, int(rng.integers(0, hkv)), int(rng.integers(0, d))] = np.inf if dtype == 1 else 1e5
                marked.add(int(slots[t]) // B)
            pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
            ref.append(layout, image, layer, k, v, slots)
        elif op == "copy":
            n = int(rng.integers(1, 6))
            blocks = rng.choice(NB, 2 * n, replace=False)
            pairs = np.stack([blocks[:n], blocks[n:]], 1).astype(np.int64)
            pool.copy_blocks(to_dev(pairs))
            ref.copy_blocks(layout, image, pairs)
            for s, t in pairs:
                marked.discard(int(t))
                if int(s) in marked:
                    marked.add(int(t))
        elif op == "swap_out":
            n = int(rng.integers(1, 5))
            dev = rng.choice(NB, n, replace=False)
            hb = rng.choice(NHOST, n, replace=False)
            pool.swap_out(np.stack([dev, hb], 1).astype(np.int64))
            for db_, h in zip(dev, hb):
                host[int(h)] = image[int(db_) * bb:(int(db_) + 1) * bb].copy()
                host_marked.discard(int(h))
                if int(db_) in marked:
                    host_marked.add(int(h))
        elif op == "swap_in" and host:
            hb = rng.choice(sorted(host), min(len(host), int(rng.integers(1, 5))), replace=False)
            dev = rng.choice(NB, len(hb), replace=False)
            pool.swap_in(np.stack([hb, dev], 1).astype(np.int64))
            for h, db_ in zip(hb, dev):
                image[int(db_) * bb:(int(db_) + 1) * bb] = host[int(h)]
                marked.discard(int(db_))
                if int(h) in host_marked:
                    marked.add(int(db_))
        elif op == "gather":
            layer = int(rng.integers(0, layers))
            slots = rng.choice(NB * B, int(rng.integers(1, 60)), replace=False).astype(np.int64)
            for fmt in (0, 1):
                wk, wv = ref.gather_slots(layout, image, layer, slots, fmt)
                ok = torch.empty(wk.shape, dtype=torch.float32 if fmt == 0 else torch.uint8,
                                 device="cuda")
                ov = torch.empty_like(ok)
                pool.gather_slots(layer, to_dev(slots), ok, ov, fmt=fmt)
                torch.cuda.synchronize()
                gk, gv = ok.cpu().numpy(), ov.cpu().numpy()
                assert np.array_equal(gk.view(np.uint8), wk.view(np.uint8)), (step, fmt, "k")
                assert np.array_equal(gv.view(np.uint8), wv.view(np.uint8)), (step, fmt, "v")
            # one sequence's block-table gather over a random table
            ctx = int(rng.integers(1, 5 * B))
            tab = rng.choice(NB, 5, replace=False).astype(np.int32)[None, :]
            wk, wv, _ = ref.gather_tables(layout, image, layer, tab, np.array([ctx]), 0)
            ok = torch.empty(wk.shape, dtype=torch.float32, device="cuda")
            ov = torch.empty_like(ok)
            pool.gather_tables(layer, to_dev(tab), to_dev(np.array([ctx], np.int32)),
                               to_dev(np.array([0], np.int64)), ctx, ok, ov)
            torch.cuda.synchronize()
            assert np.array_equal(ok.cpu().numpy().view(np.uint32), wk.view(np.uint32)), step
            assert np.array_equal(ov.cpu().numpy().view(np.uint32), wv.view(np.uint32)), step
        elif op == "fill":
            pool.fill(0)
            image[:] = 0
            marked.clear()
        torch.cuda.synchronize()
        assert np.array_equal(pool.read(), image), f"step {step} ({op}): pool image differs"
        if dtype != 0:
            assert pool.marked_blocks() == len(marked), (step, op, pool.marked_blocks(), marked)
    assert pool.take_fault_flags() == 0
    pool.close()
