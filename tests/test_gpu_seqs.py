"""The sequence block manager (fkv_seqs_*) on a real pool.

It replaces the scheduler's dense-slot KV use (crates/scheduler/src/batcher.rs):
- admission stops on Unavailable (:108-129) and allocates nothing then;
- a rollback (restore_kv, :291-308, a prefix replay) becomes a truncation that
  leaves the sequence's K/V exactly as before the rolled-back tokens;
- finish frees the blocks (:329-338).
Forks share blocks and copy the shared partial block before the first write, and
preemption round-trips through the pool's host blocks. The K/V a sequence reads
(through the manager's slots and block tables) are checked against the oracle's
encoding of its own token history, and its attention against the oracle's.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, to_dev

pytestmark = pytest.mark.gpu

HKV, D, G = 2, 64, 4


def _setup(num_blocks, num_host_blocks=0, dtype=1):
    import ferrum_amd as fa
    pool, layout = make_pools(1, HKV, D, num_blocks, dtype=dtype, num_host_blocks=num_host_blocks)
    pool.fill(0)
    return pool, layout, fa.SequenceManager(pool)


def _append(pool, mgr, seq, rows_k, rows_v):
    """Reserve, copy a shared block if the manager asks, append, commit."""
    import torch
    n = rows_k.shape[0]
    pair = mgr.reserve(seq, n)
    if pair is not None:
        pool.copy_blocks(torch.tensor([pair], dtype=torch.int64, device="cuda"))
    length, _ = mgr.length(seq)
    slots = mgr.slots(seq, length, n)
    pool.append(0, to_dev(rows_k), to_dev(rows_v), to_dev(slots))
    torch.cuda.synchronize()
    mgr.commit(seq, n)
    return pair


def _attend(pool, mgr, seqs, q):
    import torch
    tab, ctx = mgr.tables(seqs, 64)
    out = torch.full(q.shape, 9.0, dtype=torch.float32, device="cuda")
    pool.decode_attention(0, to_dev(q), out, to_dev(tab), to_dev(ctx), int(max(1, ctx.max())))
    torch.cuda.synchronize()
    return out.cpu().numpy(), tab, ctx


def _rows_of(pool, layout, mgr, seq):
    from oracle import ref
    n, _ = mgr.length(seq)
    return ref.gather_slots(layout, pool.read(), 0, mgr.slots(seq, 0, n), 0)


def _enc(rows):
    from oracle import ref
    return ref.f16_to_f32(ref.f32_to_f16(rows))


def test_admission_by_free_blocks():
    import ferrum_amd as fa
    pool, layout, mgr = _setup(10)
    a = mgr.add(100)                       # 7 blocks
    assert pool.free_block_count() == 3
    with pytest.raises(fa.errors.Unavailable) as e:
        mgr.add(60)                        # 4 blocks: refused, nothing taken
    assert str(e.value) == "no free kv blocks"
    assert pool.free_block_count() == 3
    b = mgr.add(48)                        # exactly 3
    assert pool.free_block_count() == 0
    with pytest.raises(fa.errors.Unavailable):
        mgr.reserve(b, 49)                 # a 4th block for b: none left, nothing changes
    assert mgr.length(b) == (0, False)
    mgr.free(a)
    assert pool.free_block_count() == 7
    with pytest.raises(fa.errors.CacheError) as e:
        mgr.free(a)
    assert str(e.value) == "cache: unknown sequence"
    mgr.close()
    assert pool.free_block_count() == 10
    pool.close()


def test_histories_through_slots_and_tables_match_the_oracle():
    from oracle import ref
    import ferrum_amd as fa
    pool, layout, mgr = _setup(64)
    rng = np.random.default_rng(0)
    lens = [1, 16, 33, 100]
    seqs, hist = [], []
    for n in lens:
        s = mgr.add(n)
        k = rng.standard_normal((n, HKV, D), dtype=np.float32)
        v = rng.standard_normal((n, HKV, D), dtype=np.float32)
        _append(pool, mgr, s, k[:n // 2], v[:n // 2])     # in two appends
        _append(pool, mgr, s, k[n // 2:], v[n // 2:])
        seqs.append(s)
        hist.append((k, v))
    for s, (k, v) in zip(seqs, hist):
        kg, vg = _rows_of(pool, layout, mgr, s)
        assert np.array_equal(kg, _enc(k)) and np.array_equal(vg, _enc(v))
    q = rng.standard_normal((len(seqs), HKV * G, D), dtype=np.float32)
    got, tab, ctx = _attend(pool, mgr, seqs, q)
    assert list(ctx) == lens
    want = ref.attention(layout, pool.read(), 0, q, tab, ctx, fa.default_scale(D))
    assert_close(got, want)
    mgr.close()
    pool.close()


def test_fork_copies_the_shared_block_before_writing():
    pool, layout, mgr = _setup(32)
    rng = np.random.default_rng(1)
    k = rng.standard_normal((41, HKV, D), dtype=np.float32)
    v = rng.standard_normal((41, HKV, D), dtype=np.float32)
    parent = mgr.add(40)
    _append(pool, mgr, parent, k[:40], v[:40])
    child = mgr.fork(parent)
    tab, _ = mgr.tables([parent, child], 8)
    assert np.array_equal(tab[0, :3], tab[1, :3])
    assert all(pool.refcount(int(b)) == 2 for b in tab[0, :3])
    # the child writes position 40 into the shared, partly filled block 2: a private copy
    kc, vc = rng.standard_normal((1, HKV, D), dtype=np.float32), rng.standard_normal((1, HKV, D), dtype=np.float32)
    pair = _append(pool, mgr, child, kc, vc)
    assert pair is not None and pair[0] == tab[0, 2]
    assert pool.refcount(int(tab[0, 2])) == 1
    # the parent is the block's only user now: no copy
    assert _append(pool, mgr, parent, k[40:], v[40:]) is None
    kg, vg = _rows_of(pool, layout, mgr, parent)
    assert np.array_equal(kg, _enc(k)) and np.array_equal(vg, _enc(v))
    kg, vg = _rows_of(pool, layout, mgr, child)
    assert np.array_equal(kg, _enc(np.concatenate([k[:40], kc])))
    assert np.array_equal(vg, _enc(np.concatenate([v[:40], vc])))
    # a fork of the child copies the child's partly filled block in turn
    grand = mgr.fork(child)
    assert _append(pool, mgr, grand, k[:7], v[:7]) is not None
    mgr.close()
    assert pool.free_block_count() == 32
    pool.close()


def test_truncation_rolls_back_exactly():
    """Rollback by truncation: after appending 5 tokens and truncating them away, the
    sequence reads what it read before, bit for bit, and the blocks past it are free."""
    pool, layout, mgr = _setup(32)
    rng = np.random.default_rng(2)
    k = rng.standard_normal((50, HKV, D), dtype=np.float32)
    v = rng.standard_normal((50, HKV, D), dtype=np.float32)
    s = mgr.add(50)
    _append(pool, mgr, s, k, v)
    q = rng.standard_normal((1, HKV * G, D), dtype=np.float32)
    before, _, _ = _attend(pool, mgr, [s], q)
    free_before = pool.free_block_count()
    extra = rng.standard_normal((15, HKV, D), dtype=np.float32)
    _append(pool, mgr, s, extra, extra)
    assert pool.free_block_count() == free_before - 1           # 65 tokens: 5 blocks
    mgr.truncate(s, 50)
    assert pool.free_block_count() == free_before
    after, _, ctx = _attend(pool, mgr, [s], q)
    assert list(ctx) == [50]
    assert np.array_equal(before.view(np.uint32), after.view(np.uint32))
    import ferrum_amd as fa
    with pytest.raises(fa.errors.CacheError) as e:
        mgr.truncate(s, 51)
    assert str(e.value) == "cache: truncate past the sequence length"
    with pytest.raises(fa.errors.CacheError) as e:
        mgr.commit(s, 100)
    assert str(e.value) == "cache: commit past the reserved blocks"
    mgr.close()
    pool.close()


def test_swap_preemption_round_trip():
    import ferrum_amd as fa
    import torch
    pool, layout, mgr = _setup(16, num_host_blocks=8)
    rng = np.random.default_rng(3)
    k = rng.standard_normal((100, HKV, D), dtype=np.float32)
    v = rng.standard_normal((100, HKV, D), dtype=np.float32)
    s = mgr.add(100)
    _append(pool, mgr, s, k, v)
    other = mgr.add(16)
    q = rng.standard_normal((1, HKV * G, D), dtype=np.float32)
    before, tab0, _ = _attend(pool, mgr, [s], q)
    mgr.swap_out(s)
    torch.cuda.synchronize()
    assert mgr.length(s) == (100, True)
    assert pool.free_block_count() == 16 - 1
    with pytest.raises(fa.errors.CacheError) as e:
        mgr.reserve(s, 1)
    assert str(e.value) == "cache: sequence is swapped out"
    # reuse the released blocks, so the sequence comes back elsewhere
    filler = mgr.add(16 * 8)
    mgr.swap_in(s)
    torch.cuda.synchronize()
    after, tab1, _ = _attend(pool, mgr, [s], q)
    assert not np.array_equal(tab0[0, :7], tab1[0, :7])
    assert np.array_equal(before.view(np.uint32), after.view(np.uint32))
    kg, vg = _rows_of(pool, layout, mgr, s)
    assert np.array_equal(kg, _enc(k)) and np.array_equal(vg, _enc(v))
    # s's 7 committed blocks take 7 of the 8 host blocks (other has none committed);
    # big's 2 blocks do not fit in the last one
    mgr.free(filler)
    big = mgr.add(32)
    _append(pool, mgr, big, k[:32], v[:32])
    mgr.swap_out(s)
    mgr.swap_out(other)          # length 0: nothing to copy
    with pytest.raises(fa.errors.Unavailable) as e:
        mgr.swap_out(big)
    assert str(e.value) == "no free host blocks"
    torch.cuda.synchronize()
    mgr.close()
    assert pool.free_block_count() == 16
    pool.close()


def test_destroying_the_pool_detaches_its_manager():
    """A manager that outlives its pool holds no pointer into it: its calls fail and
    closing it releases only its own memory."""
    import ferrum_amd as fa
    pool, layout, mgr = _setup(8)
    s = mgr.add(20)
    pool.close()
    with pytest.raises(fa.errors.InvalidRequest) as e:
        mgr.add(1)
    assert str(e.value) == "pool destroyed"
    with pytest.raises(fa.errors.CacheError):
        mgr.length(s)
    mgr.close()


@pytest.mark.parametrize("dtype", [1, 8])
@pytest.mark.parametrize("seed", range(3))
def test_random_scheduler_operations_match_the_model(seed, dtype):
    """Seeded random admissions, appends, forks, truncations, swaps and frees on a small
    pool (some refused with Unavailable, which must change nothing). After every step each
    resident sequence's K/V, read through its slots, is its own token history through the
    storage's encoding (binary16, or Q8_0 blocks of 32 along each head) bit for bit; every
    20 steps the attention over all resident sequences matches the oracle's."""
    import ferrum_amd as fa
    from oracle import ref
    rng = np.random.default_rng(6000 + 10 * dtype + seed)
    pool, layout, mgr = _setup(24, num_host_blocks=40, dtype=dtype)
    if dtype == 1:
        enc = _enc
    else:
        def enc(rows):
            return ref.q8_dequant(ref.q8_quantize_row(rows), rows.size).reshape(rows.shape)
    model = {}  # seq -> (k rows, v rows, swapped)
    done = {}
    for step in range(100):
        live = sorted(model)
        resident = [q for q in live if not model[q][2]]
        op = rng.choice(["add", "append", "append", "fork", "truncate", "swap_out",
                         "swap_in", "free"])
        free_before = pool.free_block_count()
        try:
            if op == "add" or not live:
                seq = mgr.add(int(rng.integers(0, 160)))
                model[seq] = (np.zeros((0, HKV, D), np.float32), np.zeros((0, HKV, D), np.float32), False)
            elif op == "append" and resident:
                seq = int(rng.choice(resident))
                n = int(rng.integers(1, 40))
                k = rng.standard_normal((n, HKV, D)).astype(np.float32)
                v = rng.standard_normal((n, HKV, D)).astype(np.float32)
                _append(pool, mgr, seq, k, v)
                mk, mv, _ = model[seq]
                model[seq] = (np.concatenate([mk, k]), np.concatenate([mv, v]), False)
            elif op == "fork" and resident:
                parent = int(rng.choice(resident))
                child = mgr.fork(parent)
                mk, mv, _ = model[parent]
                model[child] = (mk.copy(), mv.copy(), False)
            elif op == "truncate" and resident:
                seq = int(rng.choice(resident))
                mk, mv, _ = model[seq]
                m = int(rng.integers(0, mk.shape[0] + 1))
                mgr.truncate(seq, m)
                model[seq] = (mk[:m], mv[:m], False)
            elif op == "swap_out" and resident:
                seq = int(rng.choice(resident))
                mgr.swap_out(seq)
                mk, mv, _ = model[seq]
                model[seq] = (mk, mv, True)
            elif op == "swap_in":
                swapped = [q for q in live if model[q][2]]
                if swapped:
                    seq = int(rng.choice(swapped))
                    mgr.swap_in(seq)
                    mk, mv, _ = model[seq]
                    model[seq] = (mk, mv, False)
            elif op == "free" and live:
                seq = int(rng.choice(live))
                mgr.free(seq)
                del model[seq]
            done[op] = done.get(op, 0) + 1
        except fa.Unavailable:
            assert pool.free_block_count() == free_before, (step, op)
            done["unavailable"] = done.get("unavailable", 0) + 1
        import torch
        torch.cuda.synchronize()
        for seq, (mk, mv, swapped) in model.items():
            assert mgr.length(seq) == (mk.shape[0], swapped), (step, op, seq)
            if swapped or mk.shape[0] == 0:
                continue
            gk, gv = _rows_of(pool, layout, mgr, seq)
            assert np.array_equal(gk.view(np.uint32), enc(mk).view(np.uint32)), (step, op, seq)
            assert np.array_equal(gv.view(np.uint32), enc(mv).view(np.uint32)), (step, op, seq)
        resident = [q for q in sorted(model) if not model[q][2] and model[q][0].shape[0] > 0]
        if step % 20 == 19 and resident:
            q = rng.standard_normal((len(resident), HKV * G, D)).astype(np.float32)
            got, tab, ctx = _attend(pool, mgr, resident, q)
            want = ref.attention(layout, pool.read(), 0, q, tab, ctx, fa.default_scale(D))
            assert_close(got, want, what=f"step {step}")
            done["attention"] = done.get("attention", 0) + 1
    assert pool.take_fault_flags() == 0
    # the walk must have reached every kind of step, a refusal and the attention check
    for kind in ("add", "append", "fork", "truncate", "swap_out", "swap_in", "free",
                 "unavailable", "attention"):
        assert done.get(kind, 0) > 0, (kind, done)
