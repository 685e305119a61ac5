"""GPU: the revision-1 KvPool surface over device storage.

Ports the unit tests of crates/kvcache/src/pool.rs:233-308 onto the C ABI, then
drives the device pool and the oracle's restated dense pool with the same random
operation sequence and requires identical status, message and data at every step.
"""
import numpy as np
import pytest

import ferrum_amd as fa

pytestmark = pytest.mark.gpu


def tiny_config():
    # pool.rs:237-245
    return fa.KvPoolConfig(n_layers=2, n_kv_heads=1, head_dim=4, max_seq_len=3, max_slots=2)


def test_append_commit_round_trip():
    # pool.rs:247-261
    pool = fa.PreallocatedKvPool.new(tiny_config())
    slot = pool.alloc()
    assert pool.seq_len(slot) == 0
    k = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    v = np.array([5.0, 6.0, 7.0, 8.0], np.float32)
    pool.append_layer(slot, 0, k, v)
    pool.append_layer(slot, 1, k, v)
    pool.commit_token(slot)
    assert pool.seq_len(slot) == 1
    assert np.array_equal(pool.k(slot, 0, 0).view(np.uint32), k.view(np.uint32))
    assert np.array_equal(pool.v(slot, 1, 0).view(np.uint32), v.view(np.uint32))
    pool.free(slot)


def test_append_must_be_in_layer_order_and_commit_needs_all_layers():
    # pool.rs:263-275
    pool = fa.PreallocatedKvPool.new(tiny_config())
    slot = pool.alloc()
    k = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    v = np.array([5.0, 6.0, 7.0, 8.0], np.float32)
    with pytest.raises(fa.CacheError, match="^cache: layers must append in order$"):
        pool.append_layer(slot, 1, k, v)
    pool.append_layer(slot, 0, k, v)
    with pytest.raises(fa.CacheError, match="^cache: not every layer appended$"):
        pool.commit_token(slot)
    pool.append_layer(slot, 1, k, v)
    pool.commit_token(slot)
    with pytest.raises(fa.CacheError, match="^cache: position not yet committed$"):
        pool.k(slot, 0, 1)


def test_uncommit_and_abandon_let_the_next_append_start_over():
    # pool.rs:277-291
    pool = fa.PreallocatedKvPool.new(tiny_config())
    slot = pool.alloc()
    k = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    v = np.array([5.0, 6.0, 7.0, 8.0], np.float32)
    pool.append_layer(slot, 0, k, v)
    pool.abandon_partial(slot)
    pool.append_layer(slot, 0, k, v)
    pool.append_layer(slot, 1, k, v)
    pool.commit_token(slot)
    pool.uncommit_token(slot)
    assert pool.seq_len(slot) == 0
    pool.append_layer(slot, 0, k, v)


def test_constructor_allocates_dense_storage_without_later_growth():
    # pool.rs:293-307
    cfg = tiny_config()
    expected = cfg.max_slots * cfg.n_layers * cfg.max_seq_len * cfg.n_kv_heads * cfg.head_dim * 2
    pool = fa.PreallocatedKvPool.new(cfg)
    assert pool.storage_len() == expected
    slot = pool.alloc()
    k = np.array([9.0, 8.0, 7.0, 6.0], np.float32)
    v = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    pool.append_layer(slot, 0, k, v)
    pool.append_layer(slot, 1, k, v)
    pool.commit_token(slot)
    assert pool.storage_len() == expected


def test_exhaustion_is_unavailable():
    pool = fa.PreallocatedKvPool.new(tiny_config())
    pool.alloc()
    pool.alloc()
    with pytest.raises(fa.Unavailable, match="^no free kv slots$") as e:
        pool.alloc()
    assert e.value.http_status == 503


def _apply(op, args, dev, ora):
    """Run one op on both pools; return (dev_result, oracle_result) normalised to
    (code, message, value)."""
    codes = {fa.CacheError: 1, fa.Unavailable: 2}
    try:
        val = getattr(dev, op)(*args)
        d = (0, "", val)
    except fa.FerrumError as e:
        d = (codes.get(type(e), 9), str(e), None)
    code, msg, val = getattr(ora, op)(*args)
    o = (code, msg if code else "", val if code == 0 else None)
    return d, o


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_operation_sequence_matches_oracle(seed):
    from oracle import ref
    rng = np.random.default_rng(seed)
    L, hkv, d, maxseq, slots = 3, 2, 8, 5, 3
    dev = fa.PreallocatedKvPool.new(fa.KvPoolConfig(L, hkv, d, maxseq, slots))
    ora = ref.DensePool(L, hkv, d, maxseq, slots)
    ops = ["alloc", "free", "seq_len", "append_layer", "append_layer", "append_layer",
           "commit_token", "k", "v", "abandon_partial", "uncommit_token"]
    for step in range(400):
        op = ops[rng.integers(len(ops))]
        slot = int(rng.integers(0, slots + 1))  # includes an out-of-range slot
        if op == "alloc":
            args = ()
        elif op in ("free", "seq_len", "commit_token", "abandon_partial", "uncommit_token"):
            args = (slot,)
        elif op == "append_layer":
            n = hkv * d if rng.random() > 0.05 else hkv * d - 1
            k = rng.standard_normal(n).astype(np.float32)
            v = rng.standard_normal(hkv * d).astype(np.float32)
            layer = int(rng.integers(0, L + 1))
            args = (slot, layer, k, v)
        else:
            args = (slot, int(rng.integers(0, L + 1)), int(rng.integers(0, maxseq + 1)))
        dres, ores = _apply(op, args, dev, ora)
        assert dres[0] == ores[0], f"step {step} {op}{args[:3]}: {dres[:2]} vs {ores[:2]}"
        assert dres[1] == ores[1], f"step {step} {op}: {dres[1]!r} vs {ores[1]!r}"
        if op in ("k", "v") and dres[0] == 0:
            assert np.array_equal(dres[2].view(np.uint32), ores[2].view(np.uint32))
        elif op in ("alloc", "seq_len") and dres[0] == 0:
            assert dres[2] == ores[2]
