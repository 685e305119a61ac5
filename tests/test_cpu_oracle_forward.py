"""CPU: the oracle's restatement of Llama::forward's KV sequence (oracle.ref.forward_kv,
crates/model/src/llama.rs:345-389) over the oracle's dense pool.

Pinned by the reference's own test crates/model/src/tests.rs:176-192 (two tokens from
position 0 commit two positions; a call whose position0 is not the sequence length is
a Model error that leaves the length alone) and by what the sequence fixes whatever
the model computes: a call that succeeds commits one position per token, each holding
its token's rows; a call that fails anywhere (embed, before or after a layer's append,
the pool's own capacity error) leaves the committed length and every committed row as
they were, with no partial layers (the next append must be layer 0).
"""
import itertools

import numpy as np
import pytest

from oracle import ref

L, HKV, D = 3, 2, 4


def rows(rng, n):
    return [[(rng.standard_normal(HKV * D).astype(np.float32),
              rng.standard_normal(HKV * D).astype(np.float32)) for _ in range(L)]
            for _ in range(n)]


def state(pool, slot):
    code, msg, n = pool.seq_len(slot)
    assert code == 0, msg
    ks = [[pool.k(slot, layer, p)[2].copy() for layer in range(L)] for p in range(n)]
    vs = [[pool.v(slot, layer, p)[2].copy() for layer in range(L)] for p in range(n)]
    return n, ks, vs


def test_reference_forward_logit_shape_and_position0():
    # crates/model/src/tests.rs:176-192 (MockModel::tiny: 1 layer)
    pool = ref.DensePool(1, HKV, D, 4, 1)
    code, _, slot = pool.alloc()
    assert code == 0 and pool.seq_len(slot)[2] == 0
    rng = np.random.default_rng(0)
    toks = [[(rng.standard_normal(HKV * D).astype(np.float32),
              rng.standard_normal(HKV * D).astype(np.float32))] for _ in range(2)]
    assert ref.forward_kv(pool, slot, 0, toks) == (0, "")
    assert pool.seq_len(slot)[2] == 2
    code, msg = ref.forward_kv(pool, slot, 0, toks[:1])
    assert code == ref.MODEL
    assert msg == "model: position0 0 does not match sequence length 2"
    assert pool.seq_len(slot)[2] == 2
    assert pool.free(slot)[0] == 0


def test_success_commits_one_position_per_token_with_its_rows():
    pool = ref.DensePool(L, HKV, D, 8, 1)
    slot = pool.alloc()[2]
    rng = np.random.default_rng(1)
    a, b = rows(rng, 3), rows(rng, 2)
    assert ref.forward_kv(pool, slot, 0, a) == (0, "")
    assert ref.forward_kv(pool, slot, 3, b) == (0, "")
    n, ks, vs = state(pool, slot)
    assert n == 5
    for p, tok in enumerate(a + b):
        for layer, (k, v) in enumerate(tok):
            assert np.array_equal(ks[p][layer], k) and np.array_equal(vs[p][layer], v)


FAILS = [(t, layer, where) for t, layer, where in
         itertools.product(range(3), range(L), ["before", "after"])] + [(t, 0, "embed")
                                                                         for t in range(3)]


@pytest.mark.parametrize("fail", FAILS)
def test_a_failed_call_rewinds_to_the_entry_state(fail):
    pool = ref.DensePool(L, HKV, D, 8, 1)
    slot = pool.alloc()[2]
    rng = np.random.default_rng(2)
    assert ref.forward_kv(pool, slot, 0, rows(rng, 2)) == (0, "")
    before = state(pool, slot)
    code, msg = ref.forward_kv(pool, slot, 2, rows(rng, 3), fail=fail)
    assert (code, msg) == (ref.MODEL, "model: injected failure")
    after = state(pool, slot)
    assert after[0] == before[0] == 2
    for x, y in zip(before[1] + before[2], after[1] + after[2]):
        for p, q in zip(x, y):
            assert np.array_equal(p, q)
    # no partial layers remain: layer 1 is out of order, layer 0 is accepted
    k, v = rows(rng, 1)[0][0]
    assert pool.append_layer(slot, 1, k, v)[:2] == (1, "cache: layers must append in order")
    assert pool.append_layer(slot, 0, k, v)[0] == 0
    assert pool.k(slot, 0, 2)[:2] == (1, "cache: position not yet committed")


def test_capacity_error_of_the_pool_rewinds_and_is_returned():
    pool = ref.DensePool(L, HKV, D, 4, 1)
    slot = pool.alloc()[2]
    rng = np.random.default_rng(3)
    assert ref.forward_kv(pool, slot, 0, rows(rng, 2)) == (0, "")
    # positions 2, 3 fit; position 4 fails at layer 0 of the third token
    assert ref.forward_kv(pool, slot, 2, rows(rng, 3)) == (1, "cache: sequence length exceeds max")
    assert pool.seq_len(slot)[2] == 2
    assert ref.forward_kv(pool, slot, 2, rows(rng, 2)) == (0, "")
    assert pool.seq_len(slot)[2] == 4


def test_unknown_slot_is_the_pools_error():
    pool = ref.DensePool(L, HKV, D, 4, 1)
    assert ref.forward_kv(pool, 5, 0, rows(np.random.default_rng(4), 1)) == \
        (1, "cache: unknown slot")
