"""GPU: Llama::forward's KV sequence (crates/model/src/llama.rs:345-389) over the device pools.

The oracle's restatement (oracle.ref.forward_kv: position0 check, per token
abandon_partial -> append_layer per layer -> commit_token, rewind_forward on any
error) drives two things with the same script of calls, successes and failures
(injected at embed, before or after a layer's append, and the pools' own capacity
errors, tests.rs:176-192 among them):

1. the device compat pool (fkv_kvpool_*, through the C ABI) against the oracle's dense
   pool: every call's status and message, the committed length after it, and at the
   end every committed K/V row, bit for bit;
2. the paged revision as its caller runs it: per token fkv_seqs_reserve (copy-on-write
   pair copied), the fused step fkv_append_decode_attention per layer at ctx = length
   + 1, fkv_seqs_commit; rollback by fkv_seqs_truncate to the entry length. Against
   the dense oracle: the committed length after every call and the committed rows (as
   the storage encodes them); against the paged oracle: every step's attention output
   (the attention bar) and the whole pool image at the end, bit for bit.
"""
import ctypes

import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, to_dev

pytestmark = pytest.mark.gpu

L, HKV, D, G = 3, 2, 64, 4


class DeviceCompat:
    """The device KvPool (fkv_kvpool_*) in the oracle DensePool's protocol: every
    method returns (status, FerrumError Display string, value)."""

    def __init__(self, pool):
        self.lib, self.h = pool._lib, pool._h

    def _r(self, code, value=None):
        return code, ("" if code == 0 else self.lib.fkv_last_error().decode()), value

    def seq_len(self, slot):
        n = ctypes.c_uint64()
        c = self.lib.fkv_kvpool_seq_len(self.h, slot, ctypes.byref(n))
        return self._r(c, n.value)

    def abandon_partial(self, slot):
        return self._r(self.lib.fkv_kvpool_abandon_partial(self.h, slot))

    def uncommit_token(self, slot):
        return self._r(self.lib.fkv_kvpool_uncommit_token(self.h, slot))

    def commit_token(self, slot):
        return self._r(self.lib.fkv_kvpool_commit_token(self.h, slot))

    def append_layer(self, slot, layer, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        return self._r(self.lib.fkv_kvpool_append_layer(self.h, slot, layer, k.ctypes.data,
                                                        k.size, v.ctypes.data, v.size))

    def _read(self, fn, slot, layer, pos):
        out = np.zeros(HKV * D, np.float32)
        return self._r(fn(self.h, slot, layer, pos, out.ctypes.data, out.size), out)

    def k(self, slot, layer, pos):
        return self._read(self.lib.fkv_kvpool_k, slot, layer, pos)

    def v(self, slot, layer, pos):
        return self._read(self.lib.fkv_kvpool_v, slot, layer, pos)


def token_rows(rng, n):
    return [[(rng.standard_normal(HKV * D).astype(np.float32),
              rng.standard_normal(HKV * D).astype(np.float32)) for _ in range(L)]
            for _ in range(n)]


# (slot, position0, tokens, fail); max_seq_len is 24
COMPAT_SCRIPT = [
    (0, 0, 5, None),
    (1, 0, 3, None),
    (0, 5, 3, (1, 2, "after")),
    (0, 4, 2, None),              # position0 mismatch
    (1, 3, 4, (0, 0, "embed")),
    (0, 5, 10, None),
    (1, 3, 2, (1, 0, "before")),
    (0, 15, 12, None),            # position 24 fails "sequence length exceeds max"
    (0, 15, 9, None),
    (0, 24, 1, None),             # full: fails at its first append
    (1, 3, 6, None),
]


def test_compat_pool_follows_the_forward_sequence():
    import ferrum_amd as fa
    from oracle import ref
    rng = np.random.default_rng(17)
    want = ref.DensePool(L, HKV, D, 24, 2)
    dev = fa.PreallocatedKvPool.new(fa.KvPoolConfig(L, HKV, D, 24, 2))
    got = DeviceCompat(dev)
    assert want.alloc()[2] == 0 and want.alloc()[2] == 1
    assert dev.alloc() == 0 and dev.alloc() == 1
    for i, (slot, p0, n, fail) in enumerate(COMPAT_SCRIPT):
        print(f"compat forward call {i}: slot={slot} position0={p0} tokens={n} fail={fail}",
              flush=True)
        toks = token_rows(rng, n)
        r_want = ref.forward_kv(want, slot, p0, toks, fail)
        r_got = ref.forward_kv(got, slot, p0, toks, fail)
        assert r_got == r_want, f"call {i}"
        assert got.seq_len(slot) == want.seq_len(slot), f"call {i}"
    assert [want.seq_len(s)[2] for s in (0, 1)] == [24, 9]
    for slot in (0, 1):
        n = want.seq_len(slot)[2]
        for layer in range(L):
            for p in range(n):
                for which in ("k", "v"):
                    c1, m1, a = getattr(want, which)(slot, layer, p)
                    c2, m2, b = getattr(got, which)(slot, layer, p)
                    assert (c1, m1) == (c2, m2) == (0, "")
                    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
            assert got.k(slot, layer, n)[:2] == want.k(slot, layer, n)[:2] == \
                (1, "cache: position not yet committed")
    dev.close()


# (position0, tokens, fail); the paged pool holds 2 blocks (32 tokens) per sequence
PAGED_SCRIPT = [
    (0, 5, None),
    (5, 3, (1, 2, "after")),
    (5, 2, (1, 0, "embed")),
    (3, 1, None),                 # position0 mismatch
    (5, 10, None),
    (15, 20, None),               # position 32 has no block: Unavailable, rewound
    (15, 4, (2, 1, "before")),
    (15, 17, None),
]


def _paged_forward(ref, m, pool, layout, image, seq, p0, toks, qs, fail, max_blocks, outs):
    """Llama::forward over the paged revision (llama.rs:345-389), as its caller runs it:
    fkv_seqs_reserve / fused step per layer / fkv_seqs_commit per token, truncate back
    to the entry length on an error. Mirrors every device write into the oracle image
    and checks each step's attention against the oracle on it."""
    import torch
    import ferrum_amd as fa
    seq_len = m.length(seq)[0]
    if p0 != seq_len:
        return ref.MODEL, f"model: position0 {p0} does not match sequence length {seq_len}"
    for idx, layers in enumerate(toks):
        err = None
        if fail is not None and fail[0] == idx and fail[2] == "embed":
            err = (ref.MODEL, "model: injected failure")
        else:
            try:
                pair = m.reserve(seq, 1)
            except fa.FerrumError as e:
                err = ({fa.Unavailable: 2, fa.CacheError: 1}.get(type(e), 5), str(e))
            if err is None:
                if pair is not None:
                    pool.copy_blocks(to_dev(np.array([pair], np.int64)))
                    ref.copy_blocks(layout, image, np.array([pair], np.int64))
                tab, ctx = m.tables([seq], max_blocks)
                pos = int(ctx[0])
                slot = m.slots(seq, pos, 1)
                step_ctx = np.array([pos + 1], np.int32)
                for layer, (k, v) in enumerate(layers):
                    if fail == (idx, layer, "before"):
                        err = (ref.MODEL, "model: injected failure")
                        break
                    kk, vv = k.reshape(1, HKV, D), v.reshape(1, HKV, D)
                    q = qs[idx][layer]
                    out = torch.zeros((1, HKV * G, D), dtype=torch.float32, device="cuda")
                    pool.append_decode_attention(layer, to_dev(kk), to_dev(vv), to_dev(q), out,
                                                 to_dev(tab), to_dev(step_ctx), pos + 1)
                    ref.append(layout, image, layer, kk, vv, slot)
                    outs.append((out, ref.attention(layout, image, layer, q, tab, step_ctx,
                                                    fa.default_scale(D))))
                    if fail == (idx, layer, "after"):
                        err = (ref.MODEL, "model: injected failure")
                        break
                if err is None:
                    m.commit(seq, 1)
        if err is not None:
            m.truncate(seq, seq_len)
            return err
    return 0, ""


@pytest.mark.parametrize("dtype", [0, 1, 8])
def test_paged_step_follows_the_forward_sequence(dtype):
    import torch
    import ferrum_amd as fa
    from oracle import ref
    rng = np.random.default_rng(23 + dtype)
    max_blocks = 2
    pool, layout = make_pools(L, HKV, D, max_blocks, dtype=dtype)
    pool.fill(0)
    image = ref.new_pool(layout)
    m = fa.SequenceManager(pool)
    seq = m.add(0)
    dense = ref.DensePool(L, HKV, D, 4096, 1)
    dslot = dense.alloc()[2]
    outs = []
    for i, (p0, n, fail) in enumerate(PAGED_SCRIPT):
        print(f"paged forward call {i} dtype={dtype}: position0={p0} tokens={n} fail={fail}",
              flush=True)
        toks = token_rows(rng, n)
        qs = [[rng.standard_normal((1, HKV * G, D), dtype=np.float32) for _ in range(L)]
              for _ in range(n)]
        got = _paged_forward(ref, m, pool, layout, image, seq, p0, toks, qs, fail, max_blocks,
                             outs)
        # the dense oracle sees a missing block as a failure before the token's first layer
        pfail = fail
        if i == 5:
            assert got == (2, "no free kv blocks")
            pfail = (32 - p0, 0, "before")
        want = ref.forward_kv(dense, dslot, p0, toks, pfail)
        if i != 5:
            assert got == want, f"call {i}"
        assert m.length(seq)[0] == dense.seq_len(dslot)[2], f"call {i}"
        assert pool.take_fault_flags() == 0
    torch.cuda.synchronize()
    for out, want in outs:
        assert_close(out.cpu().numpy(), want)
    assert np.array_equal(pool.read(), image), "pool image differs from the oracle's"

    # committed rows as the storage encodes the dense oracle's rows
    n = m.length(seq)[0]
    assert n == 32
    slots = m.slots(seq, 0, n)
    for layer in range(L):
        ok = torch.zeros((n, HKV, D), dtype=torch.float32, device="cuda")
        ov = torch.zeros_like(ok)
        pool.gather_slots(layer, to_dev(slots), ok, ov)
        torch.cuda.synchronize()
        for which, got_rows in (("k", ok), ("v", ov)):
            rows = np.stack([getattr(dense, which)(dslot, layer, p)[2] for p in range(n)])
            if dtype == 1:
                rows = ref.f16_to_f32(ref.f32_to_f16(rows))
            elif dtype == 8:
                rows = ref.q8_dequant(ref.q8_quantize_row(rows.ravel()), rows.size)
            assert np.array_equal(got_rows.cpu().numpy().reshape(n, -1).view(np.uint32),
                                  rows.reshape(n, -1).view(np.uint32)), (which, layer)
    m.close()
    pool.close()
