"""GPU parity: chunked-prefill attention (f16 KV, matrix cores) against the CPU
oracle's token-by-token restatement of crates/model/src/llama.rs:363-378.

Bar: |got - want| <= 2e-3 + 1e-2 * |want| elementwise; q_len = 1 agrees with
decode attention; output rows outside the chunk are never written."""
import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _pool(d, hkv, ctxs, seed, layers=1):
    rng = np.random.default_rng(seed)
    nb = [(c + 15) // 16 for c in ctxs]
    nblk = sum(nb) + 4
    pool, layout = make_pools(layers, hkv, d, nblk, dtype=1)
    pool.fill(0)
    perm = rng.permutation(nblk).astype(np.int32)
    tab = np.zeros((len(ctxs), max(nb)), np.int32)
    off = 0
    for i, n in enumerate(nb):
        tab[i, :n] = perm[off:off + n]
        off += n
    k = rng.standard_normal((sum(ctxs), hkv, d), dtype=np.float32)
    v = rng.standard_normal((sum(ctxs), hkv, d), dtype=np.float32)
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
    for layer in range(layers):
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
    return pool, layout, tab


def _prefill(pool, layer, q, tab, ctxs, qls, offs, fill=5.0):
    import torch
    out = torch.full(q.shape, fill, dtype=torch.float32, device="cuda")
    pool.prefill_attention(layer, to_dev(q), out, to_dev(tab), to_dev(np.array(ctxs, np.int32)),
                           to_dev(np.array(qls, np.int32)), to_dev(offs), max(qls), max(ctxs))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("d,g", [(128, 4), (64, 8), (128, 1), (64, 16), (128, 3), (128, 8)])
def test_prefill_matches_oracle(d, g):
    import ferrum_amd as fa
    from oracle import ref
    hkv = 2
    ctxs = [1, 17, 64, 300, 777]
    qls = [1, 17, 5, 300, 129]  # fresh chunks and chunks after history
    pool, layout, tab = _pool(d, hkv, ctxs, seed=d + g)
    rows = sum(qls) + 3
    offs = np.concatenate([[2], 2 + np.cumsum(qls)[:-1]]).astype(np.int64)
    q = np.random.default_rng(g).standard_normal((rows, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = ref.prefill_attention(layout, pool.read(), 0, q, tab, np.array(ctxs, np.int32),
                                 np.array(qls, np.int32), offs, fa.default_scale(d))
    used = np.zeros(rows, bool)
    for o, n in zip(offs, qls):
        used[o:o + n] = True
    assert_close(got[used], want[used], what="prefill")
    assert np.all(got[~used] == 5.0)  # rows outside every chunk are untouched


def test_prefill_with_one_query_is_decode():
    hkv, g, d = 8, 4, 128
    ctxs = [5, 100, 1000, 4097]
    pool, _, tab = _pool(d, hkv, ctxs, seed=3)
    q = np.random.default_rng(1).standard_normal((len(ctxs), hkv * g, d), dtype=np.float32)
    offs = np.arange(len(ctxs), dtype=np.int64)
    got = _prefill(pool, 0, q, tab, ctxs, [1] * len(ctxs), offs)
    import torch
    dec = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    pool.decode_attention(0, to_dev(q), dec, to_dev(tab), to_dev(np.array(ctxs, np.int32)),
                          max(ctxs))
    # Different schedules round the f16 weights against different running maxima, so
    # the two paths agree to the north-star tolerance, not bit for bit.
    assert_close(got, dec.cpu().numpy(), what="prefill vs decode")


def test_prefill_c3_chunk_shape():
    """BASELINE configs[2]'s prefill part at full size: 4 sequences appending 512-token
    chunks behind 0 / 700 / 1500 / 3000 tokens of history, Llama-3-8B heads."""
    import ferrum_amd as fa
    from oracle import ref
    hkv, g, d = 8, 4, 128
    hist = [0, 700, 1500, 3000]
    ctxs = [h + 512 for h in hist]
    qls = [512] * 4
    pool, layout, tab = _pool(d, hkv, ctxs, seed=21)
    offs = (np.arange(4) * 512).astype(np.int64)
    q = np.random.default_rng(2).standard_normal((2048, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    # the scalar oracle checks the shortest and the longest history (rows 0..511, 1536..2047)
    pick = [0, 3]
    want = ref.prefill_attention(layout, pool.read(), 0, q, tab[pick],
                                 np.array(ctxs, np.int32)[pick], np.array(qls, np.int32)[pick],
                                 offs[pick], fa.default_scale(d))
    rows = np.r_[0:512, 1536:2048]
    assert_close(got[rows], want[rows], what="c3 prefill")


def test_prefill_rejects_non_f16_pools():
    import torch

    import ferrum_amd as fa
    pool, _ = make_pools(1, 2, 64, 4, dtype=0)
    q = torch.zeros((1, 8, 64), dtype=torch.float32, device="cuda")
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(fa.KernelError, match="prefill attention needs f16 kv"):
        pool.prefill_attention(0, q, q.clone(), torch.zeros((1, 1), dtype=torch.int32,
                                                            device="cuda"),
                               z + 1, z + 1, torch.zeros(1, dtype=torch.int64, device="cuda"), 1,
                               1)
