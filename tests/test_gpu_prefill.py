"""GPU parity: chunked-prefill attention (F16 and Q8_0 KV, matrix cores) against the CPU
oracle's token-by-token restatement of crates/model/src/llama.rs:363-378.

Bar: |got - want| <= 2e-3 + 1e-2 * |want| elementwise on finite values, the same Inf
and NaN positions and values elsewhere; q_len = 1 agrees with decode attention;
output rows outside the chunk are never written. Also:
- an Inf or NaN V inside a chunk reaches exactly the queries whose causal range holds
  it (the reference's token loop never reads a later position), through the
  leak-safe instance that workgroups over a block marked as holding such a value run,
  which also meets the bar on finite data; an infinite K (stored by the bulk append or
  the fused decode step) marks its block the same way, and its +-Inf scores come out as
  the reference's dot gives them;
- a sequence whose q_len exceeds the call's max_q_len (the grid holds no more) is
  clamped to it and raises FKV_FAULT_CTX_RANGE; a table entry outside the pool raises
  FKV_FAULT_BLOCK_RANGE and its block is skipped, other sequences unaffected;
- Q8_0 pools, with ordinary values and with values up to +-1e6 (the exact instance);
- key ranges cut into pieces (the workspace path, down to one-block pieces through
  fkv_set_tuning's prefill piece knob) and read whole (no workspace): both meet the bar, every
  instance.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _pool(d, hkv, ctxs, seed, layers=1, dtype=1, kv=None):
    rng = np.random.default_rng(seed)
    nb = [(c + 15) // 16 for c in ctxs]
    nblk = sum(nb) + 4
    pool, layout = make_pools(layers, hkv, d, nblk, dtype=dtype)
    pool.fill(0)
    perm = rng.permutation(nblk).astype(np.int32)
    tab = np.zeros((len(ctxs), max(nb)), np.int32)
    off = 0
    for i, n in enumerate(nb):
        tab[i, :n] = perm[off:off + n]
        off += n
    if kv is None:
        k = rng.standard_normal((sum(ctxs), hkv, d), dtype=np.float32)
        v = rng.standard_normal((sum(ctxs), hkv, d), dtype=np.float32)
    else:
        k, v = kv(rng, sum(ctxs))
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
    for layer in range(layers):
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
    return pool, layout, tab


def _prefill(pool, layer, q, tab, ctxs, qls, offs, fill=5.0, max_q_len=None, split=True,
             max_ctx_len=None):
    import torch
    out = torch.full(q.shape, fill, dtype=torch.float32, device="cuda")
    pool.prefill_attention(layer, to_dev(q), out, to_dev(tab), to_dev(np.array(ctxs, np.int32)),
                           to_dev(np.array(qls, np.int32)), to_dev(offs),
                           max(qls) if max_q_len is None else max_q_len,
                           max(ctxs) if max_ctx_len is None else max_ctx_len, split=split)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _want(pool, layout, q, tab, ctxs, qls, offs, d):
    import ferrum_amd as fa
    from oracle import ref
    return ref.prefill_attention(layout, pool.read(), 0, q, tab, np.array(ctxs, np.int32),
                                 np.array(qls, np.int32), offs, fa.default_scale(d))


def _used(rows, offs, qls):
    used = np.zeros(rows, bool)
    for o, n in zip(offs, qls):
        used[o:o + n] = True
    return used


def assert_close_nonfinite(got, want, what="prefill"):
    """The attention bar on finite values; Inf and NaN where, and as, the oracle has them."""
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN positions differ"
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf]), f"{what}: infinities differ"
    assert_close(got[fin], want[fin], what=what)


SHAPES = [(1, 128, 4), (1, 64, 8), (1, 128, 1), (1, 64, 16), (1, 128, 3), (1, 128, 8),
          (8, 128, 4), (8, 64, 8), (8, 128, 1)]


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("dtype,d,g", SHAPES)
def test_prefill_matches_oracle(dtype, d, g, split):
    hkv = 2
    ctxs = [1, 17, 64, 300, 777, 1100]
    qls = [1, 17, 5, 300, 129, 40]  # fresh chunks and chunks after history
    pool, layout, tab = _pool(d, hkv, ctxs, seed=d + g, dtype=dtype)
    if split:  # max_ctx 1,100 = 69 blocks: pieces of 34-35 blocks
        assert pool.prefill_workspace_bytes(hkv * g, len(ctxs), max(qls), max(ctxs)) > 0
    rows = sum(qls) + 3
    offs = np.concatenate([[2], 2 + np.cumsum(qls)[:-1]]).astype(np.int64)
    q = np.random.default_rng(g).standard_normal((rows, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs, split=split)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    used = _used(rows, offs, qls)
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


@pytest.mark.parametrize("pieces", [1, 3, 7])
@pytest.mark.parametrize("dtype,g", [(1, 4), (8, 4), (1, 16), (1, 1)])
def test_prefill_small_pieces(dtype, g, pieces, tune):
    """Key ranges cut into pieces of `pieces` blocks (at most 32 a workgroup, so longer
    ranges get longer pieces): odd and one-block pieces, pieces past a wave's own
    causal end, ranges shorter than one piece; against the oracle."""
    tune(prefill_split_blocks=pieces)
    hkv, d = 2, 128
    ctxs = [3, 16, 33, 190, 520, 1029]
    qls = [3, 9, 33, 61, 200, 17]
    pool, layout, tab = _pool(d, hkv, ctxs, seed=71 + g, dtype=dtype)
    assert pool.prefill_workspace_bytes(hkv * g, len(ctxs), max(qls), max(ctxs)) > 0
    offs = np.concatenate([[0], np.cumsum(qls)[:-1]]).astype(np.int64)
    q = np.random.default_rng(8).standard_normal((sum(qls), hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert_close(got, want, what=f"prefill, {pieces}-block pieces")


def test_prefill_workspace_too_small_is_rejected():
    import torch

    import ferrum_amd as fa
    hkv, g, d = 2, 4, 128
    ctxs, qls = [3000], [100]  # 188 blocks over a 14-workgroup grid: split
    pool, _, tab = _pool(d, hkv, ctxs, seed=81)
    need = pool.prefill_workspace_bytes(hkv * g, 1, 100, 3000)
    assert need > 0
    q = torch.zeros((100, hkv * g, d), dtype=torch.float32, device="cuda")
    ws = torch.empty(need - 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(fa.InvalidRequest, match="prefill workspace too small"):
        pool.prefill_attention(0, q, q.clone(), to_dev(tab), to_dev(np.array(ctxs, np.int32)),
                               to_dev(np.array(qls, np.int32)), to_dev(np.zeros(1, np.int64)),
                               100, 3000, workspace=ws)


@pytest.mark.parametrize("dtype", [1, 8])
def test_prefill_c3_chunk_shape(dtype):
    """BASELINE configs[2]'s prefill part at full size: 4 sequences appending 512-token
    chunks behind 0 / 700 / 1500 / 3000 tokens of history, Llama-3-8B heads; every row
    of every chunk against the oracle."""
    hkv, g, d = 8, 4, 128
    hist = [0, 700, 1500, 3000]
    ctxs = [h + 512 for h in hist]
    qls = [512] * 4
    pool, layout, tab = _pool(d, hkv, ctxs, seed=21, dtype=dtype)
    offs = (np.arange(4) * 512).astype(np.int64)
    q = np.random.default_rng(2).standard_normal((2048, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    whole = _prefill(pool, 0, q, tab, ctxs, qls, offs, split=False)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert_close(got, want, what="c3 prefill")
    assert_close(whole, want, what="c3 prefill, whole key ranges")


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("pieces", [0, 1, 2])
@pytest.mark.parametrize("g", [4, 1, 16])
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_nonfinite_v_reaches_only_later_queries(bad, g, pieces, d, tune):
    """V of position p0 + 9 of a fresh 40-token chunk (and of position 3 of a chunk after
    100 tokens of history) holds an Inf/NaN in a few dims: queries before it must be
    finite, the ones at or after it what the oracle gives; with whole key ranges (0)
    and with pieces of 1 and 2 blocks; head_dim 128 and 64 (the staged V tiles' chunks
    fall differently over the two staging slots)."""
    tune(prefill_split_blocks=pieces)
    hkv = 2
    ctxs, qls = [40, 140], [40, 40]
    marks = [(0, 9), (1, 100 + 3)]

    def kv(rng, n):
        k = rng.standard_normal((n, hkv, d), dtype=np.float32)
        v = rng.standard_normal((n, hkv, d), dtype=np.float32)
        base = [0, ctxs[0]]
        for s, pos in marks:
            v[base[s] + pos, 1, [3, d // 2 + 6, d - 1]] = bad
        return k, v
    pool, layout, tab = _pool(d, hkv, ctxs, seed=31, kv=kv)
    offs = np.array([0, 40], np.int64)
    q = np.random.default_rng(4).standard_normal((80, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert np.all(np.isfinite(want[:9])) and np.all(np.isfinite(want[40:43]))
    assert not np.all(np.isfinite(want[9:40]))
    assert_close_nonfinite(got, want)


@pytest.mark.parametrize("append", ["bulk", "fused"])
@pytest.mark.parametrize("bad", [np.inf, -np.inf])
def test_infinite_k_marks_the_pool_and_matches_the_oracle(bad, append):
    """K (V finite) holds +-Inf at dims 5 and 77 of some positions the chunks read. q is
    1.0 on dim 77, exact in f16, so q's lo part there is 0: the f16 hi + lo split gives
    inf * 0 = NaN in the lo chain where the reference's dot gives +-Inf. Only workgroups
    over a block marked as holding a non-finite K run the instance that repairs it, and
    the store must mark the block: by the bulk append (positions inside and before the
    chunks) and by the fused decode step (the last position of sequence 1)."""
    import torch
    hkv, g, d = 2, 4, 128
    ctxs, qls = [60, 160], [40, 40]
    marks = [(0, 30), (1, 100 + 15), (1, 20)] if append == "bulk" else []
    base = [0, ctxs[0]]

    def kv(rng, n):
        k = rng.standard_normal((n, hkv, d), dtype=np.float32)
        v = rng.standard_normal((n, hkv, d), dtype=np.float32)
        for s, pos in marks:
            k[base[s] + pos, 1, [5, 77]] = bad
        return k, v
    pool_ctxs = ctxs if append == "bulk" else [60, 159]
    pool, layout, tab = _pool(d, hkv, pool_ctxs, seed=33, kv=kv)
    if append == "fused":  # sequence 1's position 159 through the fused step
        kn = np.random.default_rng(3).standard_normal((1, hkv, d)).astype(np.float32)
        kn[0, 1, [5, 77]] = bad
        vn = np.ones((1, hkv, d), np.float32)
        qd = np.ones((1, hkv * g, d), np.float32)
        out = torch.zeros(qd.shape, dtype=torch.float32, device="cuda")
        pool.append_decode_attention(0, to_dev(kn), to_dev(vn), to_dev(qd), out,
                                     to_dev(tab[1:2]), to_dev(np.array([160], np.int32)), 160)
        torch.cuda.synchronize()
    offs = np.array([0, 40], np.int64)
    q = np.random.default_rng(9).standard_normal((80, hkv * g, d), dtype=np.float32)
    q[:, :, 77] = 1.0
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert not np.all(np.isfinite(want))
    assert_close_nonfinite(got, want)


def test_leak_safe_instance_on_finite_data():
    """Every block the chunks read holds a NaN V in layer 1 (marking it), so every
    workgroup of a layer-0 prefill runs the leak-safe instance: on layer 0's finite
    values it meets the same bar."""
    hkv, g, d = 8, 4, 128
    ctxs, qls = [600, 1300], [600, 256]
    pool, layout, tab = _pool(d, hkv, ctxs, seed=41, layers=2)
    import torch
    used = np.concatenate([tab[i, :(c + 15) // 16] for i, c in enumerate(ctxs)])
    bad = np.full((len(used), hkv, d), np.nan, np.float32)
    pool.append(1, to_dev(bad), to_dev(bad), to_dev(used.astype(np.int64) * 16))
    torch.cuda.synchronize()
    assert pool.marked_blocks() == len(used)
    offs = np.array([0, 600], np.int64)
    q = np.random.default_rng(5).standard_normal((856, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert_close(got, want, what="leak-safe prefill")


@pytest.mark.parametrize("pieces", [0, 3])
def test_q_len_past_max_q_len_is_clamped_and_flagged(pieces, tune):
    """Sequence 1 says 300 queries but the call's max_q_len is 200: its first 200 rows are
    computed, the rest untouched, FKV_FAULT_CTX_RANGE raised; sequence 0 is unaffected
    (whole key ranges, and 3-block pieces merged under the same clamp)."""
    import ferrum_amd as fa
    tune(prefill_split_blocks=pieces)
    hkv, g, d = 2, 4, 128
    ctxs, qls = [150, 500], [150, 300]
    pool, layout, tab = _pool(d, hkv, ctxs, seed=51)
    offs = np.array([0, 150], np.int64)
    q = np.random.default_rng(6).standard_normal((450, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs, max_q_len=200)
    assert pool.take_fault_flags() == fa.FAULT_CTX_RANGE
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert_close(got[:350], want[:350], what="clamped prefill")
    assert np.all(got[350:] == 5.0)


@pytest.mark.parametrize("dtype", [1, 8])
@pytest.mark.parametrize("pieces", [0, 3])
def test_table_entry_outside_the_pool_is_flagged_and_skipped(dtype, pieces, tune):
    """Two of sequence 1's table entries point outside the pool (-1 and past the last
    block): FKV_FAULT_BLOCK_RANGE is raised, those blocks are skipped (no read outside the
    pool; the rows stay finite), sequence 0 still matches the oracle, and rows outside the
    chunks are untouched. F16 and Q8_0, whole key ranges and 3-block pieces."""
    import ferrum_amd as fa
    tune(prefill_split_blocks=pieces)
    hkv, g, d = 2, 4, 128
    ctxs, qls = [100, 70], [20, 30]
    pool, layout, tab = _pool(d, hkv, ctxs, seed=61, dtype=dtype)
    bad = tab.copy()
    bad[1, 1] = -1
    bad[1, 3] = int(tab.max()) + 40  # the pool holds sum(blocks) + 4
    rows = sum(qls) + 2
    offs = np.array([1, 1 + qls[0]], np.int64)
    q = np.random.default_rng(7).standard_normal((rows, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, bad, ctxs, qls, offs)
    assert pool.take_fault_flags() & fa.FAULT_BLOCK_RANGE
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    s0 = slice(1, 1 + qls[0])
    assert_close(got[s0], want[s0], what="prefill beside a bad table entry")
    s1 = slice(1 + qls[0], 1 + qls[0] + qls[1])
    assert np.all(np.isfinite(got[s1]))
    assert np.all(got[0] == 5.0) and np.all(got[rows - 1] == 5.0)


@pytest.mark.parametrize("d,g", [(128, 4), (64, 8), (128, 1), (64, 16)])
def test_q8_staged_prefill_is_bit_identical_to_in_kernel_dequant(d, g, tune):
    """With a workspace, a Q8_0 call dequantises its blocks once into binary16 staging
    tiles (the F16 pool layout) and runs the F16 fast instance over them; without one,
    every workgroup dequantises what it stages into LDS. Both form f16(scale x quant)
    with one rounding and run the same score/P.V code, so with whole key ranges (no
    pieces on either side) the outputs agree bit for bit, including a sequence whose
    history holds a block marked for a wide scale (computed by the exact instance in
    both) and contexts that end mid-block; and both meet the oracle's bar."""
    tune(prefill_split_blocks=0)
    hkv = 2
    ctxs, qls = [300, 17, 1000, 520], [300, 17, 100, 33]

    def kv(rng, n):
        k = rng.standard_normal((n, hkv, d), dtype=np.float32)
        v = rng.standard_normal((n, hkv, d), dtype=np.float32)
        k[317 + 5, 1, 3] = 3e5  # sequence 2's block 0 (its rows start at 300 + 17)
        return k, v
    pool, layout, tab = _pool(d, hkv, ctxs, seed=71, dtype=8, kv=kv)
    assert pool.marked_blocks() == 1
    offs = np.array([0, 300, 317, 417], np.int64)
    q = np.random.default_rng(8).standard_normal((450, hkv * g, d), dtype=np.float32)
    staged = _prefill(pool, 0, q, tab, ctxs, qls, offs, split=True)
    assert pool.take_fault_flags() == 0
    direct = _prefill(pool, 0, q, tab, ctxs, qls, offs, split=False)
    assert pool.take_fault_flags() == 0
    assert np.array_equal(staged.view(np.uint32), direct.view(np.uint32))
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    rows = _used(450, offs, qls)
    assert_close(staged[rows], want[rows], what="staged q8 prefill")
    assert np.all(staged[~rows] == 5.0)


@pytest.mark.parametrize("dtype,split", [(1, True), (1, False), (8, True), (8, False)])
def test_context_past_max_ctx_len_is_clamped_and_flagged(dtype, split, tune):
    """A context longer than the call's max_ctx_len (300 here: 19 blocks, 304 tokens) is
    clamped to 304 tokens with FKV_FAULT_CTX_RANGE, by every kernel of the call alike
    (the staged Q8_0 path holds no more): the sequence's queries end at position 303, as
    the oracle gives them for a 304-token context; the other sequence is unaffected.
    F16 and Q8_0, with a workspace (key-range pieces of 4 blocks; Q8_0 staged) and
    without."""
    import ferrum_amd as fa
    tune(prefill_split_blocks=4)
    hkv, g, d = 2, 4, 128
    ctxs, qls = [120, 400], [40, 50]
    pool, layout, tab = _pool(d, hkv, ctxs, seed=81, dtype=dtype)
    offs = np.array([0, 40], np.int64)
    q = np.random.default_rng(9).standard_normal((90, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs, split=split, max_ctx_len=300)
    assert pool.take_fault_flags() == fa.FAULT_CTX_RANGE
    want = _want(pool, layout, q, tab, [120, 304], qls, offs, d)
    assert_close(got, want, what="prefill past max_ctx_len")


def _term_sums(layout, image, q, tab, ctxs, qls, offs, scale):
    """sum_p |w_p * V[p][d]| per output value, in f64 from the pool's decoded K/V (the
    reference's f32 dequantisation, scalar.rs:268-275) and f64 softmax weights: the size
    of the terms an output is the sum of, which bounds what rounding the terms can do."""
    from oracle import ref
    ctx = np.array(ctxs, np.int32)
    kk, vv, koffs = ref.gather_tables(layout, image, 0, tab, ctx, 0)
    hq, d = q.shape[1], q.shape[2]
    g = hq // layout.n_kv_heads
    out = np.zeros(q.shape, np.float64)
    for s, (c, ql, o) in enumerate(zip(ctxs, qls, offs)):
        ks = kk[koffs[s]:koffs[s] + c].astype(np.float64)
        vs = np.abs(vv[koffs[s]:koffs[s] + c].astype(np.float64))
        for h in range(hq):
            qq = q[o:o + ql, h].astype(np.float64)            # [ql, d]
            sc = qq @ ks[:, h // g].T * scale                  # [ql, c]
            pos = c - ql + np.arange(ql)
            sc[np.arange(c)[None, :] > pos[:, None]] = -np.inf
            w = np.exp(sc - sc.max(1, keepdims=True))
            w /= w.sum(1, keepdims=True)
            out[o:o + ql, h] = w @ vs[:, h // g]
    return out


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("pieces", [0, 5])
def test_q8_prefill_with_wide_values(pieces, d, tune):
    """Q8_0 K and V with +-1e6 values of both signs (scales ~7,874): the blocks are
    marked and the exact instance computes, with whole key ranges and with 5-block
    pieces; q is small enough that the scores stay O(1); head_dim 128 and 64.

    The exact instance forms each weight x V scale in f32 and carries it as bf16 hi + lo
    (16 significant bits) against the int8 V, so every term of an output is exact to
    2^-16 of itself. With 64 dims a dim of V holds ~11 outliers in the longer context,
    and outliers of both signs cancel some outputs to ~1e-6 of their terms, below any
    bar relative to the output alone. The bar is the elementwise one plus 2^-16 of the
    sum of the terms' magnitudes (sum_p |w_p V_p|, computed in f64 from the decoded
    K/V), the rounding the terms are allowed."""
    tune(prefill_split_blocks=pieces)
    import ferrum_amd as fa
    hkv, g = 2, 4
    ctxs, qls = [300, 700], [300, 200]

    def kv(rng, n):
        k = rng.standard_normal((n, hkv, d), dtype=np.float32)
        v = rng.standard_normal((n, hkv, d), dtype=np.float32)
        for x in (k, v):
            idx = rng.integers(0, d, size=(n, hkv))
            big = rng.choice([-1e6, 1e6], size=(n, hkv, 1))
            np.put_along_axis(x, idx[..., None], big, -1)
        return k, v
    pool, layout, tab = _pool(d, hkv, ctxs, seed=61, dtype=8, kv=kv)
    offs = np.array([0, 300], np.int64)
    q = np.random.default_rng(7).standard_normal((500, hkv * g, d), dtype=np.float32) * 2e-6
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert np.abs(want).max() > 1e3
    terms = _term_sums(layout, pool.read(), q, tab, ctxs, qls, offs, fa.default_scale(d))
    err = np.abs(got.astype(np.float64) - want)
    lim = 2e-3 + 1e-2 * np.abs(want) + 2.0 ** -16 * terms
    assert np.all(err <= lim), (f"q8 wide prefill: {(err > lim).sum()} values out of tolerance, "
                                f"max err/lim {np.max(err / lim):.3f}")
    # the outliers cancel in some outputs: the elementwise bar alone would not hold there
    cancel = np.abs(want) < 1e-3 * terms
    assert cancel.any()


def test_prefill_rejects_f32_pools():
    import torch

    import ferrum_amd as fa
    pool, _ = make_pools(1, 2, 64, 4, dtype=0)
    q = torch.zeros((1, 8, 64), dtype=torch.float32, device="cuda")
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(fa.KernelError, match="prefill attention needs f16 or q8_0 kv"):
        pool.prefill_attention(0, q, q.clone(), torch.zeros((1, 1), dtype=torch.int32,
                                                            device="cuda"),
                               z + 1, z + 1, torch.zeros(1, dtype=torch.int64, device="cuda"), 1,
                               1)


@pytest.mark.parametrize("case", range(24))
def test_prefill_randomized_shapes_against_oracle(case, tune):
    """Seeded random cases: F16 or Q8_0, head_dim, group size, sequences with random
    histories and chunk lengths (q_len <= context, block and tile edges among them, rows
    in a shuffled order with gaps between them), whole key ranges or pieces of 1 to 40
    blocks; against the oracle at the attention bar, rows outside every chunk untouched."""
    rng = np.random.default_rng(2000 + case)
    dtype = [1, 8][case % 2]
    d = [64, 128][(case // 2) % 2]
    g = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    hkv = int(rng.choice([1, 2]))
    n = int(rng.integers(1, 6))
    edges = [1, 4, 15, 16, 17, 31, 32, 33, 64, 65]
    ctxs, qls = [], []
    for _ in range(n):
        ql = int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(1, 200))
        hist = int(rng.choice([0, 1, 16, 17])) if rng.random() < 0.4 else int(rng.integers(0, 900))
        ctxs.append(hist + ql)
        qls.append(ql)
    pieces = int(rng.choice([-1, 0, 1, 3, 40]))
    tune(prefill_split_blocks=pieces)
    pool, layout, tab = _pool(d, hkv, ctxs, seed=case, dtype=dtype)
    order = rng.permutation(n)
    gaps = rng.integers(0, 3, n)
    offs = np.zeros(n, np.int64)
    row = int(rng.integers(0, 3))
    for i in order:  # chunks placed in a shuffled order with gaps
        offs[i] = row
        row += qls[i] + int(gaps[i])
    rows = row + 1
    q = (rng.standard_normal((rows, hkv * g, d)) * rng.choice([0.3, 1.0, 3.0])).astype(np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    used = _used(rows, offs, qls)
    assert_close(got[used], want[used], what=f"case {case}: dtype {dtype} d {d} g {g} hkv {hkv} "
                 f"pieces {pieces} ctxs {ctxs} qls {qls}")
    assert np.all(got[~used] == 5.0)
