"""GPU parity: paged decode attention against the CPU oracle (llama.rs:220-247).

Bar: |got - want| <= 2e-3 + 1e-2 * |want| elementwise,
against the oracle's restatement of the reference loop and against an f64 brute
force; bit-identical outputs when only the physical block placement changes;
the non-finite-max rule of scalar.rs:125-130.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, attention_f64, make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu

CTXS = [1, 15, 16, 17, 255, 256, 257, 700, 1500]


def _build(dtype, d, hkv, ctxs, seed=0, perm_seed=None, layers=2, extra_blocks=8):
    """Pool with every sequence's K/V appended through a scattered block table."""
    rng = np.random.default_rng(seed)
    nb = [(c + 15) // 16 for c in ctxs]
    nblk = sum(nb) + extra_blocks
    pool, layout = make_pools(layers, hkv, d, nblk, dtype=dtype)
    pool.fill(0)
    prng = np.random.default_rng(seed if perm_seed is None else perm_seed)
    perm = prng.permutation(nblk).astype(np.int32)
    max_blocks = max(1, max(nb))
    tab = np.zeros((len(ctxs), max_blocks), np.int32)
    off = 0
    for i, n in enumerate(nb):
        tab[i, :n] = perm[off: off + n]
        off += n
    total = sum(ctxs)
    for layer in range(layers):
        k = rng.standard_normal((total, hkv, d), dtype=np.float32)
        v = rng.standard_normal((total, hkv, d), dtype=np.float32)
        slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
    return pool, layout, tab


def _run(pool, layer, q, tab, ctxs):
    import torch
    out = torch.full(q.shape, 123.0, dtype=torch.float32, device="cuda")
    ctx = np.array(ctxs, np.int32)
    pool.decode_attention(layer, to_dev(q), out, to_dev(tab), to_dev(ctx), int(ctx.max()))
    torch.cuda.synchronize()
    return out.cpu().numpy()


SHAPES = [(1, 128, 4), (1, 128, 8), (1, 64, 8), (1, 128, 1), (1, 64, 2), (1, 128, 16),
          (1, 128, 3), (1, 64, 5), (1, 64, 16), (1, 128, 12),
          (0, 128, 4), (0, 64, 8), (8, 128, 4), (8, 128, 8), (8, 64, 1), (8, 128, 16),
          (8, 64, 3), (8, 128, 1)]


@pytest.fixture(params=["split", "stream", "valu"])
def f16_schedule(request, tune):
    """F16 runs on the MFMA split kernel by default; the stream knob of fkv_set_tuning
    selects the persistent schedule, the engine knob the VALU partition kernel (group
    sizes 1, 2, 4, 8, 16; others stay on the matrix cores). All meet the same bar."""
    if request.param == "stream":
        tune(attn_stream=1)
    elif request.param == "valu":
        tune(attn_stream=0, attn_engine=1)
    else:
        tune(attn_stream=0)
    return request.param


@pytest.mark.parametrize("dtype,d,g", SHAPES)
def test_attention_matches_oracle(dtype, d, g, f16_schedule):
    if dtype != 1 and f16_schedule != "split":
        pytest.skip("the schedule and engine switches only apply to F16 storage")
    import ferrum_amd as fa
    from oracle import ref
    hkv = 2
    pool, layout, tab = _build(dtype, d, hkv, CTXS, seed=d + g)
    rng = np.random.default_rng(7)
    q = rng.standard_normal((len(CTXS), hkv * g, d), dtype=np.float32)
    got = _run(pool, 1, q, tab, CTXS)
    assert pool.take_fault_flags() == 0
    image = pool.read()
    scale = fa.default_scale(d)
    want = ref.attention(layout, image, 1, q, tab, np.array(CTXS), scale)
    err = assert_close(got, want)
    # independent f64 brute force on decoded rows for a few (seq, head)
    for s in (0, 4, len(CTXS) - 1):
        c = CTXS[s]
        slots = slots_for(tab[s], c)
        kr, vr = ref.gather_slots(layout, image, 1, slots, 0)
        for h in (0, hkv * g - 1):
            exp = attention_f64(q[s, h], kr[:, h // g], vr[:, h // g], scale)
            assert_close(got[s, h], exp, what="f64 brute force")
    print(f"max abs err vs oracle {err:.2e}")


@pytest.mark.parametrize("dtype,d,g", [(1, 128, 4), (8, 128, 8), (1, 64, 16)])
def test_workgroups_per_cu_cap_changes_nothing_but_occupancy(dtype, d, g, tune):
    """FKV_TUNE_ATTN_WGS_PER_CU only enlarges each decode workgroup's LDS request: the
    outputs with a cap of 2 or 3 are the uncapped call's, bit for bit."""
    hkv = 2
    pool, layout, tab = _build(dtype, d, hkv, CTXS, seed=31 + d + g)
    q = np.random.default_rng(5).standard_normal((len(CTXS), hkv * g, d), dtype=np.float32)
    tune(attn_stream=0)
    want = _run(pool, 1, q, tab, CTXS)
    for cap in (2, 3):
        tune(attn_wgs_per_cu=cap)
        got = _run(pool, 1, q, tab, CTXS)
        assert pool.take_fault_flags() == 0
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), cap


def test_attention_long_context_uses_combine(f16_schedule):
    import ferrum_amd as fa
    from oracle import ref
    ctxs = [20000, 3, 4097]
    pool, layout, tab = _build(1, 128, 8, ctxs, seed=11, layers=1)
    q = np.random.default_rng(5).standard_normal((3, 32, 128), dtype=np.float32)
    got = _run(pool, 0, q, tab, ctxs)
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array(ctxs), fa.default_scale(128))
    assert_close(got, want)


ORDER_CTXS = [0, 1, 511, 512, 513, 1024, 1500, 3000, 17, 4100, 0, 2048, 700]


@pytest.mark.parametrize("dtype", [1, 8])
def test_work_orders_are_bit_identical(dtype, tune):
    """The split kernel's workgroups take the (sequence, KV head, split) items in
    grid order, full-first order or longest-first order (fkv_set_tuning order 0/1/2).
    An item is computed the same way whichever workgroup takes it, so the three
    outputs agree bit for bit; empty contexts, contexts of whole splits and a
    9-split context are in the batch."""
    import ferrum_amd as fa
    from oracle import ref
    hkv, g, d = 2, 4, 128
    pool, layout, tab = _build(dtype, d, hkv, ORDER_CTXS, seed=21, layers=1)
    q = np.random.default_rng(8).standard_normal((len(ORDER_CTXS), hkv * g, d), dtype=np.float32)
    outs = []
    for order in ("0", "1", "2"):
        tune(attn_order=order)
        outs.append(_run(pool, 0, q, tab, ORDER_CTXS))
    assert pool.take_fault_flags() == 0
    assert np.all(outs[0][0] == 0.0) and np.all(outs[0][10] == 0.0)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array(ORDER_CTXS), fa.default_scale(d))
    assert_close(outs[2], want)
    pool.close()


@pytest.mark.parametrize("order", ["0", "1", "2"])
def test_context_outside_the_table_is_flagged(order, tune):
    """A context length past the table row (or negative) raises FKV_FAULT_CTX_RANGE in
    every work order; the sequence is read up to the row's end (or not at all, with
    a zero output) and the other sequences are unaffected."""
    import ferrum_amd as fa
    from oracle import ref
    tune(attn_order=order)
    ctxs = [40, 1100, 600]
    pool, layout, tab = _build(1, 128, 2, ctxs, seed=6, layers=1)
    cap = tab.shape[1] * 16
    q = np.random.default_rng(2).standard_normal((3, 8, 128), dtype=np.float32)
    bad = [40, cap + 5, -3]
    import torch
    out = torch.full(q.shape, 123.0, dtype=torch.float32, device="cuda")
    # max_ctx_len is checked on the host; the device-side lengths are not
    pool.decode_attention(0, to_dev(q), out, to_dev(tab), to_dev(np.array(bad, np.int32)), cap)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert pool.take_fault_flags() & fa.FAULT_CTX_RANGE
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array([40, cap, 0]), fa.default_scale(128))
    assert_close(got, want)
    assert np.all(got[2] == 0.0)
    pool.close()


@pytest.mark.parametrize("dtype,order", [(1, "0"), (1, "1"), (1, "2"), (8, "2"), (0, "2")])
def test_context_past_max_ctx_len_is_flagged(dtype, order, tune):
    """A device context longer than the call's max_ctx_len (but inside the table row)
    is clamped to what the launch's splits hold (512 here for every path: 64-token
    splits on the matrix cores, 256-token partitions on F32) and raises
    FKV_FAULT_CTX_RANGE; the merge reads only the workspace slots the launch was sized
    for (the offending sequence is the last, whose slots end the workspace), and the
    other sequences are unaffected."""
    import ferrum_amd as fa
    from oracle import ref
    tune(attn_order=order)
    ctxs = [40, 300, 1100]
    pool, layout, tab = _build(dtype, 128, 2, ctxs, seed=11, layers=1)
    q = np.random.default_rng(3).standard_normal((3, 8, 128), dtype=np.float32)
    import torch
    out = torch.full(q.shape, 123.0, dtype=torch.float32, device="cuda")
    pool.decode_attention(0, to_dev(q), out, to_dev(tab), to_dev(np.array(ctxs, np.int32)), 512)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert pool.take_fault_flags() & fa.FAULT_CTX_RANGE
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array([40, 300, 512]),
                         fa.default_scale(128))
    assert_close(got, want)
    pool.close()


@pytest.mark.parametrize("n_seqs", [300, 1100])
def test_large_batches_match_oracle(n_seqs, tune):
    """300 sequences take the full-first order (three or fewer per thread of the
    ranking), 1,100 the grid order; both against the oracle and the grid order."""
    import ferrum_amd as fa
    from oracle import ref
    hkv, g, d = 1, 4, 64
    ctxs = [int(c) for c in np.random.default_rng(n_seqs).integers(0, 1100, n_seqs)]
    pool, layout, tab = _build(1, d, hkv, ctxs, seed=2, layers=1)
    q = np.random.default_rng(4).standard_normal((n_seqs, hkv * g, d), dtype=np.float32)
    tune(attn_order=-1)
    got = _run(pool, 0, q, tab, ctxs)
    tune(attn_order="0")
    grid = _run(pool, 0, q, tab, ctxs)
    assert pool.take_fault_flags() == 0
    assert np.array_equal(got.view(np.uint32), grid.view(np.uint32))
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array(ctxs), fa.default_scale(d))
    assert_close(got, want)
    pool.close()


def test_attention_is_invariant_to_block_placement():
    q = np.random.default_rng(9).standard_normal((len(CTXS), 8, 128), dtype=np.float32)
    outs = []
    for perm_seed in (1, 2):
        pool, _, tab = _build(1, 128, 2, CTXS, seed=3, perm_seed=perm_seed)
        outs.append(_run(pool, 1, q, tab, CTXS))
        pool.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_attention_zero_context_gives_zeros():
    pool, _, tab = _build(1, 64, 2, [5, 16], seed=4)
    q = np.ones((2, 4, 64), np.float32)
    import torch
    out = torch.full(q.shape, 9.0, dtype=torch.float32, device="cuda")
    ctx = np.array([0, 16], np.int32)
    pool.decode_attention(0, to_dev(q), out, to_dev(tab), to_dev(ctx), 16)
    o = out.cpu().numpy()
    assert np.all(o[0] == 0.0)
    assert np.all(np.isfinite(o[1])) and np.any(o[1] != 0.0)


@pytest.mark.parametrize("dtype,engine", [(0, 0), (1, 0), (1, 1)])
@pytest.mark.parametrize("ctx", [40, 600])
def test_attention_non_finite_scores(ctx, dtype, engine, tune):
    """One K row is (+inf, 0, ..., 0). Head 0 (q0 > 0) scores it +inf: a non-finite
    max gives zeros (scalar.rs:127-130). Head 1 (q0 < 0) scores it -inf: the token
    only drops out. Head 2 (q0 == 0) scores it 0*inf = NaN with a finite max: the
    output is NaN. A second pool where every score of a head is -inf gives zeros.
    engine 1: F16 on the VALU partition kernel."""
    import ferrum_amd as fa
    from oracle import ref
    tune(attn_engine=engine)
    d, hkv, g = 64, 1, 4
    nb = (ctx + 15) // 16
    pool, layout = make_pools(1, hkv, d, nb + 2, dtype=dtype)
    pool.fill(0)
    rng = np.random.default_rng(0)
    k = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    v = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    k[ctx // 3, 0, :] = 0.0
    k[ctx // 3, 0, 0] = np.inf
    tab = np.arange(nb, dtype=np.int32)[None, :]
    slots = slots_for(tab[0], ctx)
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    q = rng.standard_normal((1, g, d), dtype=np.float32)
    q[0, 0, 0], q[0, 1, 0], q[0, 2, 0], q[0, 3, 0] = 1.0, -1.0, 0.0, 2.0
    got = _run(pool, 0, q, tab, [ctx])
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array([ctx]), fa.default_scale(d))
    assert np.all(want[0, 0] == 0) and np.all(want[0, 3] == 0)
    assert np.all(np.isfinite(want[0, 1])) and np.all(np.isnan(want[0, 2]))
    assert_close(got, want)

    # every score -inf
    k2 = np.zeros((ctx, hkv, d), np.float32)
    k2[:, 0, 0] = np.inf
    pool.append(0, to_dev(k2), to_dev(v), to_dev(slots))
    q2 = rng.standard_normal((1, g, d), dtype=np.float32)
    q2[0, :, 0] = -1.0
    got2 = _run(pool, 0, q2, tab, [ctx])
    assert np.all(got2 == 0.0)


@pytest.mark.parametrize("dtype,engine", [(0, 0), (1, 0), (1, 1)])
@pytest.mark.parametrize("bad", [np.inf, -np.inf])
def test_attention_infinite_k_with_any_q(bad, dtype, engine, tune):
    """One K row holds +-Inf at two dims; 16 query heads see it with random q there. On
    the matrix cores q is split into f16 hi + lo parts after a scaling, so the lo part
    at those dims is zero or of either sign: the score must still be the reference's
    dot (+-Inf, or NaN where the two infinities meet with opposite signs), giving zeros,
    a dropped token or NaN as the oracle does. engine 1: F16 on the VALU partition kernel."""
    import ferrum_amd as fa
    from oracle import ref
    tune(attn_engine=engine)
    d, hkv, g, ctx = 128, 1, 16, 300
    nb = (ctx + 15) // 16
    pool, layout = make_pools(1, hkv, d, nb + 2, dtype=dtype)
    pool.fill(0)
    rng = np.random.default_rng(12)
    k = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    v = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    k[ctx // 2, 0, [7, 90]] = bad
    tab = np.arange(nb, dtype=np.int32)[None, :]
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots_for(tab[0], ctx)))
    q = rng.standard_normal((1, g, d), dtype=np.float32)
    q[0, :8, 7] = rng.uniform(0.3, 3.0, 8)        # same sign at both dims
    q[0, :8, 90] = rng.uniform(0.3, 3.0, 8)
    q[0, 8:12, 7] = rng.uniform(0.3, 3.0, 4)      # opposite signs: NaN
    q[0, 8:12, 90] = -rng.uniform(0.3, 3.0, 4)
    got = _run(pool, 0, q, tab, [ctx])
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array([ctx]), fa.default_scale(d))
    assert np.isnan(want[0, 8:12]).all()
    assert_close(got, want)


@pytest.mark.parametrize("dtype", [1, 8, 0])
def test_fused_step_past_max_ctx_len_stores_no_token(dtype):
    """The fused step under the same rule on every storage type: sequence 2's context
    (1,100) is past what max_ctx_len = 512 sized, so FKV_FAULT_CTX_RANGE is raised, its
    token is not stored and it attends over 512 positions; sequences 0 and 1 store their
    tokens and attend normally. Pool bytes against the oracle's append of the two
    tokens only, outputs at the attention bar."""
    import torch

    import ferrum_amd as fa
    from oracle import ref
    ctxs = [40, 300, 1100]
    pool, layout, tab = _build(dtype, 128, 2, ctxs, seed=12, layers=1)
    before = pool.read()
    rng = np.random.default_rng(7)
    q = rng.standard_normal((3, 8, 128), dtype=np.float32)
    knew = rng.standard_normal((3, 2, 128), dtype=np.float32)
    vnew = rng.standard_normal((3, 2, 128), dtype=np.float32)
    out = torch.full(q.shape, 123.0, dtype=torch.float32, device="cuda")
    pool.append_decode_attention(0, to_dev(knew), to_dev(vnew), to_dev(q), out, to_dev(tab),
                                 to_dev(np.array(ctxs, np.int32)), 512)
    torch.cuda.synchronize()
    assert pool.take_fault_flags() & fa.FAULT_CTX_RANGE
    tail = np.array([slots_for(tab[i], c)[-1] for i, c in enumerate(ctxs[:2])], np.int64)
    want_image = before.copy()
    ref.append(layout, want_image, 0, knew[:2], vnew[:2], tail)
    assert np.array_equal(pool.read(), want_image)
    want = ref.attention(layout, want_image, 0, q, tab, np.array([40, 300, 512]),
                         fa.default_scale(128))
    assert_close(out.cpu().numpy(), want)
    pool.close()


EDGE_CTXS = [0, 1, 15, 16, 17, 31, 255, 256, 257, 1023, 1024, 1025]


@pytest.mark.parametrize("case", range(40))
def test_attention_randomized_shapes_against_oracle(case, tune):
    """Seeded random cases: storage type, head_dim, group size, batch size, contexts drawn
    from split and block edges (0, 1, 15-17, 31, 255-257, 1023-1025) and random lengths,
    and the split length (the planner's, or 16, 256 or 1,024 tokens forced), each against
    the oracle at the attention bar."""
    import ferrum_amd as fa
    from oracle import ref
    rng = np.random.default_rng(1000 + case)
    dtype = [1, 8, 0][case % 3]
    d = [64, 128][(case // 3) % 2]
    groups = [1, 2, 4, 8, 16] if dtype == 0 else [1, 2, 3, 4, 5, 8, 12, 16]
    g = int(rng.choice(groups))
    hkv = int(rng.choice([1, 2, 4]))
    n = int(rng.integers(1, 10))
    ctxs = [int(rng.choice(EDGE_CTXS)) if rng.random() < 0.6 else int(rng.integers(1, 2100))
            for _ in range(n)]
    split = [0, 16, 256, 1024][int(rng.integers(0, 4))]
    tune(attn_split_tokens=split, attn_stream=0)
    pool, layout, tab = _build(dtype, d, hkv, ctxs, seed=case, layers=1)
    q = (rng.standard_normal((n, hkv * g, d)) * rng.choice([0.1, 1.0, 4.0])).astype(np.float32)
    got = _run(pool, 0, q, tab, ctxs)
    assert pool.take_fault_flags() == 0
    want = ref.attention(layout, pool.read(), 0, q, tab, np.array(ctxs), fa.default_scale(d))
    assert_close(got, want, what=f"case {case}: dtype {dtype} d {d} g {g} hkv {hkv} split {split} ctxs {ctxs}")
