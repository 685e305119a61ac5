"""GPU parity: the RoPE decode step fkv_rope_append_decode_attention.

One call must equal the reference's per-layer sequence Kernels::rope of q and k at
the token's position (crates/model/src/llama.rs:207-216; scalar.rs:77-82,167-189),
KvPool::append_layer of the rotated k (pool.rs:122-153), then the attention loop of
llama.rs:220-247. Checked against the oracle (fo_rope, pinned in
test_cpu_oracle_rope.py):
- V and K bytes bit-exact: K is rotated with the pool's (sin, cos) table, built on
  the host with the C library's sinf/cosf as the oracle's fo_rope (and the reference's
  f32::sin_cos) compute them, then stored as F16, F32 or Q8_0;
- the output meets the attention bar against the oracle's attention over the GPU's
  own pool with the oracle-rotated q;
- position 0 (a one-token context) and rope_dim = 0 are bit-identical to the
  unrotated fused step; the reference's error strings and check order.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, slots_for, to_dev
from tests.test_gpu_append_attention import _setup

pytestmark = pytest.mark.gpu

CTXS = [1, 16, 17, 300, 513, 2100]
THETA = {64: 10000.0, 128: 500000.0}


def _run_rope(pool, layer, knew, vnew, q, tab, ctxs, rope_dim, theta):
    import torch
    ctx = np.array(ctxs, np.int32)
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    pool.rope_append_decode_attention(layer, to_dev(knew), to_dev(vnew), to_dev(q), out, to_dev(tab),
                                      to_dev(ctx), int(ctx.max()), rope_dim, theta)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check_k(dtype, got, want, k_rot):
    """got/want: decoded K rows of the appended tokens [n, hkv, d], bit for bit (the
    storage's own decode of the oracle-rotated rows; k_rot, the rotated f32 rows, names
    the values in the failure message)."""
    bad = got.view(np.uint32) != want.view(np.uint32)
    assert not bad.any(), (f"stored K differs from the oracle's rotation in {int(bad.sum())} "
                           f"values (dtype {dtype}), e.g. {got[bad][:3]} vs {want[bad][:3]} "
                           f"from {k_rot[bad][:3]}")


SHAPES = [(1, 128, 8, 4, 128), (1, 128, 2, 4, 64), (1, 64, 4, 8, 64), (1, 64, 2, 16, 32),
          (8, 128, 2, 4, 128), (8, 64, 2, 8, 64), (0, 64, 2, 2, 64), (0, 128, 2, 4, 96)]


@pytest.mark.parametrize("dtype,d,hkv,g,rope_dim", SHAPES)
def test_rope_step_matches_oracle(dtype, d, hkv, g, rope_dim):
    import ferrum_amd as fa
    from oracle import ref
    layer = 1
    pool, layout, tab, knew, vnew = _setup(dtype, d, hkv, CTXS, seed=d + g + rope_dim)
    before = pool.read()
    q = np.random.default_rng(4).standard_normal((len(CTXS), hkv * g, d), dtype=np.float32)
    got = _run_rope(pool, layer, knew, vnew, q, tab, CTXS, rope_dim, THETA[d])
    assert pool.take_fault_flags() == 0
    image = pool.read()

    qr, kr = ref.rope_step(q, knew, CTXS, rope_dim, THETA[d])
    tail = np.array([slots_for(tab[i], c)[-1] for i, c in enumerate(CTXS)], np.int64)
    want_image = before.copy()
    ref.append(layout, want_image, layer, kr, vnew, tail)
    kg, vg = ref.gather_slots(layout, image, layer, tail, 0)
    kw, vw = ref.gather_slots(layout, want_image, layer, tail, 0)
    assert np.array_equal(vg.view(np.uint32), vw.view(np.uint32)), "stored V is not bit-exact"
    _check_k(dtype, kg, kw, kr)
    # every byte outside the appended tokens' blocks is the oracle's
    changed = np.nonzero(image != want_image)[0]
    tail_blocks = set(int(tab[i, (c - 1) // 16]) for i, c in enumerate(CTXS))
    assert all(int(b) // pool.block_bytes in tail_blocks for b in changed)

    want = ref.attention(layout, image, layer, qr, tab, np.array(CTXS), fa.default_scale(d))
    assert_close(got, want)
    pool.close()


@pytest.mark.parametrize("dtype", [1, 8])
def test_position_zero_and_rope_dim_zero_are_the_plain_step(dtype):
    """A one-token context rotates at position 0 (sin 0 = 0, cos 0 = 1) and rope_dim 0
    rotates nothing: both give the unrotated fused step's pool and output bit for bit."""
    import torch
    d, hkv, g = 128, 2, 4
    for ctxs, rope_dim in (([1, 1, 1], 128), ([5, 40, 300], 0)):
        pool, layout, tab, knew, vnew = _setup(dtype, d, hkv, ctxs, seed=31)
        before = pool.read()
        q = np.random.default_rng(6).standard_normal((len(ctxs), hkv * g, d), dtype=np.float32)
        got = _run_rope(pool, 0, knew, vnew, q, tab, ctxs, rope_dim, 10000.0)
        image = pool.read()
        pool.write(before)
        ctx = np.array(ctxs, np.int32)
        out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
        pool.append_decode_attention(0, to_dev(knew), to_dev(vnew), to_dev(q), out, to_dev(tab),
                                     to_dev(ctx), int(ctx.max()))
        torch.cuda.synchronize()
        assert np.array_equal(pool.read(), image)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), got.view(np.uint32))
        pool.close()


def test_long_context_position():
    """Position 70,000: the pool's table grown past the first 4,096 positions (its rows
    for large angles are the C library's own reduction), against the oracle."""
    import ferrum_amd as fa
    from oracle import ref
    ctxs = [70001, 3]
    d, hkv, g = 128, 1, 4
    pool, layout, tab, knew, vnew = _setup(1, d, hkv, ctxs, seed=8, layers=1)
    q = np.random.default_rng(5).standard_normal((2, hkv * g, d), dtype=np.float32)
    got = _run_rope(pool, 0, knew, vnew, q, tab, ctxs, d, 500000.0)
    image = pool.read()
    qr, kr = ref.rope_step(q, knew, ctxs, d, 500000.0)
    tail = np.array([slots_for(tab[i], c)[-1] for i, c in enumerate(ctxs)], np.int64)
    kg, _ = ref.gather_slots(layout, image, 0, tail, 0)
    want_k = ref.f16_to_f32(ref.f32_to_f16(kr))
    _check_k(1, kg, want_k, kr)
    assert_close(got, ref.attention(layout, image, 0, qr, tab, np.array(ctxs), fa.default_scale(d)))
    pool.close()


def test_rope_errors_in_reference_order():
    """validate.rs:64-87: theta, then parity, then shape; FerrumError::Kernel strings."""
    import ferrum_amd as fa
    d, hkv, g = 64, 2, 4
    pool, layout, tab, knew, vnew = _setup(1, d, hkv, [5, 9], seed=2, layers=1)
    before = pool.read()
    q = np.zeros((2, hkv * g, d), np.float32)
    cases = [(64, 0.0, "kernel: theta must be positive"),
             (64, -1.0, "kernel: theta must be positive"),
             (64, float("nan"), "kernel: theta must be positive"),
             (3, float("nan"), "kernel: theta must be positive"),
             (63, 10000.0, "kernel: rope_dim must be even"),
             (65, 10000.0, "kernel: rope_dim must be even"),
             (66, 10000.0, "kernel: rope_dim exceeds head_dim")]
    for rope_dim, theta, msg in cases:
        with pytest.raises(fa.errors.KernelError) as e:
            _run_rope(pool, 0, knew, vnew, q, tab, [5, 9], rope_dim, theta)
        assert str(e.value) == msg
    assert np.array_equal(pool.read(), before), "a rejected call wrote to the pool"
    pool.close()


@pytest.mark.parametrize("case", range(30))
def test_rope_step_randomized_against_oracle(case, tune):
    """Seeded random cases of the fused step: storage (F16 in either rounding, Q8_0, F32),
    head_dim, group size, batch, contexts from 1 through block and split edges, rope_dim
    (even, 0 to head_dim), theta and the split length; stored V and K bit for bit and the
    output at the attention bar against the oracle."""
    import ferrum_amd as fa
    from oracle import ref
    rng = np.random.default_rng(3000 + case)
    dtype = [1, 8, 0][case % 3]
    rounding = int(rng.integers(0, 2)) if dtype == 1 else 0
    d = [64, 128][(case // 3) % 2]
    g = int(rng.choice([1, 2, 4, 8, 16] if dtype == 0 else [1, 2, 3, 4, 6, 8, 16]))
    hkv = int(rng.choice([1, 2, 4]))
    n = int(rng.integers(1, 8))
    edges = [1, 2, 15, 16, 17, 256, 257, 1024, 1025]
    ctxs = [int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(1, 3000))
            for _ in range(n)]
    rope_dim = int(rng.choice([0, 2, 32, d // 2, d - 2, d]))
    theta = float(rng.choice([10000.0, 500000.0, 1000000.0]))
    tune(attn_split_tokens=[0, 256, 1024][int(rng.integers(0, 3))], attn_stream=0)
    pool, layout, tab, knew, vnew = _setup(dtype, d, hkv, ctxs, rounding=rounding, seed=case,
                                           layers=1)
    before = pool.read()
    q = rng.standard_normal((n, hkv * g, d)).astype(np.float32)
    got = _run_rope(pool, 0, knew, vnew, q, tab, ctxs, rope_dim, theta)
    assert pool.take_fault_flags() == 0
    image = pool.read()
    qr, kr = ref.rope_step(q, knew, ctxs, rope_dim, theta)
    tail = np.array([slots_for(tab[i], c)[-1] for i, c in enumerate(ctxs)], np.int64)
    want_image = before.copy()
    ref.append(layout, want_image, 0, kr, vnew, tail)
    kg, vg = ref.gather_slots(layout, image, 0, tail, 0)
    kw, vw = ref.gather_slots(layout, want_image, 0, tail, 0)
    what = (f"case {case}: dtype {dtype} rounding {rounding} d {d} g {g} hkv {hkv} "
            f"rope_dim {rope_dim} theta {theta} ctxs {ctxs}")
    assert np.array_equal(vg.view(np.uint32), vw.view(np.uint32)), what
    _check_k(dtype, kg, kw, kr)
    want = ref.attention(layout, image, 0, qr, tab, np.array(ctxs), fa.default_scale(d))
    assert_close(got, want, what=what)
    pool.close()
