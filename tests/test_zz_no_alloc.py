"""GPU: fkv_append_decode_attention_noalloc, the decode step that allocates nothing.

It is fkv_append_decode_attention with the split partials in the library's static
per-GPU scratch instead of a caller's workspace. Called through the C ABI, its
output and the pool bytes it leaves must be bit-identical to the workspace entry
point's on the same inputs (and so within the attention bar of the oracle), on two
calls in a row, the second with fewer sequences and shorter contexts. A call whose
scratch need exceeds the static array is rejected before anything is launched.
"""
import ctypes

import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _setup(pool, rng, hkv, d, ctxs, layers, table_base):
    """Blocks for positions 0 .. ctx - 2 of every sequence, appended in every layer."""
    nb = [max(1, (c + 15) // 16) for c in ctxs]
    tab = np.zeros((len(ctxs), max(nb)), np.int32)
    off = table_base
    for i, n in enumerate(nb):
        tab[i, :n] = np.arange(off, off + n)
        off += n
    prefix = [max(0, c - 1) for c in ctxs]
    total = sum(prefix)
    for layer in range(layers):
        if total:
            k = rng.standard_normal((total, hkv, d), dtype=np.float32)
            v = rng.standard_normal((total, hkv, d), dtype=np.float32)
            slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(prefix)])
            pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
    return tab, off


def _noalloc(pool, layer, n_heads, knew, vnew, q, out, tab, ctx, max_ctx):
    import torch
    import ferrum_amd as fa
    return pool._lib.fkv_append_decode_attention_noalloc(
        pool.handle, layer, n_heads, knew.data_ptr(), vnew.data_ptr(), q.data_ptr(),
        out.data_ptr(), tab.data_ptr(), tab.shape[1], ctx.data_ptr(), ctx.numel(), max_ctx,
        fa.default_scale(q.shape[2]), torch.cuda.current_stream().cuda_stream)


CASES = [  # (kv dtype, head_dim, kv heads, group)
    (1, 128, 8, 4),
    (8, 128, 8, 4),
    (0, 128, 2, 4),
    (1, 64, 4, 8),
]


@pytest.mark.parametrize("dtype,d,hkv,g", CASES)
def test_noalloc_step_matches_workspace_step_twice(dtype, d, hkv, g):
    import torch
    import ferrum_amd as fa
    from oracle import ref
    layers, layer = 2, 1
    calls = [[1, 16, 17, 300, 513, 2100, 4096, 3000], [5, 700, 1200]]
    nblk = sum(max(1, (c + 15) // 16) for cs in calls for c in cs) + 4
    pool, layout = make_pools(layers, hkv, d, nblk, dtype=dtype)
    # the tables of both calls hold distinct blocks, all inside the pool
    pool.fill(0)
    rng = np.random.default_rng(d * 31 + g + dtype)
    base = 0
    for call, ctxs in enumerate(calls):
        print(f"noalloc case dtype={dtype} d={d} hkv={hkv} g={g} call={call} ctxs={ctxs}",
              flush=True)
        tab, base = _setup(pool, rng, hkv, d, ctxs, layers, base)
        assert base <= nblk
        n = len(ctxs)
        knew = to_dev(rng.standard_normal((n, hkv, d), dtype=np.float32))
        vnew = to_dev(rng.standard_normal((n, hkv, d), dtype=np.float32))
        q = to_dev(rng.standard_normal((n, hkv * g, d), dtype=np.float32))
        ctx = np.array(ctxs, np.int32)
        tab_d, ctx_d = to_dev(tab), to_dev(ctx)
        need = ctypes.c_uint64()
        assert pool._lib.fkv_append_decode_attention_workspace_size(
            pool.handle, hkv * g, n, int(ctx.max()), ctypes.byref(need)) == 0
        assert 0 < need.value <= fa.STATIC_SCRATCH_BYTES  # the scratch really is used

        before = pool.read()
        out_na = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
        st = _noalloc(pool, layer, hkv * g, knew, vnew, q, out_na, tab_d, ctx_d, int(ctx.max()))
        assert st == 0, pool._lib.fkv_last_error().decode()
        torch.cuda.synchronize()
        assert pool.take_fault_flags() == 0
        image_na = pool.read()

        pool.write(before)
        out_ws = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
        pool.append_decode_attention(layer, knew, vnew, q, out_ws, tab_d, ctx_d, int(ctx.max()))
        torch.cuda.synchronize()
        assert pool.take_fault_flags() == 0
        assert np.array_equal(pool.read(), image_na), "pool bytes differ from the workspace call"
        got = out_na.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), out_ws.cpu().numpy().view(np.uint32))

        want = ref.attention(layout, image_na, layer, q.cpu().numpy(), tab, ctx,
                             fa.default_scale(d))
        assert_close(got, want)


def test_noalloc_rejects_a_call_past_the_static_scratch():
    import torch
    import ferrum_amd as fa
    hkv, d, g, n, max_ctx = 8, 128, 4, 1024, 32768
    pool, _ = make_pools(1, hkv, d, 64)
    need = ctypes.c_uint64()
    assert pool._lib.fkv_append_decode_attention_workspace_size(
        pool.handle, hkv * g, n, max_ctx, ctypes.byref(need)) == 0
    assert need.value > fa.STATIC_SCRATCH_BYTES
    tab = torch.zeros((n, max_ctx // 16), dtype=torch.int32, device="cuda")
    ctx = torch.full((n,), 100, dtype=torch.int32, device="cuda")
    knew = torch.zeros((n, hkv, d), dtype=torch.float32, device="cuda")
    q = torch.zeros((n, hkv * g, d), dtype=torch.float32, device="cuda")
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    st = _noalloc(pool, 0, hkv * g, knew, knew, q, out, tab, ctx, max_ctx)
    assert st == fa._lib.FKV_ERR_INVALID
    assert pool._lib.fkv_last_error().decode() == (
        f"decode step needs {need.value} bytes of scratch; the static scratch holds "
        f"{fa.STATIC_SCRATCH_BYTES}")
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a rejected call launched work"
