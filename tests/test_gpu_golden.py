"""GPU: the HIP path against the committed golden fixtures (tests/golden/*.npz),
called through the C ABI. Append/gather are bit-exact; attention is within the
north-star tolerance |got - want| <= 2e-3 + 1e-2 * |want| of the f64 values."""
import os
import sys

import numpy as np
import pytest

from tests.helpers import assert_close, to_dev

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)
from make_golden import C1, c1_inputs, q8_inputs  # noqa: E402


def test_c1_tinyllama_prefill_and_decode_steps():
    import torch

    import ferrum_amd as fa
    g = np.load(os.path.join(GOLDEN, "c1_tinyllama_layer.npz"))
    k, v, q, table, slots = c1_inputs()
    hkv, hq, d, bs = C1["n_kv_heads"], C1["n_heads"], C1["head_dim"], C1["block_size"]
    layer = 21
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=22, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=C1["num_blocks"], block_size=bs,
                                         kv_dtype=fa.DTYPE_F16))
    pool.fill(0)
    pre = C1["prefill"]
    pool.append(layer, to_dev(k[:pre]), to_dev(v[:pre]), to_dev(slots[:pre]))
    tab = to_dev(table[None, :].astype(np.int32))
    for s in range(C1["decode_steps"]):
        t = pre + s
        pool.append(layer, to_dev(k[t:t + 1]), to_dev(v[t:t + 1]), to_dev(slots[t:t + 1]))
        out = torch.full((1, hq, d), 7.0, dtype=torch.float32, device="cuda")
        ctx = torch.tensor([t + 1], dtype=torch.int32, device="cuda")
        pool.decode_attention(layer, to_dev(q[s:s + 1]), out, tab, ctx, t + 1,
                              scale=float(g["scale"]))
        assert_close(out.cpu().numpy()[0], g["attn"][s], what=f"decode step {s}")
    n = slots.size
    rk = torch.zeros((n, hkv * d), dtype=torch.int16, device="cuda")
    rv = torch.zeros_like(rk)
    pool.gather_slots(layer, to_dev(slots), rk, rv, fa.GATHER_RAW)
    assert np.array_equal(rk.cpu().numpy().view(np.uint16).reshape(g["k_f16"].shape), g["k_f16"])
    assert np.array_equal(rv.cpu().numpy().view(np.uint16).reshape(g["v_f16"].shape), g["v_f16"])
    fk = torch.zeros((n, hkv, d), dtype=torch.float32, device="cuda")
    fv = torch.zeros_like(fk)
    pool.gather_slots(layer, to_dev(slots), fk, fv, fa.GATHER_F32)
    want = g["k_f16"].view(np.float16).astype(np.float32)
    assert np.array_equal(fk.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert pool.take_fault_flags() == 0


@pytest.mark.parametrize("rounding,key", [(0, "blocks_rne"), (1, "blocks_away")])
def test_q8_append_matches_golden_blocks(rounding, key):
    import torch

    import ferrum_amd as fa
    g = np.load(os.path.join(GOLDEN, "q8_blocks.npz"))
    d = 64
    rows = q8_inputs().reshape(-1, 1, d)
    n = rows.shape[0]
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=1, n_kv_heads=1, head_dim=d,
                                         num_blocks=(n + 15) // 16, kv_dtype=fa.DTYPE_Q8_0,
                                         f16_rounding=rounding))
    slots = np.arange(n, dtype=np.int64)
    pool.append(0, to_dev(rows), to_dev(rows[::-1].copy()), to_dev(slots))
    rk = torch.zeros((n, d // 32 * 34), dtype=torch.uint8, device="cuda")
    rv = torch.zeros_like(rk)
    pool.gather_slots(0, to_dev(slots), rk, rv, fa.GATHER_RAW)
    blocks = g[key].reshape(n, -1)
    assert np.array_equal(rk.cpu().numpy(), blocks)
    assert np.array_equal(rv.cpu().numpy(), blocks[::-1])
