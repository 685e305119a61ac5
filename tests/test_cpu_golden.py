"""CPU: the oracle against the committed golden fixtures (tests/golden/*.npz).

The fixtures were written by tests/golden/make_golden.py from numpy arithmetic
alone (numpy float16 for roundTiesToEven, an f64 brute-force softmax(qK^T)V for
attention, a numpy statement of q8_dot.rs:46-59 for Q8_0), so matching them
pins the oracle to values it did not produce.
"""
import os
import sys

import numpy as np
import pytest

from oracle import ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)
from make_golden import C1, c1_inputs, q8_inputs  # noqa: E402
from portable_rng import digest  # noqa: E402


@pytest.fixture(scope="module")
def c1():
    return np.load(os.path.join(GOLDEN, "c1_tinyllama_layer.npz"))


def test_portable_inputs_are_the_recorded_ones(c1):
    k, v, q, table, slots = c1_inputs()
    assert digest(k, v, q) == str(c1["inputs_sha256"])
    assert np.array_equal(table, c1["table"]) and np.array_equal(slots, c1["slots"])
    assert sorted(table.tolist()) == list(range(C1["num_blocks"]))


def test_oracle_c1_append_and_attention_match_golden(c1):
    k, v, q, table, slots = c1_inputs()
    hkv, hq, d, bs = C1["n_kv_heads"], C1["n_heads"], C1["head_dim"], C1["block_size"]
    n_layers, layer = 22, 21  # TinyLlama has 22 layers; the fixture is the last one
    lay = ref.Layout(n_layers, hkv, d, bs, C1["num_blocks"], 1, 0)
    pool = ref.new_pool(lay)
    pre = C1["prefill"]
    assert ref.append(lay, pool, layer, k[:pre], v[:pre], slots[:pre]) == 0
    tab = table[None, :].astype(np.int32)
    scale = float(c1["scale"])
    for s in range(C1["decode_steps"]):
        t = pre + s
        ref.append(lay, pool, layer, k[t:t + 1], v[t:t + 1], slots[t:t + 1])
        out = ref.attention(lay, pool, layer, q[s:s + 1], tab, np.array([t + 1], np.int32), scale)
        assert np.allclose(out[0], c1["attn"][s], rtol=1e-5, atol=1e-6), s
    gk, gv = ref.gather_slots(lay, pool, layer, slots, 1)
    assert np.array_equal(gk.view(np.uint16).reshape(c1["k_f16"].shape), c1["k_f16"])
    assert np.array_equal(gv.view(np.uint16).reshape(c1["v_f16"].shape), c1["v_f16"])
    # no other layer was written
    ok, _ = ref.gather_slots(lay, pool, 0, slots, 1)
    assert not ok.any()


def test_oracle_q8_matches_golden_blocks():
    g = np.load(os.path.join(GOLDEN, "q8_blocks.npz"))
    x = q8_inputs()
    assert digest(x) == str(g["inputs_sha256"])
    assert np.array_equal(ref.q8_quantize_row(x.ravel(), 0).reshape(-1, 34), g["blocks_rne"])
    assert np.array_equal(ref.q8_quantize_row(x.ravel(), 1).reshape(-1, 34), g["blocks_away"])
    # through the paged layout: append then raw gather gives the same 34-byte blocks
    d = 64
    rows = x.reshape(-1, d)  # 2 blocks of 32 per row
    lay = ref.Layout(1, 1, d, 16, (rows.shape[0] + 15) // 16, 8, 0)
    pool = ref.new_pool(lay)
    slots = np.arange(rows.shape[0], dtype=np.int64)
    ref.append(lay, pool, 0, rows[:, None, :], rows[:, None, :], slots)
    gk, gv = ref.gather_slots(lay, pool, 0, slots, 1)
    assert np.array_equal(gk.reshape(-1, 34), g["blocks_rne"])
    assert np.array_equal(gv.reshape(-1, 34), g["blocks_rne"])
