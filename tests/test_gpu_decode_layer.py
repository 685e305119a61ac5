"""GPU parity: the attention half of a decode layer, GPU-resident (DecodeAttentionLayer).

Against the oracle chain of Llama::forward_one_token (crates/model/src/llama.rs:185-255):
fo_q8_gemm for attn_q/attn_k/attn_v, fo_rope at the token's position, the append, the
attention loop, fo_q8_gemm for attn_output. Each stage is pinned on the GPU's own
intermediates:
- q, k, v (before RoPE) bit for bit against fo_q8_gemm of the normed rows;
- the appended V and K bytes bit for bit against the oracle's rotation (the pool's
  host-built sin/cos table, as in the RoPE step's own tests);
- the attention rows at the attention bar against the oracle's attention over the GPU's
  pool with the oracle-rotated q;
- attn_output bit for bit against fo_q8_gemm of the GPU's attention rows.
End to end, the GPU's attn_output against the oracle chain run alone: within 1% of the
output's largest magnitude (the attention differences, within their bar, move a few Q8_0
activation roundings of the last product; a wrong head, position or operand moves it by
O(1)).
"""
import numpy as np
import pytest

from oracle import ref
from tests.helpers import assert_close, slots_for, to_dev
from tests.test_gpu_append_attention import _setup
from tests.test_gpu_rope_attention import _check_k

pytestmark = pytest.mark.gpu


def _q8_weights(rng, rows, cols, sigma=0.05):
    """Q8_0 rows of N(0, sigma) weights (the oracle's encoder; blocks never span rows)."""
    w = (rng.standard_normal((rows, cols)) * sigma).astype(np.float32)
    return ref.q8_quantize_row(w)


SHAPES = [
    # dtype, n_embd, n_heads, n_kv_heads, head_dim, rope_dim, theta, ctxs
    (1, 256, 8, 2, 64, 64, 10000.0, [1, 17, 300]),
    (8, 256, 8, 2, 64, 64, 10000.0, [2, 40, 513]),
    (0, 256, 4, 4, 64, 32, 10000.0, [3, 100]),
    (1, 4096, 32, 8, 128, 128, 500000.0, [5, 777, 4096]),
    (8, 4096, 32, 8, 128, 128, 500000.0, [129, 2048]),
]


@pytest.mark.parametrize("dtype,n_embd,hq,hkv,d,rope_dim,theta,ctxs", SHAPES)
def test_decode_layer_matches_the_oracle_chain(dtype, n_embd, hq, hkv, d, rope_dim, theta, ctxs):
    import torch

    import ferrum_amd as fa
    rng = np.random.default_rng(n_embd + d + dtype)
    layer = 1
    pool, layout, tab, _, _ = _setup(dtype, d, hkv, ctxs, seed=n_embd + dtype)
    before = pool.read()
    wq = _q8_weights(rng, hq * d, n_embd)
    wk = _q8_weights(rng, hkv * d, n_embd)
    wv = _q8_weights(rng, hkv * d, n_embd)
    wo = _q8_weights(rng, n_embd, hq * d)
    x = rng.standard_normal((len(ctxs), n_embd), dtype=np.float32)
    ctx = np.array(ctxs, np.int32)
    lay = fa.DecodeAttentionLayer(pool, layer, to_dev(wq), to_dev(wk), to_dev(wv), to_dev(wo),
                                  hq, n_embd, rope_dim, theta, max_seqs=len(ctxs),
                                  max_ctx_len=int(ctx.max()))
    y = torch.full((len(ctxs), n_embd), 7.0, dtype=torch.float32, device="cuda")
    lay.forward(to_dev(x), to_dev(tab), to_dev(ctx), int(ctx.max()), y)
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == 0
    n = len(ctxs)
    q_g = lay.q[:n].cpu().numpy()
    k_g = lay.k[:n].cpu().numpy()
    v_g = lay.v[:n].cpu().numpy()
    attn_g = lay.attn[:n].cpu().numpy()
    y_g = y.cpu().numpy()
    image = pool.read()

    # projections: bit for bit
    q_o = ref.q8_gemm(wq, hq * d, n_embd, x).reshape(n, hq, d)
    k_o = ref.q8_gemm(wk, hkv * d, n_embd, x).reshape(n, hkv, d)
    v_o = ref.q8_gemm(wv, hkv * d, n_embd, x).reshape(n, hkv, d)
    for got, want in ((q_g, q_o), (k_g, k_o), (v_g, v_o)):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # RoPE + append: V and K exact
    qr, kr = ref.rope_step(q_o, k_o, ctx, rope_dim, theta)
    tail = np.array([slots_for(tab[i], c)[-1] for i, c in enumerate(ctxs)], np.int64)
    want_image = before.copy()
    ref.append(layout, want_image, layer, kr, v_o, tail)
    kg, vg = ref.gather_slots(layout, image, layer, tail, 0)
    kw, vw = ref.gather_slots(layout, want_image, layer, tail, 0)
    assert np.array_equal(vg.view(np.uint32), vw.view(np.uint32))
    _check_k(dtype, kg, kw, kr)
    # attention over the GPU's pool with the oracle-rotated q
    scale = fa.default_scale(d)
    assert_close(attn_g, ref.attention(layout, image, layer, qr, tab, ctx, scale))
    # attn_output of the GPU's attention rows: bit for bit
    y_o = ref.q8_gemm(wo, n_embd, hq * d, attn_g.reshape(n, hq * d))
    assert np.array_equal(y_g.view(np.uint32), y_o.view(np.uint32))
    # end to end against the oracle chain alone
    attn_o = ref.attention(layout, want_image, layer, qr, tab, ctx, scale)
    y_chain = ref.q8_gemm(wo, n_embd, hq * d, attn_o.reshape(n, hq * d))
    assert np.max(np.abs(y_g - y_chain)) <= 1e-2 * np.max(np.abs(y_chain))
    pool.close()


def test_decode_layer_rejects_a_batch_beyond_its_buffers():
    import torch

    import ferrum_amd as fa
    pool, _, tab, _, _ = _setup(1, 64, 2, [5, 6], seed=1)
    rng = np.random.default_rng(2)
    w = [to_dev(_q8_weights(rng, r, c)) for r, c in ((256, 128), (128, 128), (128, 128), (128, 256))]
    lay = fa.DecodeAttentionLayer(pool, 0, *w, 4, 128, 64, 10000.0, max_seqs=1, max_ctx_len=6)
    x = torch.zeros((2, 128), dtype=torch.float32, device="cuda")
    y = torch.zeros_like(x)
    with pytest.raises(ValueError, match="beyond what the layer was built for"):
        lay.forward(x, to_dev(tab), to_dev(np.array([5, 6], np.int32)), 6, y)
    pool.close()
