#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from numpy arithmetic alone.

Neither the CPU oracle nor the HIP library is used here, so the fixtures are an
independent statement of the expected values:

c1_tinyllama_layer.npz  BASELINE configs[0] (TinyLlama-1.1B KV shape), one layer:
    4 KV heads, 32 query heads, head_dim 64, block 16, 256-block pool whose block
    table is a seeded permutation; a 512-token prefill then 3 decode steps, each
    appending one token and attending over the whole context. Q/K/V are N(0,1)
    from the portable splitmix64 stream of seed 0. Expected values:
      k_f16, v_f16  binary16 bits of every appended K/V value, from numpy's
                    float32 -> float16 conversion (IEEE roundTiesToEven);
      attn          softmax(q . K^T * scale) . V per query head and decode step,
                    in float64 from the decoded binary16 K/V (the loop of
                    crates/model/src/llama.rs:220-247 with kv_h = h / 8).
q8_blocks.npz  Q8_0 blocks (32 values, f16 scale first: core-types/src/dtype.rs:19-21)
    of N(0,1) data with 1% +-20 outliers plus edge blocks, quantised by the rule of
    Q8Activation::quantize_into (crates/kernels/src/q8_dot.rs:46-59) written in
    numpy; scales both in roundTiesToEven (numpy) and in Ferrum's ties-away
    encoding (q8_dot.rs:111-139).

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from portable_rng import digest, normal_f32, permutation  # noqa: E402

C1 = dict(n_kv_heads=4, n_heads=32, head_dim=64, block_size=16, num_blocks=256,
          prefill=512, decode_steps=3, seed=0, table_seed=1)


def c1_inputs(cfg=C1):
    """Seeded inputs of the C1 fixture: k, v [T][Hkv][D], q [steps][Hq][D], table, slots."""
    hkv, hq, d = cfg["n_kv_heads"], cfg["n_heads"], cfg["head_dim"]
    t = cfg["prefill"] + cfg["decode_steps"]
    z = normal_f32(cfg["seed"], 2 * t * hkv * d + cfg["decode_steps"] * hq * d)
    k = z[: t * hkv * d].reshape(t, hkv, d)
    v = z[t * hkv * d: 2 * t * hkv * d].reshape(t, hkv, d)
    q = z[2 * t * hkv * d:].reshape(cfg["decode_steps"], hq, d)
    bs = cfg["block_size"]
    table = permutation(cfg["table_seed"], cfg["num_blocks"]).astype(np.int32)
    pos = np.arange(t)
    slots = table[pos // bs].astype(np.int64) * bs + pos % bs
    return k, v, q, table, slots


def f16_bits_rne(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def ferrum_f16_bits_away(x: np.ndarray) -> np.ndarray:
    """numpy statement of Ferrum's f32_to_f16_bits (crates/kernels/src/q8_dot.rs:113-139)."""
    bits = np.asarray(x, np.float32).view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    exp = (bits >> 23) & 0xFF
    frac = bits & 0x7FFFFF
    out = np.zeros(bits.shape, np.int64)
    nan_inf = exp == 0xFF
    hf = frac >> 13
    out = np.where(nan_inf, sign | 0x7C00 | hf | ((hf == 0) & (frac != 0)), out)
    he = exp - 127 + 15
    over = ~nan_inf & (he >= 31)
    out = np.where(over, sign | 0x7C00, out)
    sub = ~nan_inf & ~over & (he <= 0)
    shift = np.clip(1 - he, 0, 40)
    fr = frac | 0x800000
    sub_val = np.where(he < -10, sign, sign | ((fr >> (shift + 13)) + ((fr >> (shift + 12)) & 1)))
    out = np.where(sub, sub_val, out)
    nrm = ~nan_inf & ~over & ~sub
    half = (np.clip(he, 0, 31) << 10) | (frac >> 13)
    out = np.where(nrm, sign | ((half + ((frac >> 12) & 1)) & 0xFFFF), out)
    return out.astype(np.uint16)


def q8_quantize_blocks(x: np.ndarray, scale_bits_fn) -> np.ndarray:
    """Q8Activation::quantize_into in numpy: rows of 32 -> [n][34] bytes."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.fmax.reduce(np.abs(x), axis=1)          # f32::max skips NaN
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        y = (x * idv[:, None]).astype(np.float32)
        t = np.trunc(y)
        r = t + np.where(np.abs(y - t) >= 0.5, np.copysign(np.float32(1.0), y), 0.0)  # round()
        r = np.where(np.isnan(r), 0.0, r)                 # `as i32`: NaN -> 0, saturating
        q = np.clip(r, -128, 127).astype(np.int8)
    s = scale_bits_fn(d)
    out = np.zeros((x.shape[0], 34), np.uint8)
    out[:, 0] = s & 0xFF
    out[:, 1] = s >> 8
    out[:, 2:] = q.view(np.uint8)
    return out


def q8_inputs(seed=7):
    z = normal_f32(seed, 256 * 32).reshape(256, 32)
    pick = normal_f32(seed + 1, 256 * 32).reshape(256, 32)
    outl = np.abs(pick) > np.float32(2.5758)  # two-sided 1% of N(0,1)
    z = np.where(outl, np.where(pick > 0, np.float32(20.0), np.float32(-20.0)), z)
    edge = np.zeros((6, 32), np.float32)
    edge[1, 3] = 1.0                                   # single outlier -> q = 127 there
    edge[2, :] = 1.0                                   # reference KAT: x == 1 -> q == 127
    edge[3, 0] = 127.0                                 # d = 1, id = 1: exact .5 ties
    edge[3, 1:] = np.arange(-15, 16, dtype=np.float32) + np.float32(0.5)
    edge[4, :] = -3.0e-41                              # subnormal amax
    edge[5, :5] = [np.float32(3.0e38), -1.0, 0.0, np.float32(1e-30), 2.0]
    # Scale ties: amax = 127 * (1 + 2^-11) * 2^e makes d = amax / 127 exactly halfway
    # between two binary16 values whose lower one is even, so roundTiesToEven and
    # Ferrum's ties-away encoder store different scale bits.
    ties = np.zeros((4, 32), np.float32)
    for i, e in enumerate((-6, 0, 3, 7)):
        amax = np.float32(127.0 * (1.0 + 2.0 ** -11) * 2.0 ** e)
        ties[i] = normal_f32(seed + 2 + i, 32) * np.float32(0.3) * amax
        ties[i, 5] = -amax
    return np.concatenate([z, edge, ties]).astype(np.float32)


def main():
    k, v, q, table, slots = c1_inputs()
    hq, hkv, d = C1["n_heads"], C1["n_kv_heads"], C1["head_dim"]
    g = hq // hkv
    kb, vb = f16_bits_rne(k), f16_bits_rne(v)
    kd = kb.view(np.float16).astype(np.float64)
    vd = vb.view(np.float16).astype(np.float64)
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(d)))  # llama.rs:169
    attn = np.zeros((C1["decode_steps"], hq, d), np.float64)
    for s in range(C1["decode_steps"]):
        ctx = C1["prefill"] + s + 1
        for h in range(hq):
            sc = kd[:ctx, h // g] @ q[s, h].astype(np.float64) * scale
            e = np.exp(sc - sc.max())
            attn[s, h] = (e[:, None] * vd[:ctx, h // g]).sum(0) / e.sum()
    np.savez_compressed(os.path.join(HERE, "c1_tinyllama_layer.npz"),
                        inputs_sha256=np.array(digest(k, v, q)), table=table, slots=slots,
                        k_f16=kb, v_f16=vb, attn=attn, scale=np.float32(scale),
                        config=np.array(repr(C1)))
    x = q8_inputs()
    np.savez_compressed(os.path.join(HERE, "q8_blocks.npz"),
                        inputs_sha256=np.array(digest(x)), x=x,
                        blocks_rne=q8_quantize_blocks(x, f16_bits_rne),
                        blocks_away=q8_quantize_blocks(x, ferrum_f16_bits_away))
    print("wrote c1_tinyllama_layer.npz, q8_blocks.npz")


if __name__ == "__main__":
    main()
