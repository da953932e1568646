"""A float64 numpy decoder layer, written from block.mojo:319-482 as prose.

Test infrastructure shared by the oracle's own tests (tests/test_oracle_layer.py)
and the GPU layer tests: weights are dequantized by tests/npquant.py (not the
oracle), products are float64, rope angles come from float64 powers
(rope.mojo:253 angle with its frequency factor).  `layer64` can also return the
intermediates a per-element error bound needs (the attention output that
feeds wo and the gated activation that feeds down).
"""

import numpy as np

import oracle
from tests import npquant

F32 = np.float32


def rope64(x, heads, head_dim, rope_dim, base, neox, pos, factors):
    """rope.mojo:253 angle / :294 rotate_scaled in float64: the angle of pair
    p is pos * base^(-2p/rope_dim) / factor[p]; elements past rope_dim stay."""
    x = x.reshape(heads, head_dim).copy()
    pairs = rope_dim // 2
    p = np.arange(pairs, dtype=np.float64)
    theta = pos * base ** (-2.0 * p / rope_dim)
    if factors is not None:
        theta = theta / np.asarray(factors[:pairs], np.float64)
    c, s = np.cos(theta), np.sin(theta)
    if neox:
        lo, hi = p.astype(int), p.astype(int) + pairs
    else:
        lo, hi = 2 * p.astype(int), 2 * p.astype(int) + 1
    a, b = x[:, lo].copy(), x[:, hi].copy()
    x[:, lo] = a * c - b * s
    x[:, hi] = a * s + b * c
    return x.reshape(-1)


def rms64(x, gain, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * gain


def attend64(q, keys, values, count, heads, kv_heads, head_dim, scale, interleave=False, pmax=None):
    group = heads // kv_heads
    K = keys.reshape(-1, kv_heads * head_dim)[:count].reshape(count, kv_heads, head_dim)
    V = values.reshape(-1, kv_heads * head_dim)[:count].reshape(count, kv_heads, head_dim)
    out = np.zeros((heads, head_dim))
    for h in range(heads):
        kh = h % kv_heads if interleave else h // group
        s = K[:, kh, :] @ q[h * head_dim:(h + 1) * head_dim] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[:, kh, :]
        if pmax is not None:
            pmax.append(float(p.max() / p.sum()))
    return out.reshape(-1)


def silu64(v):
    with np.errstate(over="ignore"):
        return v / (1 + np.exp(-v))


def gelu64(v):
    """kernel.mojo:499 gelu, the tanh approximation."""
    return 0.5 * v * (1 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))


def dq(w):
    kind, rows, cols, blob = w
    if kind == oracle.F32:
        return np.ascontiguousarray(blob).view(F32).reshape(rows, cols).astype(np.float64)
    return npquant.dequant(kind, blob, rows * cols).reshape(rows, cols).astype(np.float64)


def layer64(spec, weights, x, keys, values, slot, pos, interleave=False, parts=False):
    """One layer in float64; keys/values float64 [slots, kv_width], updated at
    slot.  parts: also return {"W": the dequantized matrices, "attn": the
    attention output wo reads, "act": the gated activation down reads}."""
    H, KV, HD = spec["heads"], spec["kv_heads"], spec["head_dim"]
    W = {k: dq(weights[k]) for k in ("wq", "wk", "wv", "wo", "gate", "up", "down") if k in weights}
    fac = weights.get("rope_factors")
    x = x.astype(np.float64)
    opt = {k: (None if weights.get(k) is None else np.asarray(weights[k], np.float64)) for k in
           ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "attn_post_norm", "ffn_post_norm")}
    eps = spec["eps"]
    n = rms64(x, weights["attn_norm"].astype(np.float64), eps)
    q = W["wq"] @ n
    keys[slot] = W["wk"] @ n
    values[slot] = W["wv"] @ n
    # block.mojo:363-384: biases, then each head of q and k normed, then rope
    if opt["q_bias"] is not None:
        q = q + opt["q_bias"]
        keys[slot] = keys[slot] + opt["k_bias"]
        values[slot] = values[slot] + opt["v_bias"]
    if opt["q_norm"] is not None:
        q = np.concatenate([rms64(h, opt["q_norm"], eps) for h in q.reshape(H, HD)])
        keys[slot] = np.concatenate([rms64(h, opt["k_norm"], eps) for h in keys[slot].reshape(KV, HD)])
    q = rope64(q, H, HD, spec["rope_dim"], spec["rope_base"], spec["neox"], pos, fac)
    keys[slot] = rope64(keys[slot], KV, HD, spec["rope_dim"], spec["rope_base"], spec["neox"], pos, fac)
    pmax = []
    heads_out = attend64(q, keys.reshape(-1), values.reshape(-1), slot + 1, H, KV, HD, spec["attn_scale"],
                         interleave, pmax)
    proj = W["wo"] @ heads_out
    post = {}
    if opt["attn_post_norm"] is not None:
        post["attn"] = (proj.copy(), opt["attn_post_norm"])
        proj = rms64(proj, opt["attn_post_norm"], eps)
    x = x + proj
    n = rms64(x, weights["ffn_norm"].astype(np.float64), eps)
    u = W["up"] @ n
    fn = gelu64 if spec.get("act", 0) else silu64
    if spec.get("ungated", 0):
        act = fn(u)
    else:
        act = fn(W["gate"] @ n) * u
    proj = W["down"] @ act
    if opt["ffn_post_norm"] is not None:
        post["ffn"] = (proj.copy(), opt["ffn_post_norm"])
        proj = rms64(proj, opt["ffn_post_norm"], eps)
    out = x + proj
    if parts:
        return out, {"W": W, "attn": heads_out, "act": act, "post": post, "eps": eps, "pmax": pmax}
    return out


def layer_bound(parts, rel=1e-4):
    """Per-element tolerance of a layer's output: rel times the absolute sums
    the two last projections add into the residual, sum_j |wo_ij a_j| +
    sum_j |down_ij h_j| -- the matvec gate (1e-4 sum |w x| per row,
    tests/test_kernel.mojo:473) carried through wo and down, which also
    covers what the rounding upstream of them (norm, q|k|v, attention)
    moves their inputs by."""
    W = parts["W"]
    e_attn = np.abs(W["wo"]) @ np.abs(parts["attn"])
    e_ffn = np.abs(W["down"]) @ np.abs(parts["act"])

    def through_post(e, key):
        # a post norm y * s * g (s = 1 / rms(y)) moves an error e in y by at
        # most s |g| (e_i + |y_i| ||e|| / ||y||) per element
        if key not in parts.get("post", {}):
            return e
        y, g = parts["post"][key]
        s = 1.0 / np.sqrt(np.mean(y * y) + parts["eps"])
        return s * np.abs(g) * (e + np.abs(y) * np.linalg.norm(e) / np.linalg.norm(y))
    return rel * (through_post(e_attn, "attn") + through_post(e_ffn, "ffn"))


def envelope_close(got, want, rel):
    """|got - want| <= rel * (|want| + rms(want)) elementwise: relative where
    an element is large, relative to the vector's scale where it is near 0."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bound = rel * (np.abs(want) + np.sqrt(np.mean(want * want)))
    return float((np.abs(got - want) / bound).max())


