"""Pins the oracle's optional layer parts (block.mojo:61 BlockSpec and :116
LayerWeights): the q|k|v biases of Qwen 2, the per-head q/k norms of Qwen 3,
the post norms of Gemma 2, the non-gated and gelu MLPs.

The hand cases port tests/test_block.mojo:430-816 (test_qk_norm,
test_qkv_bias, test_post_norms, test_mlp_shapes): identity projections and
gains of one at position zero, where every expected number is worked out by
hand or by the reference test's written-out pieces (_ref_rms, _ref_matvec,
_ref_silu, _ref_gelu).  The float64 cases hold every combination against
tests/layer64.py at a grouped, rotated, quantized layer.
"""

import math

import numpy as np
import pytest

import oracle
from tests import layer64 as l64
from tests.test_oracle_layer import _Written, _dense, _f32_weight, _model_layer, _spec

F32 = np.float32
WIDTH, HIDDEN, HEADS, HD = 8, 8, 2, 4
DIVISOR = math.sqrt(25.5 + float(F32(1e-5)))  # mean square of 1..8 is 25.5


def _identity_layer(**extra):
    eye = _f32_weight(np.eye(WIDTH, dtype=F32))
    w = dict(attn_norm=np.ones(WIDTH, F32), ffn_norm=np.ones(WIDTH, F32), wq=eye, wk=eye, wv=eye, wo=eye, gate=eye,
             up=eye, down=eye)
    w.update(extra)
    return w


def _attention(weights, spec=None):
    keep = []
    L = oracle.make_layer(spec or _spec(WIDTH, HIDDEN, HEADS, HEADS, HD), weights, keep)
    x = np.arange(1, WIDTH + 1, dtype=F32)
    keys, values = np.zeros(WIDTH, F32), np.zeros(WIDTH, F32)
    oracle.layer_step(L, x, keys, values, 0, 0, parts=1)
    return x, keys, values


def test_qk_norm():
    """test_block.mojo:430: each head of the cached key has unit root mean
    square, the value is not normed, and leaving the norms out changes the key."""
    x, keys, values = _attention(_identity_layer(q_norm=np.ones(HD, F32), k_norm=np.ones(HD, F32)))
    for h in range(HEADS):
        assert abs(math.sqrt(np.mean(keys[h * HD:(h + 1) * HD].astype(np.float64) ** 2)) - 1.0) <= 1e-4
    assert abs(values[0] - 1.0 / DIVISOR) <= 1e-6
    _, keys2, _ = _attention(_identity_layer())
    assert abs(keys[7] - keys2[7]) > 1e-4


def test_qkv_bias():
    """test_block.mojo:513: a cached value is the normed input plus its bias
    (ramps 0.5 + 0.25 i, -0.5 + 0.125 i, 0.25 + 0.5 i); zero biases are the
    same layer as none; a nonzero bias changes the cached key."""
    ramp = lambda first, step: (first + step * np.arange(WIDTH)).astype(F32)  # noqa: E731
    x, keys, values = _attention(_identity_layer(q_bias=ramp(0.5, 0.25), k_bias=ramp(-0.5, 0.125),
                                                 v_bias=ramp(0.25, 0.5)))
    assert abs(values[0] - (1.0 / DIVISOR + 0.25)) <= 1e-6
    assert abs(values[3] - (4.0 / DIVISOR + 1.75)) <= 1e-6
    z = np.zeros(WIDTH, F32)
    xa, ka, va = _attention(_identity_layer(q_bias=z, k_bias=z, v_bias=z))
    xb, kb, vb = _attention(_identity_layer())
    assert (xa == xb).all() and (ka == kb).all() and (va == vb).all()
    assert abs(keys[0] - kb[0]) > 1e-4


def test_post_norms():
    """test_block.mojo:645: a post norm of gain one over an already normed
    output leaves x + x / divisor; a gain of two doubles what the sublayer
    contributes and not the stream it joins."""
    v = np.arange(1, WIDTH + 1, dtype=np.float64)
    x, _, _ = _attention(_identity_layer(attn_post_norm=np.ones(WIDTH, F32)))
    assert np.abs(x - (v + v / DIVISOR)).max() <= 1e-4
    y, _, _ = _attention(_identity_layer(attn_post_norm=np.full(WIDTH, 2.0, F32)))
    assert np.abs(y - (v + 2.0 * v / DIVISOR)).max() <= 1e-4


def test_mlp_shapes():
    """test_block.mojo:725: a non-gated silu mlp is down(silu(up(normed
    x))); a gated gelu mlp is down(gelu(gate) * up), by the reference test's
    written-out pieces (dense weights 21, 22, 23)."""
    up, down, gate = _dense(WIDTH, HIDDEN, 21), _dense(HIDDEN, WIDTH, 22), _dense(WIDTH, HIDDEN, 23)
    start = (np.arange(WIDTH) - 3.0).astype(F32)
    ref = _Written(HEADS, HEADS, HD)
    normed = ref.rms(list(start), [1.0] * WIDTH)

    keep = []
    base = _identity_layer(up=_f32_weight(up), down=_f32_weight(down))
    del base["gate"]
    L = oracle.make_layer(dict(_spec(WIDTH, HIDDEN, HEADS, HEADS, HD), ungated=1), base, keep)
    x = start.copy()
    oracle.layer_step(L, x, np.zeros(WIDTH, F32), np.zeros(WIDTH, F32), 0, 0, parts=2)
    u = [ref.silu(v) for v in ref.matvec(up.tolist(), normed)]
    want = np.array(start, np.float64) + np.array(ref.matvec(down.tolist(), u), np.float64)
    assert np.abs(x - want).max() <= 1e-4

    def ref_gelu(v):  # test_block.mojo:198 _ref_gelu
        inner = F32(0.7978845608028654) * (v + F32(0.044715) * v * v * v)
        return F32(F32(0.5) * v * (F32(1.0) + F32(math.tanh(float(inner)))))

    L2 = oracle.make_layer(dict(_spec(WIDTH, HIDDEN, HEADS, HEADS, HD), act=1),
                           _identity_layer(gate=_f32_weight(gate), up=_f32_weight(up), down=_f32_weight(down)), keep)
    y = start.copy()
    oracle.layer_step(L2, y, np.zeros(WIDTH, F32), np.zeros(WIDTH, F32), 0, 0, parts=2)
    g = [ref_gelu(a) * b for a, b in zip(ref.matvec(gate.tolist(), normed), ref.matvec(up.tolist(), normed))]
    want2 = np.array(start, np.float64) + np.array(ref.matvec(down.tolist(), g), np.float64)
    assert np.abs(y - want2).max() <= 1e-4


FAMILIES = {
    "qwen2": dict(bias=True),
    "qwen3": dict(qk_norm=True),
    "gemma2": dict(post=True, act=1),
    "gemma3": dict(post=True, qk_norm=True, act=1),
    "ungated_silu": dict(ungated=1),
    "ungated_gelu_bias": dict(ungated=1, act=1, bias=True),
}


def family_layer(name, seed):
    """A quantized grouped layer (tests/test_oracle_layer.py _model_layer)
    with the named family's optional parts, seeded."""
    f = FAMILIES[name]
    spec, weights = _model_layer(seed)
    rng = np.random.default_rng(seed + 1000)
    qw, kvw, hd, W = spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"], spec["head_dim"], spec[
        "width"]
    if f.get("bias"):
        weights["q_bias"] = (0.5 * rng.standard_normal(qw)).astype(F32)
        weights["k_bias"] = (0.5 * rng.standard_normal(kvw)).astype(F32)
        weights["v_bias"] = (0.5 * rng.standard_normal(kvw)).astype(F32)
    if f.get("qk_norm"):
        weights["q_norm"] = (0.3 * (1 + 0.1 * rng.standard_normal(hd))).astype(F32)
        weights["k_norm"] = (0.3 * (1 + 0.1 * rng.standard_normal(hd))).astype(F32)
    if f.get("post"):
        weights["attn_post_norm"] = (1 + 0.1 * rng.standard_normal(W)).astype(F32)
        weights["ffn_post_norm"] = (1 + 0.1 * rng.standard_normal(W)).astype(F32)
    spec = dict(spec, ungated=f.get("ungated", 0), act=f.get("act", 0))
    if spec["ungated"]:
        del weights["gate"]
    return spec, weights


@pytest.mark.parametrize("name", list(FAMILIES))
def test_family_layer_against_float64(name):
    """Each family's layer at position 50 over a seeded cache: or_layer_step
    within 1e-5 of the float64 layer, keys and values included; and the
    optional parts matter (the Llama layer over the same weights lands far
    outside that gate)."""
    spec, weights = family_layer(name, 11)
    keep = []
    L = oracle.make_layer(spec, weights, keep)
    kvw = spec["kv_heads"] * spec["head_dim"]
    pos = 50
    rng = np.random.default_rng(3)
    keys = rng.standard_normal((pos + 1) * kvw).astype(F32)
    values = rng.standard_normal((pos + 1) * kvw).astype(F32)
    x = rng.standard_normal(spec["width"]).astype(F32)
    k64 = keys.astype(np.float64).reshape(pos + 1, kvw)
    v64 = values.astype(np.float64).reshape(pos + 1, kvw)
    want = l64.layer64(spec, weights, x, k64.copy(), v64.copy(), pos, pos)
    k_out, v_out = k64.copy(), v64.copy()
    l64.layer64(spec, weights, x, k_out, v_out, pos, pos)
    got = x.copy()
    oracle.layer_step(L, got, keys, values, pos, pos)
    assert l64.envelope_close(got, want, 1e-5) <= 1.0
    assert l64.envelope_close(keys[pos * kvw:], k_out[pos], 1e-5) <= 1.0
    assert l64.envelope_close(values[pos * kvw:], v_out[pos], 1e-5) <= 1.0
    plain_w = {k: v for k, v in weights.items() if k not in oracle.OPTIONAL_VECTORS}
    if spec["ungated"]:
        plain_w["gate"] = weights["up"]
    plain = l64.layer64(dict(spec, ungated=0, act=0), plain_w, x, k64.copy(), v64.copy(), pos, pos)
    assert l64.envelope_close(plain, want, 1e-5) > 10.0
