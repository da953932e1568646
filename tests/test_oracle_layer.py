"""Pins the oracle's decoder layer (or_layer_step) and forward pass (or_forward).

The arithmetic under a layer (dequant, fused dot, norm, rope, attention) is
pinned in test_oracle.py.  What a layer adds is the order of the calls and
which operand goes where, so the checks here are second implementations that
share nothing with oracle/molla_oracle.c:

* `_Written` is the reference's own written-out layer from
  tests/test_block.mojo:130-221 (`_ref_matvec`, `_ref_rope`, `_ref_attend`,
  `_ref_silu`, `_ref_rms`), restated as float32 scalar loops, and driven with
  the weights, cache and position of `test_against_reference`
  (tests/test_block.mojo:313-430).
* `_layer64` is a float64 numpy layer written from block.mojo:319-482 as
  prose: weights dequantized by tests/npquant.py (not the oracle), matrix
  products in float64, rope angles from float64 powers.  It covers what the
  Mojo case leaves at its defaults: grouped heads (4:1), adjacent-pair rope
  (Llama), rope frequency factors, a position far from zero and quantized
  weights of several kinds.
* The forward pass is checked against tests/test_nnmodel.mojo:291-421
  (`test_forward`: identity layers whose first cached key has a closed form)
  and against `_forward64`, the same float64 layer stacked under an embedding
  row and a quantized head.
"""

import math

import numpy as np
import pytest

import oracle
from tests import layer64 as l64

F32 = np.float32


def _dense(cols, rows, seed):
    """tests/test_block.mojo:100 _dense: ((13 r + 7 c + 5 seed) mod 9 - 4) / 8."""
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    return (((r * 13 + c * 7 + seed * 5) % 9 - 4) / 8.0).astype(F32)


def _f32_weight(m):
    m = np.ascontiguousarray(m, F32)
    return (oracle.F32, m.shape[0], m.shape[1], m.view(np.uint8).ravel())


# ---- the reference's written-out layer (tests/test_block.mojo:130-221) -------

class _Written:
    """Float32 scalar loops in the reference test's order.  heads, kv_heads,
    head_dim as the spec; neox pairing and no scaling (the test's _ref_rope)."""

    def __init__(self, heads, kv_heads, head_dim, eps=1e-5):
        self.heads, self.kv_heads, self.hd, self.eps = heads, kv_heads, head_dim, F32(eps)

    def rms(self, x, gain):  # _ref_rms :123
        s = 0.0
        for v in x:
            s += float(v) * float(v)
        scale = F32(1.0 / math.sqrt(s / len(x) + float(self.eps)))
        return [F32(F32(v) * scale) * F32(g) for v, g in zip(x, gain)]

    @staticmethod
    def matvec(w, x):  # _ref_matvec :130
        out = []
        for row in w:
            acc = F32(0)
            for a, b in zip(row, x):
                acc = F32(acc + F32(a) * F32(b))
            out.append(acc)
        return out

    def rope(self, x, at, pos, base):  # _ref_rope :146, neox pairing
        pairs = self.hd // 2
        step = F32(1.0)
        ratio = F32(1.0) / F32(math.sqrt(base))
        for pair in range(pairs):
            theta = F32(F32(pos) * step)
            c = F32(math.cos(float(theta)))
            s = F32(math.sin(float(theta)))
            lo, hi = at + pair, at + pair + pairs
            a, b = x[lo], x[hi]
            x[lo] = F32(a * c - b * s)
            x[hi] = F32(a * s + b * c)
            step = F32(step * ratio)

    def attend(self, q, keys, values, count):  # _ref_attend :164
        hd = self.hd
        scale = F32(1.0 / math.sqrt(hd))
        group = self.heads // self.kv_heads
        kvw = self.kv_heads * hd
        out = [F32(0)] * (self.heads * hd)
        for h in range(self.heads):
            kh = h // group
            raw = []
            for t in range(count):
                dot = F32(0)
                for d in range(hd):
                    dot = F32(dot + q[h * hd + d] * keys[t * kvw + kh * hd + d])
                raw.append(F32(dot * scale))
            top = max(raw)
            total = F32(0)
            for t in range(count):
                raw[t] = F32(math.exp(float(raw[t] - top)))
                total = F32(total + raw[t])
            for d in range(hd):
                acc = F32(0)
                for t in range(count):
                    acc = F32(acc + raw[t] / total * values[t * kvw + kh * hd + d])
                out[h * hd + d] = acc
        return out

    @staticmethod
    def silu(v):  # _ref_silu :194
        return F32(v / (F32(1.0) + F32(math.exp(-float(v)))))

    def layer(self, w, x, keys, values, slot, pos, base):
        """test_block.mojo:367-405, the written-out reference's body."""
        r = [F32(v) for v in x]
        kvw = self.kv_heads * self.hd
        normed = self.rms(r, w["attn_norm"])
        q = self.matvec(w["wq"], normed)
        keys[slot * kvw:(slot + 1) * kvw] = self.matvec(w["wk"], normed)
        values[slot * kvw:(slot + 1) * kvw] = self.matvec(w["wv"], normed)
        for h in range(self.heads):
            self.rope(q, h * self.hd, pos, base)
        for h in range(self.kv_heads):
            self.rope(keys, slot * kvw + h * self.hd, pos, base)
        mixed = self.attend(q, keys, values, slot + 1)
        projected = self.matvec(w["wo"], mixed)
        r = [F32(a + b) for a, b in zip(r, projected)]
        normed2 = self.rms(r, w["ffn_norm"])
        g = self.matvec(w["gate"], normed2)
        u = self.matvec(w["up"], normed2)
        g = [F32(self.silu(a) * b) for a, b in zip(g, u)]
        out2 = self.matvec(w["down"], g)
        return [F32(a + b) for a, b in zip(r, out2)]


def _spec(width, hidden, heads, kv_heads, head_dim, neox=1, base=10000.0, rope_dim=None):
    return dict(width=width, hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                rope_dim=head_dim if rope_dim is None else rope_dim, neox=neox, eps=1e-5, rope_base=base,
                attn_scale=float(F32(1 / math.sqrt(head_dim))))


@pytest.mark.parametrize("heads,kv_heads", [(2, 2), (4, 2)])
def test_layer_against_written_reference(heads, kv_heads):
    """tests/test_block.mojo:313-430 test_against_reference: WIDTH 8, HIDDEN 8,
    HEAD_DIM 4, dense non-identity weights, two keys already cached, the new
    token at slot 2 / position 2.  (heads, kv_heads) = (2, 2) is the
    reference's case; (4, 2) runs the same written-out layer grouped."""
    WIDTH, HIDDEN, HD = 8, 8, 4
    qw, kvw = heads * HD, kv_heads * HD
    dense = {"attn_norm": _dense(WIDTH, 1, 1)[0], "ffn_norm": _dense(WIDTH, 1, 2)[0],
             "wq": _dense(WIDTH, qw, 3), "wk": _dense(WIDTH, kvw, 4), "wv": _dense(WIDTH, kvw, 5),
             "wo": _dense(qw, WIDTH, 6), "gate": _dense(WIDTH, HIDDEN, 7), "up": _dense(WIDTH, HIDDEN, 8),
             "down": _dense(HIDDEN, WIDTH, 9)}
    start = np.array([(i % 5) - 2.0 + i / 10.0 for i in range(WIDTH)], F32)
    seeded_k = _dense(kvw * 3, 1, 11)[0]
    seeded_v = _dense(kvw * 3, 1, 12)[0]

    keep = []
    weights = {k: (_f32_weight(v) if v.ndim == 2 else v) for k, v in dense.items()}
    L = oracle.make_layer(_spec(WIDTH, HIDDEN, heads, kv_heads, HD), weights, keep)
    x = start.copy()
    keys, values = seeded_k.copy(), seeded_v.copy()
    oracle.layer_step(L, x, keys, values, 2, 2)

    ref = _Written(heads, kv_heads, HD)
    rk, rv = [F32(v) for v in seeded_k], [F32(v) for v in seeded_v]
    want = ref.layer({k: (v.tolist() if v.ndim == 2 else list(v)) for k, v in dense.items()},
                     list(start), rk, rv, 2, 2, 10000.0)

    assert np.abs(x - np.array(want, F32)).max() <= 1e-4, "the layer disagrees with the written-out reference"
    assert np.abs(keys[2 * kvw:] - np.array(rk[2 * kvw:], F32)).max() <= 1e-5, "the cached key"
    assert np.abs(values[2 * kvw:] - np.array(rv[2 * kvw:], F32)).max() <= 1e-5, "the cached value"
    assert (keys[:2 * kvw] == seeded_k[:2 * kvw]).all() and (values[:2 * kvw] == seeded_v[:2 * kvw]).all(), \
        "the slots before the new one are not written to"


# ---- the float64 layer (tests/layer64.py, block.mojo:319-482) -----------------

def _quant(kind, rows, cols, seed):
    from molla_amd import synth

    return (kind, rows, cols, synth.quant_tensor(kind, rows, cols, seed).numpy())


def _model_layer(seed, width=256, hidden=512, heads=8, kv_heads=2, head_dim=32, kinds=None, factors=True):
    """A small Llama-shaped layer of quantized weights, grouped 4:1."""
    kinds = kinds or {"wq": 12, "wk": 12, "wv": 14, "wo": 12, "gate": 12, "up": 8, "down": 14}
    spec = _spec(width, hidden, heads, kv_heads, head_dim, neox=0, base=500000.0)
    shapes = {"wq": (heads * head_dim, width), "wk": (kv_heads * head_dim, width),
              "wv": (kv_heads * head_dim, width), "wo": (width, heads * head_dim), "gate": (hidden, width),
              "up": (hidden, width), "down": (width, hidden)}
    rng = np.random.default_rng(seed)
    weights = {k: _quant(kinds[k], r, c, seed * 31 + i) for i, (k, (r, c)) in enumerate(shapes.items())}
    # gains well under one keep the synthetic weights' products near unit
    # scale, so the softmax is spread over many keys and silu is not saturated
    weights["attn_norm"] = (0.03 * (1 + 0.1 * rng.standard_normal(width))).astype(F32)
    weights["ffn_norm"] = (0.05 * (1 + 0.1 * rng.standard_normal(width))).astype(F32)
    if factors:
        weights["rope_factors"] = rng.uniform(1.0, 8.0, head_dim // 2).astype(F32)
    return spec, weights


@pytest.mark.parametrize("pos", [37, 1000])
def test_layer_against_float64(pos):
    """Quantized weights (Q4_K, Q6_K, Q8_0), 8 query heads over 2 key heads,
    adjacent-pair rope with frequency factors, a cache of `pos` seeded keys
    and the new token at slot = pos: or_layer_step within 1e-5 of a float64
    layer (the oracle accumulates in float32), keys and values included."""
    spec, weights = _model_layer(5)
    keep = []
    L = oracle.make_layer(spec, weights, keep)
    kvw = spec["kv_heads"] * spec["head_dim"]
    rng = np.random.default_rng(pos)
    keys = rng.standard_normal((pos + 1) * kvw).astype(F32)
    values = rng.standard_normal((pos + 1) * kvw).astype(F32)
    x = rng.standard_normal(spec["width"]).astype(F32)
    k64 = keys.astype(np.float64).reshape(pos + 1, kvw)
    v64 = values.astype(np.float64).reshape(pos + 1, kvw)
    want = l64.layer64(spec, weights, x, k64, v64, pos, pos)
    oracle.layer_step(L, x, keys, values, pos, pos)
    assert l64.envelope_close(x, want, 1e-5) <= 1.0
    assert l64.envelope_close(keys[pos * kvw:], k64[pos], 1e-5) <= 1.0
    assert l64.envelope_close(values[pos * kvw:], v64[pos], 1e-5) <= 1.0


def test_layer_float64_catches_the_plausible_mistakes():
    """The float64 layer tells apart what a wrong oracle would compute: no
    rope on k, gate and up swapped, no frequency factors, neox pairing, the
    wrong key head for a query head.  Each variant of the float64 layer must
    land far outside the 1e-5 gate the oracle passes."""
    spec, weights = _model_layer(6)
    kvw = spec["kv_heads"] * spec["head_dim"]
    pos = 40
    rng = np.random.default_rng(1)
    keys = rng.standard_normal((pos + 1, kvw))
    values = rng.standard_normal((pos + 1, kvw))
    x = rng.standard_normal(spec["width"]).astype(F32)
    good = l64.layer64(spec, weights, x, keys.copy(), values.copy(), pos, pos)
    swapped = dict(weights, gate=weights["up"], up=weights["gate"])
    variants = {
        "gate/up swapped": l64.layer64(spec, swapped, x, keys.copy(), values.copy(), pos, pos),
        "no factors": l64.layer64(spec, {k: v for k, v in weights.items() if k != "rope_factors"}, x, keys.copy(),
                               values.copy(), pos, pos),
        "neox pairs": l64.layer64(dict(spec, neox=1), weights, x, keys.copy(), values.copy(), pos, pos),
        "query head h on key head h mod kv_heads": l64.layer64(spec, weights, x, keys.copy(), values.copy(), pos,
                                                            pos, interleave=True),
    }
    for name, v in variants.items():
        assert l64.envelope_close(v, good, 1e-5) > 10.0, name
    # k not rotated: rebuild by hand
    H, KV, HD = spec["heads"], spec["kv_heads"], spec["head_dim"]
    W = {k: l64.dq(weights[k]) for k in ("wq", "wk", "wv", "wo", "gate", "up", "down")}
    n = l64.rms64(x.astype(np.float64), weights["attn_norm"], spec["eps"])
    k2, v2 = keys.copy(), values.copy()
    k2[pos] = W["wk"] @ n
    v2[pos] = W["wv"] @ n
    q = l64.rope64(W["wq"] @ n, H, HD, spec["rope_dim"], spec["rope_base"], 0, pos, weights["rope_factors"])
    ho = l64.attend64(q, k2.reshape(-1), v2.reshape(-1), pos + 1, H, KV, HD, spec["attn_scale"])
    r = x + W["wo"] @ ho
    n2 = l64.rms64(r, weights["ffn_norm"], spec["eps"])
    g, u = W["gate"] @ n2, W["up"] @ n2
    no_krope = r + W["down"] @ (g / (1 + np.exp(-g)) * u)
    assert l64.envelope_close(no_krope, good, 1e-5) > 10.0


# ---- forward: tests/test_nnmodel.mojo:291-421 --------------------------------

def _identity_model(n_layers=2):
    WIDTH = 4
    spec = _spec(WIDTH, WIDTH, 1, 1, WIDTH, neox=1, base=10000.0)
    eye = _f32_weight(np.eye(WIDTH, dtype=F32))
    w = dict(attn_norm=np.ones(WIDTH, F32), ffn_norm=np.ones(WIDTH, F32), wq=eye, wk=eye, wv=eye, wo=eye,
             gate=eye, up=eye, down=eye)
    keep = []
    layers = [oracle.make_layer(spec, w, keep) for _ in range(n_layers)]
    rows = np.array([[t * 10 + i + 1 for i in range(WIDTH)] for t in range(3)], F32)  # _rows :88
    return layers, rows, keep


def test_forward_identity_layers():
    """test_nnmodel.mojo:291 test_forward: two identity layers, vocabulary 3,
    width 4, one head.  Token 1's row is 11..14 (mean square 157.5), so the
    first layer caches 11 / sqrt(157.5 + eps) as key[0]; the second layer
    caches something else; nothing lands past slot 0; and a token at slot 1
    that sees the first token's cache has other logits than the same token
    alone."""
    layers, rows, keep = _identity_model()
    onorm = np.ones(4, F32)
    head = _f32_weight(rows)  # the head over the embedding rows (a tied model)
    keys = [np.zeros(8, F32) for _ in range(2)]
    values = [np.zeros(8, F32) for _ in range(2)]
    logits = oracle.forward(layers, rows, onorm, head, 1, 0, 0, keys, values)
    assert logits.size == 3
    d0 = math.sqrt(157.5 + float(F32(1e-5)))
    assert abs(keys[0][0] - 11.0 / d0) <= 1e-4, "the first layer cached the normed embedding as its key"
    assert keys[1][0] != 0.0 and keys[1][0] != keys[0][0], "the second layer cached something of its own"
    assert (keys[0][4:] == 0).all() and (keys[1][4:] == 0).all(), "nothing was written past slot zero"

    with_history = oracle.forward(layers, rows, onorm, head, 2, 1, 1, keys, values)
    fresh_k = [np.zeros(8, F32) for _ in range(2)]
    fresh_v = [np.zeros(8, F32) for _ in range(2)]
    alone = oracle.forward(layers, rows, onorm, head, 2, 0, 0, fresh_k, fresh_v)
    assert np.abs(with_history - alone).max() > 1e-5, "a token's logits depend on the tokens before it"


def test_forward_identity_closed_form():
    """The same model at one token, worked out by hand: with identity weights,
    unit gains and one cached key (softmax of one score is 1, rope at 0 is no
    rotation) a layer maps x to x + n + silu(n) n, n = x / rms(x) after the
    attention step's own norm -- so the stream stays a multiple of the
    embedding row and the logits are rows . (final normed stream)."""
    layers, rows, keep = _identity_model()
    keys = [np.zeros(8, F32) for _ in range(2)]
    values = [np.zeros(8, F32) for _ in range(2)]
    got = oracle.forward(layers, rows, np.ones(4, F32), _f32_weight(rows), 0, 0, 0, keys, values)
    x = rows[0].astype(np.float64)
    eps = float(F32(1e-5))
    for _ in range(2):
        x = x + x / math.sqrt(np.mean(x * x) + eps)
        n = x / math.sqrt(np.mean(x * x) + eps)
        x = x + n / (1 + np.exp(-n)) * n
    want = rows.astype(np.float64) @ (x / math.sqrt(np.mean(x * x) + eps))
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


def _forward64(spec, layer_ws, emb, onorm, head, tokens):
    """Embedding row -> layers -> norm -> head in float64, token i at position i."""
    kvw = spec["kv_heads"] * spec["head_dim"]
    n = len(tokens)
    K = [np.zeros((n, kvw)) for _ in layer_ws]
    V = [np.zeros((n, kvw)) for _ in layer_ws]
    out = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].astype(np.float64)
        for li, w in enumerate(layer_ws):
            x = l64.layer64(spec, w, x, K[li], V[li], pos, pos)
        out.append(l64.dq(head) @ l64.rms64(x, onorm.astype(np.float64), spec["eps"]))
    return out


def test_forward_against_float64():
    """Three quantized layers (different kinds per layer), an f32 embedding, a
    Q6_K head; four tokens decoded one position at a time: every step's
    logits within 1e-5 of a float64 stack, and the same greedy pick."""
    kinds = [{"wq": 12, "wk": 12, "wv": 12, "wo": 12, "gate": 12, "up": 12, "down": 12},
             {"wq": 14, "wk": 8, "wv": 2, "wo": 14, "gate": 12, "up": 12, "down": 14},
             {"wq": 12, "wk": 12, "wv": 14, "wo": 8, "gate": 13, "up": 3, "down": 12}]
    pairs = [_model_layer(40 + i, kinds=k) for i, k in enumerate(kinds)]
    spec = pairs[0][0]
    layer_ws = [w for _, w in pairs]
    keep = []
    layers = [oracle.make_layer(s, w, keep) for s, w in pairs]
    vocab, width = 300, spec["width"]
    rng = np.random.default_rng(9)
    emb = rng.standard_normal((vocab, width)).astype(F32)
    onorm = (1 + 0.1 * rng.standard_normal(width)).astype(F32)
    head = _quant(14, vocab, width, 77)
    tokens = [5, 299, 0, 123]
    want = _forward64(spec, layer_ws, emb, onorm, head, tokens)
    kvw = spec["kv_heads"] * spec["head_dim"]
    keys = [np.zeros(len(tokens) * kvw, F32) for _ in layers]
    values = [np.zeros(len(tokens) * kvw, F32) for _ in layers]
    for pos, tok in enumerate(tokens):
        got = oracle.forward(layers, emb, onorm, head, tok, pos, pos, keys, values)
        assert l64.envelope_close(got, want[pos], 1e-5) <= 1.0, f"logits at position {pos}"
        assert int(np.argmax(got)) == int(np.argmax(want[pos]))
