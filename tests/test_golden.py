"""The committed golden vectors (tests/golden/golden.npz, written by
tests/golden/make_golden.py) against the CPU oracle and against an
independent numpy decoder.  CPU only.

Dequant bits and the small matvecs must reproduce exactly (the oracle is
plain C compiled without FP contraction); the layer within 1e-6 of its peak.
"""

import math
import os

import numpy as np
import pytest

import oracle
from tests import npquant

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
KINDS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_k": oracle.Q4_K, "q6_k": oracle.Q6_K,
         "q4_1": oracle.Q4_1, "q5_0": oracle.Q5_0, "q5_1": oracle.Q5_1, "q5_k": oracle.Q5_K}


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN) as d:
        return {k: d[k] for k in d.files}


@pytest.mark.parametrize("name", list(KINDS))
def test_dequant_vectors(g, name):
    kind = KINDS[name]
    blocks, want = g[f"deq_{name}_blocks"], g[f"deq_{name}_out"]
    got = oracle.dequant(kind, blocks, want.size)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    indep = npquant.dequant(kind, blocks, want.size)
    assert (indep.view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("name", list(KINDS))
def test_matvec_vectors(g, name):
    kind = KINDS[name]
    w, x, want = g[f"mv_{name}_w"], g[f"mv_{name}_x"], g[f"mv_{name}_y"]
    got = oracle.matvec(kind, w, want.size, x.size, x)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    # and the float64 dot of the dequantized rows agrees to the reference's gate
    dq = npquant.dequant(kind, w, want.size * x.size).reshape(want.size, x.size).astype(np.float64)
    ref = dq @ x.astype(np.float64)
    bound = 1e-4 * (np.abs(dq) @ np.abs(x.astype(np.float64))) + 1e-6
    assert (np.abs(want - ref) <= bound).all()


def test_layer_vector(g):
    spec = dict(width=256, hidden=512, heads=4, kv_heads=2, head_dim=64, rope_dim=64, neox=0, eps=1e-5,
                rope_base=500000.0, attn_scale=float(np.float32(1 / math.sqrt(64))))
    weights = {n: (oracle.Q4_K, *shape, g[f"layer_{n}"]) for n, shape in
               {"wq": (256, 256), "wk": (128, 256), "wv": (128, 256), "wo": (256, 256), "gate": (512, 256),
                "up": (512, 256), "down": (256, 512)}.items()}
    weights["attn_norm"] = g["layer_attn_norm"]
    weights["ffn_norm"] = g["layer_ffn_norm"]
    keep = []
    L = oracle.make_layer(spec, weights, keep)
    x = g["layer_x"].copy()
    k = g["layer_k16"].astype(np.float32)
    v = g["layer_v16"].astype(np.float32)
    oracle.layer_step(L, x, k, v, 37, 37, f16_store=True)
    want = g["layer_x_out"]
    assert np.abs(x - want).max() <= 1e-6 * np.abs(want).max()
    assert (k.reshape(38, 128)[37] == g["layer_k_new"]).all()
    assert (v.reshape(38, 128)[37] == g["layer_v_new"]).all()


def test_layer_vector_against_float64(g):
    """The committed layer output is the oracle's; here it is also held to
    the float64 layer of tests/layer64.py (independent of the oracle), within
    the per-element layer gate.  The float64 layer keeps the new key and value
    unrounded where the vector rounded them through f16, which the gate
    absorbs (one of 38 attended positions, weight about 1/38)."""
    from tests import layer64 as l64
    spec = dict(width=256, hidden=512, heads=4, kv_heads=2, head_dim=64, rope_dim=64, neox=0, eps=1e-5,
                rope_base=500000.0, attn_scale=float(np.float32(1 / math.sqrt(64))))
    host = {n: (oracle.Q4_K, *shape, g[f"layer_{n}"]) for n, shape in
            {"wq": (256, 256), "wk": (128, 256), "wv": (128, 256), "wo": (256, 256), "gate": (512, 256),
             "up": (512, 256), "down": (256, 512)}.items()}
    host["attn_norm"], host["ffn_norm"] = g["layer_attn_norm"], g["layer_ffn_norm"]
    k = g["layer_k16"].astype(np.float64).reshape(38, 128).copy()
    v = g["layer_v16"].astype(np.float64).reshape(38, 128).copy()
    want, parts = l64.layer64(spec, host, g["layer_x"], k, v, 37, 37, parts=True)
    assert (np.abs(g["layer_x_out"] - want) <= l64.layer_bound(parts)).all()
    assert np.abs(g["layer_k_new"] - k[37]).max() <= 1e-3 * np.abs(k[37]).max()
