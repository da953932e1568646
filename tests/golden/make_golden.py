"""Writes tests/golden/golden.npz: small input/output vectors for the hot path.

Run from the repo root:  python tests/golden/make_golden.py

Dequant and matvec inputs come from the reference's own block generator (the
xorshift64 stream and `_blocks` of tests/test_kernel.mojo:69-126, restated in
the oracle as or_test_blocks); the layer's Q4_K weights come from the seeded
generator with the benchmark configs' distributions (scales |N|*0.01), since
raw random blocks carry f16 scales far too large for a residual stream; outputs come from the CPU oracle,
which is itself pinned against the reference's known-answer tests
(tests/test_quant.mojo, tests/test_kernel.mojo, tests/test_rope.mojo,
tests/test_attention.mojo, tests/test_block.mojo).  The fixture freezes those
results so that a later change to the oracle or to a kernel that moves any
bit shows up as a diff against committed data, and so that GPU tests can
check dequant bits without the oracle.

Contents (keys of the .npz):
  deq_<kind>_blocks, deq_<kind>_out   64 blocks of each of the eight kinds and their
                                      dequant as float32 (compared bitwise)
  mv_<kind>_w, mv_<kind>_x, mv_<kind>_y
                                      4 rows x 512 cols matvec (2 superblocks
                                      or 16 small blocks per row)
  layer_*                             one decoder layer (width 256, hidden
                                      512, 4 heads / 2 kv heads of 64, Q4_K,
                                      pos 37): weights, gains, x in/out, f16
                                      k/v caches in, new k/v slot out
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from molla_amd import synth  # noqa: E402

KINDS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_k": oracle.Q4_K, "q6_k": oracle.Q6_K,
         "q4_1": oracle.Q4_1, "q5_0": oracle.Q5_0, "q5_1": oracle.Q5_1, "q5_k": oracle.Q5_K}
LAYER_SPEC = dict(width=256, hidden=512, heads=4, kv_heads=2, head_dim=64, rope_dim=64, neox=0, eps=1e-5,
                  rope_base=500000.0, attn_scale=float(np.float32(1 / math.sqrt(64))))
LAYER_POS = 37
NAMES = ("wq", "wk", "wv", "wo", "gate", "up", "down")


def layer_shapes(s):
    qw, kvw = s["heads"] * s["head_dim"], s["kv_heads"] * s["head_dim"]
    W, H = s["width"], s["hidden"]
    return {"wq": (qw, W), "wk": (kvw, W), "wv": (kvw, W), "wo": (W, qw), "gate": (H, W), "up": (H, W),
            "down": (W, H)}


def build() -> dict:
    out = {}
    for i, (name, kind) in enumerate(KINDS.items()):
        blocks = oracle.test_blocks(kind, 64, 0x9E3779B97F4A7C15 + i)
        out[f"deq_{name}_blocks"] = blocks
        out[f"deq_{name}_out"] = oracle.dequant(kind, blocks, 64 * oracle.block_elements(kind))
        rows, cols = 4, 512
        nb = rows * cols // oracle.block_elements(kind)
        w = oracle.test_blocks(kind, nb, 1000 + i)
        x = np.random.default_rng(2000 + i).standard_normal(cols).astype(np.float32)
        out[f"mv_{name}_w"] = w
        out[f"mv_{name}_x"] = x
        out[f"mv_{name}_y"] = oracle.matvec(kind, w, rows, cols, x)

    s = LAYER_SPEC
    rng = np.random.default_rng(3000)
    weights = {}
    for j, (n, (r, c)) in enumerate(layer_shapes(s).items()):
        blob = synth.quant_tensor(oracle.Q4_K, r, c, 4000 + j).numpy()
        weights[n] = (oracle.Q4_K, r, c, blob)
        out[f"layer_{n}"] = blob
    for n in ("attn_norm", "ffn_norm"):
        g = (1.0 + 0.1 * rng.standard_normal(s["width"])).astype(np.float32)
        weights[n] = g
        out[f"layer_{n}"] = g
    kvw = s["kv_heads"] * s["head_dim"]
    count = LAYER_POS + 1
    k16 = rng.standard_normal(count * kvw).astype(np.float16)
    v16 = rng.standard_normal(count * kvw).astype(np.float16)
    x = rng.standard_normal(s["width"]).astype(np.float32)
    out["layer_k16"], out["layer_v16"], out["layer_x"] = k16, v16, x
    keep = []
    L = oracle.make_layer(s, weights, keep)
    xo, ko, vo = x.copy(), k16.astype(np.float32), v16.astype(np.float32)
    oracle.layer_step(L, xo, ko, vo, LAYER_POS, LAYER_POS, f16_store=True)
    out["layer_x_out"] = xo
    out["layer_k_new"] = ko.reshape(count, kvw)[LAYER_POS].copy()
    out["layer_v_new"] = vo.reshape(count, kvw)[LAYER_POS].copy()
    return out


def main():
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **build())
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
