"""The HIP path against the committed golden vectors (no oracle involved):
dequant bit-exact, matvec within the device-vs-host gate, one decoder layer
within the per-element layer gate (tests/layer64.py layer_bound)."""

import math
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
KINDS = {"q8_0": 8, "q4_0": 2, "q4_k": 12, "q6_k": 14, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q5_k": 13}


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN) as d:
        return {k: d[k] for k in d.files}


@pytest.fixture(scope="module")
def ctx():
    from molla_amd import gpu
    return gpu.DeviceContext(0)


@pytest.mark.parametrize("name", list(KINDS))
def test_dequant_golden(g, ctx, name):
    from molla_amd import gpu
    blocks, want = g[f"deq_{name}_blocks"], g[f"deq_{name}_out"]
    w = gpu.Tensor.from_bytes(torch.from_numpy(blocks), KINDS[name], want.size, 1)
    got = gpu.device_dequant(ctx, w).cpu().numpy()
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("name", list(KINDS))
def test_matvec_golden(g, ctx, name):
    from molla_amd import gpu
    w, x, want = g[f"mv_{name}_w"], g[f"mv_{name}_x"], g[f"mv_{name}_y"]
    t = gpu.Tensor.from_bytes(torch.from_numpy(w), KINDS[name], x.size, want.size)
    out = np.zeros(want.size, np.float32)
    gpu.device_matvec(ctx, t, x, out)
    assert np.abs(out - want).max() <= 1e-5 * np.abs(want).max()


def test_layer_golden(g, ctx):
    from molla_amd import block, gpu
    bs = block.BlockSpec(width=256, hidden=512, heads=4, kv_heads=2, head_dim=64, rope_dim=64,
                         rope_base=500000.0, neox=False, eps=1e-5)
    shapes = {"wq": (256, 256), "wk": (128, 256), "wv": (128, 256), "wo": (256, 256), "gate": (512, 256),
              "up": (512, 256), "down": (256, 512)}
    ws = {n: gpu.Tensor.from_bytes(torch.from_numpy(g[f"layer_{n}"]), 12, c, r) for n, (r, c) in shapes.items()}
    steps = torch.from_numpy(gpu.rope_steps(64, 500000.0)).cuda()
    layer = block.DeviceLayer(bs, torch.from_numpy(g["layer_attn_norm"]).cuda(),
                              torch.from_numpy(g["layer_ffn_norm"]).cuda(), ws, steps)
    assert layer.spec.attn_scale == pytest.approx(1 / math.sqrt(64))
    k = torch.from_numpy(g["layer_k16"]).cuda()
    v = torch.from_numpy(g["layer_v16"]).cuda()
    x = torch.from_numpy(g["layer_x"].copy()).cuda()
    pos = torch.full((1,), 37, dtype=torch.int32, device="cuda")
    block.device_layer(ctx, layer, x, k, v, 38 * 128, pos, 38, 1)
    ctx.synchronize()
    want = g["layer_x_out"]
    from tests import layer64 as l64
    spec = dict(width=256, hidden=512, heads=4, kv_heads=2, head_dim=64, rope_dim=64, neox=0, eps=1e-5,
                rope_base=500000.0, attn_scale=float(np.float32(1 / math.sqrt(64))))
    host = {n: (12, r, c, g[f"layer_{n}"]) for n, (r, c) in shapes.items()}
    host["attn_norm"], host["ffn_norm"] = g["layer_attn_norm"], g["layer_ffn_norm"]
    kv = [g[f"layer_{n}16"].astype(np.float64).reshape(38, 128).copy() for n in ("k", "v")]
    _, parts = l64.layer64(spec, host, g["layer_x"], kv[0], kv[1], 37, 37, parts=True)
    err = np.abs(x.cpu().numpy().astype(np.float64) - want)
    assert (err <= l64.layer_bound(parts)).all()
    kn = k.cpu().float().numpy().reshape(38, 128)
    assert np.allclose(kn[37], g["layer_k_new"], rtol=2e-3, atol=1e-3)
    assert (kn[:37] == g["layer_k16"].astype(np.float32).reshape(38, 128)[:37]).all()
