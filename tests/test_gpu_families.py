"""The decoder layer with the optional parts of other families on the GPU
(block.mojo:61-482; gpu_block.mojo:678-896): Qwen 2's q|k|v biases, Qwen 3's
per-head q/k norms, Gemma 2's post norms and gelu, non-gated MLPs.  Through
the C ABI (mi_decoder_layer with the new mi_layer_desc fields) against the
oracle's layer (pinned by tests/test_oracle_families.py) at batch 1, a batch
of 3 sequences and a 12-token prefill chunk of one sequence, under the
per-element layer gate of tests/layer64.py."""

import numpy as np
import pytest
import torch

import oracle
from molla_amd import block, gpu, synth
from tests.test_gpu_layer import assert_layer_close, spec_of
from tests import layer64 as l64

pytestmark = pytest.mark.gpu

FAMILIES = {
    "qwen2": dict(bias=True),
    "qwen3": dict(qk_norm=True),
    "gemma2": dict(post=True, act=1),
    "gemma3": dict(post=True, qk_norm=True, act=1),
    "ungated_silu": dict(ungated=1),
    "ungated_gelu_bias": dict(ungated=1, act=1, bias=True),
}


def family_host(name, spec, seed):
    f = FAMILIES[name]
    W, H = spec["width"], spec["hidden"]
    qw, kvw, hd = spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"], spec["head_dim"]
    kinds = {"wv": oracle.Q6_K, "down": oracle.Q6_K, "up": oracle.Q8_0}
    shapes = {"wq": (qw, W), "wk": (kvw, W), "wv": (kvw, W), "wo": (W, qw), "gate": (H, W), "up": (H, W),
              "down": (W, H)}
    host = {}
    for i, (n, (r, c)) in enumerate(shapes.items()):
        if n == "gate" and f.get("ungated"):
            continue
        k = kinds.get(n, oracle.Q4_K)
        host[n] = (k, r, c, synth.quant_tensor(k, r, c, seed * 100 + i).numpy())
    rng = np.random.default_rng(seed)
    # gains under one keep the random layer's activations near unit scale
    host["attn_norm"] = (0.05 * (1 + 0.1 * rng.standard_normal(W))).astype(np.float32)
    host["ffn_norm"] = (0.05 * (1 + 0.1 * rng.standard_normal(W))).astype(np.float32)
    if f.get("bias"):
        host["q_bias"] = (0.5 * rng.standard_normal(qw)).astype(np.float32)
        host["k_bias"] = (0.5 * rng.standard_normal(kvw)).astype(np.float32)
        host["v_bias"] = (0.5 * rng.standard_normal(kvw)).astype(np.float32)
    if f.get("qk_norm"):
        host["q_norm"] = (0.3 * (1 + 0.1 * rng.standard_normal(hd))).astype(np.float32)
        host["k_norm"] = (0.3 * (1 + 0.1 * rng.standard_normal(hd))).astype(np.float32)
    if f.get("post"):
        host["attn_post_norm"] = (1 + 0.1 * rng.standard_normal(W)).astype(np.float32)
        host["ffn_post_norm"] = (1 + 0.1 * rng.standard_normal(W)).astype(np.float32)
    spec = dict(spec, ungated=f.get("ungated", 0), act=f.get("act", 0))
    return spec, host


def device_family_layer(spec, host):
    bs = block.BlockSpec(width=spec["width"], hidden=spec["hidden"], heads=spec["heads"], kv_heads=spec["kv_heads"],
                         head_dim=spec["head_dim"], rope_dim=spec["rope_dim"], rope_base=spec["rope_base"],
                         neox=bool(spec["neox"]), eps=spec["eps"], ungated=bool(spec["ungated"]),
                         act=gpu.ACT_BIT if spec["act"] else 0)
    weights = {n: gpu.Tensor.from_bytes(torch.from_numpy(host[n][3]), host[n][0], host[n][2], host[n][1])
               for n in block.DeviceLayer.NAMES if n in host}
    steps = torch.from_numpy(gpu.rope_steps(spec["rope_dim"], spec["rope_base"])).cuda()
    extras = {k: torch.from_numpy(host[k]).cuda() for k in oracle.OPTIONAL_VECTORS if k in host}
    layer = block.DeviceLayer(bs, torch.from_numpy(host["attn_norm"]).cuda(), torch.from_numpy(host["ffn_norm"]).cuda(),
                              weights, steps, None, extras)
    return bs, layer


def oracle_spec(spec):
    return dict(spec, act=1 if spec["act"] else 0)


@pytest.mark.parametrize("name", list(FAMILIES))
@pytest.mark.parametrize("tokens", [1, 3])
def test_family_layer_decode(name, tokens):
    spec, host = family_host(name, spec_of(512, 1024, 8, 2, 64, base=1000000.0), 31)
    ctx = gpu.DeviceContext(0)
    bs, layer = device_family_layer(spec, host)
    kvw = bs.kv_width()
    pos = 70
    count = pos + 1
    stride = count * kvw
    keys16 = synth.normal(tokens * stride, 40).half()
    vals16 = synth.normal(tokens * stride, 41).half()
    x = synth.normal(tokens * bs.width, 42).numpy()
    kd, vd = keys16.clone().cuda(), vals16.clone().cuda()
    xd = torch.from_numpy(x.copy()).cuda()
    posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")
    block.device_layer(ctx, layer, xd, kd, vd, stride, posd, count, tokens)
    ctx.synchronize()
    got = xd.cpu().numpy().reshape(tokens, -1)
    got_k = kd.cpu().float().numpy().reshape(tokens, count, kvw)
    keep = []
    L = oracle.make_layer(oracle_spec(spec), host, keep)
    for t in range(tokens):
        xr = x.reshape(tokens, -1)[t].copy()
        kr = keys16.float().numpy().reshape(tokens, -1)[t].copy()
        vr = vals16.float().numpy().reshape(tokens, -1)[t].copy()
        _, parts = l64.layer64(oracle_spec(spec), host, xr, kr.astype(np.float64).reshape(count, kvw).copy(),
                               vr.astype(np.float64).reshape(count, kvw).copy(), pos, pos, parts=True)
        oracle.layer_step(L, xr, kr, vr, pos, pos, f16_store=True, threads=8)
        assert_layer_close(got[t], xr, l64.layer_bound(parts), f"{name} seq {t}:")
        assert np.allclose(got_k[t, pos], kr.reshape(count, kvw)[pos], rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("name", list(FAMILIES))
def test_family_layer_prefill_chunk(name):
    """A 12-token chunk of one sequence (cache stride 0) through the prefill
    layer, token by token against the oracle."""
    spec, host = family_host(name, spec_of(512, 1024, 8, 2, 64, base=1000000.0), 37)
    ctx = gpu.DeviceContext(0)
    bs, layer = device_family_layer(spec, host)
    kvw = bs.kv_width()
    first, tokens = 20, 12
    count = first + tokens
    keys16 = synth.normal(count * kvw, 50).half().numpy().reshape(count, kvw)
    vals16 = synth.normal(count * kvw, 51).half().numpy().reshape(count, kvw)
    x = synth.normal(tokens * bs.width, 52).numpy()
    xd = torch.from_numpy(x.copy()).cuda()
    kd = torch.from_numpy(keys16.reshape(-1).copy()).cuda()
    vd = torch.from_numpy(vals16.reshape(-1).copy()).cuda()
    posd = torch.arange(first, count, dtype=torch.int32, device="cuda")
    block.device_layer(ctx, layer, xd, kd, vd, 0, posd, count, tokens)
    ctx.synchronize()
    got_x = xd.cpu().numpy().reshape(tokens, -1)
    got_k = kd.cpu().float().numpy().reshape(count, kvw)
    got_v = vd.cpu().float().numpy().reshape(count, kvw)
    keep = []
    L = oracle.make_layer(oracle_spec(spec), host, keep)
    for i in range(tokens):
        p = first + i
        kr = keys16.astype(np.float32).copy()
        vr = vals16.astype(np.float32).copy()
        kr[first:p], vr[first:p] = got_k[first:p], got_v[first:p]
        xr = x.reshape(tokens, -1)[i].copy()
        _, parts = l64.layer64(oracle_spec(spec), host, xr, kr[:p + 1].astype(np.float64).copy(),
                               vr[:p + 1].astype(np.float64).copy(), p, p, parts=True)
        kr, vr = kr.reshape(-1), vr.reshape(-1)
        oracle.layer_step(L, xr, kr, vr, p, p, f16_store=True, threads=8)
        assert_layer_close(got_x[i], xr, l64.layer_bound(parts), f"{name} token {i}:")
        assert np.allclose(got_k[p], kr.reshape(count, kvw)[p], rtol=2e-3, atol=1e-3)


def test_layer_refuses_partial_families():
    """block.mojo:116 LayerWeights.check: two of three biases, a q norm
    without a k norm, an unknown activation are refused before launch."""
    from molla_amd._lib import MiError
    spec, host = family_host("qwen2", spec_of(256, 512, 4, 2, 64), 5)
    ctx = gpu.DeviceContext(0)
    bs, layer = device_family_layer(spec, host)
    x = torch.zeros(bs.width, device="cuda")
    k = torch.zeros(4 * bs.kv_width(), dtype=torch.float16, device="cuda")
    posd = torch.zeros(1, dtype=torch.int32, device="cuda")
    layer.desc.v_bias = None
    with pytest.raises(MiError, match="biases"):
        block.device_layer(ctx, layer, x, k, k.clone(), 4 * bs.kv_width(), posd, 4, 1)
    spec3, host3 = family_host("qwen3", spec_of(256, 512, 4, 2, 64), 5)
    bs3, layer3 = device_family_layer(spec3, host3)
    layer3.desc.k_norm = None
    with pytest.raises(MiError, match="norms"):
        block.device_layer(ctx, layer3, x, k, k.clone(), 4 * bs.kv_width(), posd, 4, 1)
    layer3.desc.k_norm = layer3.extras["k_norm"].data_ptr()
    layer3.desc.act = 3
    with pytest.raises(MiError, match="act"):
        block.device_layer(ctx, layer3, x, k, k.clone(), 4 * bs.kv_width(), posd, 4, 1)
