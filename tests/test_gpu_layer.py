"""GPU parity of the decoder layer and the decode step against the CPU oracle
(block.mojo:466 layer, model.mojo:178 forward), through the C ABI.

The oracle is fed the same f16-rounded cache the device holds and rounds the
freshly written key and value through f16 the way the device store does
(f16_store), so both sides attend over identical data.  Gate: every element
of the residual stream after the layer within 1e-4 of the absolute sums its
last two projections add in, sum_j |wo_ij a_j| + sum_j |down_ij h_j| (the
matvec gate, tests/test_kernel.mojo:473, carried through wo and down; the
sums come from the float64 layer in tests/layer64.py), the new cache slot
within f16 rounding, and identical greedy picks for the decode tests
(tests/test_gpu_block.mojo:1407-1416).
"""

import math

import numpy as np
import pytest
import torch

import oracle
from molla_amd import synth
from tests import layer64 as l64

pytestmark = pytest.mark.gpu


def make_layer_weights(spec, seed, kinds=None):
    """Q4_K projections (or kinds[name]) and N(1, 0.1) gains: the host dict
    the oracle and device_layer_from take."""
    kinds = kinds or {}
    W, H, qw, kvw = spec["width"], spec["hidden"], spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"]
    shapes = {"wq": (qw, W), "wk": (kvw, W), "wv": (kvw, W), "wo": (W, qw), "gate": (H, W), "up": (H, W),
              "down": (W, H)}
    host = {}
    for i, (n, (r, c)) in enumerate(shapes.items()):
        k = kinds.get(n, oracle.Q4_K)
        host[n] = (k, r, c, synth.quant_tensor(k, r, c, seed * 100 + i).numpy())
    host["attn_norm"] = synth.normal(W, seed * 100 + 10, mean=1.0, std=0.1).numpy()
    host["ffn_norm"] = synth.normal(W, seed * 100 + 11, mean=1.0, std=0.1).numpy()
    return host


def device_layer_from(host, spec):
    """(BlockSpec, DeviceLayer) holding the host dict's weights (and its
    rope_factors, when present) on the device."""
    from molla_amd import block, gpu
    bs = block.BlockSpec(width=spec["width"], hidden=spec["hidden"], heads=spec["heads"],
                         kv_heads=spec["kv_heads"], head_dim=spec["head_dim"], rope_dim=spec["rope_dim"],
                         rope_base=spec["rope_base"], neox=bool(spec["neox"]), eps=spec["eps"])
    weights = {n: gpu.Tensor.from_bytes(torch.from_numpy(host[n][3]), host[n][0], host[n][2], host[n][1])
               for n in block.DeviceLayer.NAMES}
    steps = torch.from_numpy(gpu.rope_steps(spec["rope_dim"], spec["rope_base"])).cuda()
    factors = host.get("rope_factors")
    factors = None if factors is None else torch.from_numpy(factors).cuda()
    return bs, block.DeviceLayer(bs, torch.from_numpy(host["attn_norm"]).cuda(),
                                 torch.from_numpy(host["ffn_norm"]).cuda(), weights, steps, factors)


def spec_of(width, hidden, heads, kv_heads, head_dim, base=500000.0):
    return dict(width=width, hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=head_dim, rope_dim=head_dim,
                neox=0, eps=1e-5, rope_base=base, attn_scale=float(np.float32(1 / math.sqrt(head_dim))))


def layer_gate(spec, host, x, keys16, values16, pos, stats=None):
    """Per-element tolerance of one layer's output for sequence input x over
    a cache of f16 values (keys16/values16: [pos + 1, kv_width] float32
    holding halves): tests/layer64.py layer_bound.  stats (a dict): gets the
    largest softmax weight of each head ("pmax")."""
    k = np.asarray(keys16, np.float64).reshape(pos + 1, -1).copy()
    v = np.asarray(values16, np.float64).reshape(pos + 1, -1).copy()
    _, parts = l64.layer64(spec, host, x, k, v, pos, pos, parts=True)
    if stats is not None:
        stats["pmax"] = parts["pmax"]
    return l64.layer_bound(parts)


def assert_layer_close(got, want, bound, what=""):
    err = np.abs(np.asarray(got, np.float64) - want)
    ratio = float((err / bound).max())
    print(f"{what} max |dx| {err.max():.3e} (peak {np.abs(want).max():.3e}); "
          f"max |dx| / bound {ratio:.3e}", flush=True)
    assert ratio <= 1.0


def llama31_factors(pairs):
    """Per-pair rope factors shaped like a Llama 3.1 file's rope_freqs.weight:
    1 for the fast pairs, rising to 8 for the slow ones."""
    return np.concatenate([np.ones(pairs - pairs // 2), np.linspace(1.5, 8.0, pairs // 2)]).astype(np.float32)


@pytest.mark.parametrize("dims,pos,tokens,factors", [
    ((256, 512, 4, 2, 64), 0, 1, False),
    ((256, 512, 4, 2, 64), 37, 1, False),
    ((256, 512, 4, 2, 64), 37, 1, True),
    ((512, 1024, 8, 2, 64), 300, 3, False),
    ((512, 1024, 8, 2, 64), 300, 3, True),
    # 5 tokens: gate|up on the f16 tile (one-wave blocks at 512 columns, an
    # odd token count for its per-token quantize)
    ((512, 1024, 8, 2, 64), 300, 5, False),
    ((4096, 14336, 32, 8, 128), 4096, 1, False),   # config 4
    # an MLP of 8192: at 4+ tokens the batched down projection runs on the f16
    # tile split over two 4096-column parts (the GLU tile writes its hx form)
    ((1024, 8192, 8, 2, 128), 200, 4, False),
    ((1024, 8192, 8, 2, 128), 200, 8, False),
    # an MLP of 14336: four 3584-column parts, from the f16 GLU tile
    ((1024, 14336, 8, 2, 128), 200, 4, False),
    ((1024, 14336, 8, 2, 128), 200, 6, False),
    # a width of 768 (not a multiple of 512): gate|up on the int8 GLU tile,
    # which then also writes the hx form for down's f16 split
    ((768, 8192, 12, 3, 64), 150, 4, False),
    # full multi-head attention: a q|k|v of 12288 rows is more 24-row groups
    # than CUs, so the folded-norm q|k|v kernel loops (rope step and factor
    # reloaded per group)
    ((4096, 1024, 32, 32, 128), 50, 1, False),
    ((4096, 1024, 32, 32, 128), 50, 1, True),
])
def test_layer_matches_oracle(dims, pos, tokens, factors):
    _layer_vs_oracle(dims, pos, tokens, factors)


@pytest.mark.parametrize("tokens", [4, 8])
def test_batched_config_layer_spread_softmax(tokens):
    """Config 4's shape at 4 and 8 tokens with the attention norm's gain
    scaled by 0.003: q and k elements below one, scores of order one, so
    the batched attention (the 512-thread slice kernel) and the q|k|v tile's
    rope epilogue are checked where the softmax spreads over many keys (with
    N(1, 0.1) gains the scores reach thousands and one key takes all)."""
    _layer_vs_oracle((4096, 14336, 32, 8, 128), 300, tokens, False, attn_gain=0.003)


def _layer_vs_oracle(dims, pos, tokens, factors, attn_gain=1.0):
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(*dims)
    host = make_layer_weights(spec, 7)
    if factors:
        host["rope_factors"] = llama31_factors(spec["rope_dim"] // 2)
    if attn_gain != 1.0:
        host["attn_norm"] = (host["attn_norm"] * attn_gain).astype(np.float32)
    bs, layer = device_layer_from(host, spec)
    kvw = bs.kv_width()
    count = pos + 1
    cache_stride = count * kvw
    keys16 = synth.normal(tokens * cache_stride, 40).half()
    vals16 = synth.normal(tokens * cache_stride, 41).half()
    x = synth.normal(tokens * bs.width, 42).numpy()
    # device
    kd, vd = keys16.clone().cuda(), vals16.clone().cuda()
    xd = torch.from_numpy(x.copy()).cuda()
    posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")
    block.device_layer(ctx, layer, xd, kd, vd, cache_stride, posd, count, tokens)
    ctx.synchronize()
    got_x = xd.cpu().numpy().reshape(tokens, -1)
    got_k = kd.cpu().float().numpy().reshape(tokens, count, kvw)
    got_v = vd.cpu().float().numpy().reshape(tokens, count, kvw)
    # oracle, per sequence
    keep = []
    L = oracle.make_layer(spec, host, keep)
    spread = []
    for t in range(tokens):
        xr = x.reshape(tokens, -1)[t].copy()
        kr = keys16.float().numpy().reshape(tokens, -1)[t].copy()
        vr = vals16.float().numpy().reshape(tokens, -1)[t].copy()
        stats = {}
        bound = layer_gate(spec, host, xr, kr, vr, pos, stats)
        pm = np.array(stats["pmax"])
        print(f"seq {t}: largest softmax weight per head: median {np.median(pm):.3e}, max {pm.max():.3e}",
              flush=True)
        spread.extend(pm.tolist())
        oracle.layer_step(L, xr, kr, vr, pos, pos, f16_store=True, threads=8)
        assert_layer_close(got_x[t], xr, bound, f"seq {t}:")
        # earlier slots untouched, new slot within one f16 ulp of the oracle's rounding
        kr = kr.reshape(count, kvw)
        vr = vr.reshape(count, kvw)
        assert (got_k[t, :pos] == kr[:pos]).all() and (got_v[t, :pos] == vr[:pos]).all()
        assert np.allclose(got_k[t, pos], kr[pos], rtol=2e-3, atol=1e-3)
        assert np.allclose(got_v[t, pos], vr[pos], rtol=2e-3, atol=1e-3)
    if attn_gain != 1.0:
        # the point of the case: most heads spread their softmax over many keys
        assert np.median(spread) < 0.5, np.median(spread)


@pytest.mark.parametrize("tokens", [1, 4, 8])
def test_layer_q4_k_m_kinds_match_oracle(tokens):
    """The kinds of a Q4_K_M file: attn_v and ffn_down in Q6_K (the f16
    tile's split over K takes the Q6_K down at 4 and 8 tokens)."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(1024, 14336, 8, 2, 128)
    host = make_layer_weights(spec, 9, {"wv": oracle.Q6_K, "down": oracle.Q6_K})
    bs, layer = device_layer_from(host, spec)
    kvw = bs.kv_width()
    pos = 120
    count = pos + 1
    cache_stride = count * kvw
    keys16 = synth.normal(tokens * cache_stride, 43).half()
    vals16 = synth.normal(tokens * cache_stride, 44).half()
    x = synth.normal(tokens * bs.width, 45).numpy()
    kd, vd = keys16.clone().cuda(), vals16.clone().cuda()
    xd = torch.from_numpy(x.copy()).cuda()
    posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")
    block.device_layer(ctx, layer, xd, kd, vd, cache_stride, posd, count, tokens)
    ctx.synchronize()
    got_x = xd.cpu().numpy().reshape(tokens, -1)
    keep = []
    L = oracle.make_layer(spec, host, keep)
    for t in range(tokens):
        xr = x.reshape(tokens, -1)[t].copy()
        kr = keys16.float().numpy().reshape(tokens, -1)[t].copy()
        vr = vals16.float().numpy().reshape(tokens, -1)[t].copy()
        bound = layer_gate(spec, host, xr, kr, vr, pos)
        oracle.layer_step(L, xr, kr, vr, pos, pos, f16_store=True, threads=8)
        assert_layer_close(got_x[t], xr, bound, f"seq {t}:")


def test_layer_unaligned_residual_runs_separate_norms():
    """A residual row that is not 16-byte aligned makes the batch-1 layer run
    both norms as launches of their own (the kernels with the norm folded in
    load the row as float4): both calls within the oracle's per-element
    bound, and within it of each other (the folded kernels scale each row's
    sum by the norm's scale rather than the activation, so the two round
    differently)."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(512, 1024, 8, 2, 64)
    host = make_layer_weights(spec, 9)
    bs, layer = device_layer_from(host, spec)
    kvw, pos = bs.kv_width(), 300
    count = pos + 1
    keys16 = synth.normal(count * kvw, 43).half()
    vals16 = synth.normal(count * kvw, 44).half()
    x = synth.normal(bs.width, 45).numpy()
    posd = torch.full((1,), pos, dtype=torch.int32, device="cuda")
    outs = []
    for offset in (0, 1):
        buf = torch.zeros(bs.width + 4, device="cuda")
        xd = buf[offset:offset + bs.width]
        xd.copy_(torch.from_numpy(x))
        assert (xd.data_ptr() % 16 != 0) == (offset == 1)
        kd, vd = keys16.clone().cuda(), vals16.clone().cuda()
        block.device_layer(ctx, layer, xd, kd, vd, count * kvw, posd, count, 1)
        ctx.synchronize()
        outs.append((xd.cpu().numpy().astype(np.float64), kd.cpu().float().numpy(), vd.cpu().float().numpy()))
    xr = x.copy()
    kr = keys16.float().numpy().copy()
    vr = vals16.float().numpy().copy()
    keep = []
    bound = layer_gate(spec, host, xr, kr, vr, pos)
    oracle.layer_step(oracle.make_layer(spec, host, keep), xr, kr, vr, pos, pos, f16_store=True, threads=8)
    for got_x, got_k, got_v in outs:
        assert_layer_close(got_x, xr, bound)
        assert np.allclose(got_k, kr, rtol=2e-3, atol=1e-3) and np.allclose(got_v, vr, rtol=2e-3, atol=1e-3)
    assert_layer_close(outs[0][0], outs[1][0], bound)


def test_small_model_greedy_decode_matches_oracle():
    """A 2-layer model decodes 12 tokens greedily; every logit row within
    2e-3 of the peak and every pick identical (tests/test_gpu_block.mojo:1407)."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(256, 512, 4, 2, 64, base=10000.0)
    vocab, n_layers, steps = 1000, 2, 12
    hosts = [make_layer_weights(spec, 20 + i) for i in range(n_layers)]
    emb = synth.normal(vocab * spec["width"], 50).numpy().reshape(vocab, spec["width"])
    onorm = synth.normal(spec["width"], 51, mean=1.0, std=0.1).numpy()
    head = synth.quant_tensor(oracle.Q6_K, vocab, spec["width"], 52).numpy()
    layers = [device_layer_from(h, spec)[1] for h in hosts]
    bs = layers[0].spec
    model = block.DeviceModel(bs, torch.from_numpy(emb).cuda(), layers, torch.from_numpy(onorm).cuda(),
                              gpu.Tensor.from_bytes(torch.from_numpy(head), oracle.Q6_K, spec["width"], vocab))
    sess = block.DeviceSession(ctx, model, batch=1, context=steps + 1)
    keep = []
    ol = [oracle.make_layer(spec, h, keep) for h in hosts]
    kvw = bs.kv_width()
    ok = [np.zeros((steps + 1) * kvw, np.float32) for _ in range(n_layers)]
    ov = [np.zeros((steps + 1) * kvw, np.float32) for _ in range(n_layers)]
    token = 7
    sess.ids.fill_(token)
    sess.pos.zero_()
    for p in range(steps):
        sess.step()
        ctx.synchronize()
        logits = sess.logits.cpu().numpy()
        pick = int(sess.picks.cpu().numpy()[0])
        want = oracle.forward(ol, emb, onorm, (oracle.Q6_K, vocab, spec["width"], head), token, p, p, ok, ov,
                              f16_store=True)
        assert np.abs(logits - want).max() <= 2e-3 * np.abs(want).max()
        assert pick == oracle.argmax(want), p
        token = pick
        sess.advance()


def test_session_prefill_matches_oracle():
    """A prompt fed in chunks (DeviceSession.prefill: 16-token chunks through
    the prefill layer, two sequences of different prompts) leaves the model
    where the oracle's token-by-token forward leaves it: the next-token logits
    within 2e-3 of the peak with the same pick, and greedy decode continuing
    from there picking what the oracle picks (tests/test_gpu_block.mojo:1407
    gate)."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(256, 512, 4, 2, 64, base=10000.0)
    vocab, n_layers, plen, gen = 1000, 2, 40, 4
    hosts = [make_layer_weights(spec, 60 + i) for i in range(n_layers)]
    emb = synth.normal(vocab * spec["width"], 70).numpy().reshape(vocab, spec["width"])
    onorm = synth.normal(spec["width"], 71, mean=1.0, std=0.1).numpy()
    head = synth.quant_tensor(oracle.Q6_K, vocab, spec["width"], 72).numpy()
    layers = [device_layer_from(h, spec)[1] for h in hosts]
    bs = layers[0].spec
    model = block.DeviceModel(bs, torch.from_numpy(emb).cuda(), layers, torch.from_numpy(onorm).cuda(),
                              gpu.Tensor.from_bytes(torch.from_numpy(head), oracle.Q6_K, spec["width"], vocab))
    batch, context = 2, plen + gen + 1
    sess = block.DeviceSession(ctx, model, batch=batch, context=context)
    rng = np.random.default_rng(73)
    prompts = rng.integers(0, vocab, size=(batch, plen)).astype(np.int32)
    for b in range(batch):
        sess.prefill(torch.from_numpy(prompts[b]).cuda(), seq=b, start=0, chunk=16)
    sess.finish()
    ctx.synchronize()
    keep = []
    ol = [oracle.make_layer(spec, h, keep) for h in hosts]
    kvw = bs.kv_width()
    hd = (oracle.Q6_K, vocab, spec["width"], head)
    for b in range(batch):
        ok = [np.zeros(context * kvw, np.float32) for _ in range(n_layers)]
        ov = [np.zeros(context * kvw, np.float32) for _ in range(n_layers)]
        for p in range(plen):
            want = oracle.forward(ol, emb, onorm, hd, int(prompts[b, p]), p, p, ok, ov, f16_store=True)
        got = sess.logits.cpu().numpy().reshape(batch, vocab)[b]
        assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max(), b
        assert int(sess.picks.cpu().numpy()[b]) == oracle.argmax(want), b
    # decode on from the prefilled caches: the first sequence against the oracle
    ok = [np.zeros(context * kvw, np.float32) for _ in range(n_layers)]
    ov = [np.zeros(context * kvw, np.float32) for _ in range(n_layers)]
    for p in range(plen):
        want = oracle.forward(ol, emb, onorm, hd, int(prompts[0, p]), p, p, ok, ov, f16_store=True)
    token = oracle.argmax(want)
    sess.ids.copy_(sess.picks)
    for p in range(plen, plen + gen):
        sess.step()
        ctx.synchronize()
        want = oracle.forward(ol, emb, onorm, hd, token, p, p, ok, ov, f16_store=True)
        got = sess.logits.cpu().numpy().reshape(batch, vocab)[0]
        assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max(), p
        pick = int(sess.picks.cpu().numpy()[0])
        assert pick == oracle.argmax(want), p
        token = pick
        sess.advance()


def test_graph_replay_matches_eager():
    """The decode step captured as a HIP graph (DeviceSession.capture) gives
    the eager step's logits and picks bit for bit, on every replay, with
    eager work and synchronizations between the replays."""
    from molla_amd import block, gpu
    stream = torch.cuda.Stream()
    ctx = gpu.DeviceContext(0, stream=stream)
    spec = spec_of(256, 512, 4, 2, 64, base=10000.0)
    vocab, n_layers, steps = 1000, 2, 10
    hosts = [make_layer_weights(spec, 40 + i) for i in range(n_layers)]
    emb = synth.normal(vocab * spec["width"], 60).numpy().reshape(vocab, spec["width"])
    onorm = synth.normal(spec["width"], 61, mean=1.0, std=0.1).numpy()
    head = synth.quant_tensor(oracle.Q6_K, vocab, spec["width"], 62).numpy()
    layers = [device_layer_from(h, spec)[1] for h in hosts]
    model = block.DeviceModel(layers[0].spec, torch.from_numpy(emb).cuda(), layers, torch.from_numpy(onorm).cuda(),
                              gpu.Tensor.from_bytes(torch.from_numpy(head), oracle.Q6_K, spec["width"], vocab))
    with torch.cuda.stream(stream):
        eager = block.DeviceSession(ctx, model, batch=2, context=steps + 2)
        graphed = block.DeviceSession(ctx, model, batch=2, context=steps + 2)
        for s in (eager, graphed):
            s.ids.copy_(torch.tensor([7, 11], dtype=torch.int32, device="cuda"))
            s.pos.zero_()
        want_logits, want_picks = [], []
        for _ in range(steps):
            eager.step()
            want_logits.append(eager.logits.clone())
            want_picks.append(eager.picks.clone())
            eager.advance()
        graphed.step()  # eager first position: every kernel loaded before capture
        assert torch.equal(graphed.logits, want_logits[0])
        graphed.advance()
        g = graphed.capture()
        for p in range(1, steps):
            g.replay()
            stream.synchronize()
            got_logits = graphed.logits.clone()
            assert torch.equal(got_logits, want_logits[p]), p
            assert torch.equal(graphed.picks, want_picks[p]), p
            # unrelated eager work between replays
            torch.randn(4096, device="cuda").sum().item()
        assert graphed.pos.cpu().tolist() == [steps, steps]


@pytest.mark.parametrize("dims,pos,tokens", [
    ((256, 512, 4, 2, 64), 37, 1),
    ((512, 1024, 8, 2, 64), 300, 3),
    ((4096, 14336, 32, 8, 128), 2048, 1),
])
def test_layer_q8_cache_matches_oracle(dims, pos, tokens):
    """The layer over a q8_0 KV cache (repack.mojo:181 CACHE_Q8): the residual
    within the layer gate of the oracle attending over the values the cache
    holds, earlier slots untouched, the new slot within one quant step of the
    oracle's q8-rounded key and value."""
    from molla_amd import block, gpu
    from tests.test_gpu_kernels import q8_decode, q8_rows
    ctx = gpu.DeviceContext(0)
    spec = spec_of(*dims)
    host = make_layer_weights(spec, 9)
    bs, layer = device_layer_from(host, spec)
    kvw = bs.kv_width()
    row = gpu.cache_row(gpu.CACHE_Q8, kvw)
    count = pos + 1
    cache_stride = count * row
    raw_k = synth.normal(tokens * count * kvw, 50).numpy()
    raw_v = synth.normal(tokens * count * kvw, 51).numpy()
    kh = np.concatenate([q8_rows(raw_k.reshape(tokens, -1)[t], kvw) for t in range(tokens)])
    vh = np.concatenate([q8_rows(raw_v.reshape(tokens, -1)[t], kvw) for t in range(tokens)])
    x = synth.normal(tokens * bs.width, 52).numpy()
    kd = torch.from_numpy(kh.view(np.int16).copy()).view(torch.float16).cuda()
    vd = torch.from_numpy(vh.view(np.int16).copy()).view(torch.float16).cuda()
    xd = torch.from_numpy(x.copy()).cuda()
    posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")
    block.device_layer(ctx, layer, xd, kd, vd, cache_stride, posd, count, tokens, form=gpu.CACHE_Q8)
    ctx.synchronize()
    got_x = xd.cpu().numpy().reshape(tokens, -1)
    got_kh = kd.cpu().view(torch.int16).numpy().view(np.uint16).reshape(tokens, -1)
    got_vh = vd.cpu().view(torch.int16).numpy().view(np.uint16).reshape(tokens, -1)
    keep = []
    L = oracle.make_layer(spec, host, keep)
    for t in range(tokens):
        kr = q8_decode(kh.reshape(tokens, -1)[t], kvw, count).reshape(-1).copy()
        vr = q8_decode(vh.reshape(tokens, -1)[t], kvw, count).reshape(-1).copy()
        xr = x.reshape(tokens, -1)[t].copy()
        bound = layer_gate(spec, host, xr, kr, vr, pos)
        oracle.layer_step(L, xr, kr, vr, pos, pos, q8_store=True, threads=8)
        assert_layer_close(got_x[t], xr, bound, f"seq {t}:")
        old = slice(0, pos * row)
        assert np.array_equal(got_kh[t][old], kh.reshape(tokens, -1)[t][old])
        assert np.array_equal(got_vh[t][old], vh.reshape(tokens, -1)[t][old])
        gk = q8_decode(got_kh[t], kvw, count)[pos]
        gv = q8_decode(got_vh[t], kvw, count)[pos]
        wk, wv = kr.reshape(count, kvw)[pos], vr.reshape(count, kvw)[pos]
        for got, want in ((gk, wk), (gv, wv)):
            step = np.repeat(np.abs(want).reshape(-1, 32).max(axis=1) / 127, 32) * 1.01 + 1e-7
            assert (np.abs(got - want) <= step).all()


def paged_from_contiguous(caches, count, row, tokens, extra, seed):
    """A pool holding the rows of per-sequence caches (uint16 [tokens, count *
    row]) in shuffled cells, and the index [tokens, count] of each position's
    cell."""
    rng = np.random.default_rng(seed)
    cells = rng.permutation(tokens * count + extra)[: tokens * count].reshape(tokens, count).astype(np.int32)
    pool = np.zeros(((tokens * count + extra) * row,), np.uint16)
    for t in range(tokens):
        for j in range(count):
            pool[cells[t, j] * row:(cells[t, j] + 1) * row] = caches[t, j * row:(j + 1) * row]
    return pool, cells


@pytest.mark.parametrize("form", ["f16", "q8"])
@pytest.mark.parametrize("dims,pos,tokens", [((256, 512, 4, 2, 64), 77, 1), ((512, 1024, 8, 2, 64), 300, 3)])
def test_layer_paged_matches_contiguous(form, dims, pos, tokens, kinds=None):
    """The paged layer (cells scattered over a shared pool, gpu.mojo:571
    DevicePaging) gives the contiguous layer's residual and new cache rows
    bit for bit: only the addressing differs."""
    from molla_amd import block, gpu
    from tests.test_gpu_kernels import q8_rows
    ctx = gpu.DeviceContext(0)
    f = gpu.CACHE_Q8 if form == "q8" else gpu.CACHE_F16
    spec = spec_of(*dims)
    bs, layer = device_layer_from(make_layer_weights(spec, 11, kinds), spec)
    kvw = bs.kv_width()
    row = gpu.cache_row(f, kvw)
    count = pos + 1
    raw = [synth.normal(tokens * count * kvw, 60 + i).numpy() for i in (0, 1)]
    if f == gpu.CACHE_Q8:
        caches = [np.stack([q8_rows(r.reshape(tokens, -1)[t], kvw) for t in range(tokens)]) for r in raw]
    else:
        caches = [r.astype(np.float16).view(np.uint16).reshape(tokens, -1) for r in raw]
    x = synth.normal(tokens * bs.width, 62).numpy()
    posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16).cuda()

    kd, vd, xd = dev(caches[0]), dev(caches[1]), torch.from_numpy(x.copy()).cuda()
    block.device_layer(ctx, layer, xd, kd, vd, count * row, posd, count, tokens, form=f)
    extra = 5
    kp, cells = paged_from_contiguous(caches[0], count, row, tokens, extra, 7)
    vp, _ = paged_from_contiguous(caches[1], count, row, tokens, extra, 7)
    kpd, vpd, xpd = dev(kp), dev(vp), torch.from_numpy(x.copy()).cuda()
    idx = torch.from_numpy(cells).cuda()
    block.device_layer_paged(ctx, layer, xpd, kpd, vpd, idx, count, posd, count, tokens, form=f)
    ctx.synchronize()
    assert torch.equal(xd, xpd)
    kc = kd.cpu().view(torch.int16).numpy().reshape(tokens, -1)
    kpool = kpd.cpu().view(torch.int16).numpy()
    vc = vd.cpu().view(torch.int16).numpy().reshape(tokens, -1)
    vpool = vpd.cpu().view(torch.int16).numpy()
    for t in range(tokens):
        for j in (0, pos // 2, pos):
            c = cells[t, j]
            assert np.array_equal(kc[t, j * row:(j + 1) * row], kpool[c * row:(c + 1) * row])
            assert np.array_equal(vc[t, j * row:(j + 1) * row], vpool[c * row:(c + 1) * row])


@pytest.mark.parametrize("tokens", [3, 4])
def test_layer_paged_matches_contiguous_q4_k_m_kinds(tokens):
    """The same with a Q6_K attn_v and ffn_down: the batched q|k and v
    launches store k and v through the cell index too."""
    test_layer_paged_matches_contiguous("f16", (1024, 1024, 8, 2, 64), 300, tokens,
                                        {"wv": oracle.Q6_K, "down": oracle.Q6_K})


@pytest.mark.parametrize("kinds,tokens,width", [
    ({}, 1, 512), ({}, 4, 512), ({}, 8, 512),
    ({"wv": oracle.Q6_K, "down": oracle.Q6_K}, 1, 512),
    ({"wv": oracle.Q6_K, "down": oracle.Q6_K}, 3, 512),
    ({"wv": oracle.Q6_K, "down": oracle.Q6_K}, 4, 512),
    # width 1024 (Q6_K rows of four superblocks): the batched q|k and v
    # launches of a Q6_K attn_v
    ({"wv": oracle.Q6_K, "down": oracle.Q6_K}, 4, 1024),
    ({"wv": oracle.Q6_K}, 8, 1024),
])
def test_layer_ignores_prior_workspace_contents(kinds, tokens, width):
    """The layer reads nothing of its workspace it has not written in the
    same call: runs over workspaces filled with different bytes agree bit
    for bit."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(width, 1024, 8, 2, 64)
    bs, layer = device_layer_from(make_layer_weights(spec, 11, kinds), spec)
    kvw, pos = bs.kv_width(), 300
    count = pos + 1
    need = block.layer_workspace(layer, count, tokens)
    outs = []
    for fill in (0, 0x7F, 0x3C, 0xFF):
        k = synth.normal(tokens * count * kvw, 60).half().cuda()
        v = synth.normal(tokens * count * kvw, 61).half().cuda()
        x = synth.normal(tokens * bs.width, 62).cuda()
        posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")
        work = torch.full((need + 256,), fill, dtype=torch.uint8, device="cuda")
        block.device_layer(ctx, layer, x, k, v, count * kvw, posd, count, tokens, work=work)
        ctx.synchronize()
        outs.append((x.cpu(), k.cpu(), v.cpu()))
    for o in outs[1:]:
        assert all(torch.equal(a, b) for a, b in zip(outs[0], o))


def test_layer_paged_skips_positions_it_does_not_hold():
    """A negative cell is a position the sequence does not hold
    (gpu_ops.mojo:662 _row_of): attention leaves it out.  The oracle attends
    over the held positions only (slot = how many it holds, rope at pos)."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    spec = spec_of(256, 512, 4, 2, 64)
    host = make_layer_weights(spec, 13)
    bs, layer = device_layer_from(host, spec)
    kvw = bs.kv_width()
    pos = 90
    count = pos + 1
    held = np.ones(count, bool)
    held[[3, 10, 11, 12, 64, 65, 89]] = False  # windows trimmed out
    raw_k = synth.normal(count * kvw, 70).half().numpy().reshape(count, kvw)
    raw_v = synth.normal(count * kvw, 71).half().numpy().reshape(count, kvw)
    cells = np.full(count, -1, np.int32)
    order = np.random.default_rng(9).permutation(count + 4)
    pool_k = np.zeros(((count + 4), kvw), np.float16)
    pool_v = np.zeros(((count + 4), kvw), np.float16)
    for j in range(count):
        if held[j] or j == pos:
            cells[j] = order[j]
            pool_k[order[j]] = raw_k[j]
            pool_v[order[j]] = raw_v[j]
    x = synth.normal(bs.width, 72).numpy()
    xd = torch.from_numpy(x.copy()).cuda()
    kpd = torch.from_numpy(pool_k.reshape(-1)).cuda()
    vpd = torch.from_numpy(pool_v.reshape(-1)).cuda()
    posd = torch.tensor([pos], dtype=torch.int32, device="cuda")
    block.device_layer_paged(ctx, layer, xd, kpd, vpd, torch.from_numpy(cells).cuda(), count, posd, count, 1)
    ctx.synchronize()
    keep = []
    L = oracle.make_layer(spec, host, keep)
    kept = [j for j in range(pos) if held[j]]
    slot = len(kept)
    kr = np.zeros(((slot + 1), kvw), np.float32)
    vr = np.zeros(((slot + 1), kvw), np.float32)
    kr[:slot], vr[:slot] = raw_k[kept].astype(np.float32), raw_v[kept].astype(np.float32)
    xr = x.copy()
    kr, vr = kr.reshape(-1).copy(), vr.reshape(-1).copy()
    bound = layer_gate(spec, host, xr, kr, vr, slot)
    oracle.layer_step(L, xr, kr, vr, slot, pos, f16_store=True, threads=8)
    assert_layer_close(xd.cpu().numpy(), xr, bound)


@pytest.mark.parametrize("paged,tokens,dims", [(False, 4, (512, 1024, 8, 2, 64)), (True, 4, (512, 1024, 8, 2, 64)),
                                               (False, 40, (512, 1024, 8, 2, 64)), (True, 40, (512, 1024, 8, 2, 64)),
                                               (False, 256, (512, 1024, 8, 2, 64)),
                                               (False, 72, (1024, 1024, 8, 4, 128)),
                                               (True, 33, (512, 1024, 4, 4, 128)),
                                               (False, 48, "q4_k_m")])
def test_layer_chunk_of_one_sequence(paged, tokens, dims):
    """Stride 0: the tokens are one sequence's chunk at consecutive positions
    (gpu.mojo:617 `bases` all zero).  Each token attends over the positions up
    to its own, the chunk's earlier tokens included; the oracle runs them one
    at a time over the same cache (fed the rows the device stored for the
    chunk's earlier tokens).  Above 8 tokens the layer runs the prefill path
    (f32 activations through the prefill matmul, gpu_block.mojo:1654
    forward over a chunk)."""
    from molla_amd import block, gpu
    ctx = gpu.DeviceContext(0)
    kinds = None
    if dims == "q4_k_m":  # a Q4_K_M file's mix: v and down Q6_K (q|k one launch, v its own)
        dims, kinds = (512, 1024, 8, 2, 64), {"wv": oracle.Q6_K, "down": oracle.Q6_K, "wo": oracle.Q5_K}
    spec = spec_of(*dims)
    host = make_layer_weights(spec, 17, kinds)
    host["rope_factors"] = llama31_factors(spec["rope_dim"] // 2)
    # Attention logits of a real model's size: with N(1, 0.1) gains these
    # random Q4_K projections make q and k elements ~50 and scaled scores of
    # a few thousand, where a softmax turns f32 rounding of a score into ~1e-3
    # of a weight and only the oracle's own summation order agrees to 1e-4.
    host["attn_norm"] = (host["attn_norm"] * 0.05).astype(np.float32)
    bs, layer = device_layer_from(host, spec)
    kvw = bs.kv_width()
    first = 200
    count = first + tokens
    keys16 = synth.normal(count * kvw, 80).half().numpy().reshape(count, kvw)
    vals16 = synth.normal(count * kvw, 81).half().numpy().reshape(count, kvw)
    keys16[first:] = 0
    vals16[first:] = 0
    x = synth.normal(tokens * bs.width, 82).numpy()
    xd = torch.from_numpy(x.copy()).cuda()
    posd = torch.arange(first, count, dtype=torch.int32, device="cuda")
    if paged:
        order = np.random.default_rng(3).permutation(count + 7).astype(np.int32)[:count]
        pk = np.zeros((count + 7, kvw), np.float16)
        pv = np.zeros((count + 7, kvw), np.float16)
        pk[order], pv[order] = keys16, vals16
        kd, vd = torch.from_numpy(pk.reshape(-1)).cuda(), torch.from_numpy(pv.reshape(-1)).cuda()
        block.device_layer_paged(ctx, layer, xd, kd, vd, torch.from_numpy(order).cuda(), 0, posd, count, tokens)
        ctx.synchronize()
        got_k = kd.cpu().numpy().reshape(-1, kvw)[order].astype(np.float32)
        got_v = vd.cpu().numpy().reshape(-1, kvw)[order].astype(np.float32)
    else:
        kd, vd = torch.from_numpy(keys16.reshape(-1).copy()).cuda(), torch.from_numpy(vals16.reshape(-1).copy()).cuda()
        block.device_layer(ctx, layer, xd, kd, vd, 0, posd, count, tokens)
        ctx.synchronize()
        got_k = kd.cpu().float().numpy().reshape(count, kvw)
        got_v = vd.cpu().float().numpy().reshape(count, kvw)
    got_x = xd.cpu().numpy().reshape(tokens, -1)
    assert (got_k[:first] == keys16[:first].astype(np.float32)).all()
    keep = []
    L = oracle.make_layer(spec, host, keep)
    for i in range(tokens):
        p = first + i
        kr = keys16.astype(np.float32).copy()
        vr = vals16.astype(np.float32).copy()
        kr[first:p], vr[first:p] = got_k[first:p], got_v[first:p]
        kr, vr = kr.reshape(-1), vr.reshape(-1)
        xr = x.reshape(tokens, -1)[i].copy()
        bound = layer_gate(spec, host, xr, kr[:(p + 1) * kvw], vr[:(p + 1) * kvw], p)
        oracle.layer_step(L, xr, kr, vr, p, p, f16_store=True, threads=8)
        assert_layer_close(got_x[i], xr, bound, f"token {i}:")
        kr, vr = kr.reshape(count, kvw), vr.reshape(count, kvw)
        assert np.allclose(got_k[p], kr[p], rtol=2e-3, atol=1e-3)
        assert np.allclose(got_v[p], vr[p], rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("dims,tokens,family", [
    ((1024, 14336, 8, 2, 128), 4, None),  # down split in four parts: add and norm in one launch
    ((1024, 8192, 8, 2, 128), 8, None),   # two parts
    ((512, 1024, 8, 2, 64), 3, None),     # int8 tiles: the next norm as its own launch
    ((512, 1024, 8, 2, 64), 4, "qwen2"),  # the layer of other families: its own launches
    ((512, 1024, 8, 2, 64), 4, "gemma2"),
])
def test_chained_layers_match_unchained(dims, tokens, family):
    """Three layers chained (mi_layer_desc next_norm / prenormed: each layer
    norms its output for the next on the shared workspace) leave exactly the
    residual stream and caches of the same layers run one by one."""
    from molla_amd import block, gpu
    from molla_amd._lib import MiLayerDesc, check, lib
    import ctypes
    ctx = gpu.DeviceContext(0)
    spec = spec_of(*dims)
    if family:
        from tests.test_gpu_families import device_family_layer, family_host
        layers = [device_family_layer(*family_host(family, spec, 31 + i))[1] for i in range(3)]
    else:
        layers = [device_layer_from(make_layer_weights(spec, 11 + i), spec)[1] for i in range(3)]
    bs = block.BlockSpec(width=spec["width"], hidden=spec["hidden"], heads=spec["heads"], kv_heads=spec["kv_heads"],
                         head_dim=spec["head_dim"], rope_dim=spec["rope_dim"], rope_base=spec["rope_base"])
    kvw = bs.kv_width()
    pos = 150
    count = pos + 1
    cache_stride = count * kvw
    k0 = synth.normal(tokens * cache_stride, 50).half().cuda()
    v0 = synth.normal(tokens * cache_stride, 51).half().cuda()
    x0 = synth.normal(tokens * bs.width, 52).cuda()
    posd = torch.full((tokens,), pos, dtype=torch.int32, device="cuda")
    need = max(block.layer_workspace(l, count, tokens) for l in layers)
    L = lib()

    def run(chained):
        descs = [MiLayerDesc.from_buffer_copy(l.desc) for l in layers]
        if chained:
            block.chain_layers(descs)
        x = x0.clone()
        ks = [k0.clone() for _ in layers]
        vs = [v0.clone() for _ in layers]
        work = torch.zeros(need + 256, dtype=torch.uint8, device="cuda")
        for i, d in enumerate(descs):
            check(L.mi_decoder_layer(ctx.handle, ctypes.byref(d), x.data_ptr(), ks[i].data_ptr(), vs[i].data_ptr(),
                                     cache_stride, posd.data_ptr(), count, tokens, work.data_ptr(), work.numel()))
        ctx.synchronize()
        return x.cpu(), [k.cpu() for k in ks], [v.cpu() for v in vs]

    xa, ka, va = run(False)
    xb, kb, vb = run(True)
    assert torch.equal(xa, xb)
    assert all(torch.equal(a, b) for a, b in zip(ka + va, kb + vb))
