"""A GGUF file through molla_amd.load onto the device, decoding greedily as the
CPU oracle does on the same bytes (tests/test_gpu_block.mojo:1407-1416 gate:
every logit row within 2e-3 of its peak, every pick identical).  The files are
written by tests/gguf_writer.py with mixed kinds (Q4_K / Q6_K / Q8_0 / Q5_K /
Q4_1 / Q5_0), with and without Llama 3.1 rope frequency factors, with a
separate or a tied head."""

import numpy as np
import pytest
import torch

import oracle
from tests.gguf_writer import llama_file

pytestmark = pytest.mark.gpu


def f32(host, name):
    return np.frombuffer(host[name][1], dtype=np.float32).copy()


@pytest.mark.parametrize("tied,factors,kinds", [
    (False, True, None),
    (True, False, {"embd": oracle.Q4_K, "ffn": oracle.Q5_K, "attn_v": oracle.Q4_1, "down": oracle.Q5_0}),
])
def test_gguf_model_decodes_like_the_oracle(tmp_path, tied, factors, kinds):
    from molla_amd import block, gpu, load
    path = str(tmp_path / "m.gguf")
    host = llama_file(path, tied=tied, factors=factors, kinds=kinds)
    ctx = gpu.DeviceContext(0)
    plan, model = load.load_llama(ctx, path)
    assert plan.tied == tied and (plan.rope_factors is not None) == factors
    steps = 8
    sess = block.DeviceSession(ctx, model, batch=1, context=steps + 1)

    W, vocab = plan.width, plan.vocab
    spec = dict(width=W, hidden=plan.hidden, heads=plan.heads, kv_heads=plan.kv_heads, head_dim=plan.head_dim,
                rope_dim=plan.rope_dim, neox=0, eps=plan.eps, rope_base=plan.rope_base,
                attn_scale=model.spec.attn_scale)
    keep = []
    layers = []
    short = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    shapes = {"wq": (plan.heads * plan.head_dim, W), "wk": (plan.kv_heads * plan.head_dim, W),
              "wv": (plan.kv_heads * plan.head_dim, W), "wo": (W, plan.heads * plan.head_dim),
              "gate": (plan.hidden, W), "up": (plan.hidden, W), "down": (W, plan.hidden)}
    for i in range(plan.n_layers):
        w = {"attn_norm": f32(host, f"blk.{i}.attn_norm.weight"), "ffn_norm": f32(host, f"blk.{i}.ffn_norm.weight")}
        for n, s in short.items():
            kind, data = host[f"blk.{i}.{s}.weight"]
            w[n] = (kind, *shapes[n], np.frombuffer(data, dtype=np.uint8))
        if factors:
            w["rope_factors"] = f32(host, "rope_freqs.weight")
        layers.append(oracle.make_layer(spec, w, keep))
    ekind, edata = host["token_embd.weight"]
    emb = oracle.dequant(ekind, np.frombuffer(edata, dtype=np.uint8), vocab * W).reshape(vocab, W)
    okind, odata = host["token_embd.weight" if tied else "output.weight"]
    head = (okind, vocab, W, np.frombuffer(odata, dtype=np.uint8))
    onorm = f32(host, "output_norm.weight")
    # the device embedding table is the oracle's dequant, bit for bit
    assert np.array_equal(model.embedding.cpu().numpy().view(np.uint32), emb.astype(np.float32).view(np.uint32))

    kvw = plan.kv_heads * plan.head_dim
    ok = [np.zeros((steps + 1) * kvw, np.float32) for _ in layers]
    ov = [np.zeros((steps + 1) * kvw, np.float32) for _ in layers]
    token = 11
    sess.ids.fill_(token)
    sess.pos.zero_()
    for p in range(steps):
        sess.step()
        ctx.synchronize()
        logits = sess.logits.cpu().numpy()
        pick = int(sess.picks.cpu().numpy()[0])
        want = oracle.forward(layers, emb, onorm, head, token, p, p, ok, ov, f16_store=True)
        assert np.abs(logits - want).max() <= 2e-3 * np.abs(want).max(), p
        assert pick == oracle.argmax(want), p
        token = pick
        sess.advance()
    del sess
    # the same file prefilling a 20-token prompt in chunks of 16 (the prefill
    # layer at 16 tokens, then at 4): next-token logits and pick as the oracle
    prompt = np.array([(11 + 37 * i) % vocab for i in range(20)], dtype=np.int32)
    sess = block.DeviceSession(ctx, model, batch=1, context=len(prompt) + 1)
    sess.prefill(torch.from_numpy(prompt).cuda(), seq=0, start=0, chunk=16)
    sess.finish()
    ctx.synchronize()
    ok = [np.zeros((len(prompt) + 1) * kvw, np.float32) for _ in layers]
    ov = [np.zeros((len(prompt) + 1) * kvw, np.float32) for _ in layers]
    for p, tok in enumerate(prompt):
        want = oracle.forward(layers, emb, onorm, head, int(tok), p, p, ok, ov, f16_store=True)
    logits = sess.logits.cpu().numpy()
    assert np.abs(logits - want).max() <= 2e-3 * np.abs(want).max()
    assert int(sess.picks.cpu().numpy()[0]) == oracle.argmax(want)
    del sess
    torch.cuda.empty_cache()
