"""Config 5 at its real size: the synthetic 8B decode step against the oracle.

32 Q4_K layers of width 4096 (32 query / 8 key heads of 128, MLP 14336), a
Q6_K head over 128256 tokens and an f32 embedding, built on the device from
the benchmark's seeds (block.synthetic_model).  A 16-token prompt goes
through the prefill layer in one chunk; then three greedy steps.  Checks
(tests/test_gpu_block.mojo:1407-1416's gate):

* batch 1: the logits after the prompt and after each greedy step within
  2e-3 of their peak of oracle.forward (model.mojo:178) run token by token
  over the same weights (copied back to the host), with identical picks;
* batch 4 and 8 (different prompts): each sequence's logits within the same
  gate of its own batch-1 run, with identical picks;
* the step replayed from a captured HIP graph equal to the eager step, bit
  for bit, at batch 1, 4 and 8.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from molla_amd import block, gpu, synth

pytestmark = pytest.mark.gpu

VOCAB, PROMPT, STEPS = 128256, 16, 3
THREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def model8b():
    spec = block.BlockSpec()
    model = block.synthetic_model(spec, 32, VOCAB, device="cuda")
    torch.cuda.synchronize()
    return model


def _host_oracle_model(model):
    """The same weights as the oracle takes them (host copies)."""
    s = model.spec
    ospec = dict(width=s.width, hidden=s.hidden, heads=s.heads, kv_heads=s.kv_heads, head_dim=s.head_dim,
                 rope_dim=s.rope_dim, neox=int(s.neox), eps=s.eps, rope_base=s.rope_base, attn_scale=s.attn_scale)
    keep, layers = [], []
    for layer in model.layers:
        w = {n: (t.kind, t.rows, t.cols, t.keep.cpu().numpy()) for n, t in layer.weights.items()}
        w["attn_norm"] = layer.attn_norm.cpu().numpy()
        w["ffn_norm"] = layer.ffn_norm.cpu().numpy()
        layers.append(oracle.make_layer(ospec, w, keep))
    head = (model.output.kind, model.output.rows, model.output.cols, model.output.keep.cpu().numpy())
    return layers, model.embedding.cpu().numpy(), model.output_norm.cpu().numpy(), head, keep


def _prompts(batch):
    return synth.tokens(PROMPT * batch, VOCAB, 1234).numpy().reshape(batch, PROMPT)


def _run(model, prompts, graph=False):
    """Prefill each sequence's prompt, then STEPS greedy steps: the logits
    and picks after the prompt and after every step, [STEPS + 1][batch]."""
    batch = prompts.shape[0]
    stream = torch.cuda.Stream()
    ctx = gpu.DeviceContext(0, stream=stream)
    logits, picks = [], []
    with torch.cuda.stream(stream):
        sess = block.DeviceSession(ctx, model, batch=batch, context=PROMPT + STEPS + 2)
        for b in range(batch):
            sess.prefill(torch.from_numpy(prompts[b].copy()).cuda(), seq=b, start=0, chunk=PROMPT)
        sess.finish()
        stream.synchronize()
        logits.append(sess.logits.view(batch, -1).cpu().numpy().copy())
        picks.append(sess.picks.cpu().numpy().copy())
        sess.ids.copy_(sess.picks)
        g = None
        for i in range(STEPS):
            if graph and i == 1:
                g = sess.capture(advance=True)  # step 0 ran eagerly: every kernel is loaded
            if g is not None:
                g.replay()
            else:
                sess.step()
                sess.advance()
            stream.synchronize()
            logits.append(sess.logits.view(batch, -1).cpu().numpy().copy())
            picks.append(sess.picks.cpu().numpy().copy())
        del g
    return logits, picks


def _close(got, want):
    err = np.abs(got.astype(np.float64) - want).max()
    return err, err <= 2e-3 * np.abs(want).max()


def test_8b_batch1_matches_oracle(model8b):
    prompts = _prompts(1)
    logits, picks = _run(model8b, prompts)
    layers, emb, onorm, head, keep = _host_oracle_model(model8b)
    kvw = model8b.spec.kv_width()
    ctxlen = PROMPT + STEPS + 1
    keys = [np.zeros(ctxlen * kvw, np.float32) for _ in layers]
    values = [np.zeros(ctxlen * kvw, np.float32) for _ in layers]
    for p in range(PROMPT):
        want = oracle.forward(layers, emb, onorm, head, int(prompts[0, p]), p, p, keys, values, f16_store=True,
                              threads=THREADS)
    for i in range(STEPS + 1):
        err, ok = _close(logits[i][0], want)
        top2 = np.sort(want)[-2:]
        print(f"step {i}: max |dlogit| {err:.3e} peak {np.abs(want).max():.3e} pick {picks[i][0]} "
              f"oracle {oracle.argmax(want)} top-2 margin {top2[1] - top2[0]:.3e}", flush=True)
        assert ok, i
        assert int(picks[i][0]) == oracle.argmax(want), i
        if i < STEPS:
            p = PROMPT + i
            want = oracle.forward(layers, emb, onorm, head, int(picks[i][0]), p, p, keys, values, f16_store=True,
                                  threads=THREADS)


@pytest.mark.parametrize("batch", [4, 8])
def test_8b_batch_matches_batch1(model8b, batch):
    # batch 4: int8 gate|up tile; batch 8: the f16 GLU tile; both run q|k|v
    # with rope and down (split over K) on the f16 tile
    prompts = _prompts(batch)
    logits4, picks4 = _run(model8b, prompts)
    for b in range(batch):
        logits1, picks1 = _run(model8b, prompts[b:b + 1])
        for i in range(STEPS + 1):
            err, ok = _close(logits4[i][b], logits1[i][0])
            print(f"seq {b} step {i}: max |dlogit| batch {batch} vs 1 {err:.3e} picks {picks4[i][b]} {picks1[i][0]}",
                  flush=True)
            assert ok, (b, i)
            assert picks4[i][b] == picks1[i][0], (b, i)


@pytest.mark.parametrize("batch", [1, 4, 8])
def test_8b_graph_replay_matches_eager(model8b, batch):
    prompts = _prompts(batch)
    eager_logits, eager_picks = _run(model8b, prompts)
    graph_logits, graph_picks = _run(model8b, prompts, graph=True)
    for i in range(STEPS + 1):
        assert np.array_equal(graph_logits[i], eager_logits[i]), i
        assert np.array_equal(graph_picks[i], eager_picks[i]), i
