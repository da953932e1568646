"""mi_matvec_noalloc (no counterpart in the reference): mi_matvec with its
workspace in the library's static per-device scratch, for callers that
cannot allocate.  Through the C ABI, against mi_matvec with a caller
workspace of the same size on the same inputs: bit for bit at every size
(both run the same kernels on the same arithmetic, with the same split-K
choice), on two calls in a row, the second with a
smaller input (the scratch keeps the first call's contents), at batch 1, a
batched decode and a prefill chunk; and a shape whose workspace is above the
static size is refused before any launch."""

import numpy as np
import pytest
import torch

from molla_amd import gpu, synth
from molla_amd._lib import MiError, check, lib

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 32 << 20


def _run_pair(ctx, kind, rows, cols, tokens, seed, epi=0, aux=None):
    L = lib()
    blob = synth.quant_tensor(kind, rows, cols, seed, device="cuda")
    rb = gpu.row_bytes(kind, cols)
    x = synth.normal(tokens * cols, seed + 1, device="cuda")
    want = torch.full((tokens * rows,), 7.0, device="cuda")
    got = torch.full((tokens * rows,), 7.0, device="cuda")
    # the same workspace budget as the static scratch, so a prefill chunk
    # splits its reduction the same way
    need = max(L.mi_matvec_workspace(cols, tokens), NOALLOC_BYTES)
    work = torch.empty(need, dtype=torch.uint8, device="cuda")
    ap = None if aux is None else aux.data_ptr()
    check(L.mi_matvec(ctx.handle, kind, blob.data_ptr(), rb, rows, cols, x.data_ptr(), tokens, want.data_ptr(),
                      epi, ap, work.data_ptr(), need))
    check(L.mi_matvec_noalloc(ctx.handle, kind, blob.data_ptr(), rb, rows, cols, x.data_ptr(), tokens,
                              got.data_ptr(), epi, ap))
    ctx.synchronize()
    return want.cpu().numpy(), got.cpu().numpy()


@pytest.mark.parametrize("calls", [
    [(gpu.Q_Q4_K, 14336, 4096, 1), (gpu.Q_Q4_K, 4096, 4096, 1)],
    [(gpu.Q_Q6_K, 4096, 14336, 4), (gpu.Q_Q8_0, 1024, 896, 2)],
    [(gpu.Q_Q4_K, 4096, 4096, 256), (gpu.Q_Q4_0, 1024, 2048, 40)],
])
def test_noalloc_matches_matvec(calls):
    ctx = gpu.DeviceContext(0)
    for i, (kind, rows, cols, tokens) in enumerate(calls):
        want, got = _run_pair(ctx, kind, rows, cols, tokens, 100 + i)
        print(f"kind {kind} {rows}x{cols} tokens {tokens}: equal {np.array_equal(want, got)}", flush=True)
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32))


def test_noalloc_epilogue():
    ctx = gpu.DeviceContext(0)
    rows, cols = 2048, 4096
    aux = synth.normal(rows, 9, device="cuda")
    want, got = _run_pair(ctx, gpu.Q_Q4_K, rows, cols, 1, 300, epi=gpu.EPI_GLU, aux=aux)
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))


def test_noalloc_refuses_beyond_its_scratch():
    ctx = gpu.DeviceContext(0)
    L = lib()
    cols, tokens = 8192, 2048  # a workspace of 64 MiB
    assert L.mi_matvec_workspace(cols, tokens) > NOALLOC_BYTES
    blob = synth.quant_tensor(gpu.Q_Q4_K, 256, cols, 1, device="cuda")
    x = torch.zeros(tokens * cols, device="cuda")
    y = torch.zeros(tokens * 256, device="cuda")
    with pytest.raises(MiError, match="static"):
        check(L.mi_matvec_noalloc(ctx.handle, gpu.Q_Q4_K, blob.data_ptr(), gpu.row_bytes(gpu.Q_Q4_K, cols), 256,
                                  cols, x.data_ptr(), tokens, y.data_ptr(), 0, None))


@pytest.mark.parametrize("kind,rows,cols,tokens", [(gpu.Q_Q4_K, 4096, 4096, 1), (gpu.Q_Q4_K, 4096, 4096, 4)])
def test_noalloc_under_graph_capture(kind, rows, cols, tokens):
    """The use the entry point is for: after a first eager call on the device
    (which resolves the scratch address), calls captured in a HIP graph;
    every replay, with eager work and synchronizations between them, equals
    the eager result bit for bit."""
    L = lib()
    ctx = gpu.DeviceContext(0)
    blob = synth.quant_tensor(kind, rows, cols, 77, device="cuda")
    rb = gpu.row_bytes(kind, cols)
    x = synth.normal(tokens * cols, 78, device="cuda")
    want = torch.empty(tokens * rows, device="cuda")
    check(L.mi_matvec_noalloc(ctx.handle, kind, blob.data_ptr(), rb, rows, cols, x.data_ptr(), tokens,
                              want.data_ptr(), 0, None))
    ctx.synchronize()
    stream = torch.cuda.Stream()
    sctx = gpu.DeviceContext(0, stream=stream)
    got = torch.full((tokens * rows,), 7.0, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        check(L.mi_matvec_noalloc(sctx.handle, kind, blob.data_ptr(), rb, rows, cols, x.data_ptr(), tokens,
                                  got.data_ptr(), 0, None))
    for r in range(3):
        got.fill_(7.0)
        # eager work on the same scratch between replays
        other = torch.empty(tokens * rows, device="cuda")
        check(L.mi_matvec_noalloc(ctx.handle, kind, blob.data_ptr(), rb, rows, cols, x.data_ptr(), tokens,
                                  other.data_ptr(), 0, None))
        ctx.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), r
