"""The prefill matmul (mi_matvec at tokens > 8: a prompt chunk, gpu.mojo:1695
PREFILL_CHUNK; the matrix-core tile of gpu.mojo:2665) against the CPU oracle.

Gate: the one every matvec here is held to (tests/test_gpu_kernels.py
assert_matvec_close): 1e-4 of each output's magnitude sum |w||x| and 1e-5 of
the peak, which is the reference's gate for its float tiles
(tests/test_gpu.mojo:255-300; its half-precision tile gets 2e-3).  Shapes
cover ragged token counts (padding inside a 32-token tile and a 64-token
block), rows that end inside a tile, widths with a partial 256-value chunk,
split-K, every epilogue, and the runs-of-eight route for widths the tile does
not take.
"""

import numpy as np
import pytest
import torch

import oracle
from molla_amd import synth
from tests.test_gpu_kernels import assert_matvec_close, dequant_abs, upload

pytestmark = pytest.mark.gpu

KINDS = [oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.Q8_0, oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1]
K_QUANTS = (oracle.Q4_K, oracle.Q5_K, oracle.Q6_K)


@pytest.fixture(scope="module")
def ctx():
    from molla_amd import gpu
    return gpu.DeviceContext(0)


def run(ctx, kind, rows, cols, tokens, seed, epi=0, aux=None, base=None):
    from molla_amd import gpu
    blob = synth.quant_tensor(kind, rows, cols, seed).numpy()
    x = synth.normal(tokens * cols, seed + 1).numpy()
    w = upload(blob, kind, cols, rows)
    out = torch.from_numpy(base.copy()) if base is not None else torch.zeros(tokens * rows, dtype=torch.float32)
    out = out.cuda()
    gpu.device_matmul_into(ctx, w, torch.from_numpy(x).cuda(), out, tokens, epi=epi,
                           aux=None if aux is None else torch.from_numpy(aux).cuda())
    ctx.synchronize()
    return blob, x, out.cpu().numpy()


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows,cols,tokens", [(200, 512, 9), (200, 512, 77), (96, 768, 256)])
def test_prefill_matches_oracle(ctx, kind, rows, cols, tokens):
    blob, x, got = run(ctx, kind, rows, cols, tokens, 300 + kind)
    want = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8)
    assert_matvec_close(got, want, dequant_abs(kind, blob, rows, cols), x)


@pytest.mark.parametrize("kind", [oracle.Q8_0, oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1])
def test_prefill_partial_chunk(ctx, kind):
    """320 values: the last 256-value chunk holds two blocks (the min term's
    empty slots, the stage walk stopping inside a chunk)."""
    rows, cols, tokens = 70, 320, 40
    blob, x, got = run(ctx, kind, rows, cols, tokens, 400 + kind)
    want = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8)
    assert_matvec_close(got, want, dequant_abs(kind, blob, rows, cols), x)


@pytest.mark.parametrize("kind", [oracle.Q4_K, oracle.Q6_K, oracle.Q4_1])
def test_prefill_split_k(ctx, kind):
    """Few output tiles over a long reduction: K splits across blocks and the
    partial sums are added in split order."""
    rows, cols, tokens = 64, 4096, 64
    blob, x, got = run(ctx, kind, rows, cols, tokens, 500 + kind)
    want = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8)
    assert_matvec_close(got, want, dequant_abs(kind, blob, rows, cols), x)


@pytest.mark.parametrize("kind", [oracle.Q4_K, oracle.Q8_0])
@pytest.mark.parametrize("cols", [512, 4096])
def test_prefill_epilogues(ctx, kind, cols):
    from molla_amd import gpu
    rows, tokens = 160, 40
    blob = synth.quant_tensor(kind, rows, cols, 600).numpy()
    x = synth.normal(tokens * cols, 601).numpy()
    dot = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8).astype(np.float64)
    tol = 1e-5 * np.abs(dot).max() + 1e-4 * np.abs(dot)
    bias = synth.normal(rows, 602).numpy()
    gate_aux = synth.normal(tokens * rows, 603).numpy()
    base = synth.normal(tokens * rows, 604).numpy()
    _, _, got = run(ctx, kind, rows, cols, tokens, 600, epi=gpu.EPI_BIAS, aux=bias)
    assert (np.abs(got.reshape(tokens, rows) - (dot + bias)) <= tol).all()
    _, _, got = run(ctx, kind, rows, cols, tokens, 600, epi=gpu.EPI_ADD, base=base)
    assert (np.abs(got.reshape(tokens, rows) - (dot + base.reshape(tokens, rows))) <= tol).all()
    _, _, got = run(ctx, kind, rows, cols, tokens, 600, epi=gpu.EPI_GLU, aux=gate_aux)
    silu = dot / (1.0 + np.exp(-np.clip(dot, -80, 80)))
    assert (np.abs(got.reshape(tokens, rows) - silu * gate_aux.reshape(tokens, rows)) <= tol * 4 + 1e-6).all()


def test_prefill_without_split_room(ctx):
    """Given only mi_matvec_workspace bytes, K is not split; same result."""
    from molla_amd import gpu
    from molla_amd._lib import lib
    kind, rows, cols, tokens = oracle.Q4_K, 64, 4096, 64
    blob = synth.quant_tensor(kind, rows, cols, 700).numpy()
    x = synth.normal(tokens * cols, 701).numpy()
    w = upload(blob, kind, cols, rows)
    need = lib().mi_matvec_workspace(cols, tokens)
    assert need < lib().mi_matmul_workspace(rows, cols, tokens)
    work = torch.empty(need, dtype=torch.uint8, device="cuda")
    dx = torch.from_numpy(x).cuda()
    out = torch.zeros(tokens * rows, device="cuda")
    rc = lib().mi_matvec(ctx.handle, kind, w.address, w.row_bytes(), rows, cols, dx.data_ptr(), tokens,
                         out.data_ptr(), 0, out.data_ptr(), work.data_ptr(), need)
    assert rc == 0
    ctx.synchronize()
    want = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8)
    assert_matvec_close(out.cpu().numpy(), want, dequant_abs(kind, blob, rows, cols), x)
    split = torch.zeros_like(out)
    gpu.device_matmul_into(ctx, w, dx, split, tokens)
    ctx.synchronize()
    assert_matvec_close(split.cpu().numpy(), want, dequant_abs(kind, blob, rows, cols), x)


def test_prefill_fallback_unaligned(ctx):
    """A weight the tile does not take (Q5_K 4 bytes off 16-byte alignment,
    which the decode kernels accept) runs the decode kernels eight tokens at
    a time, the GLU aux and the output moving along with each run."""
    from molla_amd import gpu
    kind, rows, cols, tokens = oracle.Q5_K, 50, 512, 21
    blob = synth.quant_tensor(kind, rows, cols, 800).numpy()
    x = synth.normal(tokens * cols, 801).numpy()
    aux = synth.normal(tokens * rows, 802).numpy()
    dev = torch.zeros(blob.size + 16, dtype=torch.uint8, device="cuda")
    dev[4:4 + blob.size].copy_(torch.from_numpy(blob))
    w = gpu.Tensor(dev.data_ptr() + 4, kind, cols, rows, keep=dev)
    out = torch.zeros(tokens * rows, device="cuda")
    gpu.device_matmul_into(ctx, w, torch.from_numpy(x).cuda(), out, tokens, epi=gpu.EPI_GLU,
                           aux=torch.from_numpy(aux).cuda())
    ctx.synchronize()
    dot = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8).astype(np.float64)
    want = dot / (1.0 + np.exp(-np.clip(dot, -80, 80))) * aux.reshape(tokens, rows)
    assert np.abs(out.cpu().numpy().reshape(tokens, rows) - want).max() <= 1e-4 * np.abs(want).max()


def test_prefill_large_activations(ctx):
    """Tokens of very different magnitude (1e-3 .. 1e5): each token carries
    its own power-of-two scale, so none loses precision to another and none
    overflows half precision."""
    kind, rows, cols, tokens = oracle.Q4_K, 64, 512, 12
    blob = synth.quant_tensor(kind, rows, cols, 900).numpy()
    x = synth.normal(tokens * cols, 901).numpy().reshape(tokens, cols)
    x *= (10.0 ** np.linspace(-3, 5, tokens)).astype(np.float32)[:, None]
    from molla_amd import gpu
    w = upload(blob, kind, cols, rows)
    out = torch.zeros(tokens * rows, device="cuda")
    gpu.device_matmul_into(ctx, w, torch.from_numpy(x.reshape(-1).copy()).cuda(), out, tokens)
    ctx.synchronize()
    want = oracle.matvec(kind, blob, rows, cols, x, threads=8)
    got = out.cpu().numpy().reshape(tokens, rows)
    wabs = dequant_abs(kind, blob, rows, cols)
    mag = np.abs(x.astype(np.float64)) @ wabs.T
    assert (np.abs(got - want) <= 1e-5 * mag).all()


@pytest.mark.parametrize("kind", KINDS)
def test_prefill_reference_blocks(ctx, kind):
    """Random blocks with the reference tests' scale fields (both signs, the
    full int8 range of Q6_K scales, tests/test_kernel.mojo:106): every code
    path of the weight decode, including Q6_K products above 2048."""
    from molla_amd import gpu
    rows, cols, tokens = 96, 512, 33
    per = oracle.block_elements(kind)
    blob = oracle.test_blocks(kind, rows * cols // per, 0xBEEF + kind)
    x = synth.normal(tokens * cols, 950 + kind).numpy()
    w = upload(blob, kind, cols, rows)
    out = torch.zeros(tokens * rows, device="cuda")
    gpu.device_matmul_into(ctx, w, torch.from_numpy(x).cuda(), out, tokens)
    ctx.synchronize()
    want = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8)
    assert_matvec_close(out.cpu().numpy(), want, dequant_abs(kind, blob, rows, cols), x, peak_gate=False)


def test_prefill_q6k_wide_scales(ctx):
    """Q6_K scales across the whole int8 range, so sc * (q - 32) reaches 4096
    and odd products above 2048 (the even part and the low bit as two MFMA
    operands)."""
    kind, rows, cols, tokens = oracle.Q6_K, 64, 1024, 40
    blob = synth.quant_tensor(kind, rows, cols, 960).numpy().reshape(-1, 210).copy()
    rng = np.random.default_rng(961)
    blob[:, 192:208] = rng.integers(-128, 128, size=(blob.shape[0], 16)).astype(np.int8).view(np.uint8)
    blob = blob.reshape(-1)
    x = synth.normal(tokens * cols, 962).numpy()
    from molla_amd import gpu
    w = upload(blob, kind, cols, rows)
    out = torch.zeros(tokens * rows, device="cuda")
    gpu.device_matmul_into(ctx, w, torch.from_numpy(x).cuda(), out, tokens)
    ctx.synchronize()
    want = oracle.matvec(kind, blob, rows, cols, x.reshape(tokens, cols), threads=8)
    assert_matvec_close(out.cpu().numpy(), want, dequant_abs(kind, blob, rows, cols), x)
