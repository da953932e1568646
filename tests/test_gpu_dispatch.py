"""The batched dispatch swept over shapes on the GPU: for Q4_K, Q6_K, Q4_0
and Q8_0, every multiple of 256 columns from 256 to 4096 plus 14336, at 1..8
tokens, over few rows (so long rows split over K where the dispatch does),
mi_matvec against the oracle within the matvec gate of test_gpu_kernels, and
bit for bit the same whether its workspace held one byte pattern or another
before the call (a kernel that reads workspace it did not write differs)."""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from molla_amd import synth

pytestmark = pytest.mark.gpu

COLS = [256 * i for i in range(1, 17)] + [14336]
ROUTE_SPLIT = 16


@pytest.fixture(scope="module")
def ctx():
    from molla_amd import gpu
    return gpu.DeviceContext(0)


@pytest.mark.parametrize("kind", [oracle.Q4_K, oracle.Q6_K, oracle.Q4_0, oracle.Q8_0])
def test_dispatch_grid(ctx, kind):
    from molla_amd import gpu
    from molla_amd._lib import check, lib
    L = lib()
    rows = 48
    routes = set()
    for cols in COLS:
        print(f"kind {kind} cols {cols}", flush=True)
        blob = synth.quant_tensor(kind, rows, cols, 900 + cols // 256 + kind).numpy()
        x = synth.normal(8 * cols, 901 + cols // 256).numpy()
        want_all = oracle.matvec(kind, blob, rows, cols, x.reshape(8, cols), threads=8).reshape(8, rows)
        wabs = np.abs(oracle.dequant(kind, blob, rows * cols).reshape(rows, cols).astype(np.float64))
        w = gpu.Tensor.from_bytes(torch.from_numpy(blob), kind, cols, rows)
        xd = torch.from_numpy(x).cuda()
        for tokens in range(1, 9):
            need = L.mi_matmul_workspace(rows, cols, tokens)
            part = ctypes.c_int32(0)
            r = L.mi_matvec_route(kind, rows, cols, tokens, need, ctypes.byref(part))
            routes.add(r)
            outs = []
            for fill in (0xA5, 0x7F):
                work = torch.full((need + 256,), fill, dtype=torch.uint8, device="cuda")
                y = torch.full((tokens * rows,), float("nan"), device="cuda")
                check(L.mi_matvec(ctx.handle, kind, w.address, w.row_bytes(), rows, cols, xd.data_ptr(), tokens,
                                  y.data_ptr(), gpu.EPI_NONE, y.data_ptr(), work.data_ptr(), need))
                ctx.synchronize()
                outs.append(y.cpu().numpy())
            what = f"kind {kind} cols {cols} tokens {tokens} route {r} part {part.value}"
            assert (outs[0].view(np.uint32) == outs[1].view(np.uint32)).all(), what
            got = outs[0].astype(np.float64).reshape(tokens, rows)
            want = want_all[:tokens]
            mag = np.abs(x.astype(np.float64).reshape(8, cols)[:tokens]) @ wabs.T
            err = np.abs(got - want)
            assert np.isfinite(got).all(), what
            assert (err <= 1e-4 * mag + 1e-6).all(), (what, float((err / (mag + 1e-30)).max()))
    print(f"kind {kind}: routes taken {sorted(routes)}", flush=True)
    if kind in (oracle.Q4_K, oracle.Q6_K):
        assert any(r & ROUTE_SPLIT for r in routes), routes
