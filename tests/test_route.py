"""The batched matvec dispatch (mi_matvec_route, pure host logic: no GPU
needed) only admits each tile's shapes.  The preconditions here are the
tiles' own, written out independently of the predicates in the library:

  f16 tile (matvec_htile.hip): 2..8 tokens, Q4_K or Q6_K, a row (or a split
    part's row) of whole 512-column wave slices, at most 8 of them, copied
    to LDS in 8-byte words, so a Q6_K part holds a multiple of four 210-byte
    superblocks; a split cuts cols into >= 2 equal parts;
  int8 tiles: Q4_K (matvec_tile.hip), Q4_0 / Q8_0 (matvec_tile_b32.hip),
    Q6_K (matvec_tile_q6k.hip), 2..8 tokens;
  batch-1 row kernels: one token, at most 4 waves of 64 units of 64 values.
"""

import ctypes

import pytest

import oracle
from molla_amd import _lib

ROUTE_ROWS, ROUTE_Q6K_ROWS, ROUTE_HTILE, ROUTE_Q4K_TILE, ROUTE_B32_TILE, ROUTE_Q6K_TILE, ROUTE_GENERAL, \
    ROUTE_PREFILL = range(1, 9)
SPLIT = 16
KINDS = [oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K]
COLS = [256 * i for i in range(1, 17)] + [5120, 8192, 11008, 14336]


def route(lib, kind, rows, cols, tokens, work):
    part = ctypes.c_int32(0)
    r = lib.mi_matvec_route(kind, rows, cols, tokens, work, ctypes.byref(part))
    return r, part.value


@pytest.mark.parametrize("kind", KINDS)
def test_route_admits_only_tile_shapes(kind):
    lib = _lib.lib()
    seen = set()
    for cols in COLS:
        for rows in (16, 48, 4096):
            for tokens in range(1, 9):
                work = lib.mi_matmul_workspace(rows, cols, tokens)
                r, part = route(lib, kind, rows, cols, tokens, work)
                assert r > 0, (kind, rows, cols, tokens, r)
                seen.add(r)
                base, split = r & ~SPLIT, bool(r & SPLIT)
                what = (kind, rows, cols, tokens, r, part)
                if tokens == 1:
                    assert not split and base in (ROUTE_ROWS, ROUTE_Q6K_ROWS, ROUTE_GENERAL), what
                    if base in (ROUTE_ROWS, ROUTE_Q6K_ROWS):
                        assert cols // 64 <= 4 * 64, what
                        assert (base == ROUTE_Q6K_ROWS) == (kind == oracle.Q6_K), what
                    continue
                assert base not in (ROUTE_ROWS, ROUTE_Q6K_ROWS, ROUTE_PREFILL), what
                if base == ROUTE_HTILE:
                    assert kind in (oracle.Q4_K, oracle.Q6_K), what
                    assert part % 512 == 0 and part // 512 <= 8, what
                    assert (part // 256) * oracle.block_bytes(kind) % 8 == 0, what
                    if split:
                        assert cols % part == 0 and cols // part >= 2, what
                    else:
                        assert part == cols, what
                elif base == ROUTE_Q4K_TILE:
                    assert kind == oracle.Q4_K, what
                elif base == ROUTE_B32_TILE:
                    assert kind in (oracle.Q4_0, oracle.Q8_0) and not split, what
                elif base == ROUTE_Q6K_TILE:
                    assert kind == oracle.Q6_K and not split, what
                else:
                    assert base == ROUTE_GENERAL and not split, what
                # without room for the parts nothing splits
                r1, _ = route(lib, kind, rows, cols, tokens, lib.mi_matvec_workspace(cols, tokens))
                assert not (r1 & SPLIT), what
    if kind == oracle.Q4_K:
        assert {ROUTE_ROWS, ROUTE_HTILE, ROUTE_HTILE | SPLIT} <= seen, seen
    if kind == oracle.Q6_K:
        assert {ROUTE_Q6K_ROWS, ROUTE_HTILE, ROUTE_Q6K_TILE} <= seen, seen


def test_route_prefill_and_refusals():
    lib = _lib.lib()
    assert route(lib, oracle.Q4_K, 64, 4096, 9, 0)[0] == ROUTE_PREFILL
    assert route(lib, oracle.Q4_K, 64, 4000, 1, 0)[0] < 0   # not whole superblocks
    assert route(lib, 99, 64, 4096, 1, 0)[0] < 0            # no such kind
    assert route(lib, oracle.Q4_K, 0, 4096, 1, 0)[0] < 0
