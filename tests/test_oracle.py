"""Pins the CPU oracle (oracle/) against the reference's own known answers.

Every expected number here comes from the reference's tests (cited file:line
under /root/reference/tests), from a closed form, or from an independent
implementation (tests/npquant.py, float64 numpy) -- never from re-running the
oracle's own formula.
"""

import math

import numpy as np
import pytest

import oracle
from tests import npquant

HALF_ONE = 0x3C00


def put16(b, at, v):
    b[at] = v & 0xFF
    b[at + 1] = (v >> 8) & 0xFF


# ---- geometry: tests/test_quant.mojo:85-157 ---------------------------------

def test_geometry():
    table = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
             8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
    for kind, (el, by) in table.items():
        assert oracle.block_elements(kind) == el
        assert oracle.block_bytes(kind) == by
    assert oracle.block_elements(19) == 0 and oracle.block_bytes(19) == 0


def test_scalars():
    # tests/test_quant.mojo:160-186
    assert oracle.f16(0x3C00) == 1.0
    assert oracle.f16(0xBC00) == -1.0
    # every half widens exactly: compare all 65536 patterns against numpy
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16(int(b)) for b in bits[::7]], dtype=np.float32)
    w = want[::7]
    same = (got.view(np.uint32) == w.view(np.uint32)) | (np.isnan(got) & np.isnan(w))
    assert same.all()


def test_f32_to_f16_round_trip():
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10.0,
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-5, -3e-7], np.float32)])
    got = oracle.f32_to_f16_bits(v)
    want = v.astype(np.float16).view(np.uint16)
    assert (got == want).all()


# ---- block known answers: tests/test_quant.mojo:187-464 --------------------

def test_q4_0_kat():
    b = np.zeros(18, np.uint8)
    put16(b, 0, HALF_ONE)
    b[2] = 0x91
    b[3] = 0x08
    out = oracle.dequant(oracle.Q4_0, b, 32)
    assert out[0] == -7.0 and out[16] == 1.0 and out[1] == 0.0 and out[17] == -8.0


def test_q4_1_kat():
    b = np.zeros(20, np.uint8)
    put16(b, 0, HALF_ONE)
    put16(b, 2, 0xC000)
    b[4] = 0x91
    out = oracle.dequant(oracle.Q4_1, b, 32)
    assert out[0] == -1.0 and out[16] == 7.0 and out[1] == -2.0


def test_q5_0_kat():
    b = np.zeros(22, np.uint8)
    put16(b, 0, HALF_ONE)
    b[2] = 0x01
    b[4] = 0x01
    b[6] = 0x10
    b[7] = 0x0F
    out = oracle.dequant(oracle.Q5_0, b, 32)
    assert out[0] == 0.0 and out[16] == 1.0 and out[1] == -1.0 and out[17] == -16.0


def test_q5_1_kat():
    b = np.zeros(24, np.uint8)
    put16(b, 0, HALF_ONE)
    put16(b, 2, 0xC000)
    b[4] = 0x01
    b[8] = 0x10
    out = oracle.dequant(oracle.Q5_1, b, 32)
    assert out[0] == 14.0 and out[16] == -1.0 and out[1] == -2.0


def test_q8_0_kat():
    b = np.zeros(34, np.uint8)
    put16(b, 0, HALF_ONE)
    b[2:6] = [1, 127, 128, 255]
    out = oracle.dequant(oracle.Q8_0, b, 32)
    assert list(out[:4]) == [1.0, 127.0, -128.0, -1.0]


def _scales_of_one():
    s = np.zeros(12, np.uint8)
    s[0:4] = 1
    s[8:12] = 1
    return s


def test_q4_k_kat():
    b = np.zeros(144, np.uint8)
    put16(b, 0, HALF_ONE)
    b[4:16] = _scales_of_one()
    b[16] = 0x53
    b[16 + 32] = 0x27
    out = oracle.dequant(oracle.Q4_K, b, 256)
    assert out[0] == 3.0 and out[32] == 5.0 and out[64] == 7.0 and out[96] == 2.0
    c = np.zeros(144, np.uint8)
    put16(c, 2, HALF_ONE)
    c[4:16] = 3
    assert oracle.dequant(oracle.Q4_K, c, 256)[0] == -3.0


def test_q5_k_kat():
    four = np.zeros(144, np.uint8)
    five = np.zeros(176, np.uint8)
    put16(four, 0, HALF_ONE)
    put16(five, 0, HALF_ONE)
    four[4:16] = _scales_of_one()
    five[4:16] = _scales_of_one()
    for l in range(128):
        four[16 + l] = (l * 37) & 0xFF
        five[48 + l] = (l * 37) & 0xFF
    a = oracle.dequant(oracle.Q4_K, four, 256)
    e = oracle.dequant(oracle.Q5_K, five, 256)
    assert (a == e).all()
    five[16] = 0xFF
    lifted = oracle.dequant(oracle.Q5_K, five, 256)
    assert lifted[0] == a[0] + 16 and lifted[32] == a[32] + 16 and lifted[64] == a[64] + 16
    assert lifted[1] == a[1]


def test_q6_k_kat():
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    put16(b, 208, HALF_ONE)
    b[0] = 0x50
    b[32] = 0x03
    b[128] = 0b01000001
    out = oracle.dequant(oracle.Q6_K, b, 256)
    assert out[0] == -16.0 and out[32] == -29.0 and out[64] == -27.0 and out[96] == -16.0
    b[192] = 0xFF
    assert oracle.dequant(oracle.Q6_K, b, 256)[0] == 16.0


def test_errors_and_run_stride():
    # tests/test_quant.mojo:467-530
    with pytest.raises(ValueError):
        oracle.dequant(19, np.zeros(210, np.uint8), 256)
    with pytest.raises(ValueError):
        oracle.dequant(oracle.Q4_K, np.zeros(210, np.uint8), 300)
    two = np.zeros(68, np.uint8)
    put16(two, 0, HALF_ONE)
    two[2] = 5
    put16(two, 34, HALF_ONE)
    two[36] = 7
    out = oracle.dequant(oracle.Q8_0, two, 64)
    assert out[0] == 5.0 and out[32] == 7.0


# ---- closed forms and the independent decoder --------------------------------

KINDS = [oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K]


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_matches_independent_decoder(kind):
    per = oracle.block_elements(kind)
    blob = oracle.test_blocks(kind, 64, 0x9E3779B97F4A7C15 + kind)
    got = oracle.dequant(kind, blob, 64 * per)
    want = npquant.dequant(kind, blob, 64 * per)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("kind", KINDS)
def test_all_zero_bytes_decode_to_zero(kind):
    per, nb = oracle.block_elements(kind), oracle.block_bytes(kind)
    out = oracle.dequant(kind, np.zeros(nb * 3, np.uint8), 3 * per)
    assert (out == 0).all()


def test_q4_k_scale_one_min_zero_is_the_nibble():
    # d = 1, every sc = 1, every m = 0 -> value = nibble
    rng = np.random.default_rng(3)
    b = np.zeros(144, np.uint8)
    put16(b, 0, HALF_ONE)
    b[4:16] = _scales_of_one()
    b[16:144] = rng.integers(0, 256, 128, dtype=np.uint8)
    out = oracle.dequant(oracle.Q4_K, b, 256)
    qs = b[16:144].reshape(4, 32).astype(np.int32)
    want = np.concatenate([np.concatenate([qs[h] & 0xF, qs[h] >> 4]) for h in range(4)])
    assert (out == want).all()


def test_q6_k_linear_in_d():
    blob = oracle.test_blocks(oracle.Q6_K, 1, 77)
    put16(blob, 208, HALF_ONE)
    one = oracle.dequant(oracle.Q6_K, blob, 256)
    put16(blob, 208, 0x4000)  # 2.0
    two = oracle.dequant(oracle.Q6_K, blob, 256)
    assert (two == 2 * one).all()


# ---- fused dot: tests/test_kernel.mojo:437-478 -------------------------------

@pytest.mark.parametrize("kind", KINDS)
def test_fused_matches_dequant(kind):
    per = oracle.block_elements(kind)
    n = per * 4
    packed = oracle.test_blocks(kind, 4, 0x9E3779B97F4A7C15 + kind)
    w = oracle.dequant(kind, packed, n)
    x = oracle.test_units(0x1234567 + kind, n)
    terms = (w * x).astype(np.float32)
    slow = np.float32(0)
    for t in terms:
        slow = np.float32(slow + t)
    mag = float(np.abs(terms.astype(np.float64)).sum())
    fast = oracle.row_dot(kind, packed, x)
    assert abs(fast - float(slow)) <= 1e-4 * mag + 1e-6


@pytest.mark.parametrize("kind", KINDS)
def test_matvec_against_float64_brute_force(kind):
    per = oracle.block_elements(kind)
    rows, cols = 5, per * 3
    blob = oracle.test_blocks(kind, rows * 3, 0xABCDEF + kind)
    w = npquant.dequant(kind, blob, rows * cols).reshape(rows, cols).astype(np.float64)
    x = oracle.test_units(99 + kind, cols)
    y = oracle.matvec(kind, blob, rows, cols, x)
    exact = w @ x.astype(np.float64)
    mag = np.abs(w) @ np.abs(x.astype(np.float64))
    assert (np.abs(y - exact) <= 1e-4 * mag + 1e-6).all()


def test_matvec_hand():
    # tests/test_kernel.mojo:481-512: rows [1 2 3], [4 5 6]
    w = np.array([1, 2, 3, 4, 5, 6], np.float32).view(np.uint8)
    assert list(oracle.matvec(oracle.F32, w, 2, 3, np.array([1, 0, -1], np.float32))) == [-2.0, -2.0]
    assert list(oracle.matvec(oracle.F32, w, 2, 3, np.array([1, 1, -1], np.float32))) == [0.0, 3.0]


def test_row_dot_plain_types():
    # tests/test_kernel.mojo:347-384
    x = np.array([1, 2, 3, 4], np.float32)
    assert oracle.row_dot(oracle.F32, np.array([1, 2, -3, 0.5], np.float32).view(np.uint8), x) == -2.0
    h = np.array([0x3C00, 0x4000, 0x3C00, 0x4000], np.uint16).view(np.uint8)
    assert oracle.row_dot(oracle.F16, h, x) == 16.0
    bf = np.array([0x3F80, 0x4000, 0x3F80, 0x4000], np.uint16).view(np.uint8)
    assert oracle.row_dot(oracle.BF16, bf, x) == 16.0


# ---- scalars: tests/test_kernel.mojo:161-304 ----------------------------------

def test_kernel_scalars():
    assert oracle.silu(0.0) == 0.0
    assert abs(oracle.silu(1.0) - 0.7310586) <= 1e-6
    assert oracle.silu(-20.0) > -1e-6
    assert abs(oracle.gelu(1.0) - 0.8411920) <= 1e-5
    assert abs(oracle.gelu(-1.0) + 0.1588080) <= 1e-5
    assert oracle.argmax(np.array([1, 9, 3], np.float32)) == 1
    assert oracle.argmax(np.array([1, 9, 9], np.float32)) == 1


def test_softmax_cases():
    x = oracle.softmax([1.0, 2.0, 3.0])
    assert abs(x.sum() - 1) <= 1e-6 and abs(x[0] - 0.09003057) <= 1e-6
    big = oracle.softmax([800.0, 801.0])
    assert abs(big.sum() - 1) <= 1e-6 and not np.isnan(big).any()
    assert oracle.softmax([-5.0])[0] == 1.0


def test_rms_norm_mean_square_7_5():
    x = np.array([1, 2, 3, 4], np.float32)
    out = oracle.rms_norm(x, np.ones(4, np.float32), 1e-5)
    expect = 1.0 / math.sqrt(7.5 + 1e-5)
    assert abs(out[0] - expect) <= 1e-6 and abs(out[3] - 4 * expect) <= 1e-5
    half = oracle.rms_norm(x, np.full(4, 0.5, np.float32), 1e-5)
    assert abs(half[0] - 0.5 * expect) <= 1e-6
    zero = oracle.rms_norm(np.zeros(4, np.float32), np.ones(4, np.float32), 1e-5)
    assert (zero == 0).all()


# ---- rope: tests/test_rope.mojo:93-190 ----------------------------------------

def test_rope_plain_and_adjacent_pairs():
    fresh = np.arange(1, 9, dtype=np.float32)
    assert (oracle.rotate(fresh, 1, 8, 8, 10000.0, True, 0) == fresh).all()
    neox = oracle.rotate(fresh, 1, 8, 8, 10000.0, True, 3)
    want_neox = [-1.6955925, 0.1375517, 2.7886816, 3.9759820, -4.8088425, 6.3230593, 7.0868367, 8.0119640]
    assert np.allclose(neox, want_neox, atol=1e-5, rtol=0)
    adj = oracle.rotate(fresh, 1, 8, 8, 10000.0, False, 3)
    want_adj = [-1.2722325, -1.8388650, 1.6839286, 4.7079066, 4.8177772, 6.1472777, 6.9759685, 8.0209640]
    assert np.allclose(adj, want_adj, atol=1e-5, rtol=0)
    c, s = oracle.rope_angle(8, 10000.0, 3, 1)
    assert abs(c - 0.9553365) <= 1e-6 and abs(s - 0.2955202) <= 1e-6
    part = oracle.rotate(fresh, 1, 8, 4, 10000.0, True, 3)
    assert (part[4:] == fresh[4:]).all() and part[0] != 1.0


def test_rope_per_pair_factors():
    # tests/test_rope.mojo:321-373: Llama 3.1's rope_freqs.weight divides each
    # pair's angle by its own factor; factors of one are no scaling at all.
    # RopeSpec(8, 10000.0) is half-split pairing (neox), the default there.
    x = np.arange(1, 9, dtype=np.float32)
    got = oracle.rotate(x, 1, 8, 8, 10000.0, True, 3, factors=[1.0, 2.0, 4.0, 8.0])
    want = [-1.6955925, 1.0809134, 2.9474161, 3.9969997, -4.8088425, 6.2315027, 7.0223029, 8.0014994]
    assert np.allclose(got, want, atol=1e-5)
    for neox in (True, False):
        ones = oracle.rotate(x, 1, 8, 8, 10000.0, neox, 3, factors=[1.0] * 4)
        assert np.array_equal(ones, oracle.rotate(x, 1, 8, 8, 10000.0, neox, 3))
    with pytest.raises(ValueError):
        oracle.rotate(x, 1, 8, 8, 10000.0, True, 3, factors=[1.0])


def test_q8_cache_round():
    # The q8_0 cache quantizer (tests/test_gpu_ops.mojo:925 _quantize_q8):
    # per 32-value block, the largest magnitude maps to +-127 exactly; every
    # value reads back within half a factor; a block of zeros stays zero;
    # rounding is half away from zero.
    rng = np.random.default_rng(3)
    v = rng.standard_normal(256).astype(np.float32)
    got = oracle.q8_cache_round(v)
    for b in range(8):
        blk, out = v[32 * b:32 * b + 32], got[32 * b:32 * b + 32]
        amax = np.abs(blk).max()
        s = np.float32(np.float16(amax / np.float32(127)))
        q = out / s
        assert np.allclose(q, np.rint(q), atol=1e-4) and np.abs(q).max() == 127.0
        assert np.abs(out - blk).max() <= s * 0.5 + abs(amax - 127 * s) + 1e-6
    assert not oracle.q8_cache_round(np.zeros(32, np.float32)).any()
    half = np.zeros(32, np.float32)
    half[0], half[1], half[2] = 127.0, 2.5, -2.5  # factor 1: 2.5 -> 3, -2.5 -> -3
    assert list(oracle.q8_cache_round(half)[:3]) == [127.0, 3.0, -3.0]


def test_rope_steps():
    # tests/test_rope.mojo:420-457: one step per pair, first is 1, falling.
    steps = oracle.rope_steps(64, 10000.0)
    assert steps.size == 32 and steps[0] == 1.0 and (np.diff(steps) < 0).all()
    want = (10000.0 ** (-2.0 * np.arange(32) / 64.0)).astype(np.float32)
    assert np.allclose(steps, want, rtol=2e-7, atol=0)


def test_rope_preserves_length_at_long_positions():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(8 * 128).astype(np.float32)
    y = oracle.rotate(x, 8, 128, 128, 500000.0, False, 4096)
    assert np.allclose(np.linalg.norm(x.reshape(8, 128), axis=1), np.linalg.norm(y.reshape(8, 128), axis=1),
                       rtol=1e-5)


# ---- attention: tests/test_attention.mojo:150-236 ----------------------------

def test_attention_paper_case():
    q = np.array([1, 0], np.float32)
    kv = np.array([1, 0, 0, 1, 1, 1], np.float32)
    scale = float(np.float32(1.0 / math.sqrt(2.0)))
    out = oracle.attend(1, 1, 2, scale, q, kv, kv, 3)
    assert abs(out[0] - 0.8022242) <= 1e-6 and abs(out[1] - 0.5988879) <= 1e-6
    one = oracle.attend(1, 1, 2, scale, q, kv, kv, 1)
    assert one[0] == 1.0 and one[1] == 0.0


def test_attention_grouped():
    out = oracle.attend(4, 2, 1, 1.0, np.ones(4, np.float32), np.array([1, 10], np.float32),
                        np.array([3, 30], np.float32), 1)
    assert list(out) == [3.0, 3.0, 30.0, 30.0]


# ---- layer: tests/test_block.mojo:246-313 -------------------------------------

def _f32_weight(m):
    m = np.ascontiguousarray(m, np.float32)
    return (oracle.F32, m.shape[0], m.shape[1], m.view(np.uint8).ravel())


def test_layer_identity_hand_case():
    W, H = 8, 8
    spec = dict(width=W, hidden=H, heads=2, kv_heads=2, head_dim=4, rope_dim=4, neox=1, eps=1e-5,
                rope_base=10000.0, attn_scale=float(np.float32(1 / math.sqrt(4))))
    eye = np.eye(W, dtype=np.float32)
    weights = dict(attn_norm=np.ones(W), ffn_norm=np.ones(W), wq=_f32_weight(eye), wk=_f32_weight(eye),
                   wv=_f32_weight(eye), wo=_f32_weight(eye), gate=_f32_weight(eye), up=_f32_weight(eye),
                   down=_f32_weight(eye))
    keep = []
    L = oracle.make_layer(spec, weights, keep)
    x = np.arange(1, 9, dtype=np.float32)
    keys = np.zeros(W, np.float32)
    values = np.zeros(W, np.float32)
    oracle.layer_step(L, x, keys, values, 0, 0)
    div = math.sqrt(25.5 + float(np.float32(1e-5)))
    v = np.arange(1, 9, dtype=np.float64)
    after_attn = v + v / div
    normed = v / div
    silu = normed / (1 + np.exp(-normed))
    want = after_attn + silu * normed
    assert np.allclose(x, want, atol=1e-5, rtol=0)
    assert abs(keys[0] - 1 / div) <= 1e-6 and abs(values[3] - 4 / div) <= 1e-6
