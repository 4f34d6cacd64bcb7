"""Pins the CPU oracle (oracle/lowbit_oracle.py) before it is trusted as the GPU checker.

Each check is chosen so that a plausible slip in the oracle (nibble order, sign of the
int4 decode, double rounding of q*s, tie direction of the quantizer, a dropped
correction stage) fails at least one of them.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import lowbit_oracle as o

GOLDEN = Path(__file__).resolve().parent / 'golden'
KA = json.loads((GOLDEN / 'known_answers.json').read_text())


def fixtures():
    data = np.load(GOLDEN / 'linear_small.npz', allow_pickle=False)
    names = sorted({key.split('/')[0] for key in data.files})
    return data, names


def test_pack_known_answers():
    for key in ('pack_arange16', 'pack_odd3'):
        case = KA[key]
        assert o.pack(np.array(case['codes'], np.uint8)).hex() == case['packed_hex'], case['source']


def test_unpack_round_trip_and_nibble_order():
    rng = np.random.default_rng(1)
    for count in (1, 2, 3, 17, 64, 1001):
        codes = rng.integers(0, 16, count).astype(np.uint8)
        data = o.pack(codes)
        assert len(data) == (count + 1) // 2
        np.testing.assert_array_equal(o.nibbles(data, count), codes)
        if count % 2:
            assert data[-1] >> 4 == 0
    # element 0 lives in the low nibble
    assert o.nibbles(bytes([0xA5]), 2).tolist() == [5, 10]


def test_int4_and_nf4_all_codes_known_answers():
    packed = bytes.fromhex(KA['int4_all_codes_scale1']['packed_hex'])
    got = o.dequantize('int4', (1, 16), 16, packed, np.float16(1).tobytes()).ravel()
    np.testing.assert_array_equal(got, np.array(KA['int4_all_codes_scale1']['values'], np.float16))
    case = KA['nf4_all_codes_scale1_f16_bits']
    literal16 = np.array([np.float32(v) for v in case['literals']], np.float32).astype(np.float16)
    np.testing.assert_array_equal(literal16.view(np.uint16), np.array(case['bits'], np.uint16))
    np.testing.assert_array_equal(o.NF4_F32, np.array([np.float32(v) for v in case['literals']], np.float32))
    got = o.dequantize('nf4', (1, 16), 16, packed, np.float16(1).tobytes()).ravel()
    np.testing.assert_array_equal(got.view(np.uint16), np.array(case['bits'], np.uint16))
    # int4 decode is the two's complement nibble
    assert o.unpack('int4', packed, 16).tolist() == [c - 16 if c >= 8 else c for c in range(16)]


def test_int8_codec_known_answer():
    case = KA['int8_codec_eighth']
    codes = np.array(case['codes'], np.int8)
    got = o.dequantize('int8', (1, 256), 256, codes.tobytes(), np.float16(case['scale']).tobytes()).ravel()
    np.testing.assert_array_equal(got, codes.astype(np.float16) * np.float16(case['scale']))
    np.testing.assert_array_equal(got.astype(np.float64), codes.astype(np.float64) * 0.125)


def test_dequantize_brute_force_single_rounding():
    """Every int4 code and every int8 code against a sample of fp16 scales, including
    subnormal products: fp64 route (oracle) == fp32 multiply then RNE to fp16."""
    rng = np.random.default_rng(2)
    bits = np.concatenate([np.arange(1, 0x7C00, 97, dtype=np.uint16), rng.integers(1, 0x7C00, 300).astype(np.uint16),
                           np.array([1, 2, 3, 0x3C00, 0x0400, 0x03FF, 0x7BFF], np.uint16)])
    scales = bits.view(np.float16)
    for fmt, codes in (('int4', np.arange(16, dtype=np.uint8)), ('int8', np.arange(-128, 128).astype(np.int8)),
                       ('nf4', np.arange(16, dtype=np.uint8))):
        n, k = scales.size, codes.size
        data = o.pack(np.tile(codes, n)) if fmt != 'int8' else np.tile(codes, n).tobytes()
        got = o.dequantize(fmt, (n, k), k, data, scales.tobytes())
        if fmt == 'int4':
            q = np.where(codes >= 8, codes.astype(np.int16) - 16, codes).astype(np.float32)
        elif fmt == 'nf4':
            q = o.NF4_F32.astype(np.float16).astype(np.float32)
        else:
            q = codes.astype(np.float32)
        with np.errstate(over='ignore'):
            expected = (q[None, :] * scales.astype(np.float32)[:, None]).astype(np.float16)
        np.testing.assert_array_equal(got.view(np.uint16), expected.view(np.uint16), err_msg=fmt)


def test_quantize_ties_and_invariants():
    # int4 rint ties go to even: scale 1 (absmax 7), values k+0.5.
    w = np.array([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]], np.float32)
    data, scales = o.quantize(w, 'int4')
    assert np.frombuffer(scales, np.float16)[0] == 1.0
    assert o.unpack('int4', data, 8).tolist() == [7, 0, 2, 2, 0, -2, -2, 4]
    # nf4: exactly at an fp32 midpoint goes to the lower code (searchsorted side='left')
    mids = ((o.NF4_F32[:-1] + o.NF4_F32[1:]) / np.float32(2)).astype(np.float32)
    w = np.concatenate([[1.0], mids, np.nextafter(mids, np.float32(2))]).astype(np.float32)[None, :]
    data, scales = o.quantize(w, 'nf4')
    assert np.frombuffer(scales, np.float16)[0] == 1.0
    codes = o.unpack('nf4', data, w.size)
    assert codes[0] == 15
    assert codes[1:16].tolist() == list(range(15))
    assert codes[16:].tolist() == list(range(1, 16))
    # invariants on random data: |q| <= limit, s >= 2^-24, zero rows stay zero, error <= s/2
    rng = np.random.default_rng(3)
    for fmt, limit in (('int4', 7), ('int8', 127)):
        w = (rng.standard_normal((9, 64)) * 0.02).astype(np.float32)
        w[3] = 0
        data, scales = o.quantize(w, fmt, 32)
        q = o.unpack(fmt, data, w.size).reshape(9, 2, 32)
        s = np.frombuffer(scales, np.float16).reshape(9, 2).astype(np.float64)
        assert np.abs(q).max() <= limit and s.min() >= 2.0 ** -24
        assert not q[3].any()
        err = np.abs(q * s[:, :, None] - w.reshape(9, 2, 32).astype(np.float64))
        assert (err <= s[:, :, None] * 0.5 * (1 + 1e-3) + 1e-12).all()
    with pytest.raises(ValueError):
        o.quantize(np.full((1, 4), 1e7, np.float32), 'int8')
    with pytest.raises(ValueError):
        o.quantize(np.array([[np.nan, 1.0]], np.float32), 'int4')


def test_linear_textbook_and_identity():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((12, 64)) * 0.02).astype(np.float32)
    x = rng.standard_normal((3, 64)).astype(np.float16)
    for fmt in ('int4', 'nf4', 'int8'):
        data, scales = o.quantize(w, fmt, 32)
        deq = o.dequantize(fmt, (12, 64), 32, data, scales).astype(np.float64)
        # textbook triple loop on a small slice pins the matmul orientation
        ref = np.array([[sum(float(x[m, k]) * deq[n, k] for k in range(64)) for n in range(12)] for m in range(3)])
        np.testing.assert_array_equal(o.linear(x, fmt, (12, 64), 32, data, scales), ref.astype(np.float16))
    # identity input reproduces the dequantized weights bit-exactly (demo :124-128)
    for fmt in ('int4', 'nf4'):
        for scale in KA['identity_input_exact']['scales']:
            packed = bytes.fromhex(KA['pack_arange16']['packed_hex'])
            s = np.float16(scale).tobytes()
            y = o.linear(np.eye(16, dtype=np.float16), fmt, (1, 16), 16, packed, s)
            np.testing.assert_array_equal(y[:, 0], o.dequantize(fmt, (1, 16), 16, packed, s)[0])


def test_correction_staging():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((16, 32)) * 0.02).astype(np.float32)
    data, scales = o.quantize(w, 'int8')
    x = rng.standard_normal((2, 32)).astype(np.float16)
    base = o.linear(x, 'int8', (16, 32), 32, data, scales)
    zero = o.linear(x, 'int8', (16, 32), 32, data, scales, down=np.zeros((4, 32), np.float16),
                    up=np.zeros((16, 4), np.float16))
    np.testing.assert_array_equal(base, zero)  # zero factors: bitwise unchanged
    down = (rng.standard_normal((4, 32)) * 0.1).astype(np.float16)
    up = (rng.standard_normal((16, 4)) * 0.1).astype(np.float16)
    got = o.linear(x, 'int8', (16, 32), 32, data, scales, down=down, up=up)
    z = (x.astype(np.float64) @ down.astype(np.float64).T).astype(np.float16)
    d = (z.astype(np.float64) @ up.astype(np.float64).T).astype(np.float16)
    np.testing.assert_array_equal(got, (base.astype(np.float32) + d.astype(np.float32)).astype(np.float16))
    # the exact-weight W8 path differs from the fp16-dequantized path somewhere
    w16 = o.dense_linear(x, o.dequantize('int8', (16, 32), 32, data, scales))
    assert o.rel_l2(w16, base) < 1e-3


def test_fixtures_reproduce():
    data, names = fixtures()
    assert len(names) >= 8
    for name in names:
        m, n, k, g, rank = data[f'{name}/shape'].tolist()
        fmt = str(data[f'{name}/fmt'])
        raw, scales = o.quantize(data[f'{name}/weight'].astype(np.float32), fmt, g)
        assert raw == data[f'{name}/data'].tobytes() and scales == data[f'{name}/scales'].tobytes(), name
        kw = {}
        if f'{name}/bias' in data.files:
            kw['bias'] = data[f'{name}/bias']
        if rank:
            kw['down'], kw['up'] = data[f'{name}/down'], data[f'{name}/up']
        y = o.linear(data[f'{name}/x'], fmt, (n, k), g, raw, scales, **kw)
        np.testing.assert_array_equal(y.view(np.uint16), data[f'{name}/y'].view(np.uint16), err_msg=name)


# ---------------------------------------------------------------- compact_groups
def test_compact_one_group_is_the_default_graph():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((3, 64)) / 8).astype(np.float16)
    for fmt in ('int4', 'nf4', 'int8'):
        data, scales = o.quantize(rng.standard_normal((5, 64)) / 8, fmt, None)
        np.testing.assert_array_equal(o.compact_linear(x, fmt, (5, 64), 64, data, scales),
                                      o.linear(x, fmt, (5, 64), 64, data, scales))


def test_compact_reference_edges():
    # all 16 codes split over two groups of 8, identity input: the output is dequantize()^T bit
    # for bit (torch_npu_lowbit_group_demo.py edges, 'all_codes_two_groups')
    codes = o.pack(np.arange(16, dtype=np.uint8))
    for fmt in ('int4', 'nf4'):
        for scale in (0.125, 1.0, 16.0):
            scales = np.full(2, scale, np.float16).tobytes()
            got = o.compact_linear(np.eye(16, dtype=np.float16), fmt, (1, 16), 8, codes, scales)
            want = o.dequantize(fmt, (1, 16), 8, codes, scales).T
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
        # zero weights in groups of 3 ('odd_group_zero')
        data, scales = o.quantize(np.zeros((5, 9), np.float32), fmt, 3)
        assert not o.compact_linear(np.ones((7, 9), np.float16), fmt, (5, 9), 3, data, scales).any()
    # a finite full product whose fp16 partials overflow ('partial_overflow_limitation')
    for fmt, pos, neg, act, sc in (('int4', 7, 13, 1024.0, [1.0, 2.0]), ('nf4', 15, 0, 4096.0, [1.0, 0.5])):
        data = o.pack(np.array([pos] * 16 + [neg] * 16, np.uint8))
        scales = np.array(sc, np.float16).tobytes()
        x = np.full((1, 32), act, np.float16)
        full = o.linear(x, fmt, (1, 32), 16, data, scales)
        expected = float((x.astype(np.float64) @ o.dequantize(fmt, (1, 32), 16, data, scales).astype(np.float64).T)[0, 0])
        assert float(full[0, 0]) == expected
        assert float(o.compact_linear(x, fmt, (1, 32), 16, data, scales)[0, 0]) != expected


def _pieces_weight(values, group=32):
    """int8 weight row whose group g sums to values[g] against an all-ones input (scales 1)."""
    codes = np.zeros((1, group * len(values)), np.int8)
    for g, v in enumerate(values):
        q, r = divmod(v, group)
        codes[0, g * group:(g + 1) * group] = q
        codes[0, g * group:g * group + r] += 1
    return codes.tobytes(), np.ones(len(values), np.float16).tobytes()


def test_compact_tree_pairs_neighbours():
    f = lambda v: float(np.float16(v))
    # eight pieces: ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)); sequential addition would give 2048
    data, scales = _pieces_weight([2048] + [1] * 7)
    x = np.ones((1, 256), np.float16)
    tree = f(f(f(2048 + 1) + f(1 + 1)) + f(f(1 + 1) + f(1 + 1)))
    assert tree == 2054.0
    assert float(o.compact_linear(x, 'int8', (1, 256), 32, data, scales)[0, 0]) == tree
    assert float(o.linear(x, 'int8', (1, 256), 32, data, scales)[0, 0]) == 2056.0  # one fp16 rounding
    # five pieces: the odd last piece moves up unpaired: ((p0+p1)+(p2+p3))+p4
    data, scales = _pieces_weight([2048, 1, 1, 1, 1])
    x = np.ones((1, 160), np.float16)
    tree = f(f(f(2048 + 1) + f(1 + 1)) + 1)
    assert float(o.compact_linear(x, 'int8', (1, 160), 32, data, scales)[0, 0]) == tree == 2052.0
    # three pieces with bias: fp16(fp16((p0+p1)+p2) + b)
    data, scales = _pieces_weight([2048, 1, 3])
    x = np.ones((1, 96), np.float16)
    got = o.compact_linear(x, 'int8', (1, 96), 32, data, scales, bias=np.array([1.0], np.float16))
    assert float(got[0, 0]) == f(f(f(2048 + 1) + 3) + 1)


# ---------------------------------------------------------------- W8A8 (activation_scale)
def test_w8a8_all_weight_codes_exact():
    # torch_npu_int8_demo.py 'w8a8_all_weight_codes': identity input, activation scale 1/64
    codes = np.arange(-128, 128, dtype=np.int8)
    for sc in (0.125, 1.0, 16.0):
        got = o.w8a8_linear(np.eye(256, dtype=np.float16), (1, 256), codes.tobytes(), np.float16(sc).tobytes(), 1 / 64)
        np.testing.assert_array_equal(got.ravel().astype(np.float64), codes.astype(np.float64) * sc)


def test_w8a8_activation_ties_and_clipping():
    # 'all_activation_codes_ties_clipping': identity int8 weights, unit scales, activation 1/128
    grid = np.arange(-128, 128, dtype=np.float64) / 128
    x = np.stack((grid, grid + 1 / 256, grid - 1 / 256, grid * 2)).astype(np.float16)
    eye = np.eye(256, dtype=np.int8).tobytes()
    got = o.w8a8_linear(x, (256, 256), eye, np.ones(256, np.float16).tobytes(), 1 / 128)
    # independent expectation: Python's round() is half-to-even on exact binary fractions
    want = [[max(-128, min(127, round(float(v) * 128))) / 128 for v in row] for row in x]
    np.testing.assert_array_equal(got.astype(np.float64), np.array(want))
    assert got[1, 128] == 0 and got[1, 129] == np.float16(2 / 128)  # 0.5 -> 0, 1.5 -> 2
    assert got[3].max() == np.float16(127 / 128) and got[3].min() == -1.0  # clipping


def test_w8a8_large_integer_accumulation():
    # 'large_integer_accumulation_cancellation': K=4096, |sum| above 2^24 stays exact
    codes = np.stack((np.full(4096, 127, np.int8), np.tile([127, -127], 2048).astype(np.int8)))
    scales = np.full(2, 1 / 128, np.float16).tobytes()
    got = o.w8a8_linear(np.full((1, 4096), 127 / 128, np.float16), (2, 4096), codes.tobytes(), scales, 1 / 128)
    # 4096*127*127 / 128 * step, step = (fp16(127/128) + 1) / 255 = 1/128 -> 4032.25 -> fp16 4032
    assert got.tolist() == [[4032.0, 0.0]]


def test_w8a8_scale_boundaries_and_zero():
    eye = np.eye(16, dtype=np.int8).tobytes()
    ones = np.ones(16, np.float16).tobytes()
    for s in (2.0 ** -24, 2.0 ** -14, 256.0):
        x = (np.arange(-8, 8, dtype=np.float64) * s).astype(np.float16).reshape(1, 16)
        np.testing.assert_array_equal(o.w8a8_linear(x, (16, 16), eye, ones, s), x)
    data, scales = o.quantize(np.zeros((3, 17), np.float32), 'int8')
    assert not o.w8a8_linear(np.ones((2, 17), np.float16), (3, 17), data, scales, 1 / 128).any()


def test_w8a8_integer_brute_force():
    from fractions import Fraction
    rng = np.random.default_rng(11)
    for m, k, n, sx in ((1, 17, 3, 1 / 128), (5, 64, 32, 1 / 256), (7, 64, 13, 1 / 128)):
        data, scales = o.quantize(rng.standard_normal((n, k)) / 8, 'int8')
        x = (rng.standard_normal((m, k)) / 8).astype(np.float16)
        bias = (rng.standard_normal(n) / 8).astype(np.float16)
        got = o.w8a8_linear(x, (n, k), data, scales, sx, bias=bias)
        codes = np.frombuffer(data, np.int8).reshape(n, k)
        s16 = np.frombuffer(scales, np.float16)
        for i in range(m):
            qx = [max(-128, min(127, round(Fraction(float(v)) / Fraction(sx)))) for v in x[i]]
            for j in range(n):
                acc = sum(a * int(b) for a, b in zip(qx, codes[j]))
                hi = Fraction(float(np.float16(127 * float(s16[j]))))
                lo = Fraction(float(np.float16(-128 * float(s16[j]))))
                step = float((hi - lo) / 255)          # fp64 division, as the reference
                r = float(Fraction(acc) * Fraction(sx)) * step  # exact acc*sx, one fp64 product
                y = np.float16(r)
                y = np.float16(float(y) + float(bias[j]))
                assert got[i, j].view(np.uint16) == y.view(np.uint16), (m, k, n, i, j)


def test_w8a8_quantization_error_bound():
    rng = np.random.default_rng(12)
    n, k, sx = 24, 256, 1 / 128
    data, scales = o.quantize(rng.standard_normal((n, k)) / 8, 'int8')
    x = (rng.standard_normal((4, k)) / 8).astype(np.float16)
    got = o.w8a8_linear(x, (n, k), data, scales, sx).astype(np.float64)
    w = o.exact_weight('int8', (n, k), k, data, scales)
    ideal = x.astype(np.float64) @ w.T
    qw = np.frombuffer(data, np.int8).reshape(n, k).astype(np.float64)
    step = o.w8a8_weight_steps(scales)
    xq = o.quantize_activations(x, sx) * sx
    bound = (sx / 2) * np.abs(w).sum(1)[None, :] + np.abs(xq) @ (np.abs(qw) * np.abs(step - np.frombuffer(scales, np.float16))[:, None]).T
    bound += np.finfo(np.float16).eps * np.abs(got) + 1e-6
    assert (np.abs(got - ideal) <= bound).all()
