"""GPU parity of the lane-linear one-row GEMVs (line_gemv_kernel, pack_gemv_kernel) against the CPU
oracle.

One-row INT4 / INT8 calls without a correction or prologue whose rows hold at least one segment
(64 lanes x one 16-byte load: 2048 INT4 / 1024 INT8 codes) run there without any flag.  A wave
reads 4 (rows of up to 4 segments) or 8 rows of one segment, 1 KB of each row per load, and the
lane's activations once; the sum is the exact x . (q s) product (magic-bias codes on
v_dot2_f32_f16 with the bias removed per lane; group scales per lane, or per lane quad once two
reduction levels have summed it; per-row scales on the row total).  The bars are those of every linear path: rel-L2 <= 1e-3 against the
oracle and the reference's rounding-budget gate (torch_npu_lowbit_demo.py:91-106), bit-exact for
identity inputs with power-of-two scales (torch_npu_lowbit_demo.py:124-128).  NF4 codes enter as the
fp16 literals of an LDS pair table (no bias).  Shapes cover 1..8 INT4 / NF4 and 1..16 INT8 segments, a partly filled last segment, row groups and workgroups past N,
groups of one lane pair, one quad and longer, per-row scales, bias and residual.  Rows shorter
than a segment take pack_gemv_kernel, which packs whole rows across a wave's lanes: four loads per
wave over at least 16384 rows (the SmolLM tied head), one load per wave for INT4 below that (the
SmolLM projections), and one to three problems sharing the activation row in one lb_fused_linear
(q|k|v, gate|up); its cases follow the same bars.
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from test_gpu_linear import check, problem, run, to_dev

pytestmark = pytest.mark.gpu

# (fmt, N, K, group)
LINE_SHAPES = [
    ('int4', 4096, 4096, 128),     # two segments, quad scales
    ('int4', 37, 2176, 128),       # one quad in the second segment, a partial row group and workgroup
    ('int4', 1000, 14336, 128),    # seven segments: one row group per workgroup
    ('int4', 520, 16384, 128),     # eight segments
    ('int4', 2056, 4096, 64),      # groups of two lanes: per-lane scales
    ('int4', 77, 3072, 64),        # half a second segment
    ('int4', 1032, 8192, 1024),    # groups of 32 lanes, four segments
    ('int4', 4104, 4096, 4096),    # one scale per row (row total)
    ('int8', 4096, 4096, 4096),    # per-row int8
    ('int8', 129, 1056, 1056),     # per-row, two live lanes in the second segment
    ('int8', 1040, 14336, 14336),  # fourteen segments (896-thread workgroups)
    ('int8', 528, 16384, 128),     # sixteen segments, quad scales
    ('int8', 2048, 4096, 64),      # groups of one lane quad
    ('int8', 2048, 1536, 32),      # groups of two lanes
    ('int8', 3000, 1024, 1024),    # exactly one segment
    ('nf4', 4096, 4096, 128),      # NF4: literals from the LDS pair table, quad scales
    ('nf4', 37, 2176, 128),        # one quad in the second segment
    ('nf4', 1000, 14336, 128),     # seven segments
    ('nf4', 2056, 4096, 64),       # groups of two lanes
    ('nf4', 4104, 4096, 4096),     # one scale per row (per-channel NF4)
]


@pytest.mark.parametrize('spec', LINE_SHAPES, ids=lambda s: '-'.join(map(str, s)))
def test_line_matches_oracle(device, spec):
    fmt, n, k, group = spec
    announce('line', spec)
    rng = np.random.default_rng(n + 7 * k + group)
    p = problem(rng, fmt, 1, n, k, group)
    check(p, run(p, device), f'line {spec}')


@pytest.mark.parametrize('spec', [('int4', 4096, 4096, 128), ('int4', 77, 3072, 64), ('int8', 2048, 4096, 4096)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_line_with_bias(device, spec):
    fmt, n, k, group = spec
    announce('line bias', spec)
    rng = np.random.default_rng(3 * n + k)
    p = problem(rng, fmt, 1, n, k, group, bias=True)
    check(p, run(p, device), f'line bias {spec}')


@pytest.mark.parametrize('fmt,group', [('int4', 128), ('int4', 64), ('int4', 4096), ('int8', 4096), ('int8', 64),
                                       ('nf4', 128), ('nf4', 4096)])
def test_line_identity_is_bit_exact(device, fmt, group):
    """One-hot activations and power-of-two scales: y is the dequantized column, bit for bit, for
    columns in every slot of a 16-byte load (even and odd INT4 nibbles) and in both segments."""
    n, k = 1000, 4096
    announce('line identity', fmt, group)
    rng = np.random.default_rng(group + (fmt == 'int8'))
    nibbles = fmt in ('int4', 'nf4')
    codes = rng.integers(0, 16, n * k).astype(np.uint8) if nibbles else rng.integers(-128, 128, n * k)
    data = o.pack(codes) if nibbles else codes.astype(np.int8).tobytes()
    g = k // group
    scales = (2.0 ** rng.integers(-12, 3, n * g)).astype(np.float16)
    w = o.dequantize(fmt, (n, k), group, data, scales.tobytes())
    dev_codes = to_dev(np.frombuffer(data, np.uint8), device)
    dev_scales = to_dev(scales, device)
    for col in (0, 1, 2, 3, 4, 5, 6, 7, 15, 31, 32, 33, 127, 128, 2047, 2048, 2049, k // 2 + 77, k - 1):
        x = np.zeros((1, k), np.float16)
        x[0, col] = 1.0
        y = lowbit_hip.linear(to_dev(x, device), dev_codes, dev_scales, format=fmt, N=n, K=k, group_size=group)
        np.testing.assert_array_equal(y.cpu().numpy()[0].view(np.uint16), w[:, col].view(np.uint16),
                                      err_msg=f'column {col}')


def test_line_zero_input_gives_zero(device):
    announce('line zero input')
    rng = np.random.default_rng(5)
    p = problem(rng, 'int4', 1, 8192, 4096, 128)
    p['x'] = np.zeros_like(p['x'])
    got = run(p, device)
    assert (got == 0).all()


@pytest.mark.parametrize('xscale', [1e-3, 30.0])
@pytest.mark.parametrize('fmt,group', [('int4', 128), ('int8', 4096)])
def test_line_activation_magnitudes(device, xscale, fmt, group):
    """Small (fp16-subnormal after the 1/16 staging of odd INT4 codes) and large activations."""
    announce('line xscale', xscale, fmt)
    rng = np.random.default_rng(11)
    p = problem(rng, fmt, 1, 8192, 4096, group, xscale=xscale)
    check(p, run(p, device), f'line xscale {xscale} {fmt}')


def test_line_agrees_with_tiled_gemv(device):
    """The forced tiled GEMV (fp16(q s) weights) and the line kernel (exact q s) on one problem."""
    announce('line vs gemv')
    rng = np.random.default_rng(31)
    p = problem(rng, 'int4', 1, 16384, 4096, 128)
    a = run(p, device)
    b = run(p, device, lowbit_hip.FLAG_FORCE_GEMV)
    assert o.rel_l2(a, b) <= 1e-3


@pytest.mark.parametrize('group', [1536, 32])
def test_line_residual_through_fused_linear(device, group):
    """One INT8 problem without prologue or correction in lb_fused_linear (K = 1536, one and a half
    segments): y = fp16(residual + fp16(x W^T)), with y and residual the same buffer."""
    n, k = 3000, 1536
    announce('line residual', group)
    rng = np.random.default_rng(21 + group)
    data = rng.integers(-127, 128, n * k).astype(np.int8).tobytes()
    g = k // group
    scales = (rng.uniform(0.5, 1.5, n * g) * (0.02 / 127)).astype(np.float16)
    x = rng.standard_normal((1, k)).astype(np.float16)
    residual = (rng.standard_normal(n) * 0.5).astype(np.float16)
    y = to_dev(residual, device)
    lowbit_hip.fused_linear(to_dev(x[0], device), [dict(codes=to_dev(np.frombuffer(data, np.uint8), device),
                                                        scales=to_dev(scales, device), N=n, y=y, residual=y)],
                            format='int8', K=k, group_size=group)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    plain = o.linear(x, 'int8', (n, k), group, data, scales.tobytes())[0]
    want = (residual.astype(np.float32) + plain.astype(np.float32)).astype(np.float16)
    assert o.rel_l2(got, want) <= 1e-3
    budget = o.rounding_budget(x, 'int8', (n, k), group, data, scales.tobytes())[0]
    ulp = (np.abs(want.astype(np.float64)) + np.abs(plain.astype(np.float64))) * 2.0 ** -10 + 2.0 ** -24
    assert (np.abs(got.astype(np.float64) - want.astype(np.float64)) <= budget + ulp).all()


def test_line_repeated_calls_are_deterministic(device):
    """Segment sums meet in a fixed order: the same call twice gives the same bits."""
    announce('line determinism')
    rng = np.random.default_rng(41)
    p = problem(rng, 'int4', 1, 4096, 14336, 128)
    a = run(p, device)
    b = run(p, device)
    np.testing.assert_array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize('spec', [('int4', 1000, 4096, 128), ('int4', 77, 3072, 64), ('int8', 129, 1056, 1056)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_line_row_reversal_is_bit_exact(device, spec):
    """Each row's sum has one association whatever its position in a wave's row group: the weight
    rows reversed give the outputs reversed, bit for bit."""
    fmt, n, k, group = spec
    announce('line row reversal', spec)
    rng = np.random.default_rng(53 + n)
    p = problem(rng, fmt, 1, n, k, group)
    row_bytes = k // 2 if fmt == 'int4' else k
    rev = dict(p)
    rev['data'] = np.frombuffer(p['data'], np.uint8).reshape(n, row_bytes)[::-1].tobytes()
    rev['scales'] = np.frombuffer(p['scales'], np.float16).reshape(n, k // group)[::-1].tobytes()
    a = run(p, device)
    b = run(rev, device)
    np.testing.assert_array_equal(b[0][::-1].view(np.uint16), a[0].view(np.uint16))


# Rows shorter than a segment over at least 16384 rows: pack_gemv_kernel packs whole rows across a
# wave's lanes (P = 64 // S rows of S 16-byte slots per wave-wide load).  (fmt, N, K, group)
PACK_SHAPES = [
    ('int4', 49152, 576, 64),      # the SmolLM tied head: 3 rows in 54 lanes
    ('int4', 16400, 576, 576),     # one scale per row, a partial last workgroup
    ('int4', 20000, 1536, 128),    # one row per load (48 lanes)
    ('int4', 16416, 256, 32),      # eight rows per load, groups of one lane
    ('int4', 16390, 992, 32),      # two rows per load (62 lanes), ragged N
    ('int8', 20000, 576, 576),     # per-row int8, one row per load (36 lanes)
    ('int8', 16400, 992, 32),      # int8 groups of two lanes, 62 lanes
    # below 16384 rows (INT4): one load per wave
    ('int4', 576, 576, 64),        # SmolLM q / o: 3 rows per wave
    ('int4', 192, 576, 64),        # SmolLM k / v
    ('int4', 576, 1536, 128),      # SmolLM down: one row per wave (48 lanes)
    ('int4', 1536, 576, 32),       # SmolLM gate / up with groups of one lane
    ('int4', 5, 992, 32),          # two rows per load, one partly filled wave
    ('int4', 1000, 256, 64),       # eight rows per load, 125 waves
    ('int4', 16383, 576, 64),      # one row short of the four-load kernel
]


@pytest.mark.parametrize('spec', PACK_SHAPES, ids=lambda s: '-'.join(map(str, s)))
def test_pack_matches_oracle(device, spec):
    fmt, n, k, group = spec
    announce('pack', spec)
    rng = np.random.default_rng(n + 3 * k + group)
    p = problem(rng, fmt, 1, n, k, group)
    check(p, run(p, device), f'pack {spec}')


def test_pack_with_bias(device):
    announce('pack bias')
    rng = np.random.default_rng(17)
    p = problem(rng, 'int4', 1, 16400, 576, 64, bias=True)
    check(p, run(p, device), 'pack bias')


@pytest.mark.parametrize('fmt,group', [('int4', 64), ('int8', 576)])
def test_pack_identity_is_bit_exact(device, fmt, group):
    n, k = 16384, 576
    announce('pack identity', fmt, group)
    rng = np.random.default_rng(group + 5)
    codes = rng.integers(0, 16, n * k).astype(np.uint8) if fmt == 'int4' else rng.integers(-128, 128, n * k)
    data = o.pack(codes) if fmt == 'int4' else codes.astype(np.int8).tobytes()
    g = k // group
    scales = (2.0 ** rng.integers(-12, 3, n * g)).astype(np.float16)
    w = o.dequantize(fmt, (n, k), group, data, scales.tobytes())
    dev_codes = to_dev(np.frombuffer(data, np.uint8), device)
    dev_scales = to_dev(scales, device)
    for col in (0, 1, 7, 31, 32, 33, 287, 288, 289, k - 1):
        x = np.zeros((1, k), np.float16)
        x[0, col] = 1.0
        y = lowbit_hip.linear(to_dev(x, device), dev_codes, dev_scales, format=fmt, N=n, K=k, group_size=group)
        np.testing.assert_array_equal(y.cpu().numpy()[0].view(np.uint16), w[:, col].view(np.uint16),
                                      err_msg=f'column {col}')


@pytest.mark.parametrize('spec', [('int4', 16390, 576, 64), ('int4', 16390, 992, 32), ('int4', 578, 576, 64),
                                  ('int4', 1000, 1536, 128)], ids=lambda s: '-'.join(map(str, s)))
def test_pack_row_reversal_is_bit_exact(device, spec):
    """A row's sum is its slots' partials in slot order, whatever lanes the row falls to."""
    fmt, n, k, group = spec
    announce('pack row reversal', spec)
    rng = np.random.default_rng(59 + k)
    p = problem(rng, fmt, 1, n, k, group)
    row_bytes = k // 2
    rev = dict(p)
    rev['data'] = np.frombuffer(p['data'], np.uint8).reshape(n, row_bytes)[::-1].tobytes()
    rev['scales'] = np.frombuffer(p['scales'], np.float16).reshape(n, k // group)[::-1].tobytes()
    a = run(p, device)
    b = run(rev, device)
    np.testing.assert_array_equal(b[0][::-1].view(np.uint16), a[0].view(np.uint16))


def test_pack_residual_through_fused_linear(device):
    """One INT4 problem without prologue or correction in lb_fused_linear over 20000 rows of 576:
    y = fp16(residual + fp16(x W^T)), y and residual the same buffer."""
    n, k, group = 20000, 576, 64
    announce('pack residual')
    rng = np.random.default_rng(23)
    data = rng.integers(0, 256, n * k // 2).astype(np.uint8).tobytes()
    g = k // group
    scales = (rng.uniform(0.5, 1.5, n * g) * (0.02 / 7)).astype(np.float16)
    x = rng.standard_normal((1, k)).astype(np.float16)
    residual = (rng.standard_normal(n) * 0.5).astype(np.float16)
    y = to_dev(residual, device)
    lowbit_hip.fused_linear(to_dev(x[0], device), [dict(codes=to_dev(np.frombuffer(data, np.uint8), device),
                                                        scales=to_dev(scales, device), N=n, y=y, residual=y)],
                            format='int4', K=k, group_size=group)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    plain = o.linear(x, 'int4', (n, k), group, data, scales.tobytes())[0]
    want = (residual.astype(np.float32) + plain.astype(np.float32)).astype(np.float16)
    assert o.rel_l2(got, want) <= 1e-3
    budget = o.rounding_budget(x, 'int4', (n, k), group, data, scales.tobytes())[0]
    ulp = (np.abs(want.astype(np.float64)) + np.abs(plain.astype(np.float64))) * 2.0 ** -10 + 2.0 ** -24
    assert (np.abs(got.astype(np.float64) - want.astype(np.float64)) <= budget + ulp).all()


# Several problems sharing the activation row in one lb_fused_linear call (no prologue or
# correction): each problem's rows over its own waves of pack_gemv_kernel.  (fmt, group, K, rows of
# each problem, bias on, residual on)
PACK_MULTI = [
    ('int4', 64, 576, (576, 192, 192), (), ()),            # SmolLM q|k|v: one load per wave
    ('int4', 64, 576, (1536, 1536), (), ()),               # SmolLM gate|up
    ('int4', 32, 576, (100, 7, 33), (1,), (0, 2)),         # ragged rows, bias and residual
    ('int4', 128, 1536, (10000, 8000), (0,), ()),          # 18000 rows: four loads per wave
    ('int8', 576, 576, (9000, 8000, 5), (), (1,)),         # per-row int8 over 17005 rows
]


@pytest.mark.parametrize('spec', PACK_MULTI, ids=lambda s: f'{s[0]}-g{s[1]}-k{s[2]}-' + 'x'.join(map(str, s[3])))
def test_pack_problems_through_fused_linear(device, spec):
    """Every problem equals its own one-problem product: fp16(x W^T) (+ bias) (+ residual, y and
    residual the same buffer), checked against the oracle at the linear path's bars."""
    fmt, group, k, rows, with_bias, with_res = spec
    announce('pack problems', spec)
    rng = np.random.default_rng(sum(rows) + k + group)
    x = rng.standard_normal((1, k)).astype(np.float16)
    problems, refs = [], []
    for j, n in enumerate(rows):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        data, scales = o.quantize(w, fmt, group)
        bias = (rng.standard_normal(n) * 0.1).astype(np.float16) if j in with_bias else None
        res = (rng.standard_normal(n) * 0.5).astype(np.float16) if j in with_res else None
        y = to_dev(res, device) if res is not None else torch.empty(n, dtype=torch.float16, device=device)
        pr = dict(codes=to_dev(np.frombuffer(data, np.uint8), device),
                  scales=to_dev(np.frombuffer(scales, np.float16), device), N=n, y=y)
        if bias is not None:
            pr['bias'] = to_dev(bias, device)
        if res is not None:
            pr['residual'] = y
        problems.append(pr)
        refs.append((data, scales, bias, res))
    outs = lowbit_hip.fused_linear(to_dev(x[0], device), problems, format=fmt, K=k, group_size=group)
    torch.cuda.synchronize()
    for j, (n, out, (data, scales, bias, res)) in enumerate(zip(rows, outs, refs)):
        got = out.cpu().numpy()
        plain = o.linear(x, fmt, (n, k), group, data, scales)[0]
        want = plain
        if bias is not None:
            want = (want.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
        if res is not None:
            want = (res.astype(np.float32) + want.astype(np.float32)).astype(np.float16)
        assert np.isfinite(got).all(), f'problem {j}'
        assert o.rel_l2(got, want) <= 1e-3, f'problem {j}: rel-L2 {o.rel_l2(got, want):.3e}'
        if bias is None and res is None:
            budget = o.rounding_budget(x, fmt, (n, k), group, data, scales)[0]
            ulp = np.abs(want.astype(np.float64)) * 2.0 ** -10 + 2.0 ** -24
            assert (np.abs(got.astype(np.float64) - want.astype(np.float64)) <= budget + ulp).all(), f'problem {j}'


def test_pack_problems_match_single_calls(device):
    """q|k|v in one call gives, bit for bit, what three one-problem calls give."""
    announce('pack problems vs single')
    k, group, rows = 576, 64, (576, 192, 192)
    rng = np.random.default_rng(71)
    x = to_dev(rng.standard_normal(k).astype(np.float16), device)
    problems, singles = [], []
    for n in rows:
        data, scales = o.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), 'int4', group)
        codes = to_dev(np.frombuffer(data, np.uint8), device)
        sc = to_dev(np.frombuffer(scales, np.float16), device)
        problems.append(dict(codes=codes, scales=sc, N=n, y=torch.empty(n, dtype=torch.float16, device=device)))
        singles.append(lowbit_hip.fused_linear(x, [dict(codes=codes, scales=sc, N=n,
                                                        y=torch.empty(n, dtype=torch.float16, device=device))],
                                               format='int4', K=k, group_size=group)[0])
    outs = lowbit_hip.fused_linear(x, problems, format='int4', K=k, group_size=group)
    torch.cuda.synchronize()
    for a, b in zip(outs, singles):
        np.testing.assert_array_equal(a.cpu().numpy().view(np.uint16), b.cpu().numpy().view(np.uint16))
