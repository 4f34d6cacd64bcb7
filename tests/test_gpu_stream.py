"""GPU parity of the streaming one-row GEMV (stream_gemv_kernel) against the CPU oracle.

One-row lb_linear calls over at least 64 MB of INT4 weights whose rows are shorter than a segment
of the lane-linear kernel (2048 codes) run there; the tests force it (LB_FLAG_FORCE_STREAM) on
other shapes.  It sums
x . (q + magic bias) on MFMA and applies the group scale per 32- or 16-code block, so its
value is the exact x . (q s) product; the bars are those of every linear path: rel-L2 <= 1e-3
against the oracle and the reference's rounding-budget gate (torch_npu_lowbit_demo.py:91-106),
bit-exact for identity inputs with power-of-two scales (torch_npu_lowbit_demo.py:124-128).
Shapes cover both launch modes (persistent waves; K split over a workgroup's waves), every
group span (1, 2 or 4 groups per 16-byte load), partial tiles and chunks, bias and residual.
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from test_gpu_linear import check, problem, run, to_dev

pytestmark = pytest.mark.gpu
STREAM = lowbit_hip.FLAG_FORCE_STREAM

# (fmt, N, K, group)
STREAM_SHAPES = [
    ('int4', 4096, 4096, 128),     # K split over the waves (256 tiles)
    ('int4', 16384, 4096, 128),    # persistent waves
    ('int4', 49152, 576, 64),      # the SmolLM tied-head shape, two groups per load
    ('int4', 8200, 576, 32),       # four groups per load, a partial last tile
    ('int4', 2056, 4096, 64),      # two groups per load, split, partial tile
    ('int4', 520, 16384, 128),     # the longest staged row
    ('int4', 1032, 14336, 128),    # 14 chunks over 4 waves
    ('int4', 4104, 4096, 4096),    # one group per row
    ('int4', 9000, 1536, 512),     # group spanning four loads, 1536-code rows
    ('int8', 4096, 4096, 4096),    # per-row int8 (scale on the row total), split
    ('int8', 4104, 576, 576),      # per-row int8, ten loads per chunk, persistent
    ('int8', 20000, 1536, 1536),   # per-row int8, persistent
    ('int8', 2048, 4096, 64),      # int8 groups: one per load
    ('int8', 2048, 2048, 32),      # two per load
    ('int8', 2064, 1024, 16),      # four per load
]


@pytest.mark.parametrize('spec', STREAM_SHAPES, ids=lambda s: '-'.join(map(str, s)))
def test_stream_matches_oracle(device, spec):
    fmt, n, k, group = spec
    announce('stream', spec)
    rng = np.random.default_rng(n + 7 * k + group)
    p = problem(rng, fmt, 1, n, k, group)
    check(p, run(p, device, STREAM), f'stream {spec}')


@pytest.mark.parametrize('spec', [('int4', 8192, 576, 64), ('int4', 4096, 4096, 128), ('int8', 4096, 2048, 2048)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_stream_with_bias(device, spec):
    fmt, n, k, group = spec
    announce('stream bias', spec)
    rng = np.random.default_rng(3 * n + k)
    p = problem(rng, fmt, 1, n, k, group, bias=True)
    check(p, run(p, device, STREAM), f'stream bias {spec}')


@pytest.mark.parametrize('fmt,group', [('int4', 128), ('int4', 64), ('int4', 32), ('int8', 4096), ('int8', 64)])
def test_stream_identity_is_bit_exact(device, fmt, group):
    """One-hot activations and power-of-two scales: y is the dequantized column, bit for bit."""
    n, k = (4096, 4096) if group != 32 else (8192, 1024)
    announce('stream identity', fmt, group)
    rng = np.random.default_rng(group)
    codes = rng.integers(0, 16, n * k).astype(np.uint8) if fmt == 'int4' else rng.integers(-128, 128, n * k)
    data = o.pack(codes) if fmt == 'int4' else codes.astype(np.int8).tobytes()
    g = k // group
    scales = (2.0 ** rng.integers(-12, 3, n * g)).astype(np.float16)
    w = o.dequantize(fmt, (n, k), group, data, scales.tobytes())
    dev_codes = to_dev(np.frombuffer(data, np.uint8), device)
    dev_scales = to_dev(scales, device)
    for col in (0, 1, 31, 32, 33, 127, 128, k // 2 + 5, k - 1):
        x = np.zeros((1, k), np.float16)
        x[0, col] = 1.0
        y = lowbit_hip.linear(to_dev(x, device), dev_codes, dev_scales, format=fmt, N=n, K=k, group_size=group,
                              flags=STREAM)
        np.testing.assert_array_equal(y.cpu().numpy()[0].view(np.uint16), w[:, col].view(np.uint16),
                                      err_msg=f'column {col}')


def test_stream_zero_input_gives_zero(device):
    announce('stream zero input')
    rng = np.random.default_rng(5)
    p = problem(rng, 'int4', 1, 8192, 4096, 128)
    p['x'] = np.zeros_like(p['x'])
    got = run(p, device, STREAM)
    assert (got == 0).all()


@pytest.mark.parametrize('xscale', [1e-3, 30.0])
def test_stream_activation_magnitudes(device, xscale):
    """Small (fp16-subnormal after the 1/16 staging) and large activations stay within the bars."""
    announce('stream xscale', xscale)
    rng = np.random.default_rng(11)
    p = problem(rng, 'int4', 1, 8192, 4096, 128, xscale=xscale)
    check(p, run(p, device, STREAM), f'stream xscale {xscale}')


@pytest.mark.parametrize('fmt,group', [('int4', 64), ('int4', 576)])
def test_stream_residual_through_fused_linear(device, fmt, group):
    """One INT4 problem without prologue or correction in lb_fused_linear, above the size
    threshold: y = fp16(residual + fp16(x W^T)).  Random codes; the oracle checks row slices."""
    n, k = 262144 if fmt == 'int4' else 131072, 576
    announce('stream residual', fmt, group)
    rng = np.random.default_rng(21)
    if fmt == 'int4':
        data = rng.integers(0, 256, n * k // 2).astype(np.uint8).tobytes()
    else:
        data = rng.integers(-127, 128, n * k).astype(np.int8).tobytes()
    g = k // group
    scales = (rng.uniform(0.5, 1.5, n * g) * (0.02 / 7 if fmt == 'int4' else 0.02 / 127)).astype(np.float16)
    x = rng.standard_normal((1, k)).astype(np.float16)
    residual = (rng.standard_normal(n) * 0.5).astype(np.float16)
    y = to_dev(residual, device)
    lowbit_hip.fused_linear(to_dev(x[0], device), [dict(codes=to_dev(np.frombuffer(data, np.uint8), device),
                                                        scales=to_dev(scales, device), N=n, y=y, residual=y)],
                            format=fmt, K=k, group_size=group)
    torch.cuda.synchronize()
    got_all = y.cpu().numpy()
    row_bytes = k // 2 if fmt == 'int4' else k
    for lo in (0, n // 2 + 16, n - 4096):
        rows = slice(lo, lo + 4096)
        d = data[lo * row_bytes:(lo + 4096) * row_bytes]
        sc = scales[lo * g:(lo + 4096) * g].tobytes()
        plain = o.linear(x, fmt, (4096, k), group, d, sc)[0]
        want = (residual[rows].astype(np.float32) + plain.astype(np.float32)).astype(np.float16)
        got = got_all[rows]
        assert o.rel_l2(got, want) <= 1e-3
        budget = o.rounding_budget(x, fmt, (4096, k), group, d, sc)[0]
        ulp = (np.abs(want.astype(np.float64)) + np.abs(plain.astype(np.float64))) * 2.0 ** -10 + 2.0 ** -24
        assert (np.abs(got.astype(np.float64) - want.astype(np.float64)) <= budget + ulp).all(), f'rows from {lo}'


def test_stream_agrees_with_tiled_gemv(device):
    """The forced tiled GEMV (fp16(q s) weights) and the stream kernel (exact q s) on one problem."""
    announce('stream vs gemv')
    rng = np.random.default_rng(31)
    p = problem(rng, 'int4', 1, 16384, 4096, 128)
    a = run(p, device, STREAM)
    b = run(p, device, lowbit_hip.FLAG_FORCE_GEMV)
    assert o.rel_l2(a, b) <= 1e-3


@pytest.mark.parametrize('spec', [('int8', 1040, 14336, 14336), ('int8', 528, 16384, 128), ('int4', 1024, 8192, 64)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_stream_long_rows(device, spec):
    """Rows past the single-tile kernels' K limit (int8 K > 8192) or longer than 4096 codes, forced
    onto the stream kernel (unforced they take the lane-linear kernel); same bars."""
    fmt, n, k, group = spec
    announce('stream long rows', spec)
    rng = np.random.default_rng(n + k)
    p = problem(rng, fmt, 1, n, k, group)
    check(p, run(p, device, STREAM), f'long rows {spec}')


# Several activation rows (2 <= M <= 16, K <= 4096): each MFMA A row spans more code blocks as M
# grows, so INT4 needs groups >= 64 up to 8 rows and >= 128 beyond; INT8 one scale per 64 codes.
ROWS_CASES = [
    ('int4', 2, 1040, 4096, 128), ('int4', 3, 1040, 2048, 64), ('int4', 4, 2064, 4096, 64),
    ('int4', 5, 1040, 4096, 128), ('int4', 8, 1040, 1024, 64), ('int4', 11, 1040, 4096, 128),
    ('int4', 16, 1040, 4096, 4096), ('int4', 16, 16400, 1024, 128),   # the last one: persistent waves
    ('int4', 4, 16400, 576, 64),
    ('int8', 2, 1040, 4096, 4096), ('int8', 7, 1040, 2048, 2048), ('int8', 16, 1040, 4096, 4096),
    ('int8', 3, 1040, 4096, 64), ('int8', 12, 16400, 1024, 128),
    # 17 .. 32 rows (K-outer chunks): ragged N, groups of 32, K past 4096, per-row and grouped int8
    ('int4', 17, 1040, 4096, 128), ('int4', 25, 1000, 4096, 128), ('int4', 24, 2064, 1024, 32),
    ('int4', 32, 16400, 2048, 64), ('int4', 32, 1040, 8192, 128), ('int4', 29, 1040, 576, 64),
    ('int8', 20, 1040, 4096, 4096), ('int8', 32, 1040, 2048, 64),
]


@pytest.mark.parametrize('spec', ROWS_CASES, ids=lambda s: '-'.join(map(str, s)))
def test_stream_rows_match_oracle(device, spec):
    fmt, m, n, k, group = spec
    announce('stream rows', spec)
    rng = np.random.default_rng(m * 131 + n + k + group)
    p = problem(rng, fmt, m, n, k, group, bias=(m % 2 == 1))
    check(p, run(p, device, STREAM), f'stream rows {spec}')


def test_stream_rows_strided_activations_and_outputs(device):
    """x rows with ldx > K and y rows with ldy > N (views into wider buffers)."""
    m, n, k, group = 6, 2064, 2048, 128
    announce('stream rows strided')
    rng = np.random.default_rng(77)
    p = problem(rng, 'int4', m, n, k, group)
    wide = torch.zeros((m, k + 64), dtype=torch.float16, device=device)
    wide[:, 8:8 + k] = to_dev(p['x'], device)
    out = torch.full((m, n + 40), 7.0, dtype=torch.float16, device=device)
    y = lowbit_hip.linear(wide[:, 8:8 + k], to_dev(np.frombuffer(p['data'], np.uint8), device),
                          to_dev(np.frombuffer(p['scales'], np.float16), device), format='int4', N=n, K=k,
                          group_size=group, flags=STREAM, out=out[:, 16:16 + n])
    torch.cuda.synchronize()
    check(p, y.cpu().numpy(), 'stream rows strided')
    untouched = torch.cat([out[:, :16], out[:, 16 + n:]], dim=1)
    assert (untouched == 7.0).all()


def test_stream_rows_identity_is_bit_exact(device):
    """Row m of x is one-hot at column c_m (power-of-two scales): y[m] is the dequantized column."""
    m, n, k, group = 8, 1040, 2048, 64
    announce('stream rows identity')
    rng = np.random.default_rng(8)
    data = o.pack(rng.integers(0, 16, n * k).astype(np.uint8))
    scales = (2.0 ** rng.integers(-10, 3, n * (k // group))).astype(np.float16)
    w = o.dequantize('int4', (n, k), group, data, scales.tobytes())
    cols = [0, 1, 33, 64, 127, 1000, 2046, 2047]
    x = np.zeros((m, k), np.float16)
    for r, c in enumerate(cols):
        x[r, c] = 1.0
    y = lowbit_hip.linear(to_dev(x, device), to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                          format='int4', N=n, K=k, group_size=group, flags=STREAM).cpu().numpy()
    for r, c in enumerate(cols):
        np.testing.assert_array_equal(y[r].view(np.uint16), w[:, c].view(np.uint16), err_msg=f'row {r}')


@pytest.mark.parametrize('spec', [('int4', 8, 32768, 4096, 128), ('int8', 3, 16384, 4096, 4096),
                                  ('int4', 32, 32768, 4096, 128), ('int8', 20, 32768, 4096, 4096)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_stream_rows_unforced(device, spec):
    """Several rows over >= 64 MB of weights take the stream kernel without a flag; random codes,
    the oracle checks row slices (same bars)."""
    fmt, m, n, k, group = spec
    announce('stream rows auto', spec)
    rng = np.random.default_rng(n * m)
    if fmt == 'int4':
        data = rng.integers(0, 256, n * k // 2).astype(np.uint8).tobytes()
    else:
        data = rng.integers(-127, 128, n * k).astype(np.int8).tobytes()
    g = k // group
    scales = (rng.uniform(0.5, 1.5, n * g) * (0.02 / 7 if fmt == 'int4' else 0.02 / 127)).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = lowbit_hip.linear(to_dev(x, device), to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                          format=fmt, N=n, K=k, group_size=group).cpu().numpy()
    row_bytes = k // 2 if fmt == 'int4' else k
    for lo in (0, n // 2 + 16, n - 2048):
        d = data[lo * row_bytes:(lo + 2048) * row_bytes]
        sc = scales[lo * g:(lo + 2048) * g].tobytes()
        p = dict(fmt=fmt, m=m, n=2048, k=k, group=group, x=x, data=d, scales=sc, bias=None, down=None, up=None)
        check(p, np.ascontiguousarray(y[:, lo:lo + 2048]), f'stream rows auto {spec} rows from {lo}')
