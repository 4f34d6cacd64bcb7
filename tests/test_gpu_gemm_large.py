"""GPU parity of the 256 x 256 prefill GEMM (gemm4_kernel) against the CPU oracle.

Prefill calls whose 256 x 256 tiles give at least 160 workgroups (K a multiple of 64) run
there; calls with fewer, whose 256 x 128 tiles give 160 to 256 workgroups (rows past M adding at
most an eighth), run its eight-wave 256 x 128 form (4 x 2 waves of 64 x 64).  Same bars as every linear path: rel-L2 <= 1e-3 against the oracle and the reference's
rounding-budget gate (torch_npu_lowbit_demo.py:91-106), bit-exact for identity-like inputs with
power-of-two scales (torch_npu_lowbit_demo.py:124-128).  Shapes cover every format, partial
tiles in M and N, bias, per-row int8 scales and the rank-32 correction.
"""
import numpy as np
import pytest

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from test_gpu_linear import check, problem, run, to_dev

pytestmark = pytest.mark.gpu

LARGE = [
    ('int4', 2048, 6144, 256, 128), ('int4', 2000, 6100, 192, 64), ('int4', 1792, 7168, 128, 32),
    ('nf4', 2048, 6144, 128, 64), ('int8', 2048, 6144, 256, 256), ('int8', 1800, 6400, 128, 64),
    ('int4', 768, 14000, 128, 64), ('nf4', 700, 14336, 64, 64),
]


@pytest.mark.parametrize('spec', LARGE, ids=lambda s: '-'.join(map(str, s)))
def test_gemm4_matches_oracle(device, spec):
    fmt, m, n, k, group = spec
    announce('gemm4', spec)
    rng = np.random.default_rng(m + n + k + group)
    p = problem(rng, fmt, m, n, k, group)
    check(p, run(p, device), f'gemm4 {spec}')


# 256 x 128 tiles: fewer than 160 tiles of 256 x 256, 160 to 256 of 256 x 128.
TALL = [
    ('int4', 512, 12500, 256, 128), ('nf4', 480, 13000, 128, 64), ('int8', 1000, 6200, 192, 64),
    ('int8', 512, 12800, 128, 128),
]


@pytest.mark.parametrize('spec', TALL, ids=lambda s: '-'.join(map(str, s)))
def test_gemm4_tall_tiles_match_oracle(device, spec):
    fmt, m, n, k, group = spec
    announce('gemm4 256x128', spec)
    rng = np.random.default_rng(m + n + k + group + 1)
    p = problem(rng, fmt, m, n, k, group)
    check(p, run(p, device), f'gemm4 256x128 {spec}')


def test_gemm4_tall_tiles_bias_and_correction(device):
    spec = ('int4', 512, 12544, 128, 64)
    announce('gemm4 256x128 bias+correction', spec)
    rng = np.random.default_rng(77)
    p = problem(rng, *spec, rank=32, bias=True)
    check(p, run(p, device), f'gemm4 256x128 correction {spec}')


def test_gemm4_fp16_weights(device):
    """Dense fp16 weights (protected projections, tied head): fp16(x . W^T) in fp32 accumulation."""
    m, n, k = 2048, 6144, 192
    announce('gemm4 fp16')
    rng = np.random.default_rng(16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = lowbit_hip.linear(to_dev(x, device), to_dev(w, device), None, format='fp16', N=n, K=k,
                          group_size=k).cpu().numpy()
    want = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float16)
    assert o.rel_l2(y, want) <= 1e-3


@pytest.mark.parametrize('spec', [('int4', 2048, 6144, 128, 64), ('int8', 2048, 6144, 128, 128)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_gemm4_bias_and_correction(device, spec):
    fmt, m, n, k, group = spec
    announce('gemm4 bias+correction', spec)
    rng = np.random.default_rng(k * 7 + group)
    p = problem(rng, fmt, m, n, k, group, rank=32, bias=True)
    check(p, run(p, device), f'gemm4 correction {spec}')


def test_gemm4_identity_is_bit_exact(device):
    """x row m is one-hot at column m % K; power-of-two scales: y[m] is the dequantized column."""
    m, n, k, group = 2048, 6144, 128, 64
    announce('gemm4 identity')
    rng = np.random.default_rng(4)
    data = o.pack(rng.integers(0, 16, n * k).astype(np.uint8))
    scales = (2.0 ** rng.integers(-10, 3, n * (k // group))).astype(np.float16)
    w = o.dequantize('int4', (n, k), group, data, scales.tobytes())
    x = np.zeros((m, k), np.float16)
    x[np.arange(m), np.arange(m) % k] = 1.0
    y = lowbit_hip.linear(to_dev(x, device), to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                          format='int4', N=n, K=k, group_size=group).cpu().numpy()
    want = w[:, np.arange(m) % k].T
    np.testing.assert_array_equal(y.view(np.uint16), np.ascontiguousarray(want).view(np.uint16))
