"""GPU parity of the two graph variants of the low-bit linear: compact_groups and W8A8.

W8A8 (activation_scale; torch_npu_lowbit.py:224-231, reference values torch_npu_int8_demo.py:34-51):
the integer sum is exact and the scaling one fp64 product rounded once, so every path must be
bit-exact against the oracle; the reference's own exact cases are replayed first.

compact_groups (torch_npu_lowbit.py:235-256): each group's fp16 product, then the balanced fp16
tree.  Pieces built from integer products are exact, so the tree order is checked bit for bit;
random inputs meet the reference's gate (rel-L2 < 1e-3 against the fp64 ideal and the per-output
budget (depth + 3) eps16 |x||W| + 3e-4, torch_npu_lowbit_group_demo.py:161-170) and stay within
rel-L2 1e-3 of the oracle, whose pieces are accumulated in fp64.
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from torch_npu_lowbit import PackedWeight, QuantizedLinear, pack_codes, quantize_weight

pytestmark = pytest.mark.gpu
PATHS = {'gemv': lowbit_hip.FLAG_FORCE_GEMV, 'gemm': lowbit_hip.FLAG_FORCE_GEMM,
         'generic': lowbit_hip.FLAG_FORCE_GENERIC, 'auto': 0}


def dev(a, device):
    return torch.from_numpy(np.array(a, copy=True)).to(device)


def run(device, x, fmt, shape, group, data, scales, *, bias=None, flags=0, activation_scale=None):
    n, k = shape
    kw = {} if bias is None else dict(bias=dev(bias, device))
    y = lowbit_hip.linear(dev(x, device), dev(np.frombuffer(data, np.uint8), device),
                          dev(np.frombuffer(scales, np.float16), device), format=fmt, N=n, K=k, group_size=group,
                          flags=flags, activation_scale=activation_scale, **kw)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def bits(a):
    return np.asarray(a, np.float16).view(np.uint16)


# ---------------------------------------------------------------- W8A8
def test_w8a8_reference_exact_cases(device):
    """torch_npu_int8_demo.py 'numeric' / 'edges' cases with exact=True, through QuantizedLinear."""
    announce('w8a8 exact cases')
    codes = np.arange(-128, 128, dtype=np.int8)
    for sc in (0.125, 1.0, 16.0):
        q = PackedWeight((1, 256), 'int8', 256, codes.tobytes(), np.float16(sc).tobytes())
        got = QuantizedLinear(q, activation_scale=1 / 64)(torch.eye(256, dtype=torch.float16, device=device))
        np.testing.assert_array_equal(got.cpu().numpy().ravel().astype(np.float64), codes * sc)
    eye = PackedWeight((256, 256), 'int8', 256, np.eye(256, dtype=np.int8).tobytes(), np.ones(256, np.float16).tobytes())
    grid = torch.arange(-128, 128, dtype=torch.float16) / 128
    x = torch.stack((grid, grid + 1 / 256, grid - 1 / 256, grid * 2))
    got = QuantizedLinear(eye, activation_scale=1 / 128)(x.to(device)).cpu().numpy()
    want = o.w8a8_linear(x.numpy(), (256, 256), eye.data, eye.scales, 1 / 128)
    np.testing.assert_array_equal(bits(got), bits(want))
    big = np.stack((np.full(4096, 127, np.int8), np.tile([127, -127], 2048).astype(np.int8)))
    q = PackedWeight((2, 4096), 'int8', 4096, big.tobytes(), np.full(2, 1 / 128, np.float16).tobytes())
    got = QuantizedLinear(q, activation_scale=1 / 128)(torch.full((1, 4096), 127 / 128, dtype=torch.float16,
                                                                  device=device))
    assert got.cpu().tolist() == [[4032.0, 0.0]]
    eye16 = PackedWeight((16, 16), 'int8', 16, np.eye(16, dtype=np.int8).tobytes(), np.ones(16, np.float16).tobytes())
    for s in (2.0 ** -24, 2.0 ** -14, 256.0):
        x16 = (torch.arange(-8, 8, dtype=torch.float64) * s).half().view(1, 16)
        got = QuantizedLinear(eye16, activation_scale=s)(x16.to(device))
        np.testing.assert_array_equal(bits(got.cpu().numpy()), bits(x16.numpy()))
    zero = quantize_weight(torch.zeros(3, 17), format='int8')
    for scale in (None, 1 / 128):
        got = QuantizedLinear(zero, activation_scale=scale)(torch.ones(2, 17, dtype=torch.float16, device=device))
        assert not got.cpu().any()


@pytest.mark.parametrize('m,n,k', [(1, 3, 17), (5, 32, 64), (7, 13, 64), (65, 67, 256), (1, 4096, 4096),
                                   (8, 1000, 1024), (32, 576, 1536), (200, 576, 576), (512, 1536, 576)])
@pytest.mark.parametrize('path', ['auto', 'gemv', 'gemm', 'generic'])
def test_w8a8_bit_exact(device, m, n, k, path):
    if path == 'gemv' and m > 32:
        pytest.skip('GEMV takes M <= 32')
    if path in ('gemv', 'gemm') and k % 64:
        pytest.skip('the int8 MFMA paths need K % 64 == 0')
    announce('w8a8', m, n, k, path)
    x, data, scales, bias, wants = w8a8_case(m, n, k)
    for sx, want in wants.items():
        got = run(device, x, 'int8', (n, k), k, data, scales, bias=bias, flags=PATHS[path], activation_scale=sx)
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=f'{m}x{n}x{k} {path} s_x={sx}')


_W8A8_CASES = {}


def w8a8_case(m, n, k):
    """Seeded inputs and the oracle outputs at s_x = 1/128 and 1/256 (computed once per shape)."""
    if (m, n, k) not in _W8A8_CASES:
        rng = np.random.default_rng(m * 7919 + n * 31 + k)
        data, scales = o.quantize(rng.standard_normal((n, k)) / 8, 'int8')
        x = (rng.standard_normal((m, k)) / 8).astype(np.float16)
        bias = (rng.standard_normal(n) / 8).astype(np.float16) if m % 2 else None
        wants = {sx: o.w8a8_linear(x, (n, k), data, scales, sx, bias=bias) for sx in (1 / 128, 1 / 256)}
        _W8A8_CASES[(m, n, k)] = (x, data, scales, bias, wants)
    return _W8A8_CASES[(m, n, k)]


# ---------------------------------------------------------------- compact_groups
def test_compact_reference_edges(device):
    """torch_npu_lowbit_group_demo.py 'edges': all codes in two groups, zero groups of 3, and the
    documented partial-overflow limitation."""
    announce('compact edges')
    for fmt in ('int4', 'nf4'):
        for scale in (0.125, 1.0, 16.0):
            q = PackedWeight((1, 16), fmt, 8, pack_codes(np.arange(16, dtype=np.uint8)),
                             np.full(2, scale, dtype=np.float16).tobytes())
            got = QuantizedLinear(q, compact_groups=True)(torch.eye(16, dtype=torch.float16, device=device))
            np.testing.assert_array_equal(bits(got.cpu().numpy()), bits(q.dequantize().T))
        q = quantize_weight(torch.zeros(5, 9), format=fmt, group_size=3)
        got = QuantizedLinear(q, compact_groups=True)(torch.ones(7, 9, dtype=torch.float16, device=device))
        assert torch.count_nonzero(got) == 0
        positive, negative, activation = (7, 13, 1024.0) if fmt == 'int4' else (15, 0, 4096.0)
        scales = np.array([1.0, 2.0] if fmt == 'int4' else [1.0, 0.5], dtype=np.float16)
        q = PackedWeight((1, 32), fmt, 16, pack_codes(np.array([positive] * 16 + [negative] * 16, np.uint8)),
                         scales.tobytes())
        x = torch.full((1, 32), activation, dtype=torch.float16, device=device)
        expected = float((x.cpu().double() @ torch.from_numpy(q.dequantize().astype(np.float64)).t()).item())
        assert QuantizedLinear(q)(x).item() == expected
        assert QuantizedLinear(q, compact_groups=True)(x).item() != expected


def pieces_weight(values, group):
    codes = np.zeros((1, group * len(values)), np.int8)
    for g, v in enumerate(values):
        q, r = divmod(v, group)
        codes[0, g * group:(g + 1) * group] = q
        codes[0, g * group:g * group + r] += 1
    return codes.tobytes(), np.ones(len(values), np.float16).tobytes()


@pytest.mark.parametrize('path', ['auto', 'gemv', 'gemm', 'generic'])
@pytest.mark.parametrize('m', [1, 64])
def test_compact_tree_order_exact(device, path, m):
    """Integer pieces are exact, so the result shows the pairing: 2054 for eight pieces
    [2048, 1 x 7] (sequential addition gives 2048, one rounding 2056)."""
    if path == 'gemv' and m > 32:
        pytest.skip('GEMV takes M <= 32')
    announce('compact tree', path, m)
    for values, want in (([2048] + [1] * 7, 2054.0), ([2048, 1, 1, 1, 1], 2052.0), ([1] * 32, 32.0)):
        group = 64
        data, scales = pieces_weight(values, group)
        k = group * len(values)
        x = np.ones((m, k), np.float16)
        got = run(device, x, 'int8', (1, k), group, data, scales, flags=lowbit_hip.FLAG_COMPACT_GROUPS | PATHS[path])
        assert (got == want).all(), (values, path, got.ravel()[:4])
        np.testing.assert_array_equal(bits(got), bits(o.compact_linear(x, 'int8', (1, k), group, data, scales)))


def reference_gate(x, fmt, shape, group, data, scales, got, bias=None):
    n, k = shape
    real = o.exact_weight(fmt, shape, group, data, scales)
    ideal = np.asarray(x, np.float16).astype(np.float64) @ real.T
    if bias is not None:
        ideal = ideal + np.asarray(bias, np.float16).astype(np.float64)
    depth = (k // group - 1).bit_length()
    budget = (depth + 3) * float(np.finfo(np.float16).eps) * (np.abs(np.asarray(x, np.float64)) @ np.abs(real).T) + 3e-4
    err = got.astype(np.float64) - ideal
    assert o.rel_l2(got, ideal) < 1e-3
    assert (np.abs(err) <= budget).all()


@pytest.mark.parametrize('fmt', ['int4', 'nf4', 'int8'])
@pytest.mark.parametrize('m,k,n,group', [(1, 64, 32, 32), (7, 9, 5, 3), (31, 128, 64, 64), (32, 128, 64, 64),
                                         (1, 1024, 1024, 128), (128, 1024, 1024, 128), (4, 1024, 32, 32),
                                         (16, 4096, 2048, 128), (64, 2560, 960, 128)])
@pytest.mark.parametrize('path', ['auto', 'generic'])
def test_compact_random(device, fmt, m, k, n, group, path):
    """The reference group demo's configurations (torch_npu_lowbit_group_demo.py:146-147) plus two
    larger ones, on the fast (grid slice per group) and generic paths."""
    announce('compact', fmt, m, k, n, group, path)
    rng = np.random.default_rng(m * 131 + k * 7 + n + group)
    data, scales = o.quantize(rng.standard_normal((n, k)) / 8, fmt, group)
    x = (rng.standard_normal((m, k)) / 8).astype(np.float16)
    bias = (rng.standard_normal(n) / 8).astype(np.float16) if m in (7, 31) else None
    got = run(device, x, fmt, (n, k), group, data, scales, bias=bias,
              flags=lowbit_hip.FLAG_COMPACT_GROUPS | PATHS[path])
    assert np.isfinite(got).all()
    reference_gate(x, fmt, (n, k), group, data, scales, got, bias)
    want = o.compact_linear(x, fmt, (n, k), group, data, scales, bias=bias)
    assert o.rel_l2(got, want) <= 1e-3
    # pieces accumulate in fp32 here and in fp64 in the oracle: nearly all outputs agree bit for bit
    assert np.mean(bits(got) == bits(want)) >= 0.95


@pytest.mark.parametrize('fmt', ['int4', 'int8'])
def test_compact_large_grid_slices(device, fmt):
    """Grid slices of a compact call large enough for the 256 x 256 GEMM (2 x 24 tiles x 4 groups)."""
    m, k, n, group = 512, 512, 6144, 128
    announce('compact large', fmt)
    rng = np.random.default_rng(513)
    data, scales = o.quantize(rng.standard_normal((n, k)) / 8, fmt, group)
    x = (rng.standard_normal((m, k)) / 8).astype(np.float16)
    got = run(device, x, fmt, (n, k), group, data, scales, flags=lowbit_hip.FLAG_COMPACT_GROUPS)
    assert np.isfinite(got).all()
    reference_gate(x, fmt, (n, k), group, data, scales, got, None)
    want = o.compact_linear(x, fmt, (n, k), group, data, scales)
    assert o.rel_l2(got, want) <= 1e-3
    assert np.mean(bits(got) == bits(want)) >= 0.95


def test_compact_two_layer_network(device):
    """torch_npu_lowbit_group_demo.py:197-204: a 64->32->7 ReLU MLP of compact layers."""
    announce('compact mlp')
    torch.manual_seed(419)
    for fmt in ('int4', 'nf4'):
        first, second = torch.nn.Linear(64, 32).half(), torch.nn.Linear(32, 7).half()
        a = QuantizedLinear.from_float(first, format=fmt, group_size=32, compact_groups=True)
        b = QuantizedLinear.from_float(second, format=fmt, compact_groups=True)
        host = (torch.randn(7, 64) / 8).half()
        want = torch.nn.functional.linear(host, torch.from_numpy(a.weight.dequantize()), first.bias).relu()
        want = torch.nn.functional.linear(want, torch.from_numpy(b.weight.dequantize()), second.bias)
        got = b(a(host.to(device)).relu()).cpu()
        torch.testing.assert_close(got, want, rtol=3e-3, atol=3e-4)
