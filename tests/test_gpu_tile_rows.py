"""GPU parity of the one-tile multi-row GEMV (tile_rows_kernel): 2..16 activation rows over weights
below the streaming sizes take it without a flag (rows staged whole: K <= 4096, M * K <= 32768).

Bars as for every linear: rel-L2 <= 1e-3 against the oracle plus the reference's rounding-budget
gate; identity inputs with power-of-two scales are bit-exact; the result agrees with the forced
tiled GEMV (same fp16(q * s) weights) to the same bars.
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from test_gpu_linear import check, problem, run, to_dev

pytestmark = pytest.mark.gpu

# (fmt, M, N, K, group): every row count class (4, 8, 16 staged rows), ragged N, K below the
# staged length, groups of 32 .. one per row
CASES = [
    ('int4', 2, 576, 576, 64), ('int4', 3, 1000, 1536, 128), ('int4', 4, 49152, 576, 64),
    ('int4', 5, 4096, 4096, 128), ('int4', 8, 1040, 4096, 32), ('int4', 9, 1536, 576, 64),
    ('int4', 16, 576, 1536, 128), ('int4', 16, 2000, 2048, 2048),
    ('nf4', 4, 960, 2560, 64), ('nf4', 12, 2560, 960, 64),
    ('int8', 2, 1536, 576, 576), ('int8', 7, 1000, 4096, 4096), ('int8', 16, 576, 1536, 64),
]


@pytest.mark.parametrize('spec', CASES, ids=lambda s: '-'.join(map(str, s)))
def test_tile_rows_match_oracle(device, spec):
    fmt, m, n, k, group = spec
    announce('tile rows', spec)
    rng = np.random.default_rng(m * 977 + n + k + group)
    p = problem(rng, fmt, m, n, k, group, bias=(m % 2 == 0))
    got = run(p, device)
    check(p, got, f'tile rows {spec}')
    gemv = run(p, device, lowbit_hip.FLAG_FORCE_GEMV)
    assert o.rel_l2(got, gemv) <= 1e-3


def test_tile_rows_identity_is_bit_exact(device):
    m, n, k, group = 16, 1040, 2048, 64
    announce('tile rows identity')
    rng = np.random.default_rng(16)
    data = o.pack(rng.integers(0, 16, n * k).astype(np.uint8))
    scales = (2.0 ** rng.integers(-10, 3, n * (k // group))).astype(np.float16)
    w = o.dequantize('int4', (n, k), group, data, scales.tobytes())
    cols = [0, 1, 31, 32, 63, 64, 127, 128, 500, 1000, 1024, 1535, 1536, 2000, 2046, 2047]
    x = np.zeros((m, k), np.float16)
    for r, c in enumerate(cols):
        x[r, c] = 1.0
    y = lowbit_hip.linear(to_dev(x, device), to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                          format='int4', N=n, K=k, group_size=group).cpu().numpy()
    for r, c in enumerate(cols):
        np.testing.assert_array_equal(y[r].view(np.uint16), w[:, c].view(np.uint16), err_msg=f'row {r}')


def test_tile_rows_strided_activations_and_outputs(device):
    """x rows with ldx > K and y rows with ldy > N (views into wider buffers)."""
    m, n, k, group = 6, 1040, 1536, 64
    announce('tile rows strided')
    rng = np.random.default_rng(61)
    p = problem(rng, 'int4', m, n, k, group)
    wide = torch.zeros((m, k + 64), dtype=torch.float16, device=device)
    wide[:, 8:8 + k] = to_dev(p['x'], device)
    out = torch.full((m, n + 40), 7.0, dtype=torch.float16, device=device)
    y = lowbit_hip.linear(wide[:, 8:8 + k], to_dev(np.frombuffer(p['data'], np.uint8), device),
                          to_dev(np.frombuffer(p['scales'], np.float16), device), format='int4', N=n, K=k,
                          group_size=group, out=out[:, 16:16 + n])
    torch.cuda.synchronize()
    check(p, y.cpu().numpy(), 'tile rows strided')
    untouched = torch.cat([out[:, :16], out[:, 16 + n:]], dim=1)
    assert (untouched == 7.0).all()
