"""GPU parity of the one-tile multi-row GEMV (tile_rows_kernel): 2..16 activation rows over weights
below the streaming sizes, and 17..32 rows of INT4 / NF4 below the several-row kernel's 4 MB, take
it without a flag (rows staged whole up to 4096 / 2048 / 1024 codes for 8 / 16 / 32 rows, longer
ones in K slices).

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
    # 17..32 rows: two 16-row MFMA A operands per weight fragment, rows of up to 1024 codes staged
    ('int4', 17, 1000, 1024, 128), ('int4', 32, 576, 576, 64), ('nf4', 24, 960, 1024, 64),
    ('nf4', 29, 700, 1024, 128),
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


# Rows longer than the kernel stages whole go in K slices: (fmt, M, N, K, group) with 2, 3, 4 and 7
# slices, per-row INT8, NF4, ragged N.
SLICED = [
    ('int4', 8, 4096, 14336, 128), ('int4', 4, 1000, 8192, 64), ('int4', 2, 576, 12288, 32),
    ('int4', 16, 1024, 14336, 128), ('int4', 12, 600, 4096, 128), ('nf4', 6, 2048, 14336, 128),
    ('int8', 8, 1030, 8192, 8192), ('int8', 5, 2000, 6144, 128),
    ('int4', 32, 1024, 4096, 128), ('int4', 20, 600, 2048, 64), ('nf4', 32, 1024, 4096, 128),
]


@pytest.mark.parametrize('spec', SLICED, ids=lambda s: '-'.join(map(str, s)))
def test_tile_rows_slices_match_oracle(device, spec):
    fmt, m, n, k, group = spec
    announce('tile rows slices', spec)
    rng = np.random.default_rng(m * 31 + n + k + group)
    p = problem(rng, fmt, m, n, k, group, bias=(m % 2 == 0))
    got = run(p, device)
    check(p, got, f'tile rows slices {spec}')
    gemv = run(p, device, lowbit_hip.FLAG_FORCE_GEMV)
    assert o.rel_l2(got, gemv) <= 1e-3


def test_tile_rows_slices_identity_is_bit_exact(device):
    """One-hot rows over four K slices: each output is one dequantized weight, bit for bit."""
    m, n, k, group = 8, 1040, 14336, 64
    announce('tile rows slices identity')
    rng = np.random.default_rng(18)
    data = o.pack(rng.integers(0, 16, n * k).astype(np.uint8))
    scales = (2.0 ** rng.integers(-10, 3, n * (k // group))).astype(np.float16)
    w = o.dequantize('int4', (n, k), group, data, scales.tobytes())
    cols = [0, 3583, 3584, 7000, 7168, 10751, 10752, 14335]
    x = np.zeros((m, k), np.float16)
    for r, c in enumerate(cols):
        x[r, c] = 1.0
    y = lowbit_hip.linear(to_dev(x, device), to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                          format='int4', N=n, K=k, group_size=group).cpu().numpy()
    for r, c in enumerate(cols):
        np.testing.assert_array_equal(y[r].view(np.uint16), w[:, c].view(np.uint16), err_msg=f'row {r}')


@pytest.mark.parametrize('spec', [('int4', 8, 4096, 14336, 128), ('int8', 8, 1030, 8192, 8192),
                                  ('int4', 16, 1000, 14336, 128), ('int4', 32, 1024, 4096, 128),
                                  ('nf4', 27, 1032, 2048, 128)], ids=lambda s: '-'.join(map(str, s)))
def test_tile_rows_slices_added_in_kernel_equal_separate_reduction(device, spec):
    """LB_FLAG_ZEROED_WORKSPACE: the slices added by each tile column's last workgroup give the
    separate reduction launch's output bit for bit, call after call and replayed from a HIP graph,
    and leave the reserved counters zero."""
    fmt, m, n, k, group = spec
    announce('tile rows slices in kernel', spec)
    rng = np.random.default_rng(n + k)
    p = problem(rng, fmt, m, n, k, group, bias=True)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    bias = to_dev(p['bias'], device)
    x = to_dev(p['x'], device)
    y_sep = torch.empty(m, n, dtype=torch.float16, device=device)
    y_in = torch.empty(m, n, dtype=torch.float16, device=device)
    need = lowbit_hip.workspace_bytes(lowbit_hip.make_args(x, codes, scales, format=fmt, N=n, K=k, group_size=group,
                                                           y=y_sep, bias=bias))
    assert need > 0  # K slices
    garbage = torch.full((need,), 0x5A, dtype=torch.uint8, device=device)
    sep = lowbit_hip.PreparedLinear(x, codes, scales, format=fmt, N=n, K=k, group_size=group, out=y_sep, bias=bias,
                                    workspace=garbage)
    ink = lowbit_hip.PreparedLinear(x, codes, scales, format=fmt, N=n, K=k, group_size=group, out=y_in, bias=bias)
    assert ink.args.flags & lowbit_hip.FLAG_ZEROED_WORKSPACE
    counters = ink.workspace[:lowbit_hip.ZEROED_WORKSPACE_BYTES]
    for step in range(4):
        x.copy_(torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(device))
        sep.run()
        ink.run()
        ink.run()
        torch.cuda.synchronize()
        assert torch.equal(y_in, y_sep), step
        assert int(counters.count_nonzero()) == 0, step
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        ink.run()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ink.run()
    for step in range(3):
        x.copy_(torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(device))
        y_in.zero_()
        graph.replay()
        sep.run()
        torch.cuda.synchronize()
        assert torch.equal(y_in, y_sep), f'replay {step}'
        assert int(counters.count_nonzero()) == 0, f'replay {step}'
