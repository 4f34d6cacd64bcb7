"""GPU parity of the several-row GEMV on 32x32 MFMA tiles (wide_rows_kernel) against the CPU oracle.

INT4 / NF4 calls of 17..32 rows over >= 16 MB of weights (INT8: 4 MB), and of 9..16 rows over 16..64 MB
whose K slices the kernel adds itself, run there by default; the tests force it
(LB_FLAG_FORCE_WIDE) on other shapes and row counts.  Every code is decoded to its exact integer q
and a group's (or, for per-row INT8, the whole row's) integer sum is scaled in fp32, so its value
is the exact x . (q s) product: the bars are those of every linear path, rel-L2 <= 1e-3 against
the oracle and the reference's rounding-budget gate (torch_npu_lowbit_demo.py:91-106), and bit
for bit on one-hot inputs with power-of-two scales (torch_npu_lowbit_demo.py:124-128).  Shapes
cover one K slice and several (fp32 partials added in slice order, by a second launch or, with a
zeroed workspace, by each row block's last workgroup), partial 32-row blocks, every group span (2,
4, 8 loads per group, and per row), bias, and strided activation / output rows.
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from test_gpu_linear import check, problem, run, to_dev

pytestmark = pytest.mark.gpu
WIDE = lowbit_hip.FLAG_FORCE_WIDE

# (fmt, N, K, group): K a multiple of the 512-code (INT4) / 256-code (INT8) chunk
WIDE_SHAPES = [
    ('int4', 300, 1024, 128),      # 3 blocks (the last partial), K split in 2
    ('int4', 4096, 4096, 128),     # 32 blocks, split into 8 one-chunk slices
    ('int4', 14336, 1024, 128),    # 112 blocks, 2 slices
    ('int4', 28000, 512, 128),     # one chunk, one slice, a partial block
    ('int4', 1000, 2048, 256),     # four loads per group
    ('int4', 520, 1536, 512),      # eight loads per group, 3 chunks
    ('int8', 4096, 4096, 4096),    # per-row int8, split
    ('int8', 26000, 256, 256),     # per-row int8, one chunk, one slice, partial block
    ('int8', 2048, 2048, 128),     # four loads per group
    ('int8', 1030, 1024, 64),      # two loads per group
    ('int8', 777, 768, 256),       # eight loads per group
    ('nf4', 4096, 4096, 128),      # NF4 literals from the LDS table, split
    ('nf4', 300, 1024, 256),       # NF4, a partial block, four loads per group
    ('nf4', 28000, 512, 512),      # NF4, one chunk, one slice, eight loads per group
]
ROWS = [1, 2, 5, 16, 17, 31, 32]


@pytest.mark.parametrize('m', ROWS)
@pytest.mark.parametrize('spec', WIDE_SHAPES, ids=lambda s: '-'.join(map(str, s)))
def test_wide_matches_oracle(device, spec, m):
    fmt, n, k, group = spec
    announce('wide', spec, m)
    rng = np.random.default_rng(n + 7 * k + group + 1000 * m)
    p = problem(rng, fmt, m, n, k, group)
    check(p, run(p, device, WIDE), f'wide {spec} M={m}')


@pytest.mark.parametrize('spec', [('int4', 4096, 4096, 128), ('int4', 20000, 1024, 128), ('int8', 2048, 2048, 2048)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_wide_with_bias(device, spec):
    fmt, n, k, group = spec
    announce('wide bias', spec)
    rng = np.random.default_rng(3 * n + k)
    p = problem(rng, fmt, 24, n, k, group, bias=True)
    check(p, run(p, device, WIDE), f'wide bias {spec}')


def test_wide_strided_rows(device):
    """x and y as views with row strides beyond K and N (q|k|v-style slices); the rest of each
    output row is untouched."""
    announce('wide strided')
    rng = np.random.default_rng(11)
    m, n, k, group = 20, 2000, 2048, 128
    p = problem(rng, 'int4', m, n, k, group)
    xb = to_dev(np.zeros((m, k + 40), np.float16), device)
    xb[:, 8:8 + k] = to_dev(p['x'], device)
    yb = torch.full((m, n + 24), 7.0, dtype=torch.float16, device=device)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    lowbit_hip.linear(xb[:, 8:8 + k], codes, scales, format='int4', N=n, K=k, group_size=group, flags=WIDE,
                      out=yb[:, 16:16 + n])
    torch.cuda.synchronize()
    got = yb.cpu().numpy()
    check(p, got[:, 16:16 + n], 'wide strided')
    assert (got[:, :16] == 7.0).all() and (got[:, 16 + n:] == 7.0).all()


@pytest.mark.parametrize('fmt,group,n,k', [('int4', 128, 4096, 4096), ('int4', 256, 1024, 1024),
                                           ('int8', 4096, 2048, 4096), ('int8', 64, 1000, 512),
                                           ('nf4', 128, 2048, 2048)])
def test_wide_identity_is_bit_exact(device, fmt, group, n, k):
    """One-hot activation rows and power-of-two scales: row i of y is the dequantized column of its
    hot index, bit for bit, in every K slice and row position."""
    announce('wide identity', fmt, group, n, k)
    rng = np.random.default_rng(group + n)
    nibbles = fmt in ('int4', 'nf4')
    codes = rng.integers(0, 16, n * k).astype(np.uint8) if nibbles else rng.integers(-128, 128, n * k)
    data = o.pack(codes) if nibbles else codes.astype(np.int8).tobytes()
    g = k // group
    scales = (2.0 ** rng.integers(-12, 3, n * g)).astype(np.float16)
    w = o.dequantize(fmt, (n, k), group, data, scales.tobytes())
    cols = [0, 1, 31, 32, 33, 127, 128, 255, 256, k // 2 + 5, k - 129, k - 1]
    x = np.zeros((32, k), np.float16)
    for i in range(32):
        x[i, cols[i % len(cols)]] = 1.0
    y = lowbit_hip.linear(to_dev(x, device), to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                          format=fmt, N=n, K=k, group_size=group, flags=WIDE)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for i in range(32):
        np.testing.assert_array_equal(got[i], w[:, cols[i % len(cols)]], err_msg=f'row {i}')


@pytest.mark.parametrize('fmt,m', [('int4', 24), ('int4', 12), ('nf4', 16)])
def test_wide_is_the_default_on_the_tall_config5_shape(device, fmt, m):
    """14336x4096 g128 (config-5 shape) at 17..32 rows, and at 9..16 INT4 / NF4 rows (four K slices,
    added by the kernel): the default dispatch gives the forced kernel's result bit for bit, and
    the oracle's values."""
    announce('wide default dispatch', fmt, m)
    rng = np.random.default_rng(5 + m)
    p = problem(rng, fmt, m, 14336, 4096, 128)
    default = run(p, device)
    np.testing.assert_array_equal(default, run(p, device, WIDE))
    check(p, default, f'wide default {fmt} M={m}')


@pytest.mark.parametrize('over', [dict(K=4096 + 256), dict(group=64), dict(fmt='nf4', group=64), dict(M=33)])
def test_wide_refuses_shapes_it_does_not_take(device, over):
    announce('wide refuses', over)
    fmt, m, n, k, group = over.get('fmt', 'int4'), over.get('M', 4), 256, over.get('K', 4096), over.get('group', 128)
    x = torch.zeros(m, k, dtype=torch.float16, device=device)
    codes = torch.zeros(n * k // 2, dtype=torch.uint8, device=device)
    scales = torch.ones(n * (k // group), dtype=torch.float16, device=device)
    with pytest.raises(RuntimeError, match='LB_FLAG_FORCE_WIDE'):
        lowbit_hip.linear(x, codes, scales, format=fmt, N=n, K=k, group_size=group, flags=WIDE)


# (fmt, N, K, group, M, bias): 2, 3 and 4 K slices added in the kernel (partial last row blocks,
# per-row INT8 with a bias, NF4), and two calls that keep the separate reduction (14 slices, more than
# the kernel adds; N not a multiple of 4): still equal.
IN_KERNEL = [('int4', 14336, 4096, 128, 32, False), ('int4', 300, 1024, 128, 32, False),
             ('int4', 6000, 2048, 128, 17, False), ('int4', 8192, 1536, 128, 32, True),
             ('int8', 14336, 4096, 4096, 24, True), ('nf4', 14336, 2048, 128, 20, False),
             ('int4', 4096, 14336, 128, 32, False), ('int4', 1002, 2048, 256, 31, True)]


@pytest.mark.parametrize('spec', IN_KERNEL, ids=lambda s: '-'.join(map(str, s)))
def test_wide_slices_added_in_kernel_equal_separate_reduction(device, spec):
    """LB_FLAG_ZEROED_WORKSPACE: the K slices added by each row block's last workgroup give the
    separate reduction launch's output bit for bit, call after call, eagerly and replayed from a HIP
    graph (with eager calls and synchronisations between replays), and every call leaves the
    reserved counters zero."""
    fmt, n, k, group, m, bias = spec
    announce('wide in-kernel slices', spec)
    rng = np.random.default_rng(n + k + m)
    p = problem(rng, fmt, m, n, k, group, bias=bias)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    kw = dict(bias=to_dev(p['bias'], device)) if bias else {}
    x = to_dev(p['x'], device)
    y_sep = torch.empty(m, n, dtype=torch.float16, device=device)
    y_in = torch.empty(m, n, dtype=torch.float16, device=device)
    probe = lowbit_hip.make_args(x, codes, scales, format=fmt, N=n, K=k, group_size=group, y=y_sep, flags=WIDE,
                                 **kw)
    need = lowbit_hip.workspace_bytes(probe)
    assert need > 0  # several K slices
    garbage = torch.full((need,), 0xA5, dtype=torch.uint8, device=device)  # no promise: separate launch
    sep = lowbit_hip.PreparedLinear(x, codes, scales, format=fmt, N=n, K=k, group_size=group, out=y_sep,
                                    flags=WIDE, workspace=garbage, **kw)
    ink = lowbit_hip.PreparedLinear(x, codes, scales, format=fmt, N=n, K=k, group_size=group, out=y_in,
                                    flags=WIDE, **kw)
    assert ink.args.flags & lowbit_hip.FLAG_ZEROED_WORKSPACE and not sep.args.flags & lowbit_hip.FLAG_ZEROED_WORKSPACE
    assert ink.workspace_bytes == need + lowbit_hip.ZEROED_WORKSPACE_BYTES
    counters = ink.workspace[:lowbit_hip.ZEROED_WORKSPACE_BYTES]
    for step in range(4):
        x.copy_(torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(device))
        sep.run()
        ink.run()
        ink.run()  # twice: the second call starts from the counters the first left
        torch.cuda.synchronize()
        assert torch.equal(y_in, y_sep), step
        assert int(counters.count_nonzero()) == 0, step
    x.copy_(to_dev(p['x'], device))
    ink.run()
    torch.cuda.synchronize()
    check(p, y_in.cpu().numpy(), f'wide in-kernel {spec}')
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
