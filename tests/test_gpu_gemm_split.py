"""GPU parity of the split-K prefill GEMM (grids of few 64 x 64 or 128 x 128 tiles: K slices with
fp32 partials, reduced in a fixed order by splitk_reduce_kernel, which applies the epilogue).

Bars as for every linear: rel-L2 <= 1e-3 against the oracle and the reference's rounding-budget
gate; the split is deterministic (two calls agree bit for bit) and its partials are fully rewritten
on every call (a second call with other activations on the same workspace is exact against its
own oracle).  The shapes are chosen so the planner splits: the workspace query reports the fp32
partials [splits, M, N].
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from test_gpu_linear import check, problem, run, to_dev

pytestmark = pytest.mark.gpu

# (fmt, M, N, K, group, rank, bias, expected splits)
SPLIT = [
    ('nf4', 128, 960, 2560, 64, 0, False, 4),     # config 3 down at M = 128: 30 tiles
    ('nf4', 512, 960, 2560, 64, 0, False, 4),     # config 3 down at M = 512: 120 tiles
    ('int8', 96, 576, 1536, 1536, 0, True, 3),    # per-row int8 scale in the reduction's epilogue
    ('int4', 200, 1000, 2080, 32, 0, True, 4),    # ragged M / N, k steps of 32, uneven last slice
    ('int4', 64, 1536, 2048, 64, 32, True, 4),    # rank-32 correction delta and bias
    ('int8', 65, 192, 1152, 64, 0, False, 2),     # grouped int8
    ('int4', 256, 4096, 4096, 128, 0, True, 4),   # 128 x 128 tiles split (64 tiles, 64 k steps)
    ('int4', 512, 4096, 2048, 128, 0, True, 2),   # 128 tiles: two slices fill the CUs
]


def workspace_splits(p, device):
    x = to_dev(p['x'], device)
    y = torch.empty((p['m'], p['n']), dtype=torch.float16, device=device)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    kw = {}
    if p['down'] is not None:
        kw = dict(down=to_dev(p['down'], device), up=to_dev(p['up'], device), rank=p['down'].shape[0])
    args = lowbit_hip.make_args(x, codes, scales, format=p['fmt'], N=p['n'], K=p['k'], group_size=p['group'],
                                y=y, **kw)
    need = lowbit_hip.workspace_bytes(args)
    extra = 0
    if p['down'] is not None:  # z [M, r] and the fp16 delta [M, N], each rounded to 256 bytes
        extra = -(-p['m'] * p['down'].shape[0] * 2 // 256) * 256 + -(-p['m'] * p['n'] * 2 // 256) * 256
    part = need - extra
    assert part % (p['m'] * p['n'] * 4) == 0, (need, extra)
    return part // (p['m'] * p['n'] * 4)


@pytest.mark.parametrize('spec', SPLIT, ids=lambda s: '-'.join(map(str, s[:6])))
def test_split_gemm_matches_oracle(device, spec):
    fmt, m, n, k, group, rank, bias, splits = spec
    announce('split gemm', spec)
    rng = np.random.default_rng(m * 7 + n + k)
    p = problem(rng, fmt, m, n, k, group, rank=rank, bias=bias)
    assert workspace_splits(p, device) == splits
    got = run(p, device)
    check(p, got, f'split gemm {spec}')
    assert np.array_equal(run(p, device), got), 'split GEMM is not deterministic'


def test_split_gemm_partials_are_rewritten(device):
    fmt, m, n, k, group = 'nf4', 512, 960, 2560, 64
    announce('split gemm reuse', fmt, m, n, k)
    rng = np.random.default_rng(5)
    p = problem(rng, fmt, m, n, k, group)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    ws = torch.full((8 << 20,), 0x7F, dtype=torch.uint8, device=device)  # stale NaN-free garbage
    outs = []
    for xs in (1.0, 3.0):
        x = (p['x'].astype(np.float32) * xs).astype(np.float16)
        y = lowbit_hip.linear(to_dev(x, device), codes, scales, format=fmt, N=n, K=k, group_size=group,
                              workspace=ws)
        torch.cuda.synchronize()
        outs.append((x, y.cpu().numpy()))
    for x, got in outs:
        check(dict(p, x=x), got, 'split gemm with a reused workspace')
