"""GPU parity over seeded random shapes on the default dispatch: every path the planner can pick
(one-row single tile and rows kernels, one-tile rows, the streaming kernels under a forced flag,
the tiled GEMV, split-K and plain prefill GEMMs, the generic kernel) against the oracle, with the
linear path's bars (rel-L2 <= 1e-3 plus the reference's rounding-budget gate; with a bias or a
correction, rel-L2 only).  Shapes are drawn so that each row-count class and each K regime
appears; a second forced path (FORCE_GEMV where it applies, else FORCE_GENERIC) must agree too.
"""
import numpy as np
import pytest

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o
from test_gpu_linear import check, problem, run

pytestmark = pytest.mark.gpu

M_CHOICES = [1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 32, 33, 48, 64, 96, 130, 256]
K_CHOICES = [32, 64, 96, 192, 576, 640, 960, 1024, 1536, 2048, 2560, 4096]
FORMATS = ['int4', 'nf4', 'int8']


def draw(seed):
    rng = np.random.default_rng(seed)
    fmt = FORMATS[seed % 3]
    m = int(rng.choice(M_CHOICES))
    k = int(rng.choice(K_CHOICES))
    n = int(rng.integers(1, 2600))
    groups = [g for g in (32, 64, 128, k) if k % g == 0 and (g == k or (g & (g - 1)) == 0)]
    if fmt == 'int8' and rng.random() < 0.5:
        groups = [k]  # per-row int8
    group = int(rng.choice(groups))
    bias = bool(rng.random() < 0.3)
    rank = int(rng.choice([0, 0, 0, 8, 32])) if k <= 1536 else 0
    return fmt, m, n, k, group, bias, rank


@pytest.mark.parametrize('seed', range(48))
def test_random_shape_default_and_forced_paths(device, seed):
    fmt, m, n, k, group, bias, rank = draw(seed)
    spec = (fmt, m, n, k, group, bias, rank)
    announce('random shape', seed, spec)
    rng = np.random.default_rng(10_000 + seed)
    p = problem(rng, fmt, m, n, k, group, rank=rank, bias=bias)
    got = run(p, device)
    check(p, got, f'random {spec} default path')
    second = lowbit_hip.FLAG_FORCE_GEMV if m <= 32 else lowbit_hip.FLAG_FORCE_GENERIC
    other = run(p, device, second)
    check(p, other, f'random {spec} forced {second:#x}')
    assert o.rel_l2(got, other) <= 2e-3, spec
