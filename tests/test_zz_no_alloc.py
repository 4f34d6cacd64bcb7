"""GPU check of lb_linear_noalloc, the allocation-free form of lb_linear: through the C-ABI, its
output equals lb_linear's (fresh zeroed workspace) bit for bit on every path that needs scratch
(split-K prefill GEMMs, the split decode GEMV, the correction's z / d, W8A8 activations,
compact_groups pieces), on two calls in a row where the second is smaller, so what the first
call left in the library's scratch must not leak into the second."""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o

pytestmark = pytest.mark.gpu

# (label, fmt, group, flags, extra) and two (M, N, K) shapes, the second smaller.
CASES = [
    ('split-gemm-int4', 'int4', 128, 0, {}, (256, 4096, 4096), (128, 4096, 4096)),
    ('split-gemm-nf4', 'nf4', 64, 0, {}, (512, 960, 2560), (128, 960, 2560)),
    ('split-gemv-int4', 'int4', 128, lowbit_hip.FLAG_FORCE_GEMV, {}, (1, 1024, 14336), (1, 512, 8192)),
    ('correction-gemm-int8', 'int8', None, 0, dict(rank=32), (256, 576, 1536), (64, 576, 1536)),
    ('w8a8', 'int8', None, 0, dict(activation_scale=2.0 ** -5), (8, 1536, 576), (2, 1536, 576)),
    ('compact-int4', 'int4', 64, lowbit_hip.FLAG_COMPACT_GROUPS, {}, (16, 512, 1024), (4, 256, 1024)),
]


def operands(rng, fmt, group, m, n, k, extra, device):
    g = k if group is None else group
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    data, scales = o.quantize(w, fmt, g)
    x = rng.standard_normal((m, k)).astype(np.float16)
    dev = lambda a: torch.from_numpy(np.array(a, copy=True)).to(device)
    kw = dict(format=fmt, N=n, K=k, group_size=g)
    ops = dict(x=dev(x), codes=dev(np.frombuffer(data, np.uint8)), scales=dev(np.frombuffer(scales, np.float16)))
    if extra.get('rank'):
        r = extra['rank'] if m > 64 else extra['rank'] // 2
        kw.update(rank=r, down=dev((rng.standard_normal((r, k)) * 0.01).astype(np.float16)),
                  up=dev((rng.standard_normal((n, r)) * 0.01).astype(np.float16)))
    if 'activation_scale' in extra:
        kw['activation_scale'] = extra['activation_scale']
    return ops, kw, dict(x=x, data=data, scales=scales, group=g)


@pytest.mark.parametrize('case', CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_lb_linear_on_two_calls(device, case):
    label, fmt, group, flags, extra, first, second = case
    rng = np.random.default_rng(1000 + CASES.index(case))
    for call, (m, n, k) in enumerate((first, second)):
        announce('noalloc', label, call, (m, n, k))
        ops, kw, host = operands(rng, fmt, group, m, n, k, extra, device)
        out = torch.full((m, n), float('nan'), dtype=torch.float16, device=device)
        args = lowbit_hip.make_args(ops['x'], ops['codes'], ops['scales'], y=out, flags=flags, **kw)
        need = lowbit_hip.workspace_bytes(args)
        assert 0 < need <= lowbit_hip.NOALLOC_SCRATCH_BYTES, need
        want = lowbit_hip.linear(ops['x'], ops['codes'], ops['scales'], flags=flags, **kw)
        got = lowbit_hip.linear_noalloc(ops['x'], ops['codes'], ops['scales'], out=out, flags=flags, **kw)
        torch.cuda.synchronize()
        assert got is out
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (label, call)
        if fmt != 'int8' or 'rank' not in kw:
            continue
        ref = o.linear(host['x'], fmt, (n, k), host['group'], host['data'], host['scales'],
                       down=kw['down'].cpu().numpy(), up=kw['up'].cpu().numpy())
        assert o.rel_l2(got.cpu().numpy(), ref) <= 1e-3


def test_noalloc_refuses_calls_beyond_its_scratch(device):
    """32 fp16 pieces of 64 x 8200 need more than the library's scratch: refused before launch."""
    announce('noalloc oversize')
    m, n, k = 64, 8200, 1024
    x = torch.zeros(m, k, dtype=torch.float16, device=device)
    codes = torch.zeros(n * k // 2, dtype=torch.uint8, device=device)
    scales = torch.ones(n, k // 32, dtype=torch.float16, device=device)
    out = torch.zeros(m, n, dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match='scratch'):
        lowbit_hip.linear_noalloc(x, codes, scales, out=out, format='int4', N=n, K=k, group_size=32,
                                  flags=lowbit_hip.FLAG_COMPACT_GROUPS)
