"""GPU parity of liblowbit_hip against the CPU oracle (and the golden fixtures).

Bars: unpacked integer codes and dequantized fp16 weights bit-exact; linear outputs
rel-L2 <= 1e-3 against the oracle, within the reference's per-output rounding budget
(torch_npu_lowbit_demo.py:91-95), and bit-exact for the identity-input case
(torch_npu_lowbit_demo.py:124-128).  Every kernel path (decode GEMV, prefill GEMM,
generic) is forced on the same inputs.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from oracle import lowbit_oracle as o

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / 'golden'
PATHS = {'gemv': lowbit_hip.FLAG_FORCE_GEMV, 'gemm': lowbit_hip.FLAG_FORCE_GEMM,
         'generic': lowbit_hip.FLAG_FORCE_GENERIC, 'auto': 0}
REL_L2 = 1e-3


def to_dev(array, device):
    return torch.from_numpy(np.array(array, copy=True)).to(device)


def problem(rng, fmt, m, n, k, group, rank=0, bias=False, xscale=1.0):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    data, scales = o.quantize(w, fmt, group)
    x = (rng.standard_normal((m, k)) * xscale).astype(np.float16)
    b = (rng.standard_normal(n) * 0.1).astype(np.float16) if bias else None
    down = (rng.standard_normal((rank, k)) * 0.01).astype(np.float16) if rank else None
    up = (rng.standard_normal((n, rank)) * 0.01).astype(np.float16) if rank else None
    return dict(fmt=fmt, m=m, n=n, k=k, group=group, x=x, data=data, scales=scales, bias=b, down=down, up=up)


def run(p, device, flags=0):
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    kw = {}
    if p['bias'] is not None:
        kw['bias'] = to_dev(p['bias'], device)
    if p['down'] is not None:
        kw.update(down=to_dev(p['down'], device), up=to_dev(p['up'], device), rank=p['down'].shape[0])
    y = lowbit_hip.linear(to_dev(p['x'], device), codes, scales, format=p['fmt'], N=p['n'], K=p['k'],
                          group_size=p['group'], flags=flags, **kw)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def expected(p):
    return o.linear(p['x'], p['fmt'], (p['n'], p['k']), p['group'], p['data'], p['scales'], bias=p['bias'],
                    down=p['down'], up=p['up'])


def check(p, got, label):
    want = expected(p)
    assert np.isfinite(got).all(), label
    err = o.rel_l2(got, want)
    assert err <= REL_L2, f'{label}: rel-L2 {err:.3e}'
    if p['bias'] is None and p['down'] is None:
        budget = o.rounding_budget(p['x'], p['fmt'], (p['n'], p['k']), p['group'], p['data'], p['scales'])
        ideal = o.ideal(p['x'], p['fmt'], (p['n'], p['k']), p['group'], p['data'], p['scales'])
        # reference gate: |device - fp16 plain| <= budget, with one extra output ulp for our fp16 store
        ulp = np.abs(want.astype(np.float64)) * 2.0 ** -10 + 2.0 ** -24
        assert (np.abs(got.astype(np.float64) - want.astype(np.float64)) <= budget + ulp).all(), label
        assert o.rel_l2(got, ideal) <= REL_L2, label
    return err


@pytest.mark.parametrize('fmt', ['int8', 'int4', 'nf4'])
@pytest.mark.parametrize('n,k', [(3, 17), (7, 13), (5, 64), (64, 256), (33, 160)])
def test_unpack_bit_exact(device, fmt, n, k):
    announce('unpack', fmt, n, k)
    rng = np.random.default_rng(n * 1000 + k)
    if fmt == 'int8':
        data = rng.integers(-128, 128, n * k).astype(np.int8).tobytes()
    else:
        data = o.pack(rng.integers(0, 16, n * k).astype(np.uint8))
    got = lowbit_hip.unpack_codes(to_dev(np.frombuffer(data, np.uint8), device), format=fmt, N=n, K=k)
    np.testing.assert_array_equal(got.cpu().numpy().ravel(), o.unpack(fmt, data, n * k))


@pytest.mark.parametrize('fmt', ['int8', 'int4', 'nf4'])
def test_dequantize_bit_exact_all_codes_and_scales(device, fmt):
    announce('dequantize', fmt)
    rng = np.random.default_rng(7)
    bits = np.concatenate([np.arange(1, 0x7C00, 61, dtype=np.uint16), rng.integers(1, 0x7C00, 200).astype(np.uint16),
                           np.array([1, 2, 3, 0x03FF, 0x0400, 0x3C00, 0x7BFF], np.uint16)])
    scales = bits.view(np.float16)
    codes = np.arange(-128, 128).astype(np.int8) if fmt == 'int8' else np.arange(16, dtype=np.uint8)
    n, k = scales.size, codes.size
    data = np.tile(codes, n).tobytes() if fmt == 'int8' else o.pack(np.tile(codes, n))
    got = lowbit_hip.dequantize(to_dev(np.frombuffer(data, np.uint8), device), to_dev(scales, device),
                                format=fmt, N=n, K=k, group_size=k).cpu().numpy()
    want = o.dequantize(fmt, (n, k), k, data, scales.tobytes())
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize('fmt', ['int8', 'int4', 'nf4'])
@pytest.mark.parametrize('shape', [(5, 64, 32), (11, 192, 96), (3, 17, 17)])
def test_dequantize_bit_exact_quantized(device, fmt, shape):
    n, k, group = shape
    announce('dequantize-q', fmt, shape)
    rng = np.random.default_rng(n + k)
    data, scales = o.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), fmt, group)
    got = lowbit_hip.dequantize(to_dev(np.frombuffer(data, np.uint8), device),
                                to_dev(np.frombuffer(scales, np.float16), device),
                                format=fmt, N=n, K=k, group_size=group).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), o.dequantize(fmt, (n, k), group, data, scales).view(np.uint16))


def test_golden_fixtures_all_paths(device):
    data = np.load(GOLDEN / 'linear_small.npz', allow_pickle=False)
    names = sorted({key.split('/')[0] for key in data.files})
    for name in names:
        m, n, k, g, rank = data[f'{name}/shape'].tolist()
        p = dict(fmt=str(data[f'{name}/fmt']), m=m, n=n, k=k, group=g, x=data[f'{name}/x'],
                 data=data[f'{name}/data'].tobytes(), scales=data[f'{name}/scales'].tobytes(),
                 bias=data[f'{name}/bias'] if f'{name}/bias' in data.files else None,
                 down=data[f'{name}/down'] if rank else None, up=data[f'{name}/up'] if rank else None)
        want = data[f'{name}/y']
        for path, flags in PATHS.items():
            eligible = k % 32 == 0 and (g == k or g % 32 == 0)
            if path in ('gemv', 'gemm') and not eligible:
                continue
            if path == 'gemv' and m > 32:
                continue
            announce('golden', name, path)
            got = run(p, device, flags)
            err = o.rel_l2(got, want)
            assert err <= REL_L2, f'{name}/{path}: {err:.3e}'


@pytest.mark.parametrize('path', ['gemv', 'gemm', 'generic'])
@pytest.mark.parametrize('fmt', ['int4', 'nf4'])
@pytest.mark.parametrize('scale', [0.125, 1.0, 16.0])
def test_identity_input_is_bit_exact(device, path, fmt, scale):
    """All 16 codes x scale with eye(K) input reproduce dequantize() bit-exactly (demo :124-128)."""
    announce('identity', path, fmt, scale)
    k = 32
    codes = np.tile(np.arange(16, dtype=np.uint8), 2 * 3)  # N=3 rows of 32 codes
    data = o.pack(codes)
    scales = np.full(3, scale, np.float16).tobytes()
    p = dict(fmt=fmt, m=k, n=3, k=k, group=k, x=np.eye(k, dtype=np.float16), data=data, scales=scales,
             bias=None, down=None, up=None)
    got = run(p, device, PATHS[path])
    want = o.dequantize(fmt, (3, k), k, data, scales).T
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize('fmt', ['int8', 'int4', 'nf4'])
def test_single_row_path_identity_is_bit_exact(device, fmt):
    """One-row calls (the single-tile path) with unit vectors e_k return column k of dequantize()."""
    announce('identity single row', fmt)
    k, n, group = 64, 20, 32
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    if fmt == 'int8':
        data = rng.integers(-127, 128, (n, k), dtype=np.int8).tobytes()
    else:
        data = o.pack(codes)
    scales = (2.0 ** rng.integers(-6, 4, (n, k // group))).astype(np.float16).tobytes()
    want = o.dequantize(fmt, (n, k), group, data, scales)
    for col in range(k):
        x = np.zeros((1, k), np.float16)
        x[0, col] = 1.0
        p = dict(fmt=fmt, m=1, n=n, k=k, group=group, x=x, data=data, scales=scales, bias=None, down=None, up=None)
        got = run(p, device)
        np.testing.assert_array_equal(got[0].view(np.uint16), want[:, col].view(np.uint16))


SHAPES = [
    # (fmt, M, N, K, group) -- config shapes and awkward edges
    ('int8', 1, 1536, 576, 576),      # config 1 (without correction here)
    ('int8', 4, 576, 1536, 1536),
    ('int8', 17, 192, 576, 576),
    ('int4', 1, 576, 576, 64),        # config 2, K=576 -> g64
    ('int4', 4, 192, 576, 64),
    ('int4', 16, 1536, 576, 32),
    ('int4', 1, 576, 1536, 128),
    ('int4', 32, 100, 4096, 128),     # split-K decode, N not a multiple of 16
    ('int4', 1, 77, 4096, 4096),      # per-row 4-bit
    ('nf4', 1, 960, 2560, 64),
    ('nf4', 8, 2560, 960, 64),
    ('int4', 64, 300, 512, 128),
    ('nf4', 128, 2560, 960, 64),      # config 3 prefill shape
    ('int8', 256, 576, 576, 576),
    ('int8', 33, 1536, 576, 32),      # grouped int8
    ('int4', 130, 129, 96, 32),
    ('int4', 1, 130, 16384, 128),     # one row, long K (lane-linear kernel: eight segments)
    ('int8', 1, 300, 8192, 8192),     # one row, long K, per-row W8
    ('nf4', 1, 64, 5000 // 32 * 32, 64),
    ('int4', 1, 100, 4096, 32),       # one row, long K, group 32: falls back to the split GEMV
    # several rows and a large weight: 64-row workgroups, K split across workgroups
    ('int4', 8, 4096, 4096, 128),
    ('int4', 32, 2048, 4096, 64),
    ('int8', 16, 2048, 1536, 1536),
    ('nf4', 5, 1000, 8192, 128),      # N not a multiple of 64
    ('int8', 3, 1100, 2048, 64),      # grouped int8
    ('int4', 8, 40000, 1024, 128),    # enough 64-row tiles to fill the chip: no K split
    ('nf4', 16, 33000, 2048, 64),     # no K split, K walked in LDS chunks
    # one row over many rows: several 16-row tiles per workgroup (rows_gemv_kernel) ...
    ('int4', 1, 49152, 576, 64),      # config-2 lm_head: 4 tiles per workgroup
    ('nf4', 1, 20000, 4096, 128),     # 2 tiles per workgroup, waves split K in two
    # ... or, with rows of a whole segment, the lane-linear kernel
    ('int8', 1, 33000, 1024, 1024),   # per-row W8, one segment, row groups past N
    ('int4', 1, 32768, 2048, 128),    # one segment, quad scales
]


# Config 2: every SmolLM-135M linear shape at M = 1, 4, 16 on the default dispatch, with the
# config's groups (64 at K = 576, 128 at K = 1536) and with the SmolLM default group 32.
CONFIG2 = [(n, k) for n, k in ((576, 576), (192, 576), (1536, 576), (576, 1536), (49152, 576))]


@pytest.mark.parametrize('group', ['config', 32])
@pytest.mark.parametrize('m', [1, 4, 16])
@pytest.mark.parametrize('shape', CONFIG2, ids=lambda s: f'{s[0]}x{s[1]}')
def test_config2_cell_matches_oracle(device, shape, m, group):
    n, k = shape
    g = (64 if k == 576 else 128) if group == 'config' else group
    announce('config2 cell', n, k, m, g)
    rng = np.random.default_rng(100 + 7 * n + k + m)
    p = problem(rng, 'int4', m, n, k, g)
    check(p, run(p, device), f'config2 {n}x{k} M={m} g{g}')


@pytest.mark.parametrize('spec', SHAPES, ids=lambda s: '-'.join(map(str, s)))
def test_linear_matches_oracle(device, spec):
    fmt, m, n, k, group = spec
    rng = np.random.default_rng(m * 7919 + n * 31 + k)
    p = problem(rng, fmt, m, n, k, group)
    for path, flags in PATHS.items():
        if path == 'gemv' and m > 32:
            continue
        announce('linear', spec, path)
        check(p, run(p, device, flags), f'{spec}/{path}')


@pytest.mark.parametrize('spec', [('int8', 1, 1536, 576, 576, 32), ('int8', 3, 576, 1536, 1536, 32),
                                  ('int8', 40, 192, 576, 576, 32), ('int8', 256, 1536, 576, 576, 32),
                                  ('int4', 2, 64, 128, 32, 8), ('nf4', 70, 96, 64, 32, 5)],
                         ids=lambda s: '-'.join(map(str, s)))
def test_correction_and_bias(device, spec):
    fmt, m, n, k, group, rank = spec
    rng = np.random.default_rng(99 + m + n)
    for bias in (False, True):
        p = problem(rng, fmt, m, n, k, group, rank=rank, bias=bias)
        for path, flags in PATHS.items():
            if path == 'gemv' and m > 32:
                continue
            if path == 'gemm' and k % 32:
                continue
            announce('correction', spec, bias, path)
            check(p, run(p, device, flags), f'{spec}/{bias}/{path}')


def test_config1_exact_spec(device):
    """Config 1: W8A16 576->1536, seed 0, rank-32 correction, y = x.(q s)^T + (x.V^T).U^T."""
    announce('config1')
    g = torch.Generator().manual_seed(0)
    w = torch.randn(1536, 576, generator=g) * 0.02
    x = torch.randn(1, 576, generator=g).half()
    up = (torch.randn(1536, 32, generator=g) * 0.01).half()
    down = (torch.randn(32, 576, generator=g) * 0.01).half()
    data, scales = o.quantize(w.numpy(), 'int8')
    p = dict(fmt='int8', m=1, n=1536, k=576, group=576, x=x.numpy(), data=data, scales=scales, bias=None,
             down=down.numpy(), up=up.numpy())
    got = run(p, device)
    want = expected(p)
    assert o.rel_l2(got, want) <= REL_L2
    # fp32-accumulate spec without the fp16 staging, as a second reference
    exact = o.exact_weight('int8', (1536, 576), 576, data, scales)
    x64 = x.double().numpy()
    spec = x64 @ exact.T + (x64 @ down.double().numpy().T) @ up.double().numpy().T
    assert o.rel_l2(got, spec) <= REL_L2


def test_noncontiguous_and_strided_activations(device):
    announce('strided')
    rng = np.random.default_rng(11)
    p = problem(rng, 'int4', 6, 64, 128, 32)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    wide = torch.zeros(6, 200, dtype=torch.float16, device=device)
    wide[:, 8:136] = to_dev(p['x'], device)
    view = wide[:, 8:136]                          # row stride 200, 16-byte aligned start
    transposed = to_dev(np.ascontiguousarray(p['x'].T), device).t()   # column-major view
    want = expected(p)
    other = torch.zeros(6, 200, dtype=torch.float16, device=device)
    misaligned = other[:, 1:129]                   # 2-byte aligned start: generic kernel
    misaligned.copy_(view)
    for x in (view, transposed, misaligned):
        y = lowbit_hip.linear(x, codes, scales, format='int4', N=64, K=128, group_size=32)
        assert o.rel_l2(y.cpu().numpy(), want) <= REL_L2


@pytest.mark.parametrize('spec', [('int4', 1, 1024, 14336, 128), ('int8', 8, 256, 4096, 4096),
                                  ('nf4', 32, 520, 8192, 64)], ids=lambda s: '-'.join(map(str, s)))
def test_split_k_repeated_calls_reuse_workspace(device, spec):
    """Split-K partials: repeated calls on one workspace agree bit-for-bit."""
    fmt, m, n, k, group = spec
    announce('split-k repeat', spec)
    rng = np.random.default_rng(5 + n)
    p = problem(rng, fmt, m, n, k, group)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    x = to_dev(p['x'], device)
    out = torch.empty(m, n, dtype=torch.float16, device=device)
    call = lowbit_hip.PreparedLinear(x, codes, scales, format=fmt, N=n, K=k, group_size=group, out=out,
                                     flags=lowbit_hip.FLAG_FORCE_GEMV)
    assert call.workspace_bytes > 0  # the split decode GEMV splits this shape along K
    want = expected(p)
    first = None
    for _ in range(3):
        got = call.run().cpu().numpy()
        torch.cuda.synchronize()
        assert o.rel_l2(got, want) <= REL_L2
        if first is None:
            first = got.copy()
        np.testing.assert_array_equal(got.view(np.uint16), first.view(np.uint16))  # deterministic


def test_host_or_mismatched_operands_raise_before_launch(device):
    """A host tensor among device operands is refused with ValueError instead of being read
    as device memory; so are strided codes/scales views."""
    announce('operand devices')
    rng = np.random.default_rng(12)
    p = problem(rng, 'int4', 2, 64, 128, 32, rank=4, bias=True)
    x = to_dev(p['x'], device)
    codes = to_dev(np.frombuffer(p['data'], np.uint8), device)
    scales = to_dev(np.frombuffer(p['scales'], np.float16), device)
    kw = dict(format='int4', N=64, K=128, group_size=32)
    good = dict(bias=to_dev(p['bias'], device), down=to_dev(p['down'], device), up=to_dev(p['up'], device), rank=4)
    for name in ('bias', 'down', 'up'):
        with pytest.raises(ValueError, match=name):
            lowbit_hip.linear(x, codes, scales, **kw, **dict(good, **{name: good[name].cpu()}))
    with pytest.raises(ValueError, match='scales'):
        lowbit_hip.linear(x, codes, scales.cpu(), **kw)
    with pytest.raises(ValueError, match='codes'):
        lowbit_hip.linear(x, codes.cpu(), scales, **kw)
    with pytest.raises(ValueError, match='out'):
        lowbit_hip.linear(x, codes, scales, **kw, out=torch.empty(2, 64, dtype=torch.float16))
    with pytest.raises(ValueError, match='scales'):
        wide = torch.zeros(scales.numel() * 2, dtype=torch.float16, device=device)
        lowbit_hip.linear(x, codes, wide[::2], **kw)
    y = lowbit_hip.linear(x, codes, scales, **kw, **good)
    assert o.rel_l2(y.cpu().numpy(), expected(p)) <= REL_L2


@pytest.mark.parametrize('m,n,k,group', [(1, 20000, 4096, 128), (64, 4096, 1024, 64), (512, 2560, 960, 64)])
def test_nf4_gemm_repeated_launches(device, m, n, k, group):
    """NF4 GEMM tiles decode their weights through an LDS table that the workgroup's threads build
    together; the first decode waits for the whole table.  Twelve launches of the forced GEMM path
    each match the oracle and give the same bits."""
    announce('nf4 gemm repeated', m, n, k, group)
    rng = np.random.default_rng(m + n + k)
    p = problem(rng, 'nf4', m, n, k, group)
    first = run(p, device, lowbit_hip.FLAG_FORCE_GEMM)
    check(p, first, f'nf4 gemm {m}x{n}x{k}')
    for i in range(11):
        again = run(p, device, lowbit_hip.FLAG_FORCE_GEMM)
        np.testing.assert_array_equal(again.view(np.uint16), first.view(np.uint16), err_msg=f'launch {i + 2}')
