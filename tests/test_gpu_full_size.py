"""GPU checks at BASELINE.json's full sizes, through properties that hold bit for bit whatever the
size, plus the oracle on row slices.

- Homogeneity: y(4 x) == 4 y(x) bit for bit wherever y is an fp16 normal number.  Every kernel
  forms exact products (fp16 x fp16 in fp32, or exact integer-code sums) and fp32 sums, so scaling
  the activations by a power of two scales every partial sum exactly (activations are kept away
  from the fp16 subnormal range, where the 1/16 staging of odd INT4 codes would round).  An output
  below 2^-14 is rounded to a subnormal, on a fixed 2^-24 grid, so there 4 y(x) carries 4 times
  that rounding: |y(4 x) - 4 y(x)| <= 2^-23.
- Row equivariance: reversing the weight rows (codes and scales) reverses y bit for bit; a row's
  arithmetic does not depend on which tile, wave or workgroup computes it.
- Oracle: the restated reference (rel-L2 <= 1e-3 and its rounding-budget gate) on row slices.
Shapes: every config-5 cell (Llama-3-8B projections 4096x4096, 1024x4096, 14336x4096, 4096x14336
and the 128256x4096 head, INT4 g128, at M = 1, 8, 32, 256, 1024), every config-3 cell (NF4 g64
2560x960 and 960x2560 at M = 128, 512, 2048), config 2's lm_head 49152x576 g64 at M = 4 and 16,
the W8 GEMV at M = 1 on the Llama head (per-row int8) and a grouped int8 32768x2048.
"""
import numpy as np
import pytest
import torch

import lowbit_hip
from conftest import announce
from test_gpu_linear import check

pytestmark = pytest.mark.gpu

CONFIG5 = [('int4', m, n, k, 128) for m in (1, 8, 32, 256, 1024)
           for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096))]
CONFIG3 = [('nf4', m, n, k, 64) for m in (128, 512, 2048) for n, k in ((2560, 960), (960, 2560))]
FULL = CONFIG5 + CONFIG3 + [('int4', 4, 49152, 576, 64), ('int4', 16, 49152, 576, 64),
                            ('int8', 1, 128256, 4096, 4096), ('int8', 1, 32768, 2048, 64)]


def packed_random(rng, fmt, n, k, group):
    """Random codes and scales of the quantizer's range (no CPU quantization of a full-size matrix)."""
    data = rng.integers(0, 256, n * k // 2, dtype=np.uint8) if fmt != 'int8' else rng.integers(-127, 128, n * k).astype(np.int8)
    limit = {'int4': 7, 'nf4': 1, 'int8': 127}[fmt]
    scales = (rng.uniform(0.5, 1.5, n * (k // group)) * 0.05 / limit).astype(np.float16)
    return data.tobytes(), scales


def activations(rng, m, k):
    x = rng.standard_normal((m, k)).astype(np.float32)
    x = np.where(np.abs(x) < 0.0625, np.sign(x + 1e-9) * 0.0625, x)  # no fp16-subnormal staging
    return x.astype(np.float16)


@pytest.mark.parametrize('spec', FULL, ids=lambda s: '-'.join(map(str, s)))
def test_full_size_properties_and_slices(device, spec):
    fmt, m, n, k, group = spec
    announce('full size', spec)
    rng = np.random.default_rng(n + m)
    data, scales = packed_random(rng, fmt, n, k, group)
    x = activations(rng, m, k)
    codes = torch.from_numpy(np.frombuffer(data, np.uint8).copy()).to(device)
    sc = torch.from_numpy(scales).to(device)
    xd = torch.from_numpy(x).to(device)

    def run(xx, cc, ss):
        y = lowbit_hip.linear(xx, cc, ss, format=fmt, N=n, K=k, group_size=group)
        torch.cuda.synchronize()
        return y

    y = run(xd, codes, sc)
    assert bool(torch.isfinite(y).all())
    # homogeneity
    y4 = run(xd * 4, codes, sc)
    normal = y.abs() >= 2.0 ** -14
    assert torch.equal(y4[normal], (y * 4)[normal]), 'y(4x) != 4 y(x)'
    tiny = (y4.float() - 4 * y.float())[~normal]
    assert tiny.numel() == 0 or float(tiny.abs().max()) <= 2.0 ** -23
    # row equivariance
    row_bytes = k // 2 if fmt != 'int8' else k
    codes_rev = codes.view(n, row_bytes).flip(0).reshape(-1).contiguous()
    sc_rev = sc.view(n, k // group).flip(0).reshape(-1).contiguous()
    y_rev = run(xd, codes_rev, sc_rev)
    assert torch.equal(y_rev, y.flip(1)), 'reversed rows do not give the reversed output'
    # oracle on row slices
    got = y.cpu().numpy()
    rows = min(1024 if m <= 16 else 256, n // 2)
    g = k // group
    for lo in (0, n // 2 - rows // 2 + 16, n - rows):
        d = data[lo * row_bytes:(lo + rows) * row_bytes]
        s = scales[lo * g:(lo + rows) * g].tobytes()
        p = dict(fmt=fmt, m=m, n=rows, k=k, group=group, x=x, data=d, scales=s, bias=None, down=None, up=None)
        check(p, np.ascontiguousarray(got[:, lo:lo + rows]), f'full size {spec} rows from {lo}')
