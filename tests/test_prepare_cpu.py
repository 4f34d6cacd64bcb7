"""CPU checks of the preparation side of the path (no GPU): GPTQ W8 calibration, low-rank
correction fitting, quantizer guards and the QuantizedLinear option surface.

The properties are the ones the reference's own offline tests hold for these functions
(test_torch_npu_lowbit.py:9-31, 43-58, 60-112; test_torch_npu_lowbit_correction.py:10-57),
restated against this package.  They pin the algorithms through what the mathematics
fixes: an exact low-rank error is reconstructed, a full-rank fit restores the weight,
GPTQ never raises any row's reconstruction loss and lowers the total, dead input columns
keep their plain codes, zero error gives a zero correction.
"""
import numpy as np
import pytest
import torch

from torch_npu_lowbit import NF4, PackedWeight, QuantizedLinear, calibrate_int8, pack_codes, quantize_weight
from torch_npu_lowbit_correction import LowRankCorrection, fit_lowrank_correction


def codes_of(q):
    return np.frombuffer(q.data, dtype=np.int8).reshape(q.shape)


def scales_of(q):
    return np.frombuffer(q.scales, dtype=np.float16).astype(np.float64)


def test_calibration_never_worse_and_guards():
    g = torch.Generator().manual_seed(647)
    weight = (torch.randn(7, 129, generator=g) / 8).half().requires_grad_()
    snapshot = weight.detach().clone()
    inputs = torch.randn(48, 129, generator=g).half()
    inputs[:, 1] = inputs[:, 0]      # duplicate column: singular Hessian before damping
    inputs[:, -1] = 0                # dead column
    inputs = inputs.t().contiguous().t()
    plain = quantize_weight(weight.detach(), format='int8')
    tuned = calibrate_int8(weight, inputs)
    assert tuned.scales == plain.scales and len(tuned.data) == len(plain.data)
    assert torch.equal(weight, snapshot) and weight.grad is None

    x = inputs.double().numpy()
    target = x @ snapshot.double().numpy().T

    def loss(q):
        return (((x @ codes_of(q).astype(np.float64).T) * scales_of(q)[None] - target) ** 2).sum(0)

    assert np.all(loss(tuned) <= loss(plain) + 1e-18)
    assert loss(tuned).sum() < loss(plain).sum()
    assert calibrate_int8(weight, inputs) == tuned
    np.testing.assert_array_equal(codes_of(tuned)[:, -1], codes_of(plain)[:, -1])
    assert calibrate_int8(weight, torch.zeros_like(inputs)) == plain
    zero = torch.zeros_like(weight)
    assert calibrate_int8(zero, inputs) == quantize_weight(zero.detach(), format='int8')
    for bad in (None, torch.zeros(0, 129), torch.zeros(2, 128), torch.zeros(1, 2, 129), inputs.double(),
                torch.full_like(inputs, float('nan')), torch.full_like(inputs, float('inf')), torch.zeros(4097, 129)):
        with pytest.raises(ValueError):
            calibrate_int8(weight, bad)
    with pytest.raises(ValueError):
        calibrate_int8(torch.ones(1, 4097), torch.ones(1, 4097))
    with pytest.raises(ValueError):
        calibrate_int8(torch.ones(8192, 1), torch.ones(513, 1))


def test_calibration_reduces_loss_on_correlated_inputs():
    """A strongly correlated input distribution is where error feedback pays most."""
    g = torch.Generator().manual_seed(5)
    basis = torch.randn(16, 96, generator=g)
    inputs = (torch.randn(256, 16, generator=g) @ basis + 0.05 * torch.randn(256, 96, generator=g)).float()
    weight = torch.randn(32, 96, generator=g) * 0.05
    plain = quantize_weight(weight, format='int8')
    tuned = calibrate_int8(weight, inputs)
    x = inputs.double().numpy()
    target = x @ weight.double().numpy().T

    def loss(q):
        return (((x @ codes_of(q).astype(np.float64).T) * scales_of(q)[None] - target) ** 2).sum()

    assert loss(tuned) < 0.8 * loss(plain)
    assert np.abs(codes_of(tuned)).max() <= 127


def test_exact_low_rank_error_is_reconstructed():
    g = torch.Generator().manual_seed(441)
    x = torch.randn(64, 7, generator=g)
    x[:, -1] = 0
    weight = (torch.randn(5, 2, generator=g) @ torch.randn(2, 7, generator=g) / 32).half()
    packed = PackedWeight((5, 7), 'int8', 7, bytes(35), np.ones(5, dtype=np.float16).tobytes())
    down, up = fit_lowrank_correction(weight, packed, x, rank=2).tensors()
    actual = (x.double() @ down.double().t()) @ up.double().t()
    expected = x.double() @ weight.double().t()
    torch.testing.assert_close(actual, expected, rtol=.02, atol=2e-4)
    assert float((actual - expected).square().sum()) < float(expected.square().sum()) * 1e-5


def test_full_rank_restores_weight_and_truncation_is_a_prefix():
    g = torch.Generator().manual_seed(442)
    weight = torch.randn(4, 7, generator=g).half()
    x = torch.randn(50, 7, generator=g)
    packed = quantize_weight(weight, format='int8')
    fit = fit_lowrank_correction(weight, packed, x, rank=4)
    down, up = fit.tensors()
    decoded = torch.from_numpy(codes_of(packed).astype(np.float64) * scales_of(packed)[:, None])
    torch.testing.assert_close(decoded + up.double() @ down.double(), weight.double(), rtol=1e-3, atol=1e-5)
    short = fit.truncated(2)
    d2, u2 = short.tensors()
    assert torch.equal(d2, down[:2]) and torch.equal(u2, up[:, :2])
    down.fill_(99)
    assert fit.tensors()[0][0, 0] != 99


def test_zero_error_gives_zero_correction_and_guards():
    weight = torch.full((4, 8), .125)
    packed = PackedWeight((4, 8), 'int8', 8, bytes([1]) * 32, np.full(4, .125, dtype=np.float16).tobytes())
    down, up = fit_lowrank_correction(weight, packed, torch.zeros(10, 8), rank=2).tensors()
    assert int(torch.count_nonzero(down)) == 0 and int(torch.count_nonzero(up)) == 0
    weight = torch.ones(4, 8)
    packed = quantize_weight(weight, format='int8')
    x = torch.ones(12, 8)
    for rank in (0, 5, True):
        with pytest.raises(ValueError):
            fit_lowrank_correction(weight, packed, x, rank=rank)
    for bad in (torch.ones(12, 7), torch.full((12, 8), float('nan')), torch.ones(4097, 8)):
        with pytest.raises(ValueError):
            fit_lowrank_correction(weight, packed, bad, rank=2)
    with pytest.raises(ValueError):
        fit_lowrank_correction(weight, quantize_weight(weight, format='int4'), x, rank=2)
    for shape, rank, d, u in (((4, 8), True, bytes(32), bytes(16)), ((4, 8), 2, bytearray(32), bytes(16)),
                              ((4, 8), 2, np.full(16, np.inf, dtype=np.float16).tobytes(), bytes(16)),
                              ((4, 8), 2, bytes(30), bytes(16))):
        with pytest.raises(ValueError):
            LowRankCorrection(shape, rank, d, u)


def test_quantizer_groups_zero_and_guards():
    g = torch.Generator().manual_seed(41)
    for shape, size in (((3, 17), None), ((8, 64), 32), ((4, 128), 128)):
        original = torch.randn(shape, generator=g) / 8
        for fmt in ('int4', 'nf4', 'int8'):
            q = quantize_weight(original, format=fmt, group_size=size)
            assert q.dequantize().shape == shape
            assert len(q.data) == (original.numel() if fmt == 'int8' else (original.numel() + 1) // 2)
    for fmt in ('int4', 'nf4', 'int8'):
        np.testing.assert_array_equal(quantize_weight(torch.zeros(3, 17), format=fmt).dequantize(),
                                      np.zeros((3, 17), dtype=np.float16))
    for kwargs in (dict(format='fp4'), dict(group_size=3), dict(group_size=True)):
        with pytest.raises(ValueError):
            quantize_weight(torch.ones(2, 16), **kwargs)
    for value in (float('inf'), float('nan')):
        with pytest.raises(ValueError):
            quantize_weight(torch.full((2, 16), value))
    with pytest.raises(ValueError):
        PackedWeight((1, 3), 'int4', 3, b'\x10\xf2', np.float16(1).tobytes())
    codes = np.arange(16, dtype=np.uint8)
    for fmt in ('int4', 'nf4'):
        w = PackedWeight((1, 16), fmt, 16, pack_codes(codes), np.float16(1).tobytes())
        expected = np.arange(-8, 8, dtype=np.float16)[(codes + 8) % 16] if fmt == 'int4' else NF4.astype(np.float16)
        np.testing.assert_array_equal(w.dequantize().ravel(), expected)


def test_quantized_linear_option_surface():
    q = quantize_weight(torch.randn(5, 9), group_size=3)
    layer = QuantizedLinear(q, compact_groups=True)
    assert layer.compact_groups
    with pytest.raises(AttributeError):
        layer.compact_groups = False
    with pytest.raises(ValueError):
        QuantizedLinear(q, compact_groups=1)
    with pytest.raises(ValueError):
        QuantizedLinear(quantize_weight(torch.ones(1, 33), group_size=1), compact_groups=True)
    codes = np.arange(-128, 128, dtype=np.int8)
    w8 = PackedWeight((1, 256), 'int8', 256, codes.tobytes(), np.float16(.125).tobytes())
    np.testing.assert_array_equal(w8.dequantize().ravel(), codes.astype(np.float16) * .125)
    layer = QuantizedLinear(w8, activation_scale=1 / 128)
    assert layer.activation_scale == 1 / 128
    with pytest.raises(AttributeError):
        layer.activation_scale = 1 / 64
    for scale in (True, 0, -1, 2 ** -25, 512, .0037, float('nan'), float('inf'), '0.125'):
        with pytest.raises(ValueError):
            QuantizedLinear(w8, activation_scale=scale)
    for fmt, size in (('int4', 256), ('nf4', 256), ('int8', 128)):
        with pytest.raises(ValueError):
            QuantizedLinear(quantize_weight(torch.ones(1, 256), format=fmt, group_size=size), activation_scale=1 / 128)
    with pytest.raises(ValueError):
        QuantizedLinear(w8, activation_scale=1 / 128, compact_groups=True)
    for data in (codes.tobytes()[:-1], codes.tobytes() + b'\0', bytearray(codes)):
        with pytest.raises(ValueError):
            PackedWeight(w8.shape, w8.format, w8.group_size, data, w8.scales)
    large = PackedWeight((1, 256), 'int8', 256, codes.tobytes(), np.float16(512).tobytes())
    with pytest.raises(ValueError):
        QuantizedLinear(large, activation_scale=1 / 128)


# --- the product quantizer against the oracle's restatement (reference torch_npu_lowbit.py:78-105) ---------

def _oracle_quantize(weight, fmt, group):
    from oracle import lowbit_oracle as lo
    return lo.quantize(weight.float().numpy(), fmt, group)


def test_quantize_weight_matches_oracle_on_ties():
    """rint's half-to-even ties (int4 / int8) and searchsorted(side='left') at the NF4 midpoints."""
    from oracle import lowbit_oracle as lo
    ties = torch.tensor([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]])
    q = quantize_weight(ties, format='int4')
    assert (q.data, q.scales) == _oracle_quantize(ties, 'int4', None)
    assert lo.unpack('int4', q.data, 8).tolist() == [7, 0, 2, 2, 0, -2, -2, 4]
    ties8 = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -125.5]])
    q = quantize_weight(ties8, format='int8')
    assert (q.data, q.scales) == _oracle_quantize(ties8, 'int8', None)
    assert np.frombuffer(q.data, np.int8).tolist() == [127, 0, 2, 2, 0, -2, 126, -126]
    mids = ((lo.NF4_F32[:-1] + lo.NF4_F32[1:]) / np.float32(2)).astype(np.float32)
    values = np.concatenate([[1.0], mids, np.nextafter(mids, np.float32(2)), -np.nextafter(mids, np.float32(-2))])
    w = torch.from_numpy(values.astype(np.float32)[None, :])
    q = quantize_weight(w, format='nf4')
    assert (q.data, q.scales) == _oracle_quantize(w, 'nf4', None)
    codes = lo.unpack('nf4', q.data, w.numel())
    assert codes[1:16].tolist() == list(range(15)) and codes[16:31].tolist() == list(range(1, 16))


@pytest.mark.parametrize('fmt', ['int4', 'nf4', 'int8'])
def test_quantize_weight_matches_oracle_random(fmt):
    """Seeded sweep over shapes, group sizes, dtypes and magnitudes (tiny, zero and odd-count rows)."""
    g = torch.Generator().manual_seed({'int4': 41, 'nf4': 42, 'int8': 43}[fmt])
    for n, k, groups in ((3, 64, (None, 1, 8, 32, 64)), (7, 96, (None, 3, 32, 48)), (1, 5, (None, 1, 5)),
                         (16, 576, (None, 32, 64)), (5, 1536, (None, 128))):
        for std in (0.02, 1.0, 1e-6):
            for dtype in (torch.float32, torch.float16):
                w = (torch.randn(n, k, generator=g) * std).to(dtype)
                w[0, : k // 2] = 0
                if n > 2:
                    w[2] = 0
                for group in groups:
                    q = quantize_weight(w, format=fmt, group_size=group)
                    data, scales = _oracle_quantize(w, fmt, group)
                    assert q.data == data, (fmt, n, k, group, std, dtype)
                    assert q.scales == scales, (fmt, n, k, group, std, dtype)


# --- GPTQ against a plain OBS column loop (reference torch_npu_lowbit.py:108-152) --------------------------

def _obs_codes(weight, inputs, scales, order_descending=True):
    """Textbook optimal-brain-surgeon quantization: for each column in activation order,
    quantize it, spread its error over the remaining columns through the explicit inverse
    Hessian, then eliminate the column from that inverse (Schur complement).  fp64, no
    Cholesky factor, no column blocks."""
    x = inputs.double().numpy()
    k = x.shape[1]
    h = x.T @ x / x.shape[0]
    energy = np.diag(h).copy()
    order = np.argsort(-energy if order_descending else energy, kind='stable')
    h = h[np.ix_(order, order)]
    dead = energy[order] == 0
    h[dead, dead] = 1.0
    h += 0.01 * max(np.diag(h).mean(), 1e-20) * np.eye(k)
    hinv = np.linalg.inv(h)
    w = weight.double().numpy()[:, order].copy()
    codes = np.zeros(w.shape, np.int64)
    for j in range(k):
        q = np.clip(np.round(w[:, j] / scales), -127, 127)
        codes[:, j] = q
        d = hinv[j, j]
        err = (w[:, j] - q * scales) / d
        w[:, j + 1:] -= np.outer(err, hinv[j, j + 1:])
        hinv = hinv - np.outer(hinv[:, j], hinv[j, :]) / d
    out = np.empty_like(codes)
    out[:, order] = codes
    return out


def test_calibration_matches_plain_obs_loop():
    g = torch.Generator().manual_seed(73)
    n, k = 6, 300                     # three 128-column blocks in the product
    basis = torch.randn(24, k, generator=g)
    inputs = (torch.randn(400, 24, generator=g) @ basis + 0.1 * torch.randn(400, k, generator=g)).float()
    inputs[:, 17] = 0                 # a dead column
    weight = torch.randn(n, k, generator=g) * 0.05
    plain = quantize_weight(weight, format='int8')
    scales = scales_of(plain)
    tuned = calibrate_int8(weight, inputs)
    proposed = _obs_codes(weight, inputs, scales)
    # the product keeps a row's OBS codes exactly where they lower that row's loss, else the plain codes
    x = inputs.double().numpy()
    target = x @ weight.double().numpy().T

    def row_loss(c):
        return (((x @ c.astype(np.float64).T) * scales[None] - target) ** 2).sum(0)

    better = row_loss(proposed) < row_loss(codes_of(plain))
    assert better.any()
    expected = np.where(better[:, None], proposed, codes_of(plain))
    np.testing.assert_array_equal(codes_of(tuned), expected)
    # a wrong activation order changes the codes: the check is sensitive to it
    assert (_obs_codes(weight, inputs, scales, order_descending=False) != proposed).any()
