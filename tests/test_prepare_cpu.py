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
