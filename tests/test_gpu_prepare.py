"""Preparation on the GPU: calibrate_int8 and fit_lowrank_correction with device='cuda' (fp64
rocBLAS / rocSOLVER instead of the CPU's LAPACK).  The same algebraic properties as on the CPU
must hold (tests/test_prepare_cpu.py); against the CPU result the codes agree except at exact
rounding ties and the correction product U.V agrees to the fp16 storage precision (singular
vectors may flip sign in pairs).  Bitwise equality with the CPU result is not claimed."""
import numpy as np
import pytest
import torch

from conftest import announce
from torch_npu_lowbit import PackedWeight, calibrate_int8, quantize_weight
from torch_npu_lowbit_correction import fit_lowrank_correction

pytestmark = pytest.mark.gpu


def codes_of(q):
    return np.frombuffer(q.data, dtype=np.int8).reshape(q.shape)


def scales_of(q):
    return np.frombuffer(q.scales, dtype=np.float16).astype(np.float64)


def test_calibrate_int8_on_device(device):
    announce('calibrate_int8 on device')
    g = torch.Generator().manual_seed(5)
    basis = torch.randn(16, 192, generator=g)
    inputs = (torch.randn(256, 16, generator=g) @ basis + 0.05 * torch.randn(256, 192, generator=g)).float()
    inputs[:, -1] = 0  # a dead column keeps its plain codes
    weight = torch.randn(48, 192, generator=g) * 0.05
    plain = quantize_weight(weight, format='int8')
    cpu = calibrate_int8(weight, inputs)
    gpu = calibrate_int8(weight, inputs, device=device)
    assert gpu.scales == plain.scales
    x = inputs.double().numpy()
    target = x @ weight.double().numpy().T

    def loss(q):
        return (((x @ codes_of(q).astype(np.float64).T) * scales_of(q)[None] - target) ** 2).sum(0)

    assert np.all(loss(gpu) <= loss(plain) + 1e-18)
    assert loss(gpu).sum() < 0.8 * loss(plain).sum()
    np.testing.assert_array_equal(codes_of(gpu)[:, -1], codes_of(plain)[:, -1])
    assert np.mean(codes_of(gpu) == codes_of(cpu)) >= 0.99
    assert calibrate_int8(weight, torch.zeros_like(inputs), device=device) == plain


def test_fit_lowrank_correction_on_device(device):
    announce('fit_lowrank_correction on device')
    g = torch.Generator().manual_seed(441)
    x = torch.randn(64, 7, generator=g)
    x[:, -1] = 0
    weight = (torch.randn(5, 2, generator=g) @ torch.randn(2, 7, generator=g) / 32).half()
    packed = PackedWeight((5, 7), 'int8', 7, bytes(35), np.ones(5, dtype=np.float16).tobytes())
    down, up = fit_lowrank_correction(weight, packed, x, rank=2, device=device).tensors()
    actual = (x.double() @ down.double().t()) @ up.double().t()
    expected = x.double() @ weight.double().t()
    assert float((actual - expected).square().sum()) < float(expected.square().sum()) * 1e-5
    # a SmolLM-shaped projection: the device fit and the CPU fit give the same U.V
    g = torch.Generator().manual_seed(7)
    weight = torch.randn(576, 576, generator=g) * 0.02
    inputs = torch.randn(512, 576, generator=g)
    packed = quantize_weight(weight, format='int8')
    products = []
    for dev in (None, device):
        d, u = fit_lowrank_correction(weight, packed, inputs, rank=32, device=dev).tensors()
        products.append(u.double() @ d.double())
    rel = float((products[0] - products[1]).norm() / products[0].norm())
    assert rel < 1e-2, rel
