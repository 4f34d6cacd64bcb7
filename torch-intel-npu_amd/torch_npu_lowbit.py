"""Low-bit frozen linear weights (INT4 / NF4 / INT8) with fp16 IO on MI355X.

Drop-in for the reference module of the same name (LCS-Official/torch-intel-npu,
torch_npu_lowbit.py): same NF4 table, pack_codes, PackedWeight byte layout and
validation, quantize_weight, calibrate_int8 and QuantizedLinear API.  The NPU graph
path (weight_graph / compile_weight / dpu_modes, :169-297) is replaced by gfx950 HIP
kernels behind the C-ABI of liblowbit_hip.so (see lowbit_hip).

Deviation: the reference bounds every PackedWeight at N*K <= 1,048,576 elements
(npunlock/npu4000.py:23); the DPU limit does not apply here, so the bound is
MAX_TENSOR_ELEMENTS = 2**31 - 1 (the kernels index rows with 32-bit ints).
"""
from dataclasses import dataclass
from math import frexp, isfinite, prod

import numpy as np
import torch

import lowbit_hip

MAX_TENSOR_ELEMENTS = 2 ** 31 - 1

# NormalFloat4 codebook, fp32 literals (reference :17-21; OpenVINO nf4.cpp / bitsandbytes).
NF4 = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
                0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)
NF4.flags.writeable = False

_LIMITS = {'int4': 7, 'nf4': 1, 'int8': 127}


def pack_codes(codes):
    """Two 4-bit codes per byte, flat element 2i in the low nibble (reference :24-30)."""
    values = np.asarray(codes)
    if values.dtype != np.uint8 or values.size == 0 or (values > 15).any():
        raise ValueError('Codes must be a nonempty uint8 array in 0..15')
    flat = values.reshape(-1)
    if flat.size % 2:
        flat = np.append(flat, np.uint8(0))
    pairs = flat.reshape(-1, 2)
    return (pairs[:, 0] | (pairs[:, 1] << 4)).astype(np.uint8).tobytes()


def _unpack_nibbles(data, count):
    raw = np.frombuffer(data, dtype=np.uint8)
    return np.stack((raw & 0x0F, raw >> 4), axis=1).reshape(-1)[:count]


@dataclass(frozen=True)
class PackedWeight:
    """Immutable packed weight; byte layout identical to the reference (:33-65)."""
    shape: tuple
    format: str
    group_size: int
    data: bytes
    scales: bytes

    def __post_init__(self):
        shape = self.shape
        if (type(shape) is not tuple or len(shape) != 2 or any(type(v) is not int or v <= 0 for v in shape)
                or prod(shape) > MAX_TENSOR_ELEMENTS or self.format not in _LIMITS
                or type(self.group_size) is not int or not 1 <= self.group_size <= shape[1]
                or shape[1] % self.group_size):
            raise ValueError('Weight requires bounded (N,K), int4/nf4/int8, and a group size dividing K')
        if not isinstance(self.data, bytes) or not isinstance(self.scales, bytes):
            raise ValueError('Packed data/scales must be immutable bytes')
        count = prod(shape)
        expected = count if self.format == 'int8' else (count + 1) // 2
        odd_pad = self.format != 'int8' and count % 2 == 1 and (self.data[-1] & 0xF0) != 0
        if len(self.data) != expected or odd_pad:
            raise ValueError('Packed weight extent/padding differs')
        if len(self.scales) != 2 * count // self.group_size:
            raise ValueError('Scale extent differs')
        scales = np.frombuffer(self.scales, dtype=np.float16)
        if not np.isfinite(scales).all() or (scales <= 0).any():
            raise ValueError('Scales must be finite, positive FP16 values')

    @property
    def dtype(self):
        return {'int4': 'i4', 'nf4': 'nf4', 'int8': 'i8'}[self.format]

    @property
    def grouped_shape(self):
        n, k = self.shape
        return n, k // self.group_size, self.group_size

    def dequantize(self):
        """CPU reference: fp16(q * s) with both fp16 rounding stages (reference :67-75)."""
        n, k = self.shape
        if self.format == 'int8':
            q = np.frombuffer(self.data, dtype=np.int8).astype(np.float16)
        else:
            c = _unpack_nibbles(self.data, n * k)
            q = ((c.astype(np.int8) ^ 8) - 8).astype(np.float16) if self.format == 'int4' \
                else NF4.astype(np.float16)[c]
        s = np.frombuffer(self.scales, dtype=np.float16).reshape(n, k // self.group_size, 1)
        return (q.reshape(self.grouped_shape) * s).reshape(self.shape)

    def device_tensors(self, device):
        """(codes uint8, scales fp16 [N,G]) on `device`; uploaded once and cached per device."""
        device = torch.device(device)
        cache = self.__dict__.setdefault('_device_cache', {})
        key = (device.type, device.index if device.index is not None else torch.cuda.current_device())
        if key not in cache:
            codes = torch.frombuffer(bytearray(self.data), dtype=torch.uint8).to(device)
            scales = torch.frombuffer(bytearray(self.scales), dtype=torch.float16).view(
                self.shape[0], -1).to(device)
            cache[key] = (codes, scales)
        return cache[key]


def quantize_weight(weight, *, format='int4', group_size=None):
    """Symmetric CPU preparation with fp16 scales (reference :78-105)."""
    if (not isinstance(weight, torch.Tensor) or weight.device.type != 'cpu' or weight.ndim != 2
            or weight.dtype not in (torch.float16, torch.float32)):
        raise ValueError('Quantization preparation requires a CPU 2D Tensor')
    n, k = weight.shape
    size = k if group_size is None else group_size
    if (format not in _LIMITS or type(size) is not int or not 1 <= size <= k or k % size
            or not 0 < n * k <= MAX_TENSOR_ELEMENTS):
        raise ValueError('Requires int4/nf4/int8 and a group size dividing bounded K')
    values = weight.detach().float().numpy().reshape(n, k // size, size)
    if not np.isfinite(values).all():
        raise ValueError('Nonfinite weights cannot be quantized')
    limit = _LIMITS[format]
    scale = np.abs(values).max(axis=-1, keepdims=True) / limit
    if (scale > np.finfo(np.float16).max).any():
        raise ValueError('Weight scale overflows FP16')
    scale = np.maximum(scale, np.float32(2 ** -24)).astype(np.float16)
    normalized = values / scale.astype(np.float32)
    if format == 'nf4':
        midpoints = (NF4[:-1] + NF4[1:]) / 2
        data = pack_codes(np.searchsorted(midpoints, normalized, side='left').astype(np.uint8))
    else:
        codes = np.clip(np.rint(normalized), -limit, limit).astype(np.int8)
        data = codes.tobytes() if format == 'int8' else pack_codes((codes & 0x0F).astype(np.uint8))
    return PackedWeight((n, k), format, size, data, scale.tobytes())


@torch.no_grad()
def calibrate_int8(weight, inputs, *, device=None):
    """GPTQ-style W8 preparation (reference :108-152), fp64.

    Same contract as the reference: fixed fp16 per-row scales from quantize_weight,
    codes in [-127,127], descending-energy activation order with stable ties, 1% mean
    diagonal damping, dead columns keep their original codes, 128-column blocks, and a
    per-row fallback to the plain codes when calibration does not reduce the
    reconstruction error on `inputs`.  The arguments are CPU tensors as in the reference;
    `device` (e.g. 'cuda') runs the fp64 linear algebra there instead of on the CPU (its
    BLAS sums in another order, so a code at an exact rounding tie may differ).
    """
    original = quantize_weight(weight, format='int8')
    n, k = weight.shape
    if (not isinstance(inputs, torch.Tensor) or inputs.device.type != 'cpu'
            or inputs.dtype not in (torch.float16, torch.float32) or inputs.ndim != 2
            or inputs.shape[1] != k or not 1 <= inputs.shape[0] <= 4096 or k > 4096
            or max(inputs.numel(), inputs.shape[0] * n) > 4 * 1048576
            or not torch.isfinite(inputs).all()):
        raise ValueError('Calibration requires bounded finite CPU FP16/FP32 (rows,K), rows/K<=4096, matching weight K')
    dev = torch.device('cpu' if device is None else device)
    x = inputs.detach().to(dev, torch.float64)
    hessian = x.T @ x / x.shape[0]
    energy = hessian.diagonal().clone()
    order = torch.argsort(energy, descending=True, stable=True)
    hessian = hessian[order][:, order]
    dead = energy[order] == 0
    hessian[dead, dead] = 1.0
    damp = 0.01 * hessian.diagonal().mean().clamp_min(1e-20)
    hessian += damp * torch.eye(k, dtype=torch.float64, device=dev)
    # Upper Cholesky factor of H^-1 drives the column-by-column error feedback.
    inverse_factor = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(hessian)), upper=True)
    work = weight.detach().to(dev, torch.float64)[:, order].clone()
    scales = torch.from_numpy(np.frombuffer(original.scales, dtype=np.float16).astype(np.float64)).to(dev)
    codes = torch.empty((n, k), dtype=torch.int8, device=dev)
    for start in range(0, k, 128):
        stop = min(start + 128, k)
        block = work[:, start:stop].clone()
        errors = torch.zeros_like(block)
        for i in range(stop - start):
            col = start + i
            pivot = inverse_factor[col, col]
            q = (block[:, i] / scales).round().clamp(-127, 127)
            codes[:, col] = q.to(torch.int8)
            err = (block[:, i] - q * scales) / pivot
            block[:, i:] -= err[:, None] * inverse_factor[col, col:stop][None, :]
            errors[:, i] = err
        work[:, stop:] -= errors @ inverse_factor[start:stop, stop:]
    proposed = codes[:, torch.argsort(order)].contiguous().cpu().numpy()
    plain = np.frombuffer(original.data, dtype=np.int8).reshape(n, k).copy()
    target = x @ weight.detach().to(dev, torch.float64).T

    def row_error(c):
        predicted = (x @ torch.from_numpy(c.astype(np.float64)).to(dev).T) * scales[None, :]
        return (predicted - target).square().sum(0).cpu().numpy()

    better = row_error(proposed) < row_error(plain)
    plain[better] = proposed[better]
    return PackedWeight(original.shape, 'int8', original.group_size, plain.tobytes(), original.scales)


def _activation_scale(weight, scale, compact_groups):
    """W8A8 activation grid validation (reference :155-166)."""
    if scale is None:
        return None
    if (type(scale) not in (int, float) or not isfinite(scale) or not 2 ** -24 <= scale <= 511
            or weight.format != 'int8' or weight.group_size != weight.shape[1] or compact_groups):
        raise ValueError('Activation quantization requires per-channel INT8, no compact groups, '
                         'and a finite scale in [2^-24,511]')
    if frexp(scale)[0] != 0.5:
        raise ValueError('Activation scale must be an exact power of two')
    if (np.frombuffer(weight.scales, dtype=np.float16) > 511).any():
        raise ValueError('INT8 weight quantization range overflows FP16')
    return float(np.float16(scale))


def _validate_activation(x, k):
    if not isinstance(x, torch.Tensor) or x.device.type != 'cuda':
        raise ValueError('QuantizedLinear requires a ROCm device tensor')
    if x.requires_grad and torch.is_grad_enabled():
        raise ValueError('QuantizedLinear is inference-only; use no_grad/inference_mode')
    if x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != k:
        raise ValueError('QuantizedLinear requires 2D FP16 activations with matching K')


class QuantizedLinear(torch.nn.Module):
    """Frozen inference with fp16 IO (reference :300-360), executed by liblowbit_hip."""

    def __init__(self, weight, *, bias=None, compact_groups=False, activation_scale=None):
        super().__init__()
        if not isinstance(weight, PackedWeight):
            raise ValueError('Requires a PackedWeight')
        if type(compact_groups) is not bool or (compact_groups and weight.shape[1] // weight.group_size > 32):
            raise ValueError('compact_groups requires bool and at most 32 groups')
        self._weight = weight
        self._compact_groups = compact_groups
        self._activation_scale = _activation_scale(weight, activation_scale, compact_groups)
        if bias is not None:
            if (not isinstance(bias, torch.Tensor) or bias.device.type != 'cpu' or tuple(bias.shape) != (weight.shape[0],)
                    or bias.dtype not in (torch.float16, torch.float32) or not torch.isfinite(bias).all()):
                raise ValueError('Bias preparation requires N finite CPU FP16/FP32 values')
            half = bias.detach().half()
            if not torch.isfinite(half).all():
                raise ValueError('Bias overflows FP16')
            self._bias = half.contiguous().numpy().tobytes()
        else:
            self._bias = None
        self._bias_device = {}

    @property
    def weight(self):
        return self._weight

    @property
    def bias(self):
        return self._bias

    @property
    def compact_groups(self):
        return self._compact_groups

    @property
    def activation_scale(self):
        return self._activation_scale

    @classmethod
    def from_float(cls, module, *, format='int4', group_size=None, compact_groups=False, activation_scale=None):
        if not isinstance(module, torch.nn.Linear) or module.weight.device.type != 'cpu':
            raise ValueError('Requires a CPU nn.Linear for preparation')
        return cls(quantize_weight(module.weight, format=format, group_size=group_size), bias=module.bias,
                   compact_groups=compact_groups, activation_scale=activation_scale)

    def _device_bias(self, device):
        if self._bias is None:
            return None
        key = str(device)
        if key not in self._bias_device:
            self._bias_device[key] = torch.frombuffer(bytearray(self._bias), dtype=torch.float16).to(device)
        return self._bias_device[key]

    def forward(self, x):
        """y = x . W^T (+ bias) in fp16 (reference :339-360).  compact_groups selects the per-group
        fp16 products and balanced add tree of the reference's compact graph (:235-256);
        activation_scale selects W8A8 (:224-231), int8 activations on that power-of-two grid."""
        n, k = self._weight.shape
        _validate_activation(x, k)
        codes, scales = self._weight.device_tensors(x.device)
        flags = lowbit_hip.FLAG_COMPACT_GROUPS if self._compact_groups else 0
        return lowbit_hip.linear(x, codes, scales, format=self._weight.format, N=n, K=k,
                                 group_size=self._weight.group_size, bias=self._device_bias(x.device),
                                 flags=flags, activation_scale=self._activation_scale)
