"""Immutable rank-r corrections of W8 quantization error (LQER-style).

Drop-in for the reference module of the same name (torch_npu_lowbit_correction.py):
LowRankCorrection keeps the fp16 factor layout -- down = V [rank, K], up = U [N, rank],
both row-major -- and fit_lowrank_correction the ridge-regularised fitting contract.
On the device the correction is applied inside lb_linear with the reference staging
z = fp16(x.V^T), d = fp16(z.U^T), y = fp16(y + d) (torch_npu_smollm.py:160-163).
"""
from dataclasses import dataclass
from math import prod

import numpy as np
import torch

from torch_npu_lowbit import MAX_TENSOR_ELEMENTS, PackedWeight


@dataclass(frozen=True)
class LowRankCorrection:
    """Correction factors (reference :15-39)."""
    shape: tuple
    rank: int
    down: bytes
    up: bytes

    def __post_init__(self):
        shape = self.shape
        if (type(shape) is not tuple or len(shape) != 2 or any(type(v) is not int or v <= 0 for v in shape)
                or prod(shape) > MAX_TENSOR_ELEMENTS or type(self.rank) is not int
                or not 1 <= self.rank <= min(shape)):
            raise ValueError('Correction requires bounded (N,K) and rank in 1..min(N,K)')
        for data, count in ((self.down, self.rank * shape[1]), (self.up, shape[0] * self.rank)):
            if (type(data) is not bytes or len(data) != 2 * count
                    or not np.isfinite(np.frombuffer(data, dtype=np.float16)).all()):
                raise ValueError('Correction factors require finite immutable FP16 data of the declared shape')

    def tensors(self, rank=None):
        """(down[:rank] fp16 [rank,K], up[:, :rank] fp16 [N,rank]) as fresh CPU tensors."""
        rank = self.rank if rank is None else rank
        if type(rank) is not int or not 1 <= rank <= self.rank:
            raise ValueError('Invalid correction rank')
        n, k = self.shape
        down = torch.from_numpy(np.frombuffer(self.down, dtype=np.float16).reshape(self.rank, k).copy())
        up = torch.from_numpy(np.frombuffer(self.up, dtype=np.float16).reshape(n, self.rank).copy())
        return down[:rank].contiguous(), up[:, :rank].contiguous()

    def truncated(self, rank):
        down, up = self.tensors(rank)
        return LowRankCorrection(self.shape, rank, down.numpy().tobytes(), up.numpy().tobytes())

    def device_tensors(self, device):
        """(down fp16 [rank,K], up fp16 [N,rank]) on `device`, uploaded once per device."""
        device = torch.device(device)
        cache = self.__dict__.setdefault('_device_cache', {})
        key = (device.type, device.index if device.index is not None else torch.cuda.current_device())
        if key not in cache:
            down, up = self.tensors()
            cache[key] = (down.to(device), up.to(device))
        return cache[key]


@torch.no_grad()
def fit_lowrank_correction(weight, packed, inputs, *, rank=32, device=None):
    """Fit E ~= U V for E = W - q*s, minimising ||E L||_F with L L^T = X^T X / m + ridge.

    Same contract as the reference (:42-69): per-row W8 only, fp64, 1% mean-diagonal ridge,
    SVD of E.L, balanced sqrt(sigma) split, factors stored in fp16.  The arguments are CPU
    tensors; `device` (e.g. 'cuda') runs the Cholesky / SVD there instead of on the CPU
    (singular vectors are defined up to sign, so U and V may both flip sign column-wise).
    """
    if (not isinstance(packed, PackedWeight) or packed.format != 'int8' or packed.group_size != packed.shape[1]
            or not isinstance(weight, torch.Tensor) or weight.device.type != 'cpu' or tuple(weight.shape) != packed.shape
            or weight.dtype not in (torch.float16, torch.float32) or not torch.isfinite(weight).all()
            or not isinstance(inputs, torch.Tensor) or inputs.device.type != 'cpu'
            or inputs.dtype not in (torch.float16, torch.float32) or inputs.ndim != 2
            or inputs.shape[1] != packed.shape[1] or not 1 <= inputs.shape[0] <= 4096
            or max(packed.shape) > 4096 or not torch.isfinite(inputs).all()
            or type(rank) is not int or not 1 <= rank <= min(packed.shape)):
        raise ValueError('Correction fitting requires finite matching CPU W8A16 weights/activations, '
                         'rows/K<=4096 and a valid rank')
    n, k = packed.shape
    dev = torch.device('cpu' if device is None else device)
    q = torch.from_numpy(np.frombuffer(packed.data, dtype=np.int8).reshape(n, k).astype(np.float64)).to(dev)
    s = torch.from_numpy(np.frombuffer(packed.scales, dtype=np.float16).astype(np.float64)).to(dev)
    error = weight.detach().to(dev, torch.float64) - q * s[:, None]
    x = inputs.detach().to(dev, torch.float64)
    covariance = x.T @ x / x.shape[0]
    covariance += 0.01 * covariance.diagonal().mean().clamp_min(1e-20) * torch.eye(k, dtype=torch.float64, device=dev)
    lower = torch.linalg.cholesky(covariance)
    left, sigma, right_h = torch.linalg.svd(error @ lower, full_matrices=False)
    root = sigma[:rank].sqrt()
    up = (left[:, :rank] * root).half().contiguous()
    # V = (L^-T right_h[:rank]^T)^T scaled by sqrt(sigma): undo the whitening on the input side.
    down = (torch.linalg.solve_triangular(lower.T, right_h[:rank].T, upper=True).T * root[:, None]).half().contiguous()
    return LowRankCorrection(packed.shape, rank, down.cpu().numpy().tobytes(), up.cpu().numpy().tobytes())
