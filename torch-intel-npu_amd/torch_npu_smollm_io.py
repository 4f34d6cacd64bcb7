"""Tied embedding and final RMSNorm + lm_head of SmolLM (reference torch_npu_smollm_io.py).

Same constructor, buffers (`embedding`, `norm`, fp16) and methods (embed_tokens, logits) as
the reference FrozenSmolIO.  The reference runs both endpoints on the CPU only
(:39-43); here the module may be moved to a ROCm device, where the tied lm_head runs as an
fp16 GEMV/GEMM of liblowbit_hip with the same staging: fp32 RMS, fp16 normalize, fp16
gamma, fp32-accumulated product rounded to fp16 (:57-61).  On the CPU the reference
computation is used unchanged.

head_format ('int8' per-row, 'int4' or 'nf4' with head_group_size) quantizes the tied head with
quantize_weight (the embedding lookup stays fp16): the logits are then the low-bit linear of the
normalized rows with the SmolLM projection semantics (reference torch_npu_smollm.py:150-157: W8
with the exact q*s, 4-bit with fp16(q*s)), on the device through lb_linear, on the CPU as that
reference CPU computation.  The reference keeps its head fp16 on the CPU; this option has no
counterpart there.
"""
import json
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

import lowbit_hip
from torch_npu_lowbit import quantize_weight


class FrozenSmolIO(torch.nn.Module):
    """Inference-only embedding and norm/output head for the frozen decoder."""

    def __init__(self, config, embedding, norm, *, head_format=None, head_group_size=None):
        super().__init__()
        if (config.get('model_type') != 'llama' or config.get('hidden_size') != 576
                or config.get('tie_word_embeddings') is not True or config.get('rms_norm_eps') != 1e-5
                or type(config.get('vocab_size')) is not int or config['vocab_size'] <= 0):
            raise ValueError('Requires tied SmolLM endpoints with D576 and RMSNorm eps=1e-5')
        for name, value, shape in (('embedding', embedding, (config['vocab_size'], 576)), ('norm', norm, (576,))):
            if (not isinstance(value, torch.Tensor) or value.device.type != 'cpu' or tuple(value.shape) != shape
                    or value.dtype not in (torch.float16, torch.bfloat16, torch.float32)
                    or not torch.isfinite(value).all()):
                raise ValueError('Requires finite CPU floating endpoint weights of the expected shape')
            half = value.detach().to(dtype=torch.float16, copy=True, memory_format=torch.contiguous_format)
            if not torch.isfinite(half).all():
                raise ValueError('Endpoint weight overflows FP16')
            self.register_buffer(name, half)
        self.vocab_size = config['vocab_size']
        if head_format not in (None, 'int8', 'int4', 'nf4') or (head_format == 'int8' and head_group_size is not None):
            raise ValueError('head_format must be None (fp16), int8 (per-row) or int4/nf4 with a group size')
        self.head = None if head_format is None else quantize_weight(
            self.embedding, format=head_format, group_size=head_group_size)
        self.eval()

    @classmethod
    def from_checkpoint(cls, directory, **options):
        from safetensors import safe_open
        directory = Path(directory)
        config = json.loads((directory / 'config.json').read_text())
        with safe_open(directory / 'model.safetensors', framework='pt', device='cpu') as file:
            if 'lm_head.weight' in file.keys():
                raise ValueError('Requires the canonical tied checkpoint without a separate lm_head weight')
            return cls(config, file.get_tensor('model.embed_tokens.weight'), file.get_tensor('model.norm.weight'),
                       **options)

    def _check(self, device):
        if self.training:
            raise ValueError('FrozenSmolIO requires eval mode')
        if self.embedding.dtype != torch.float16 or self.norm.dtype != torch.float16:
            raise ValueError('FrozenSmolIO endpoints require FP16')
        if self.embedding.device != device or self.norm.device != device:
            raise ValueError('FrozenSmolIO buffers and inputs must be on the same device')

    def embed_tokens(self, ids):
        if (not isinstance(ids, torch.Tensor) or ids.device.type not in ('cpu', 'cuda') or ids.dtype != torch.int64
                or ids.ndim != 2 or any(size <= 0 for size in ids.shape)):
            raise ValueError('Embedding requires nonempty int64 (B,S) token IDs')
        self._check(ids.device)
        if ids.device.type == 'cpu':
            return F.embedding(ids, self.embedding)
        return self.embedding.index_select(0, ids.reshape(-1)).view(*ids.shape, 576)

    def normalize(self, hidden):
        """fp32 variance / inverse, then fp16 scaling: the checkpoint's RMSNorm rounding (:57-60)."""
        value = hidden.float()
        inverse = torch.rsqrt(value.square().mean(-1, keepdim=True) + 1e-5)
        return (value * inverse).half() * self.norm

    def logits(self, hidden):
        if (not isinstance(hidden, torch.Tensor) or hidden.device.type not in ('cpu', 'cuda')
                or hidden.dtype != torch.float16 or hidden.ndim != 3 or hidden.shape[-1] != 576
                or any(size <= 0 for size in hidden.shape)):
            raise ValueError('Output head requires nonempty FP16 (B,S,576) hidden states')
        self._check(hidden.device)
        normalized = self.normalize(hidden)
        b, s, _ = hidden.shape
        if self.head is not None:
            return self._quantized_logits(normalized.reshape(b * s, 576)).view(b, s, self.vocab_size)
        if hidden.device.type == 'cpu':
            return F.linear(normalized, self.embedding)
        y = lowbit_hip.linear(normalized.reshape(b * s, 576), self.embedding, None, format='fp16',
                              N=self.vocab_size, K=576, group_size=576)
        return y.view(b, s, self.vocab_size)

    def head_tensors(self, device):
        """(codes, scales) of the quantized head on `device` (uploaded once)."""
        return self.head.device_tensors(device)

    def _quantized_logits(self, rows):
        q = self.head
        if rows.device.type != 'cpu':
            codes, scales = q.device_tensors(rows.device)
            return lowbit_hip.linear(rows, codes, scales, format=q.format, N=self.vocab_size, K=576,
                                     group_size=q.group_size)
        if q.format == 'int8':
            codes = np.frombuffer(q.data, dtype=np.int8).reshape(q.shape).astype(np.float64)
            scales = np.frombuffer(q.scales, dtype=np.float16).astype(np.float64)
            return (rows.double() @ torch.from_numpy(codes * scales[:, None]).T).half()
        return F.linear(rows.float(), torch.from_numpy(q.dequantize().copy()).float()).half()
