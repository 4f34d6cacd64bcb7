"""Frozen SmolLM2-135M decoder layers on MI355X with low-bit projections.

Drop-in for the reference module of the same name (torch_npu_smollm.py): FrozenSmolLayer,
SmolKVCache and FrozenSmolStack keep their constructor arguments (config, weights, mode in
{fp16, w8a16, w4a16, nf4a16}, packed_weights, fp16_projections, corrections), their
forward / prefill / decode / reference_cpu methods and their fp16 staging (reference
:142-193).  The reference compiles each layer into one NPU graph; here every projection is
an lb_linear call of liblowbit_hip (W8 per-row, INT4/NF4 group-32, optional rank-r
correction) and the glue (RMSNorm, RoPE, attention, SiLU) is staged PyTorch-ROCm ops with
the same fp16 rounding points.

Deviations (the reference limits come from its NPU graph and are lifted):
  * rope_theta: any positive value from the config (the reference accepts only 1e5, :81);
  * capacity: KV slots per layer, default 64 as in the reference (:111-116), settable;
  * batch / sequence: B >= 1, S <= capacity (the reference caps B <= 8, S <= 64, :133-135).
KV snapshots keep the reference contract (decode never changes an earlier snapshot's
valid positions): snapshots of one sequence share storage and append in place; decoding
from a snapshot that is no longer the newest copies the storage first.
"""
from dataclasses import dataclass, replace
import json
from math import isfinite, prod
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

import lowbit_hip
from torch_npu_lowbit import PackedWeight, quantize_weight
from torch_npu_lowbit_correction import LowRankCorrection

_PROJECTIONS = frozenset(('self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight',
                          'self_attn.o_proj.weight', 'mlp.gate_proj.weight', 'mlp.up_proj.weight',
                          'mlp.down_proj.weight'))
_WEIGHT_FORMATS = {'fp16': None, 'w8a16': 'int8', 'w4a16': 'int4', 'nf4a16': 'nf4'}
_SHAPES = {'self_attn.q_proj.weight': (576, 576), 'self_attn.k_proj.weight': (192, 576),
           'self_attn.v_proj.weight': (192, 576), 'self_attn.o_proj.weight': (576, 576),
           'mlp.gate_proj.weight': (1536, 576), 'mlp.up_proj.weight': (1536, 576),
           'mlp.down_proj.weight': (576, 1536), 'input_layernorm.weight': (576,),
           'post_attention_layernorm.weight': (576,)}
_REQUIRED = dict(model_type='llama', hidden_size=576, intermediate_size=1536, num_attention_heads=9,
                 num_key_value_heads=3, hidden_act='silu', attention_bias=False, mlp_bias=False,
                 rms_norm_eps=1e-5, rope_scaling=None, pretraining_tp=1)
HEADS, KV_HEADS, HEAD_DIM, HIDDEN = 9, 3, 64, 576


def _projection_policy(mode, names):
    """Validated fp16-protected projection names (reference :31-37)."""
    if (type(names) is not tuple or any(type(name) is not str for name in names)
            or len(set(names)) != len(names) or not set(names) <= _PROJECTIONS):
        raise ValueError('fp16_projections requires a tuple of distinct SmolLM projection weight names')
    if names and (mode != 'w8a16' or len(names) == len(_PROJECTIONS)):
        raise ValueError('FP16 protection requires w8a16 with at least one INT8 projection; use mode=fp16 for all FP16')
    return frozenset(names)


def _half(tensor, shape):
    """fp16 copy of a finite CPU fp16/bf16/fp32 parameter of the expected shape."""
    if (not isinstance(tensor, torch.Tensor) or tensor.device.type != 'cpu' or tuple(tensor.shape) != shape
            or tensor.dtype not in (torch.float16, torch.bfloat16, torch.float32)
            or not torch.isfinite(tensor).all()):
        raise ValueError('Preparation requires finite CPU FP16/BF16/FP32 weights of the expected shape')
    value = tensor.detach().float().half().contiguous()
    if not torch.isfinite(value).all():
        raise ValueError('Parameter overflows FP16')
    return value


def _rope_tables(theta, positions):
    freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2).float() / HEAD_DIM))
    angles = torch.outer(torch.arange(positions).float(), freq)
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos().half(), angles.sin().half()


class _KVStorage:
    """Device K/V slots shared by the snapshots of one sequence; `high` is the written length."""

    def __init__(self, keys, values, high):
        self.keys, self.values, self.high = keys, values, high


@dataclass(frozen=True, eq=False)
class SmolKVCache:
    """KV snapshot (reference :547-556): keys/values [B,3,capacity,64] fp16; positions
    [0, length) are valid.  Tensor contents must not be edited by callers."""
    _owner: object
    _sequence: object
    keys: torch.Tensor
    values: torch.Tensor
    length: int
    _position: torch.Tensor
    _storage: object = None


class FrozenSmolLayer(torch.nn.Module):
    """One frozen SmolLM2-135M decoder layer (reference :66-544)."""

    def __init__(self, config, weights, *, mode='w8a16', packed_weights=None, fp16_projections=(), corrections=None,
                 capacity=64):
        super().__init__()
        if mode not in _WEIGHT_FORMATS:
            raise ValueError('Requires fp16, w8a16, w4a16 or nf4a16')
        fmt = _WEIGHT_FORMATS[mode]
        self._fp16_projections = _projection_policy(mode, fp16_projections)
        theta = config.get('rope_theta') if isinstance(config, dict) else None
        if (not isinstance(config, dict) or any(config.get(k) != v for k, v in _REQUIRED.items())
                or config.get('rope_interleaved', False) or type(theta) not in (int, float)
                or not isfinite(theta) or theta <= 0):
            raise ValueError('Requires the SmolLM2-135M configuration (positive rope_theta)')
        if type(capacity) is not int or not 1 <= capacity <= 1 << 20:
            raise ValueError('capacity must be a positive int')
        if corrections is not None and (
                type(corrections) is not dict or mode != 'w8a16' or packed_weights is None
                or not set(corrections) <= _PROJECTIONS or set(corrections) & self._fp16_projections
                or any(not isinstance(c, LowRankCorrection) or c.shape != _SHAPES[name] or c.rank > 32
                       for name, c in corrections.items())):
            raise ValueError('Corrections require matching rank<=32 factors, explicit packed W8 weights, '
                             'and unprotected projections')
        if not isinstance(weights, dict) or set(weights) != set(_SHAPES):
            raise ValueError('Unexpected layer weight names')
        if packed_weights is not None:
            if (fmt is None or type(packed_weights) is not dict
                    or set(packed_weights) != {n for n, s in _SHAPES.items() if len(s) == 2}):
                raise ValueError('Prepared weights require all seven projections in a matching lowbit mode')
            for name, q in packed_weights.items():
                if (not isinstance(q, PackedWeight) or q.shape != _SHAPES[name] or q.format != fmt
                        or (fmt == 'int8' and q.group_size != _SHAPES[name][1])):
                    raise ValueError('Prepared weights require matching formats/shapes; W8 uses per-row scales')
        self._mode = mode
        self._theta = float(theta)
        self._capacity = capacity
        self._corrections = {} if corrections is None else dict(corrections)
        self._weights = {name: _half(weights[name], shape) for name, shape in _SHAPES.items()}
        self._packed = {}
        if fmt is not None:
            for name, shape in _SHAPES.items():
                if len(shape) == 2:
                    # The reference quantizes the fp16-rounded weight with group 32 for 4-bit (:109-110).
                    self._packed[name] = (quantize_weight(self._weights[name], format=fmt,
                                                          group_size=None if fmt == 'int8' else 32)
                                          if packed_weights is None else packed_weights[name])
        self._cos, self._sin = _rope_tables(self._theta, capacity)
        self._cache_owner = object()
        self._device = {}
        self.eval()

    @classmethod
    def from_checkpoint(cls, directory, *, layer_index=0, mode='w8a16', packed_weights=None, fp16_projections=(),
                        corrections=None, capacity=64):
        from safetensors import safe_open
        _projection_policy(mode, fp16_projections)
        directory = Path(directory)
        config = json.loads((directory / 'config.json').read_text())
        if type(layer_index) is not int or not 0 <= layer_index < config.get('num_hidden_layers', 0):
            raise ValueError('Invalid layer index')
        prefix = f'model.layers.{layer_index}.'
        with safe_open(directory / 'model.safetensors', framework='pt', device='cpu') as file:
            weights = {n[len(prefix):]: file.get_tensor(n) for n in file.keys() if n.startswith(prefix)}
        return cls(config, weights, mode=mode, packed_weights=packed_weights, fp16_projections=fp16_projections,
                   corrections=corrections, capacity=capacity)

    @property
    def mode(self):
        return self._mode

    @property
    def fp16_projections(self):
        return self._fp16_projections

    @property
    def capacity(self):
        return self._capacity

    def _shape(self, shape, limit=None):
        limit = self._capacity if limit is None else limit
        if (len(shape) != 3 or any(type(v) is not int or v <= 0 for v in shape) or shape[2] != HIDDEN
                or shape[1] > limit):
            raise ValueError(f'Requires FP16 (B,S,576) with S <= {limit}')
        return tuple(shape)

    # ------------------------------------------------------------------ CPU reference
    def _cpu_linear(self, v, name, quantized):
        if quantized and self._mode != 'fp16' and name not in self._fp16_projections:
            q = self._packed[name]
            if q.format == 'int8':
                codes = np.frombuffer(q.data, dtype=np.int8).reshape(q.shape).astype(np.float64)
                scales = np.frombuffer(q.scales, dtype=np.float16).astype(np.float64)
                value = (v.double() @ torch.from_numpy(codes * scales[:, None]).T).half()
            else:
                value = F.linear(v.float(), torch.from_numpy(q.dequantize().copy()).float()).half()
            if name in self._corrections:
                down, up = self._corrections[name].tensors()
                delta = F.linear(F.linear(v.float(), down.float()).half().float(), up.float()).half()
                value = (value + delta).half()
            return value
        return F.linear(v.float(), self._weights[name].float()).half()

    def _cpu_norm(self, v, name):
        f = v.float()
        normalized = (f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half()
        return (normalized * self._weights[name]).half()

    def reference_cpu(self, x, *, quantized=True, segment=None, normalized=None):
        """Explicit staged CPU reference (reference :142-193); never called by forward."""
        if (not isinstance(x, torch.Tensor) or x.device.type != 'cpu' or x.dtype not in (torch.float16, torch.float32)
                or not torch.isfinite(x).all()):
            raise ValueError('Reference requires finite CPU FP16/FP32 input')
        b, s, d = self._shape(tuple(x.shape))
        x = x.detach().half()
        if not torch.isfinite(x).all():
            raise ValueError('Reference input overflows FP16')
        if segment not in (None, 'attention', 'ffn') or (segment is not None and (
                not isinstance(normalized, torch.Tensor) or normalized.device.type != 'cpu'
                or normalized.dtype != torch.float16 or normalized.shape != x.shape)):
            raise ValueError('CPU segment requires matching FP16 normalization')
        trace = {}
        supplied = normalized
        n1 = supplied if segment == 'attention' else self._cpu_norm(x, 'input_layernorm.weight')
        trace['norm1'] = n1
        q = self._cpu_linear(n1, 'self_attn.q_proj.weight', quantized).view(b, s, HEADS, HEAD_DIM).transpose(1, 2)
        k = self._cpu_linear(n1, 'self_attn.k_proj.weight', quantized).view(b, s, KV_HEADS, HEAD_DIM).transpose(1, 2)
        v = self._cpu_linear(n1, 'self_attn.v_proj.weight', quantized).view(b, s, KV_HEADS, HEAD_DIM).transpose(1, 2)
        cos, sin = self._cos[:s][None, None], self._sin[:s][None, None]

        def rotate(t):
            return (t * cos + torch.cat((-t[..., 32:], t[..., :32]), -1) * sin).half()

        q, k = rotate(q), rotate(k)
        trace['keys'], trace['values'] = k, v
        k, v = k.repeat_interleave(3, dim=1), v.repeat_interleave(3, dim=1)
        scores = (q.float() @ k.float().transpose(-1, -2)).half()
        scores = (scores * 0.125).half()
        mask = torch.triu(torch.full((s, s), float('-inf')), diagonal=1)
        probs = (scores + mask).float().softmax(-1).half()
        attended = (probs.float() @ v.float()).half().transpose(1, 2).reshape(b, s, d)
        trace['attention'] = attended
        delta = self._cpu_linear(attended, 'self_attn.o_proj.weight', quantized)
        trace['attention_output'] = delta
        value = (x + delta).half()
        trace['residual1'] = value
        if segment == 'attention':
            return value, trace
        if segment == 'ffn':
            value = x
        n2 = supplied if segment == 'ffn' else self._cpu_norm(value, 'post_attention_layernorm.weight')
        trace['norm2'] = n2
        gate = self._cpu_linear(n2, 'mlp.gate_proj.weight', quantized)
        up = self._cpu_linear(n2, 'mlp.up_proj.weight', quantized)
        activated = F.silu(gate.float()).half()
        trace['silu'] = activated
        hidden = (activated * up).half()
        trace['gated'] = hidden
        delta = self._cpu_linear(hidden, 'mlp.down_proj.weight', quantized)
        trace['ffn_output'] = delta
        value = (value + delta).half()
        trace['output'] = value
        return value, trace

    # ------------------------------------------------------------------ device path
    def _dev(self, device):
        """Device copies of weights, packed codes, factors and RoPE tables (built once per device)."""
        key = str(device)
        if key not in self._device:
            state = {'norm1': self._weights['input_layernorm.weight'].to(device),
                     'norm2': self._weights['post_attention_layernorm.weight'].to(device),
                     'cos': self._cos.to(device), 'sin': self._sin.to(device), 'lin': {}}
            for name in sorted(_PROJECTIONS):
                n, k = _SHAPES[name]
                if self._mode != 'fp16' and name not in self._fp16_projections:
                    q = self._packed[name]
                    codes, scales = q.device_tensors(device)
                    entry = dict(codes=codes, scales=scales, format=q.format, group=q.group_size, N=n, K=k)
                    if name in self._corrections:
                        down, up = self._corrections[name].device_tensors(device)
                        entry.update(down=down, up=up, rank=self._corrections[name].rank)
                else:
                    entry = dict(codes=self._weights[name].to(device), scales=None, format='fp16', group=k, N=n, K=k)
                state['lin'][name] = entry
            self._device[key] = state
        return self._device[key]

    @staticmethod
    def _linear(state, x2d, name, out=None):
        e = state['lin'][name]
        return lowbit_hip.linear(x2d, e['codes'], e['scales'], format=e['format'], N=e['N'], K=e['K'],
                                 group_size=e['group'], down=e.get('down'), up=e.get('up'), rank=e.get('rank', 0),
                                 out=out)

    @staticmethod
    def _norm(x, gamma):
        f = x.float()
        return ((f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half() * gamma).half()

    @staticmethod
    def _rotate(t, cos, sin):
        return (t * cos + torch.cat((-t[..., 32:], t[..., :32]), -1) * sin).half()

    @staticmethod
    def _attend(q, k, v, mask):
        k = k.repeat_interleave(3, dim=1)
        v = v.repeat_interleave(3, dim=1)
        scores = (q.float() @ k.float().transpose(-1, -2)).half()
        scores = (scores * 0.125).half()
        probs = (scores + mask).float().softmax(-1).half()
        return (probs.float() @ v.float()).half()

    def _validate_input(self, x):
        if self.training:
            raise ValueError('FrozenSmolLayer requires eval; training is unsupported')
        if not isinstance(x, torch.Tensor) or x.device.type != 'cuda':
            raise ValueError('FrozenSmolLayer requires a ROCm device tensor')
        if x.requires_grad and torch.is_grad_enabled():
            raise ValueError('FrozenSmolLayer is inference-only; use no_grad/inference_mode')
        if x.dtype != torch.float16:
            raise ValueError('FrozenSmolLayer requires FP16 device input')
        return self._shape(tuple(x.shape))

    def _mlp(self, state, value):
        b, s, d = value.shape
        n2 = self._norm(value, state['norm2']).view(b * s, d)
        gate = self._linear(state, n2, 'mlp.gate_proj.weight')
        up = self._linear(state, n2, 'mlp.up_proj.weight')
        hidden = (F.silu(gate.float()).half() * up).half()
        delta = self._linear(state, hidden, 'mlp.down_proj.weight').view(b, s, d)
        return (value + delta).half()

    def _full(self, x):
        """Causal full-sequence layer on device; returns (out, keys [B,3,S,64], values)."""
        state = self._dev(x.device)
        b, s, d = x.shape
        n1 = self._norm(x, state['norm1']).view(b * s, d)
        q = self._linear(state, n1, 'self_attn.q_proj.weight').view(b, s, HEADS, HEAD_DIM).transpose(1, 2)
        k = self._linear(state, n1, 'self_attn.k_proj.weight').view(b, s, KV_HEADS, HEAD_DIM).transpose(1, 2)
        v = self._linear(state, n1, 'self_attn.v_proj.weight').view(b, s, KV_HEADS, HEAD_DIM).transpose(1, 2)
        cos, sin = state['cos'][:s][None, None], state['sin'][:s][None, None]
        q, k = self._rotate(q, cos, sin), self._rotate(k, cos, sin)
        mask = torch.triu(torch.full((s, s), float('-inf'), device=x.device), diagonal=1)
        att = self._attend(q, k, v, mask).transpose(1, 2).reshape(b * s, d)
        delta = self._linear(state, att, 'self_attn.o_proj.weight').view(b, s, d)
        value = (x + delta).half()
        return self._mlp(state, value), k, v

    def forward(self, x):
        self._validate_input(x)
        return self._full(x)[0]

    def prefill(self, x):
        """Full prefix; returns the output and a KV snapshot (reference :506-523)."""
        b, s, _ = self._validate_input(x)
        out, k, v = self._full(x)
        keys = torch.zeros((b, KV_HEADS, self._capacity, HEAD_DIM), dtype=torch.float16, device=x.device)
        values = torch.zeros_like(keys)
        keys[:, :, :s] = k
        values[:, :, :s] = v
        storage = _KVStorage(keys, values, s)
        position = torch.tensor([s], dtype=torch.int32, device=x.device)
        return out, SmolKVCache(self._cache_owner, object(), keys, values, s, position, storage)

    def _validate_cache(self, x, cache):
        if x.shape[1] != 1 or type(cache) is not SmolKVCache or cache._owner is not self._cache_owner:
            raise ValueError("Decode requires one token and this layer's own KV cache")
        if type(cache.length) is not int or not 1 <= cache.length < self._capacity:
            raise ValueError(f'KV cache is full or has an invalid length; total tokens must be <= {self._capacity}')
        if (tuple(cache.keys.shape) != (x.shape[0], KV_HEADS, self._capacity, HEAD_DIM)
                or cache.keys.dtype != torch.float16 or cache.keys.device != x.device):
            raise ValueError('KV cache has the wrong batch, layout or device')

    def decode(self, x, cache):
        """Append exactly one token; earlier snapshots keep their valid positions (reference :529-544)."""
        self._validate_input(x)
        self._validate_cache(x, cache)
        state = self._dev(x.device)
        storage = cache._storage
        if storage.high != cache.length:  # decoding from an older snapshot: copy on write
            storage = _KVStorage(cache.keys.clone(), cache.values.clone(), cache.length)
        p = cache.length
        b = x.shape[0]
        n1 = self._norm(x, state['norm1']).view(b, HIDDEN)
        q = self._linear(state, n1, 'self_attn.q_proj.weight').view(b, 1, HEADS, HEAD_DIM).transpose(1, 2)
        k = self._linear(state, n1, 'self_attn.k_proj.weight').view(b, 1, KV_HEADS, HEAD_DIM).transpose(1, 2)
        v = self._linear(state, n1, 'self_attn.v_proj.weight').view(b, 1, KV_HEADS, HEAD_DIM).transpose(1, 2)
        cos, sin = state['cos'][p:p + 1][None, None], state['sin'][p:p + 1][None, None]
        q, k = self._rotate(q, cos, sin), self._rotate(k, cos, sin)
        storage.keys[:, :, p:p + 1] = k
        storage.values[:, :, p:p + 1] = v
        storage.high = p + 1
        mask = torch.zeros((1, p + 1), device=x.device)
        att = self._attend(q, storage.keys[:, :, :p + 1], storage.values[:, :, :p + 1], mask)
        delta = self._linear(state, att.transpose(1, 2).reshape(b, HIDDEN), 'self_attn.o_proj.weight').view(b, 1, HIDDEN)
        value = (x + delta).half()
        out = self._mlp(state, value)
        position = torch.tensor([p + 1], dtype=torch.int32, device=x.device)
        return out, SmolKVCache(self._cache_owner, cache._sequence, storage.keys, storage.values, p + 1, position,
                                storage)


class FrozenSmolStack(torch.nn.Module):
    """Contiguous frozen decoder layers (reference :558-657)."""

    def __init__(self, directory, *, start_layer=0, num_layers=2, mode='w8a16', packed_weights=None,
                 fp16_projections=(), corrections=None, capacity=64):
        super().__init__()
        from safetensors import safe_open
        _projection_policy(mode, fp16_projections)
        directory = Path(directory)
        config = json.loads((directory / 'config.json').read_text())
        total = config.get('num_hidden_layers', 0)
        self._check_range(start_layer, num_layers, total, mode, packed_weights, corrections)
        layers = []
        with safe_open(directory / 'model.safetensors', framework='pt', device='cpu') as file:
            names = list(file.keys())
            for index in range(start_layer, start_layer + num_layers):
                prefix = f'model.layers.{index}.'
                weights = {n[len(prefix):]: file.get_tensor(n) for n in names if n.startswith(prefix)}
                layers.append(FrozenSmolLayer(
                    config, weights, mode=mode, fp16_projections=fp16_projections, capacity=capacity,
                    packed_weights=None if packed_weights is None else packed_weights[index],
                    corrections=None if corrections is None else corrections[index]))
        self._init_layers(layers, start_layer, mode, fp16_projections)

    @staticmethod
    def _check_range(start_layer, num_layers, total, mode, packed_weights, corrections):
        if (type(start_layer) is not int or type(num_layers) is not int or type(total) is not int
                or start_layer < 0 or num_layers <= 0 or start_layer + num_layers > total):
            raise ValueError('Requires a nonempty contiguous checkpoint layer range')
        if mode not in _WEIGHT_FORMATS:
            raise ValueError('Requires fp16, w8a16, w4a16 or nf4a16')
        indices = set(range(start_layer, start_layer + num_layers))
        if packed_weights is not None and (
                mode == 'fp16' or type(packed_weights) is not dict or any(type(i) is not int for i in packed_weights)
                or any(type(v) is not dict for v in packed_weights.values()) or set(packed_weights) != indices):
            raise ValueError('Prepared stack weights require a complete lowbit map indexed by checkpoint layer')
        if corrections is not None and (
                mode != 'w8a16' or packed_weights is None or type(corrections) is not dict
                or any(type(i) is not int or type(v) is not dict for i, v in corrections.items())
                or set(corrections) != indices):
            raise ValueError('Stack corrections require explicit W8 weights and a complete map indexed by checkpoint layer')

    def _init_layers(self, layers, start_layer, mode, fp16_projections):
        self.layers = torch.nn.ModuleList(layers)
        self.start_layer = start_layer
        self._mode = mode
        self._fp16_projections = _projection_policy(mode, fp16_projections)
        self.eval()

    @classmethod
    def from_checkpoint(cls, directory, **options):
        return cls(directory, **options)

    @classmethod
    def from_layers(cls, layers, *, start_layer=0):
        """Stack already-built FrozenSmolLayer objects (e.g. random-init weights without a checkpoint)."""
        if not layers or any(not isinstance(layer, FrozenSmolLayer) for layer in layers):
            raise ValueError('Requires a nonempty list of FrozenSmolLayer')
        if len({(layer.mode, layer.fp16_projections, layer.capacity) for layer in layers}) != 1:
            raise ValueError('Layers must share mode, protection policy and capacity')
        stack = cls.__new__(cls)
        torch.nn.Module.__init__(stack)
        stack._init_layers(list(layers), start_layer, layers[0].mode, tuple(sorted(layers[0].fp16_projections)))
        return stack

    @property
    def mode(self):
        return self._mode

    @property
    def num_layers(self):
        return len(self.layers)

    @property
    def fp16_projections(self):
        return self._fp16_projections

    def _check_eval(self):
        if self.training or any(layer.training for layer in self.layers):
            raise ValueError('FrozenSmolStack requires every layer in eval; training is unsupported')

    def reference_cpu(self, x, *, quantized=True):
        """Explicit staged CPU reference; never called by forward."""
        traces = []
        for layer in self.layers:
            x, trace = layer.reference_cpu(x, quantized=quantized)
            traces.append(trace)
        return x, traces

    def forward(self, x):
        self._check_eval()
        for layer in self.layers:
            x = layer(x)
        return x

    def prefill(self, x):
        self._check_eval()
        caches, sequence = [], object()
        for layer in self.layers:
            x, cache = layer.prefill(x)
            caches.append(replace(cache, _sequence=sequence))
        return x, tuple(caches)

    def decode(self, x, caches, *, group_size=None):
        """One token through every layer.  group_size (1, 2 or 4) is accepted for API
        compatibility; it grouped NPU graphs per fence in the reference (:628-657)."""
        if group_size is not None and (type(group_size) is not int or group_size not in (1, 2, 4)):
            raise ValueError('Decode group_size must be 1, 2 or 4')
        self._check_eval()
        if type(caches) is not tuple or len(caches) != self.num_layers:
            raise ValueError('Requires one KV cache per consecutive layer')
        if any(c.length != caches[0].length or c._sequence is not caches[0]._sequence for c in caches):
            raise ValueError('Stack KV caches must belong to the same snapshot and position')
        updated, sequence = [], object()
        for layer, cache in zip(self.layers, caches):
            x, cache = layer.decode(x, cache)
            updated.append(replace(cache, _sequence=sequence))
        return x, tuple(updated)


@torch.no_grad()
def generate_greedy(stack, io, ids, steps):
    """Greedy generation on the device: prefill `ids` (int64 [1, S]), then `steps` tokens.

    Same loop as the reference's hybrid generation harness (embed -> prefill -> decode per
    token -> tied logits -> argmax), with every stage on the device.  Returns
    (tokens list, fp16 logits [steps, vocab]) where logits[i] chose tokens[i].
    """
    device = io.embedding.device
    x = io.embed_tokens(ids.to(device))
    h, caches = stack.prefill(x)
    logits = io.logits(h[:, -1:])[0, 0]
    tokens, history = [], []
    for step in range(steps):
        tok = int(logits.float().argmax())
        tokens.append(tok)
        history.append(logits)
        if step == steps - 1:
            break
        h, caches = stack.decode(io.embed_tokens(torch.tensor([[tok]], device=device)), caches)
        logits = io.logits(h)[0, 0]
    return tokens, torch.stack(history)


class GraphDecoder:
    """Greedy decode of one sequence (B=1) as a replayable HIP graph.

    The per-token work of FrozenSmolStack.decode plus FrozenSmolIO.logits and the argmax is
    captured once; activations live in static buffers and the position is a device tensor,
    so generation needs no host synchronization.  Staging matches FrozenSmolLayer.decode
    (reference torch_npu_smollm.py:142-193).

    fused=True (default) issues five launches per layer from liblowbit_hip's decode-step
    entry points, the GPU counterpart of the reference's one-graph-per-layer decode
    (:195-340, chained per fence at :644-654):
      1. RMSNorm -> q | k | v projections (+ corrections)          lb_fused_linear
      2. RoPE, KV append at the position, GQA attention            lb_decode_attention
      3. o projection (+ correction) + residual                     lb_fused_linear
      4. RMSNorm -> gate | up projections (+ corrections)           lb_fused_linear
      5. SiLU(gate) * up -> down projection (+ correction) + residual  lb_fused_linear
    then RMSNorm -> tied fp16 lm_head and the greedy token with the next embedding, as one
    lb_head_next launch (head_next=True, the default, where it takes the head's format) or as
    lb_fused_linear + lb_argmax_next.  Projections of different formats (fp16-protected ones)
    get separate launches.  layer=True (default) runs those five steps of a layer as one
    lb_decode_layer launch whenever its seven projections share one format and group (the
    reference's one graph per layer); the fused launches remain for other layers.  stack=True
    (default) goes further when every layer has the same format, group and ranks: one
    lb_decode_stack launch runs all layers of the token (the reference's whole fenced chain of
    layer graphs, :644-654).  fused=False runs the same step as staged PyTorch-ROCm glue
    around one lb_linear per projection.  shared_z (default) gives every fused launch with
    corrections its own workspace, so each correction's z is computed once per launch.
    """

    def __init__(self, stack, io, *, fused=True, shared_z=True, layer=True, stack_kernel=True, head_next=True):
        self.device = io.embedding.device
        if self.device.type != 'cuda':
            raise ValueError('GraphDecoder needs FrozenSmolIO moved to a ROCm device')
        self.stack, self.io, self.fused, self.shared_z = stack, io, fused, shared_z
        self.use_head_next = head_next
        self.head_next = None
        dev = self.device
        cap = stack.layers[0].capacity
        self.capacity = cap
        z = lambda *shape, dtype=torch.float16: torch.zeros(shape, dtype=dtype, device=dev)
        self.pos = z(1, dtype=torch.int64)
        self.token = z(1, dtype=torch.int64)
        self.tokens = z(cap + 1, dtype=torch.int64)
        self.logits = z(1, io.vocab_size)
        self.keys = [z(1, KV_HEADS, cap, HEAD_DIM) for _ in stack.layers]
        self.values = [z(1, KV_HEADS, cap, HEAD_DIM) for _ in stack.layers]
        self.states = [layer._dev(dev) for layer in stack.layers]
        self.layer_kernel = fused and layer and all(self._layer_ready(st) for st in self.states)
        self.stack_kernel = self.layer_kernel and stack_kernel and self._stack_ready(self.states)
        if self.layer_kernel:
            self._build_layer(z)
        elif fused:
            self._build_fused(z)
        else:
            self._build_staged(z)
        self.graph = None
        self.graph_tokens = 1

    # ---------------------------------------------------------------- fused launches
    @staticmethod
    def _problem(entry, y, **extra):
        problem = dict(codes=entry['codes'], scales=entry['scales'], N=entry['N'], y=y, **extra)
        if entry.get('rank', 0):
            down, up = entry['down'], entry['up']
            rank = down.shape[0]
            if rank % 8:  # the fused kernel reads U rows in 8-wide pieces: pad columns with zeros
                padded = torch.zeros((up.shape[0], (rank + 7) // 8 * 8), dtype=up.dtype, device=up.device)
                padded[:, :rank] = up
                up = padded
            problem.update(down=down, up=up)
        return problem

    def _fused_group(self, lin, members, x, **options):
        """One lb_fused_linear per run of same-format projections in `members` [(name, y, extra)]."""
        import lowbit_hip as lb
        calls, run = [], []

        def flush():
            if run:
                first = lin[run[0][0]]
                calls.append(lb.PreparedFused(x, [self._problem(lin[name], y, **extra) for name, y, extra in run],
                                              format=first['format'], K=first['K'], group_size=first['group'],
                                              shared_z=self.shared_z, **options))
                run.clear()

        for member in members:
            e = lin[member[0]]
            if run and (lin[run[0][0]]['format'], lin[run[0][0]]['group']) != (e['format'], e['group']):
                flush()
            run.append(member)
        flush()
        return calls

    def _build_fused(self, z):
        import lowbit_hip as lb
        io = self.io
        self.h = z(HIDDEN)
        self.qkv = z(HIDDEN + 2 * KV_HEADS * HEAD_DIM)
        self.att = z(HIDDEN)
        self.gu = z(2 * 1536)
        q, k, v = self.qkv[:HIDDEN], self.qkv[HIDDEN:HIDDEN + 192], self.qkv[HIDDEN + 192:]
        gate, up = self.gu[:1536], self.gu[1536:]
        self.calls = []
        for state, keys, values in zip(self.states, self.keys, self.values):
            lin = state['lin']
            seq = self._fused_group(lin, [('self_attn.q_proj.weight', q, {}), ('self_attn.k_proj.weight', k, {}),
                                          ('self_attn.v_proj.weight', v, {})],
                                    self.h, prologue='rmsnorm', gamma=state['norm1'], eps=1e-5)
            seq.append(lb.PreparedAttention(q, k, v, state['cos'], state['sin'], self.pos, keys, values, self.att,
                                            heads=HEADS, kv_heads=KV_HEADS, scale=0.125))
            seq += self._fused_group(lin, [('self_attn.o_proj.weight', self.h, dict(residual=self.h))], self.att)
            seq += self._fused_group(lin, [('mlp.gate_proj.weight', gate, {}), ('mlp.up_proj.weight', up, {})],
                                     self.h, prologue='rmsnorm', gamma=state['norm2'], eps=1e-5)
            seq += self._fused_group(lin, [('mlp.down_proj.weight', self.h, dict(residual=self.h))], gate,
                                     prologue='silu_mul', x2=up)
            self.calls.append(seq)
        self._build_head(io)

    def _build_head(self, io):
        """Final RMSNorm -> tied lm_head and the greedy token with the next embedding: one
        lb_head_next launch where it takes the head (fp16, int4), else one fused launch for the head
        and lb_argmax_next."""
        import lowbit_hip as lb
        if io.head is None:
            head, head_format, head_group = dict(codes=io.embedding, scales=None), 'fp16', HIDDEN
        else:
            codes, scales = io.head_tensors(self.device)
            head, head_format, head_group = dict(codes=codes, scales=scales), io.head.format, io.head.group_size
        problem = dict(head, N=io.vocab_size, y=self.logits)
        self.head = lb.PreparedFused(self.h, [problem], format=head_format, K=HIDDEN, group_size=head_group,
                                     prologue='rmsnorm', gamma=io.norm, eps=1e-5)
        self.argmax = lb.PreparedArgmax(self.logits, io.embedding, self.h, self.tokens, self.token, self.pos,
                                        limit=self.capacity)
        if self.use_head_next and head_format in lb.PreparedHeadNext.FORMATS:
            self.head_next = lb.PreparedHeadNext(self.h, problem, io.embedding, self.tokens, self.token, self.pos,
                                                 format=head_format, K=HIDDEN, group_size=head_group, gamma=io.norm,
                                                 eps=1e-5, limit=self.capacity)

    # ---------------------------------------------------------------- one launch per layer
    _ORDER = ('self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight',
              'self_attn.o_proj.weight', 'mlp.gate_proj.weight', 'mlp.up_proj.weight', 'mlp.down_proj.weight')

    @classmethod
    def _layer_ready(cls, state):
        """One format for all seven projections, groups lb_decode_layer takes (int8 per row, or one
        power-of-two group), so the layer can run as one lb_decode_layer launch."""
        entries = [state['lin'][name] for name in cls._ORDER]
        fmt = entries[0]['format']
        if any(e['format'] != fmt for e in entries):
            return False
        if fmt == 'fp16':
            return True
        groups = {e['group'] if e['group'] != e['K'] else 0 for e in entries}
        if len(groups) != 1:
            return False
        group = groups.pop()
        return (group == 0 and fmt == 'int8') or (group >= 32 and group & (group - 1) == 0)

    @classmethod
    def _layer_key(cls, state):
        """(format, group, ranks) of a layer: the launch shape lb_decode_stack needs shared."""
        entries = [state['lin'][name] for name in cls._ORDER]
        fmt = entries[0]['format']
        group = 0 if fmt == 'fp16' or entries[0]['group'] == entries[0]['K'] else entries[0]['group']
        return fmt, group, tuple(e.get('rank', 0) for e in entries)

    @classmethod
    def _stack_ready(cls, states):
        import lowbit_hip as lb
        return (len(states) <= lb.STACK_MAX_LAYERS and len({cls._layer_key(st) for st in states}) == 1
                and all(torch.equal(st['cos'], states[0]['cos']) and torch.equal(st['sin'], states[0]['sin'])
                        for st in states))

    @classmethod
    def _projections(cls, state):
        projections = []
        for name in cls._ORDER:
            e = state['lin'][name]
            pr = dict(codes=e['codes'], scales=e['scales'], N=e['N'])
            if e.get('rank', 0):
                pr.update(down=e['down'], up=e['up'])
            projections.append(pr)
        return projections

    def _build_layer(self, z):
        """Every layer in one lb_decode_stack launch (or each layer as one lb_decode_layer launch),
        then the fused head and the argmax."""
        import lowbit_hip as lb
        io = self.io
        self.h = z(HIDDEN)
        self.calls = []
        if self.stack_kernel:
            fmt, group, _ = self._layer_key(self.states[0])
            layers = [dict(norm1=st['norm1'], norm2=st['norm2'], keys=k, values=v, projections=self._projections(st))
                      for st, k, v in zip(self.states, self.keys, self.values)]
            self.calls.append([lb.PreparedStack(self.h, layers, format=fmt, group_size=group, hidden=HIDDEN,
                                                intermediate=1536, eps=1e-5, heads=HEADS, kv_heads=KV_HEADS,
                                                cos=self.states[0]['cos'], sin=self.states[0]['sin'],
                                                position=self.pos, scale=0.125)])
            self._build_head(io)
            return
        for state, keys, values in zip(self.states, self.keys, self.values):
            fmt, group, _ = self._layer_key(state)
            projections = self._projections(state)
            self.calls.append([lb.PreparedLayer(self.h, projections, format=fmt, group_size=group, hidden=HIDDEN,
                                                intermediate=1536, norm1=state['norm1'], norm2=state['norm2'],
                                                eps=1e-5, heads=HEADS, kv_heads=KV_HEADS, cos=state['cos'],
                                                sin=state['sin'], position=self.pos, keys=keys, values=values,
                                                scale=0.125)])
        self._build_head(io)

    def _waiting_calls(self):
        """The calls that hand data between workgroups through a workspace (bounded waits)."""
        import lowbit_hip as lb
        for seq in self.calls:
            for call in (seq.values() if isinstance(seq, dict) else seq):
                if isinstance(call, lb._Prepared) and call.workspace is not None:
                    yield call

    def timeouts(self):
        """Timed-out waits recorded by the launches since construction (0 when healthy)."""
        return sum(call.counters()[1] for call in self._waiting_calls())

    def check(self):
        """Synchronise, then raise RuntimeError if a bounded hand-over wait of any launch gave up
        (its outputs, and so the tokens, are not valid); the library is then failed and refuses
        every later call, as the reference's failed context (backend.cpp:280-292)."""
        for call in self._waiting_calls():
            call.check()

    # ---------------------------------------------------------------- staged launches
    def _build_staged(self, z):
        import lowbit_hip as lb
        io = self.io
        cap = self.capacity
        self.h = z(1, HIDDEN)
        self.n1, self.att, self.o, self.n2, self.down = (z(1, HIDDEN) for _ in range(5))
        self.q, self.k, self.v = z(1, 576), z(1, 192), z(1, 192)
        self.gate, self.up, self.hidden = z(1, 1536), z(1, 1536), z(1, 1536)
        self.normed = z(1, HIDDEN)
        self.slots = torch.arange(cap, device=self.device)
        plan = (('self_attn.q_proj.weight', 'n1', 'q'), ('self_attn.k_proj.weight', 'n1', 'k'),
                ('self_attn.v_proj.weight', 'n1', 'v'), ('self_attn.o_proj.weight', 'att', 'o'),
                ('mlp.gate_proj.weight', 'n2', 'gate'), ('mlp.up_proj.weight', 'n2', 'up'),
                ('mlp.down_proj.weight', 'hidden', 'down'))
        self.calls = []
        for state in self.states:
            calls = {}
            for name, src, dst in plan:
                e = state['lin'][name]
                calls[name] = lb.PreparedLinear(getattr(self, src), e['codes'], e['scales'], format=e['format'],
                                                N=e['N'], K=e['K'], group_size=e['group'], out=getattr(self, dst),
                                                down=e.get('down'), up=e.get('up'), rank=e.get('rank', 0))
            self.calls.append(calls)
        if io.head is None:
            self.head = lb.PreparedLinear(self.normed, io.embedding, None, format='fp16', N=io.vocab_size, K=HIDDEN,
                                          group_size=HIDDEN, out=self.logits)
        else:
            codes, scales = io.head_tensors(self.device)
            self.head = lb.PreparedLinear(self.normed, codes, scales, format=io.head.format, N=io.vocab_size,
                                          K=HIDDEN, group_size=io.head.group_size, out=self.logits)

    @staticmethod
    def _norm_into(out, x, gamma):
        f = x.float()
        torch.mul((f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half(), gamma, out=out)

    def _step_staged(self):
        torch.index_select(self.io.embedding, 0, self.token, out=self.h)
        mask = torch.where(self.slots > self.pos, float('-inf'), 0.0)
        for layer_index, (state, calls) in enumerate(zip(self.states, self.calls)):
            self._norm_into(self.n1, self.h, state['norm1'])
            calls['self_attn.q_proj.weight'].run()
            calls['self_attn.k_proj.weight'].run()
            calls['self_attn.v_proj.weight'].run()
            cos = state['cos'].index_select(0, self.pos)[None]
            sin = state['sin'].index_select(0, self.pos)[None]
            q = FrozenSmolLayer._rotate(self.q.view(1, HEADS, 1, HEAD_DIM), cos, sin)
            k = FrozenSmolLayer._rotate(self.k.view(1, KV_HEADS, 1, HEAD_DIM), cos, sin)
            keys, values = self.keys[layer_index], self.values[layer_index]
            keys.index_copy_(2, self.pos, k)
            values.index_copy_(2, self.pos, self.v.view(1, KV_HEADS, 1, HEAD_DIM))
            att = FrozenSmolLayer._attend(q, keys, values, mask)
            self.att.copy_(att.view(1, HIDDEN))
            calls['self_attn.o_proj.weight'].run()
            torch.add(self.h, self.o, out=self.h)
            self._norm_into(self.n2, self.h, state['norm2'])
            calls['mlp.gate_proj.weight'].run()
            calls['mlp.up_proj.weight'].run()
            torch.mul(F.silu(self.gate.float()).half(), self.up, out=self.hidden)
            calls['mlp.down_proj.weight'].run()
            torch.add(self.h, self.down, out=self.h)
        f = self.h.float()
        torch.mul((f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half(), self.io.norm, out=self.normed)
        self.head.run()
        nxt = self.logits.float().argmax(-1)
        self.tokens.index_copy_(0, self.pos, nxt)
        self.token.copy_(nxt)
        self.pos.add_(1)

    # ---------------------------------------------------------------- common
    def load(self, caches, next_token):
        """Start from a prefill snapshot: copy its K/V, set the position and the next input token."""
        length = caches[0].length
        if not 1 <= length < self.capacity:
            raise ValueError('the snapshot leaves no free KV slot')
        for dst_k, dst_v, cache in zip(self.keys, self.values, caches):
            dst_k[:, :, :length].copy_(cache.keys[:, :, :length])
            dst_v[:, :, :length].copy_(cache.values[:, :, :length])
        self.pos.fill_(length)
        self.token.fill_(int(next_token))
        self.h.view(1, HIDDEN).copy_(self.io.embedding[int(next_token)].view(1, HIDDEN))

    def step(self):
        """One greedy token (eager; this is what capture() records)."""
        if not self.fused:
            return self._step_staged()
        for seq in self.calls:
            for call in seq:
                call.run()
        if self.head_next is not None:
            self.head_next.run()
        else:
            self.head.run()
            self.argmax.run()

    def capture(self, tokens=1):
        """Record `tokens` consecutive step()s into one HIP graph (warm-up runs first on a side
        stream, as torch requires).  Every step reads its position from the device, so one replay
        generates `tokens` tokens; more than one shares a graph launch between them."""
        if type(tokens) is not int or tokens < 1:
            raise ValueError('tokens must be a positive int')
        start = int(self.pos.item())
        if start + tokens > self.capacity:
            raise ValueError(f'capturing {tokens} steps from position {start} exceeds the KV capacity')
        saved = [t.clone() for t in [self.pos, self.token, self.h] + self.keys + self.values]
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(tokens):
                self.step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for _ in range(tokens):
                self.step()
        self.graph_tokens = tokens
        for dst, src in zip([self.pos, self.token, self.h] + self.keys + self.values, saved):
            dst.copy_(src)  # the warm-up advanced the state; restore it
        return self.graph

    def generate(self, steps):
        """Replay `steps` tokens; returns the generated token ids (one host sync at the end)."""
        if self.graph is None:
            self.capture()
        if steps % self.graph_tokens:
            raise ValueError(f'steps must be a multiple of the {self.graph_tokens} tokens per captured graph')
        start = int(self.pos.item())
        if start + steps > self.capacity:
            raise ValueError(f'{steps} steps from position {start} exceed the KV capacity {self.capacity}')
        for _ in range(steps // self.graph_tokens):
            self.graph.replay()
        lowbit_hip.synchronize(self.device)  # a device fault of the replays marks the library failed here
        self.check()  # and so does a hand-over wait that gave up
        return self.tokens[start:start + steps].tolist()
