"""On-disk form of prepared low-bit weights and corrections (safetensors).

The reference keeps PackedWeight / LowRankCorrection as in-memory bytes only: they are not
Parameters and not in state_dict (TORCH_NPU_README.md:448), and every run re-quantizes from the
checkpoint (torch_npu_smollm.py:566-595) and re-fits corrections (about 150 s for GPTQ W8 plus
rank-32 fitting of SmolLM2-135M).  This module stores the prepared objects once and loads them
back bit for bit:

    <name>.codes   uint8 [len(PackedWeight.data)]   the packed bytes, unchanged
    <name>.scales  float16 [N, K / group_size]      the fp16 scales
    <name>.down    float16 [rank, K]                LowRankCorrection.down (V)
    <name>.up      float16 [N, rank]                LowRankCorrection.up (U)

The header metadata holds, per name, a JSON record of shape / format / group_size (and rank),
plus "lowbit.version".  Loading rebuilds every object through its own constructor, so the
reference's validation (extents, odd-nibble padding, finite positive scales, finite factors)
applies to what is read.  safetensors executes nothing from the file.

Stack files name projections 'model.layers.<i>.<projection>' (the checkpoint's own names), so
load_stack returns the packed_weights / corrections maps FrozenSmolStack takes.
"""
import json
import re
from pathlib import Path

import numpy as np
import torch

from torch_npu_lowbit import PackedWeight
from torch_npu_lowbit_correction import LowRankCorrection

FORMAT_VERSION = '1'
_LAYER_NAME = re.compile(r'^model\.layers\.(\d+)\.(.+)$')


def _bytes_tensor(data, dtype, shape):
    return torch.from_numpy(np.frombuffer(data, dtype=dtype).reshape(shape).copy())


def save_prepared(path, weights, corrections=None, *, metadata=None):
    """Write {name: PackedWeight} and optional {name: LowRankCorrection} to a safetensors file."""
    from safetensors.torch import save_file
    corrections = {} if corrections is None else corrections
    if (type(weights) is not dict or type(corrections) is not dict
            or any(type(n) is not str or not isinstance(w, PackedWeight) for n, w in weights.items())
            or any(type(n) is not str or not isinstance(c, LowRankCorrection) for n, c in corrections.items())):
        raise ValueError('Requires {str: PackedWeight} and {str: LowRankCorrection} maps')
    tensors, header = {}, {'lowbit.version': FORMAT_VERSION}
    for name, w in weights.items():
        n, k = w.shape
        tensors[f'{name}.codes'] = _bytes_tensor(w.data, np.uint8, (len(w.data),))
        tensors[f'{name}.scales'] = _bytes_tensor(w.scales, np.float16, (n, k // w.group_size))
        header[f'lowbit.weight.{name}'] = json.dumps(dict(shape=list(w.shape), format=w.format,
                                                          group_size=w.group_size))
    for name, c in corrections.items():
        n, k = c.shape
        tensors[f'{name}.down'] = _bytes_tensor(c.down, np.float16, (c.rank, k))
        tensors[f'{name}.up'] = _bytes_tensor(c.up, np.float16, (n, c.rank))
        header[f'lowbit.correction.{name}'] = json.dumps(dict(shape=list(c.shape), rank=c.rank))
    for key, value in (metadata or {}).items():
        if type(key) is not str or type(value) is not str or key.startswith('lowbit.'):
            raise ValueError('metadata must map str to str outside the lowbit. namespace')
        header[key] = value
    save_file(tensors, str(path), metadata=header)


def load_prepared(path):
    """Read a file written by save_prepared -> (weights, corrections, metadata)."""
    from safetensors import safe_open
    weights, corrections = {}, {}
    with safe_open(str(path), framework='pt', device='cpu') as f:
        header = f.metadata() or {}
        if header.get('lowbit.version') != FORMAT_VERSION:
            raise ValueError(f'{path}: not a lowbit prepared-weight file of version {FORMAT_VERSION}')
        names = set(f.keys())
        for key, record in header.items():
            if key.startswith('lowbit.weight.'):
                name = key[len('lowbit.weight.'):]
                meta = json.loads(record)
                if not {f'{name}.codes', f'{name}.scales'} <= names:
                    raise ValueError(f'{path}: tensors of {name} are missing')
                codes = f.get_tensor(f'{name}.codes')
                scales = f.get_tensor(f'{name}.scales')
                if codes.dtype != torch.uint8 or scales.dtype != torch.float16:
                    raise ValueError(f'{path}: {name} has unexpected tensor types')
                weights[name] = PackedWeight(tuple(int(v) for v in meta['shape']), meta['format'],
                                             int(meta['group_size']), codes.numpy().tobytes(),
                                             scales.contiguous().numpy().tobytes())
            elif key.startswith('lowbit.correction.'):
                name = key[len('lowbit.correction.'):]
                meta = json.loads(record)
                if not {f'{name}.down', f'{name}.up'} <= names:
                    raise ValueError(f'{path}: factors of {name} are missing')
                down, up = f.get_tensor(f'{name}.down'), f.get_tensor(f'{name}.up')
                if down.dtype != torch.float16 or up.dtype != torch.float16:
                    raise ValueError(f'{path}: {name} factors must be float16')
                corrections[name] = LowRankCorrection(tuple(int(v) for v in meta['shape']), int(meta['rank']),
                                                      down.contiguous().numpy().tobytes(),
                                                      up.contiguous().numpy().tobytes())
    metadata = {k: v for k, v in header.items() if not k.startswith('lowbit.')}
    return weights, corrections, metadata


def save_stack(path, stack, *, metadata=None):
    """Store every layer's packed projections and corrections of a low-bit FrozenSmolStack."""
    weights, corrections = {}, {}
    for offset, layer in enumerate(stack.layers):
        prefix = f'model.layers.{stack.start_layer + offset}.'
        if not layer._packed:
            raise ValueError('the fp16 mode has no prepared low-bit weights to store')
        weights.update({prefix + name: w for name, w in layer._packed.items()})
        corrections.update({prefix + name: c for name, c in layer._corrections.items()})
    save_prepared(path, weights, corrections, metadata=metadata)


def load_stack(path):
    """-> (packed_weights, corrections) indexed by checkpoint layer, the maps FrozenSmolStack
    (directory, packed_weights=..., corrections=...) takes; corrections is None if the file has none."""
    weights, corrections, _ = load_prepared(Path(path))
    packed, fixes = {}, {}
    for source, target in ((weights, packed), (corrections, fixes)):
        for name, value in source.items():
            match = _LAYER_NAME.match(name)
            if not match:
                raise ValueError(f'{name}: not a model.layers.<i>.<projection> name')
            target.setdefault(int(match.group(1)), {})[match.group(2)] = value
    if fixes:
        for index in packed:
            fixes.setdefault(index, {})
    return packed, (fixes or None)
