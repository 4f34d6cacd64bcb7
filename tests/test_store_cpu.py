"""CPU checks of the on-disk form of prepared weights (torch_npu_lowbit_store): every object
comes back bit for bit through its own validating constructor, damaged files are refused."""
import numpy as np
import pytest
import torch

import smollm_random
from torch_npu_lowbit import PackedWeight, pack_codes, quantize_weight
from torch_npu_lowbit_correction import LowRankCorrection
from torch_npu_lowbit_store import load_prepared, load_stack, save_prepared, save_stack


def sample_weights():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(24, 96, generator=g) * 0.02
    weights = {
        'int8_row': quantize_weight(w, format='int8'),
        'int8_g32': quantize_weight(w, format='int8', group_size=32),
        'int4_g32': quantize_weight(w, format='int4', group_size=32),
        'nf4_g96': quantize_weight(w, format='nf4'),
        # odd element count: the last byte carries one code and a zero pad nibble
        'int4_odd': PackedWeight((3, 5), 'int4', 5, pack_codes(np.arange(15, dtype=np.uint8)),
                                 np.full(3, 0.5, np.float16).tobytes()),
    }
    down = (torch.randn(4, 96, generator=g) * 0.01).half()
    up = (torch.randn(24, 4, generator=g) * 0.01).half()
    corrections = {'int8_row': LowRankCorrection((24, 96), 4, down.numpy().tobytes(), up.numpy().tobytes())}
    return weights, corrections


def test_round_trip_is_bit_exact(tmp_path):
    weights, corrections = sample_weights()
    path = tmp_path / 'prepared.safetensors'
    save_prepared(path, weights, corrections, metadata={'source': 'unit test'})
    got_w, got_c, meta = load_prepared(path)
    assert got_w == weights and got_c == corrections  # frozen dataclasses: field-wise equality of the bytes
    assert meta == {'source': 'unit test'}
    for name, w in weights.items():
        assert got_w[name].dequantize().tobytes() == w.dequantize().tobytes()


def test_guards(tmp_path):
    weights, corrections = sample_weights()
    with pytest.raises(ValueError):
        save_prepared(tmp_path / 'a.safetensors', {'x': b'not a weight'})
    with pytest.raises(ValueError):
        save_prepared(tmp_path / 'a.safetensors', weights, metadata={'lowbit.version': '9'})
    # a safetensors file that is not a prepared-weight file
    from safetensors.torch import save_file
    save_file({'t': torch.zeros(2)}, str(tmp_path / 'other.safetensors'))
    with pytest.raises(ValueError):
        load_prepared(tmp_path / 'other.safetensors')
    # damaged contents are caught by the reference's own validation on load
    save_prepared(tmp_path / 'bad.safetensors', {'w': weights['int4_g32']})
    from safetensors import safe_open
    with safe_open(str(tmp_path / 'bad.safetensors'), framework='pt') as f:
        meta, codes, scales = f.metadata(), f.get_tensor('w.codes'), f.get_tensor('w.scales')
    scales[0, 0] = 0.0  # scales must be positive
    save_file({'w.codes': codes, 'w.scales': scales}, str(tmp_path / 'bad.safetensors'), metadata=meta)
    with pytest.raises(ValueError):
        load_prepared(tmp_path / 'bad.safetensors')
    save_file({'w.codes': codes[:-1], 'w.scales': scales.abs() + 1}, str(tmp_path / 'short.safetensors'),
              metadata=meta)
    with pytest.raises(ValueError):
        load_prepared(tmp_path / 'short.safetensors')


def test_stack_round_trip(tmp_path):
    stack, _, packed, corrections = smollm_random.build(seed=1, layers=2, rank=8, capacity=16)
    path = tmp_path / 'stack.safetensors'
    save_stack(path, stack)
    got_packed, got_corrections = load_stack(path)
    assert set(got_packed) == {0, 1} and set(got_corrections) == {0, 1}
    for i, layer in enumerate(stack.layers):
        assert got_packed[i] == layer._packed
        assert got_corrections[i] == layer._corrections


def test_loaded_stack_rebuilds_identical_layers(tmp_path):
    """Layers built from the loaded maps compute what the original layers compute (CPU reference)."""
    from torch_npu_smollm import FrozenSmolLayer
    stack, _, _, _ = smollm_random.build(seed=2, layers=2, rank=8, capacity=16)
    save_stack(tmp_path / 's.safetensors', stack)
    packed, corrections = load_stack(tmp_path / 's.safetensors')
    cfg = smollm_random.config(10000.0, 2)
    x = (torch.randn(1, 5, 576, generator=torch.Generator().manual_seed(3)) * 0.5).half()
    for i, layer in enumerate(stack.layers):
        rebuilt = FrozenSmolLayer(cfg, layer._weights, mode='w8a16', packed_weights=packed[i],
                                  corrections=corrections[i], capacity=16)
        assert torch.equal(rebuilt.reference_cpu(x)[0], layer.reference_cpu(x)[0])
