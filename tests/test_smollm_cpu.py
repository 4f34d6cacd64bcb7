"""CPU checks of the SmolLM decoder oracle and of the decoder API (no GPU).

Oracle pins (each plausible slip fails one): decode rows reproduce the causal full-sequence
forward; zero correction factors leave the staged output bitwise unchanged and a nonzero
factor changes exactly the selected projection by fp16(fp16(x.V^T).U^T) before the residual
(reference test_torch_npu_smollm_correction.py:45-85); the 4-bit value trace equals
F.linear(norm1, dequantize()) exactly (test_torch_npu_smollm_lowbit.py:46-53); protected
projections use the original fp16 weight (test_torch_npu_smollm_policy.py:65-74); tied
logits match F.rms_norm + F.linear (test_torch_npu_smollm_io.py:27-35).
"""
import json
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import smollm_oracle as so
import smollm_random
from torch_npu_lowbit import quantize_weight
from torch_npu_lowbit_correction import LowRankCorrection
from torch_npu_smollm import FrozenSmolLayer, FrozenSmolStack, _SHAPES
from torch_npu_smollm_io import FrozenSmolIO

CONFIG = dict(model_type='llama', hidden_size=576, intermediate_size=1536, num_attention_heads=9,
              num_key_value_heads=3, hidden_act='silu', attention_bias=False, mlp_bias=False, rms_norm_eps=1e-5,
              rope_theta=100000, rope_scaling=None, pretraining_tp=1)


@pytest.fixture(scope='module')
def policy_weights():
    """The reference policy fixture: seed 414, weights N(0, 0.015^2), x N(0, 0.1^2)."""
    g = torch.Generator().manual_seed(414)
    w = {n: (torch.randn(s, generator=g) * .015).half() if len(s) == 2 else torch.ones(s).half()
         for n, s in _SHAPES.items()}
    x = (torch.randn(1, 7, 576, generator=g) * .1).half()
    return w, x


def packed_of(layer):
    return {n: (q.format, q.shape, q.group_size, q.data, q.scales) for n, q in layer._packed.items()}


def test_decode_rows_reproduce_full_forward(policy_weights):
    w, x = policy_weights
    layer = FrozenSmolLayer(CONFIG, w)
    oracle = so.OracleLayer(w, packed_of(layer))
    full, _, keys, values = oracle.forward(x)
    _, _, k3, v3 = oracle.forward(x[:, :3])
    torch.testing.assert_close(k3, keys[:, :, :3], rtol=0, atol=0)
    k, v = k3, v3
    for pos in range(3, 7):
        out, k, v = oracle.decode(x[:, pos:pos + 1], k, v, pos)
        # same staging row by row; CPU BLAS order can differ with M, so allow 1-2 fp16 ulps
        torch.testing.assert_close(out, full[:, pos:pos + 1], rtol=4e-3, atol=2e-4)
    torch.testing.assert_close(k, keys, rtol=4e-3, atol=2e-4)


def test_zero_and_selected_corrections(policy_weights):
    w, x = policy_weights
    packed = {n: quantize_weight(t, format='int8') for n, t in w.items() if t.ndim == 2}
    base = FrozenSmolLayer(CONFIG, w, packed_weights=packed)
    zero = LowRankCorrection((576, 1536), 8, bytes(8 * 1536 * 2), bytes(576 * 8 * 2))
    exact = FrozenSmolLayer(CONFIG, w, packed_weights=packed, corrections={'mlp.down_proj.weight': zero})
    a, _ = exact.reference_cpu(x)
    b, old = base.reference_cpu(x)
    torch.testing.assert_close(a, b, rtol=0, atol=0)
    o = so.OracleLayer(w, packed_of(base), {'mlp.down_proj.weight': zero.tensors()})
    torch.testing.assert_close(o.forward(x)[0], b, rtol=0, atol=0)
    factor = LowRankCorrection((576, 1536), 8, np.full((8, 1536), .001, dtype=np.float16).tobytes(),
                               np.full((576, 8), .001, dtype=np.float16).tobytes())
    layer = FrozenSmolLayer(CONFIG, w, packed_weights=packed, corrections={'mlp.down_proj.weight': factor})
    _, actual = layer.reference_cpu(x)
    down, up = factor.tensors()
    delta = F.linear(F.linear(old['gated'].float(), down.float()).half().float(), up.float()).half()
    torch.testing.assert_close(actual['ffn_output'], (old['ffn_output'] + delta).half(), rtol=0, atol=0)
    oracle = so.OracleLayer(w, packed_of(layer), {'mlp.down_proj.weight': (down, up)})
    _, trace, _, _ = oracle.forward(x)
    torch.testing.assert_close(trace['ffn_output'], actual['ffn_output'], rtol=0, atol=0)
    assert not torch.equal(trace['ffn_output'], old['ffn_output'])


def test_four_bit_trace_uses_dequantized_weights(policy_weights):
    w, x = policy_weights
    for mode in ('w4a16', 'nf4a16'):
        layer = FrozenSmolLayer(CONFIG, w, mode=mode)
        assert all(q.group_size == 32 for q in layer._packed.values())
        oracle = so.OracleLayer(w, packed_of(layer))
        _, trace, _, values = oracle.forward(x)
        q = layer._packed['self_attn.v_proj.weight']
        expected = F.linear(trace['norm1'].float(), torch.from_numpy(q.dequantize().copy()).float()).half()
        torch.testing.assert_close(values, expected.view(1, 7, 3, 64).transpose(1, 2), rtol=0, atol=0)
        plain = so.OracleLayer(w).forward(x)[3]
        assert not torch.equal(values, plain)


def test_protected_projection_uses_fp16(policy_weights):
    w, x = policy_weights
    layer = FrozenSmolLayer(CONFIG, w, fp16_projections=('mlp.down_proj.weight',))
    oracle = so.OracleLayer(w, packed_of(layer), protected=('mlp.down_proj.weight',))
    _, trace, _, _ = oracle.forward(x)
    expected = F.linear(trace['gated'].float(), w['mlp.down_proj.weight'].float()).half()
    torch.testing.assert_close(trace['ffn_output'], expected, rtol=0, atol=0)
    torch.testing.assert_close(layer.reference_cpu(x)[0], oracle.forward(x)[0], rtol=0, atol=0)


def test_tied_logits_reference():
    g = torch.Generator().manual_seed(105)
    cfg = dict(model_type='llama', hidden_size=576, tie_word_embeddings=True, rms_norm_eps=1e-5, vocab_size=64)
    emb = (torch.randn(64, 576, generator=g) * .03).bfloat16()
    norm = (1 + torch.randn(576, generator=g) * .1).bfloat16()
    io = FrozenSmolIO(cfg, emb, norm)
    ids = torch.tensor([[0, 1, 63], [2, 7, 19]])
    assert torch.equal(io.embed_tokens(ids), F.embedding(ids, emb.half()))
    x = io.embed_tokens(ids)
    ref = F.rms_norm(x.float(), (576,), eps=1e-5).half() * norm.half()
    torch.testing.assert_close(io.logits(x), F.linear(ref, emb.half()), atol=.002, rtol=.002)
    model = so.OracleModel([], emb, norm)
    torch.testing.assert_close(model.logits(x), io.logits(x), rtol=0, atol=0)


def test_policy_and_correction_guards(policy_weights):
    w, _ = policy_weights
    names = tuple(n for n, t in w.items() if t.ndim == 2)
    for bad in (None, [], 'mlp.down_proj.weight', ('unknown',), ('input_layernorm.weight',), (False,),
                ('mlp.down_proj.weight',) * 2, names):
        with pytest.raises(ValueError):
            FrozenSmolLayer(CONFIG, w, fp16_projections=bad)
    with pytest.raises(ValueError):
        FrozenSmolLayer(CONFIG, w, mode='fp16', fp16_projections=('mlp.down_proj.weight',))
    packed = {n: quantize_weight(t, format='int8') for n, t in w.items() if t.ndim == 2}
    corr = LowRankCorrection((576, 576), 8, bytes(8 * 576 * 2), bytes(576 * 8 * 2))
    bad_shape = LowRankCorrection((2, 2), 1, bytes(4), bytes(4))
    for options in (dict(corrections=[]), dict(corrections={'unknown': corr}),
                    dict(corrections={'self_attn.k_proj.weight': corr}),
                    dict(corrections={'self_attn.q_proj.weight': bad_shape}),
                    dict(corrections={'self_attn.q_proj.weight': corr}, fp16_projections=('self_attn.q_proj.weight',))):
        with pytest.raises(ValueError):
            FrozenSmolLayer(CONFIG, w, packed_weights=packed, **options)
    with pytest.raises(ValueError):
        FrozenSmolLayer(CONFIG, w, corrections={'self_attn.q_proj.weight': corr})
    with pytest.raises(ValueError):
        FrozenSmolLayer(dict(CONFIG, hidden_size=512), w)
    with pytest.raises(ValueError):
        FrozenSmolLayer(dict(CONFIG, rope_theta=-1.0), w)
    four = FrozenSmolLayer(CONFIG, w, mode='w4a16')._packed
    with pytest.raises(ValueError):
        FrozenSmolLayer(CONFIG, w, mode='nf4a16', packed_weights=four)
    layer = FrozenSmolLayer(CONFIG, w, packed_weights=packed, fp16_projections=('mlp.down_proj.weight',))
    assert layer.fp16_projections == frozenset(('mlp.down_proj.weight',))
    with pytest.raises(AttributeError):
        layer.fp16_projections = ()


def test_checkpoint_round_trip():
    from safetensors.torch import save_file
    cfg = smollm_random.config(theta=10000.0, layers=2)
    cfg['vocab_size'] = 64
    layer_weights, _, _, _ = smollm_random.random_weights(seed=3, layers=2, rank=0)
    g = torch.Generator().manual_seed(9)
    tensors = {'model.embed_tokens.weight': torch.randn(64, 576, generator=g) * .02, 'model.norm.weight': torch.ones(576)}
    for i, w in enumerate(layer_weights):
        tensors.update({f'model.layers.{i}.{n}': t.contiguous() for n, t in w.items()})
    with tempfile.TemporaryDirectory() as d:
        path = Path(d)
        (path / 'config.json').write_text(json.dumps(cfg))
        save_file(tensors, str(path / 'model.safetensors'))
        stack = FrozenSmolStack.from_checkpoint(path, num_layers=2, capacity=16)
        io = FrozenSmolIO.from_checkpoint(path)
        single = FrozenSmolLayer.from_checkpoint(path, layer_index=1, capacity=16)
        assert stack.num_layers == 2 and stack.mode == 'w8a16' and io.embedding.shape == (64, 576)
        assert single._packed['mlp.up_proj.weight'] == stack.layers[1]._packed['mlp.up_proj.weight']
        x = (torch.randn(1, 3, 576, generator=g) * .1).half()
        y, _ = stack.reference_cpu(x)
        assert torch.isfinite(y).all()
        save_file(dict(tensors, **{'lm_head.weight': tensors['model.embed_tokens.weight'].clone()}),
                  str(path / 'model.safetensors'))
        with pytest.raises(ValueError):
            FrozenSmolIO.from_checkpoint(path)
