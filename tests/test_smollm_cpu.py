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


# --- independent pin of the oracle's attention half against a textbook Llama ------------------------------
# transformers' LlamaForCausalLM (built offline from a local LlamaConfig, eager attention, fp32) is the
# textbook form of the reference's decoder: rotate-half RoPE from theta (torch_npu_smollm.py:113-116,176),
# GQA by repeat_interleave (:178), scaled causal scores and softmax (:179-182), RMSNorm and the SiLU MLP.
# Loaded with the oracle's own effective weights (exact q*s plus U.V), it must agree with the staged
# oracle to fp16-staging accuracy, and each plausible wrong convention of the oracle must not.

def _hf_case(seed=11, layers=2, vocab=256, length=16):
    """Seeded W8 + rank-8 layers with peaked attention (q/k std 0.08), non-unit norms and 16 ids."""
    g = torch.Generator().manual_seed(seed)
    specs = []
    for _ in range(layers):
        w = {n: (torch.randn(_SHAPES[n], generator=g) * (.08 if n.split('.')[1] in ('q_proj', 'k_proj') else .03)).half()
             for n in so.PROJECTIONS}
        for n in ('input_layernorm.weight', 'post_attention_layernorm.weight'):
            w[n] = (1 + torch.randn(576, generator=g) * .1).half()
        packed = {n: quantize_weight(w[n], format='int8') for n in so.PROJECTIONS}
        corr = {n: ((torch.randn(8, _SHAPES[n][1], generator=g) * .02).half(),
                    (torch.randn(_SHAPES[n][0], 8, generator=g) * .02).half())
                for n in ('self_attn.o_proj.weight', 'mlp.down_proj.weight')}
        specs.append((w, {n: (q.format, q.shape, q.group_size, q.data, q.scales) for n, q in packed.items()}, corr))
    emb = (torch.randn(vocab, 576, generator=g) * .05).half()
    norm = (1 + torch.randn(576, generator=g) * .1).half()
    ids = torch.randint(0, vocab, (1, length), generator=g)
    return specs, emb, norm, ids


def _hf_reference(specs, emb, norm, ids, theta):
    """(per-layer attention outputs [S,576], logits [S,V]) of transformers' Llama in fp32."""
    transformers = pytest.importorskip('transformers')
    from oracle import lowbit_oracle as lo
    cfg = transformers.LlamaConfig(
        vocab_size=emb.shape[0], hidden_size=576, intermediate_size=1536, num_hidden_layers=len(specs),
        num_attention_heads=9, num_key_value_heads=3, head_dim=64, rms_norm_eps=1e-5, rope_theta=theta,
        tie_word_embeddings=True, max_position_embeddings=64, attention_bias=False, mlp_bias=False,
        hidden_act='silu', attn_implementation='eager')
    model = transformers.LlamaForCausalLM(cfg).eval()
    state = {'model.embed_tokens.weight': emb.float(), 'lm_head.weight': emb.float(), 'model.norm.weight': norm.float()}
    for i, (w, packed, corr) in enumerate(specs):
        for n in so.PROJECTIONS:
            effective = torch.from_numpy(lo.exact_weight(*packed[n]))
            if n in corr:
                down, up = corr[n]
                effective = effective + up.double() @ down.double()
            state[f'model.layers.{i}.{n}'] = effective.float()
        for n in ('input_layernorm.weight', 'post_attention_layernorm.weight'):
            state[f'model.layers.{i}.{n}'] = w[n].float()
    model.load_state_dict(state, strict=True)
    attention = []
    for layer in model.model.layers:
        layer.self_attn.o_proj.register_forward_pre_hook(lambda _m, args: attention.append(args[0][0].detach()))
    with torch.no_grad():
        logits = model(ids).logits[0]
    return attention, logits


def _oracle_run(layer_type, specs, emb, norm, ids, theta):
    layers = [layer_type(w, packed, corr, theta=theta, capacity=64) for w, packed, corr in specs]
    model = so.OracleModel(layers, emb, norm)
    x, attention = model.embed(ids), []
    for layer in layers:
        x, trace, _, _ = layer.forward(x)
        attention.append(trace['attention'][0])
    return attention, model.logits(x)[0]


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


class _InterleavedRope(so.OracleLayer):
    """Wrong convention: RoPE on adjacent pairs (2i, 2i+1) instead of rotate-half."""

    @staticmethod
    def _rotate(v, cos, sin):
        c, s = cos[..., :32].repeat_interleave(2, -1), sin[..., :32].repeat_interleave(2, -1)
        rot = torch.stack((-v[..., 1::2], v[..., 0::2]), -1).flatten(-2)
        return (v * c + rot * s).half()


class _TiledHeads(so.OracleLayer):
    """Wrong GQA mapping: query head h reads KV head h % 3 instead of h // 3."""

    @staticmethod
    def _attend(q, k, v, mask):
        k, v = k.repeat(1, 3, 1, 1), v.repeat(1, 3, 1, 1)
        scores = (q.float() @ k.float().transpose(-1, -2)).half()
        probs = ((scores * 0.125).half() + mask).float().softmax(-1).half()
        return (probs.float() @ v.float()).half()


class _NoMask(so.OracleLayer):
    """Wrong masking: every position attends to the whole sequence."""

    @staticmethod
    def _attend(q, k, v, mask):
        return so.OracleLayer._attend(q, k, v, torch.zeros_like(mask))


def test_oracle_attention_matches_transformers_llama():
    specs, emb, norm, ids = _hf_case()
    theta = 10000.0
    want_att, want_logits = _hf_reference(specs, emb, norm, ids, theta)
    att, logits = _oracle_run(so.OracleLayer, specs, emb, norm, ids, theta)
    errs = [_rel(a, b) for a, b in zip(att, want_att)] + [_rel(logits, want_logits)]
    assert max(errs) <= 5e-3, errs
    # Each wrong convention is far outside that tolerance, at the first layer's attention already.
    for layer_type, t in ((_InterleavedRope, theta), (_TiledHeads, theta), (_NoMask, theta), (so.OracleLayer, 1e5)):
        bad_att, bad_logits = _oracle_run(layer_type, specs, emb, norm, ids, t)
        assert _rel(bad_att[0], want_att[0]) > 0.1, (layer_type.__name__, t)
        assert _rel(bad_logits, want_logits) > 0.1, (layer_type.__name__, t)


def test_quantized_head_cpu_logits():
    """The quantized tied head on the CPU is the projection linear of the reference
    (torch_npu_smollm.py:150-157) on the normalized rows, as the oracle states it."""
    g = torch.Generator().manual_seed(106)
    cfg = dict(model_type='llama', hidden_size=576, tie_word_embeddings=True, rms_norm_eps=1e-5, vocab_size=96)
    emb = (torch.randn(96, 576, generator=g) * .03).half()
    norm = (1 + torch.randn(576, generator=g) * .1).half()
    x = (torch.randn(2, 3, 576, generator=g)).half()
    plain = FrozenSmolIO(cfg, emb, norm)
    for fmt, group in (('int8', None), ('int4', 64), ('nf4', 32)):
        io = FrozenSmolIO(cfg, emb, norm, head_format=fmt, head_group_size=group)
        q = io.head
        assert q.format == fmt and q.shape == (96, 576) and q == quantize_weight(emb, format=fmt, group_size=group)
        model = so.OracleModel([], emb, norm, head=(q.format, q.shape, q.group_size, q.data, q.scales))
        got = io.logits(x)
        torch.testing.assert_close(got, model.logits(x), rtol=0, atol=0)
        err = float((got.float() - plain.logits(x).float()).norm() / plain.logits(x).float().norm())
        assert 0 < err < (0.02 if fmt == 'int8' else 0.3), (fmt, err)
    for bad in (dict(head_format='int2'), dict(head_format='int8', head_group_size=64)):
        with pytest.raises(ValueError):
            FrozenSmolIO(cfg, emb, norm, **bad)
