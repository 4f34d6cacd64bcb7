"""Seeded random-init SmolLM-135M-architecture weights (no checkpoint is available offline).

Builds the decoder used for decode benchmarks and decoder parity tests: 30 layers, hidden
576, 9 query / 3 KV heads, SiLU MLP 1536, RMSNorm eps 1e-5 with gamma = 1 (the Hugging Face
init), tied vocab 49152 embedding, every weight and the embedding drawn from N(0, 0.02^2),
W8 per-row quantization of the fp16-cast weights (as the reference prepares them,
torch_npu_smollm.py:109), and optional rank-r corrections with U, V ~ N(0, 0.01^2).

Draw order from one torch.Generator(seed): per layer, the seven projection weights in
PROJECTIONS order; then the embedding; then, per layer and projection, V [r,K] and U [N,r].
"""
import torch

from torch_npu_lowbit import quantize_weight
from torch_npu_lowbit_correction import LowRankCorrection
from torch_npu_smollm import FrozenSmolLayer, FrozenSmolStack, _SHAPES
from torch_npu_smollm_io import FrozenSmolIO

PROJECTIONS = ('self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight',
               'self_attn.o_proj.weight', 'mlp.gate_proj.weight', 'mlp.up_proj.weight', 'mlp.down_proj.weight')
VOCAB = 49152
QK = ('self_attn.q_proj.weight', 'self_attn.k_proj.weight')


def config(theta=10000.0, layers=30):
    return dict(model_type='llama', hidden_size=576, intermediate_size=1536, num_attention_heads=9,
                num_key_value_heads=3, hidden_act='silu', attention_bias=False, mlp_bias=False, rms_norm_eps=1e-5,
                rope_theta=theta, rope_scaling=None, pretraining_tp=1, num_hidden_layers=layers,
                tie_word_embeddings=True, vocab_size=VOCAB)


def random_weights(seed=0, layers=30, rank=32, std=0.02, corr_std=0.01, qk_std=None, embed_std=None):
    """(per-layer weight dicts, embedding fp32 [V,576], norm [576], per-layer {name: (V, U)} or None).

    qk_std / embed_std (default: std) set the q/k projections' and the embedding's deviation."""
    g = torch.Generator().manual_seed(seed)
    qk_std = std if qk_std is None else qk_std
    embed_std = std if embed_std is None else embed_std
    layer_weights = []
    for _ in range(layers):
        w = {name: torch.randn(_SHAPES[name], generator=g) * (qk_std if name in QK else std) for name in PROJECTIONS}
        w['input_layernorm.weight'] = torch.ones(576)
        w['post_attention_layernorm.weight'] = torch.ones(576)
        layer_weights.append(w)
    embedding = torch.randn(VOCAB, 576, generator=g) * embed_std
    norm = torch.ones(576)
    factors = None
    if rank:
        factors = []
        for _ in range(layers):
            f = {}
            for name in PROJECTIONS:
                n, k = _SHAPES[name]
                down = (torch.randn(rank, k, generator=g) * corr_std).half()
                up = (torch.randn(n, rank, generator=g) * corr_std).half()
                f[name] = (down, up)
            factors.append(f)
    return layer_weights, embedding, norm, factors


def build(seed=0, layers=30, rank=32, theta=10000.0, capacity=384, mode='w8a16', **scales):
    """(FrozenSmolStack, FrozenSmolIO, packed per layer, corrections per layer) for the config.
    `scales` (std, qk_std, embed_std, corr_std) go to random_weights."""
    cfg = config(theta, layers)
    layer_weights, embedding, norm, factors = random_weights(seed, layers, rank, **scales)
    stack_layers, packed_all, corr_all = [], [], []
    for i, w in enumerate(layer_weights):
        fmt = {'w8a16': 'int8', 'w4a16': 'int4', 'nf4a16': 'nf4'}.get(mode)
        packed = None if fmt is None else {
            name: quantize_weight(w[name].half(), format=fmt, group_size=None if fmt == 'int8' else 32)
            for name in PROJECTIONS}
        corrections = None
        if factors is not None and mode == 'w8a16':
            corrections = {name: LowRankCorrection(_SHAPES[name], rank, down.numpy().tobytes(), up.numpy().tobytes())
                           for name, (down, up) in factors[i].items()}
        stack_layers.append(FrozenSmolLayer(cfg, w, mode=mode, packed_weights=packed, corrections=corrections,
                                            capacity=capacity))
        packed_all.append(packed)
        corr_all.append(corrections)
    stack = FrozenSmolStack.from_layers(stack_layers)
    io = FrozenSmolIO(cfg, embedding, norm)
    return stack, io, packed_all, corr_all


def prompt(seed=0, length=256):
    """Uniform-random token ids [1, length] in [0, VOCAB)."""
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randint(0, VOCAB, (1, length), generator=g)
