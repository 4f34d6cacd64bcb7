"""GPU parity of lb_decode_layer (one decoder layer for one token in one launch) against the CPU
oracle's decode step (the restated reference_cpu, torch_npu_smollm.py:142-193).

Bars: the layer output and the appended key / value rows within rel-L2 1e-2 (the decoder bar; the
stages are the fused decode kernels, each at 1e-3 against the oracle), identical bits over repeated
calls on one workspace, every workgroup counted once per call and no timed-out wait; past the
capacity the cache is left alone and the output is NaN.  Modes: W8 per row with rank-32 and rank-5
corrections, INT4 / NF4 group 32 (the SmolLM 4-bit policy), fp16.
"""
import pytest
import torch

import lowbit_hip as lb
from conftest import announce
from oracle import smollm_oracle as so
from torch_npu_lowbit import quantize_weight
from torch_npu_lowbit_correction import LowRankCorrection
from torch_npu_smollm import FrozenSmolLayer, GraphDecoder, _SHAPES
import smollm_random

pytestmark = pytest.mark.gpu
CONFIG = smollm_random.config(theta=10000.0, layers=1)
CAP = 384


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


def make_layer(mode, rank, seed):
    g = torch.Generator().manual_seed(seed)
    w = {n: (torch.randn(s, generator=g) * .03).half() if len(s) == 2 else (1 + torch.randn(s, generator=g) * .1).half()
         for n, s in _SHAPES.items()}
    packed = corr = None
    if mode == 'w8a16':
        packed = {n: quantize_weight(t, format='int8') for n, t in w.items() if t.ndim == 2}
        if rank:
            corr = {n: LowRankCorrection(_SHAPES[n], rank,
                                         (torch.randn(rank, _SHAPES[n][1], generator=g) * .02).half().numpy().tobytes(),
                                         (torch.randn(_SHAPES[n][0], rank, generator=g) * .02).half().numpy().tobytes())
                    for n in packed}
    layer = FrozenSmolLayer(CONFIG, w, mode=mode, packed_weights=packed, corrections=corr, capacity=CAP)
    oracle = so.OracleLayer(layer._weights,
                            {n: (q.format, q.shape, q.group_size, q.data, q.scales) for n, q in layer._packed.items()},
                            {n: c.tensors() for n, c in layer._corrections.items()}, theta=10000.0, capacity=CAP)
    x = (torch.randn(1, 1, 576, generator=g) * .5).half()
    keys = (torch.randn(1, 3, CAP, 64, generator=g) * .7).half()
    values = torch.randn(1, 3, CAP, 64, generator=g).half()
    return layer, oracle, x, keys, values


def prepared(layer, device, h, keys, values, position):
    state = layer._dev(device)
    order = GraphDecoder._ORDER
    entries = [state['lin'][n] for n in order]
    fmt = entries[0]['format']
    group = 0 if fmt == 'fp16' or entries[0]['group'] == entries[0]['K'] else entries[0]['group']
    projections = []
    for e in entries:
        pr = dict(codes=e['codes'], scales=e['scales'], N=e['N'])
        if e.get('rank', 0):
            pr.update(down=e['down'], up=e['up'])
        projections.append(pr)
    return lb.PreparedLayer(h, projections, format=fmt, group_size=group, hidden=576, intermediate=1536,
                            norm1=state['norm1'], norm2=state['norm2'], eps=1e-5, heads=9, kv_heads=3,
                            cos=state['cos'], sin=state['sin'], position=position, keys=keys, values=values)


CASES = [('w8a16', 32, 37), ('w8a16', 32, 383), ('w8a16', 5, 200), ('w8a16', 0, 0), ('w4a16', 0, 100),
         ('nf4a16', 0, 300), ('fp16', 0, 64)]


@pytest.mark.parametrize('mode,rank,pos', CASES, ids=['-'.join(map(str, c)) for c in CASES])
def test_decode_layer_matches_oracle(device, mode, rank, pos):
    announce('decode layer', mode, rank, pos)
    layer, oracle, x, keys, values = make_layer(mode, rank, 31 + pos)
    keys[:, :, pos + 1:] = float('nan')      # slots past the position are never read
    values[:, :, pos + 1:] = float('nan')
    want, wk, wv = oracle.decode(x, keys[:, :, :pos], values[:, :, :pos], pos)
    h = x.view(576).to(device).clone()
    dk, dv = keys[0].to(device).contiguous(), values[0].to(device).contiguous()
    position = torch.tensor([pos], dtype=torch.int64, device=device)
    call = prepared(layer, device, h, dk, dv, position)
    call.run()
    torch.cuda.synchronize()
    got = h.cpu().clone()
    err = rel_l2(got, want.view(576))
    print(f'[decode layer] {mode} rank {rank} pos {pos}: rel-L2 {err:.2e}', flush=True)
    assert bool(torch.isfinite(got).all()) and err <= 1e-2
    assert rel_l2(dk[:, pos].cpu(), wk[0, :, pos]) <= 1e-2
    assert rel_l2(dv[:, pos].cpu(), wv[0, :, pos]) <= 1e-2
    others = [i for i in range(CAP) if i != pos]
    assert torch.equal(dk[:, others].cpu(), keys[0][:, others], ) or bool(
        torch.equal(dk[:, others].cpu().isnan(), keys[0][:, others].isnan()))
    total, timeout = call.counters()
    assert timeout == 0 and total > 0
    # two more calls from the same input: the same bits, every workgroup counted once per call
    first_k = dk[:, pos].cpu().clone()
    for _ in range(2):
        h.copy_(x.view(576).to(device))
        call.run()
    torch.cuda.synchronize()
    assert torch.equal(h.cpu(), got) and torch.equal(dk[:, pos].cpu(), first_k)
    assert call.counters() == [3 * total, 0]


def test_decode_layer_past_capacity(device):
    announce('decode layer past capacity')
    layer, oracle, x, keys, values = make_layer('w8a16', 32, 5)
    h = x.view(576).to(device).clone()
    dk, dv = keys[0].to(device).contiguous(), values[0].to(device).contiguous()
    position = torch.tensor([CAP], dtype=torch.int64, device=device)
    call = prepared(layer, device, h, dk, dv, position)
    call.run()
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), keys[0]) and torch.equal(dv.cpu(), values[0])
    assert bool(torch.isnan(h.cpu()).all())
    assert call.counters()[1] == 0


def test_decode_layer_rejects_bad_arguments(device):
    layer, _, x, keys, values = make_layer('w8a16', 32, 9)
    h = x.view(576).to(device).clone()
    dk, dv = keys[0].to(device).contiguous(), values[0].to(device).contiguous()
    position = torch.tensor([3], dtype=torch.int64, device=device)
    call = prepared(layer, device, h, dk, dv, position)
    call.args.proj[0].N = 500
    with pytest.raises(ValueError, match='N=500'):
        call.run()
    call.args.proj[0].N = 576
    call.args.workspace_bytes = 64
    with pytest.raises(ValueError, match='workspace'):
        call.run()


def stack_entry(layer, device, keys, values):
    """One lb_decode_stack_layer dict (the tensors of `layer` on `device`)."""
    state = layer._dev(device)
    projections = []
    for n in GraphDecoder._ORDER:
        e = state['lin'][n]
        pr = dict(codes=e['codes'], scales=e['scales'], N=e['N'])
        if e.get('rank', 0):
            pr.update(down=e['down'], up=e['up'])
        projections.append(pr)
    return dict(norm1=state['norm1'], norm2=state['norm2'], keys=keys, values=values, projections=projections)


STACK_CASES = [('w8a16', 32, 3, 200), ('w8a16', 32, 2, 0), ('w4a16', 0, 3, 77), ('fp16', 0, 2, 383)]


@pytest.mark.parametrize('mode,rank,layers,pos', STACK_CASES, ids=['-'.join(map(str, c)) for c in STACK_CASES])
def test_decode_stack_matches_layer_calls(device, mode, rank, layers, pos):
    """lb_decode_stack over L layers gives the bits of L lb_decode_layer calls (same arithmetic), and
    the oracle's chained decode steps within the decoder bar."""
    announce('decode stack', mode, rank, layers, pos)
    made = [make_layer(mode, rank, 100 + 7 * l + pos) for l in range(layers)]
    x = made[0][2]
    position = torch.tensor([pos], dtype=torch.int64, device=device)
    # oracle chain
    want = x
    wks, wvs = [], []
    for layer, oracle, _, keys, values in made:
        want, wk, wv = oracle.decode(want, keys[:, :, :pos], values[:, :, :pos], pos)
        wks.append(wk[0, :, pos])
        wvs.append(wv[0, :, pos])
    # per-layer launches
    h1 = x.view(576).to(device).clone()
    caches1 = [(k[0].to(device).contiguous(), v[0].to(device).contiguous()) for _, _, _, k, v in made]
    for (layer, *_), (dk, dv) in zip(made, caches1):
        prepared(layer, device, h1, dk, dv, position).run()
    # one stacked launch
    h2 = x.view(576).to(device).clone()
    caches2 = [(k[0].to(device).contiguous(), v[0].to(device).contiguous()) for _, _, _, k, v in made]
    state = made[0][0]._dev(device)
    fmt, group, _ = GraphDecoder._layer_key(state)
    stack = lb.PreparedStack(h2, [stack_entry(m[0], device, dk, dv) for m, (dk, dv) in zip(made, caches2)],
                             format=fmt, group_size=group, hidden=576, intermediate=1536, eps=1e-5, heads=9,
                             kv_heads=3, cos=state['cos'], sin=state['sin'], position=position)
    stack.run()
    torch.cuda.synchronize()
    got = h2.cpu()
    err = rel_l2(got, want.view(576))
    print(f'[decode stack] {mode} rank {rank} layers {layers} pos {pos}: rel-L2 {err:.2e}', flush=True)
    assert torch.equal(got, h1.cpu())
    for (ak, av), (bk, bv) in zip(caches1, caches2):
        assert torch.equal(ak.cpu(), bk.cpu()) and torch.equal(av.cpu(), bv.cpu())
    assert bool(torch.isfinite(got).all()) and err <= 1e-2
    for l, (dk, dv) in enumerate(caches2):
        assert rel_l2(dk[:, pos].cpu(), wks[l]) <= 1e-2 and rel_l2(dv[:, pos].cpu(), wvs[l]) <= 1e-2
    total, timeout = stack.counters()
    assert timeout == 0 and total > 0
    # again from the same input: the same bits, every workgroup counted once per call
    for _ in range(2):
        h2.copy_(x.view(576).to(device))
        stack.run()
    torch.cuda.synchronize()
    assert torch.equal(h2.cpu(), got)
    assert stack.counters() == [3 * total, 0]


def test_decode_stack_refuses_unprepared_table(device):
    made = [make_layer('w8a16', 32, 11 + l) for l in range(2)]
    position = torch.tensor([5], dtype=torch.int64, device=device)
    h = made[0][2].view(576).to(device).clone()
    caches = [(k[0].to(device).contiguous(), v[0].to(device).contiguous()) for _, _, _, k, v in made]
    state = made[0][0]._dev(device)
    stack = lb.PreparedStack(h, [stack_entry(m[0], device, dk, dv) for m, (dk, dv) in zip(made, caches)],
                             format='int8', group_size=0, hidden=576, intermediate=1536, eps=1e-5, heads=9,
                             kv_heads=3, cos=state['cos'], sin=state['sin'], position=position)
    # layers that differ from the ones the table was prepared for
    n0, n1 = stack._rows[0].norm1, stack._rows[1].norm1
    stack._rows[0].norm1, stack._rows[1].norm1 = n1, n0
    with pytest.raises(ValueError, match='not prepared'):
        stack.run()
    stack._rows[0].norm1, stack._rows[1].norm1 = n0, n1
    stack.run()
    torch.cuda.synchronize()
    assert stack.counters()[1] == 0
