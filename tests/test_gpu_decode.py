"""GPU parity of the decode-step entry points (include/lowbit_decode_hip.h) against the CPU oracle.

lb_fused_linear: the prologue is applied on the CPU with the reference staging (RMSNorm
torch_npu_smollm.py:166-168, SiLU * up :188-190), then oracle.lowbit_oracle.linear gives each
projection (with its correction) and the residual is added in fp16; rel-L2 <= 1e-3.
lb_decode_attention: RoPE/attention from oracle.smollm_oracle (the restated reference_cpu);
the appended key/value rows are bit-exact, attention output rel-L2 <= 1e-3.
lb_argmax_next: torch.argmax order (first maximal index), bit-exact embedding row.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import lowbit_hip as lb
from conftest import announce
from oracle import lowbit_oracle as lo
from oracle import smollm_oracle as so
from torch_npu_lowbit import quantize_weight

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = torch.as_tensor(a).double().cpu(), torch.as_tensor(b).double().cpu()
    return float((a - b).norm() / b.norm())


def prologue_cpu(kind, x, x2=None, gamma=None):
    if kind == 'rmsnorm':
        f = x.float()
        return ((f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half() * gamma).half()
    if kind == 'silu_mul':
        return (F.silu(x.float()).half() * x2).half()
    return x


# (format, group (None = per row), K, prologue, output sizes, rank, residual, bias)
CASES = [
    ('int8', None, 576, 'rmsnorm', (576, 192, 192), 32, False, False),   # SmolLM q|k|v, W8 + rank 32
    ('int8', None, 576, 'none', (576,), 32, True, False),                # o_proj + residual
    ('int8', None, 576, 'rmsnorm', (1536, 1536), 32, False, False),      # gate|up
    ('int8', None, 1536, 'silu_mul', (576,), 32, True, False),           # down + residual
    ('int4', 32, 576, 'rmsnorm', (576, 192, 192), 0, False, False),      # w4a16 policy
    ('nf4', 32, 1536, 'silu_mul', (200,), 0, True, False),               # partial last tile
    ('int8', 64, 576, 'none', (40, 8, 100), 8, False, True),             # grouped int8, rank 8, bias
    ('int4', 576, 576, 'none', (33,), 16, True, True),                   # one group per row
    ('nf4', 64, 1024, 'rmsnorm', (40, 300), 24, False, True),
    ('fp16', None, 576, 'rmsnorm', (4096,), 0, False, False),            # tied-head shape (smaller N)
    ('fp16', None, 1536, 'silu_mul', (64, 64), 8, True, False),
    # one problem over many rows (rows_gemv_kernel): the full tied head, epilogue operands, 2 tiles
    ('fp16', None, 576, 'rmsnorm', (49152,), 0, False, False),
    ('int8', None, 1536, 'silu_mul', (32768,), 0, True, True),
    ('int4', 64, 576, 'none', (16400,), 0, True, False),
    # four tiles per workgroup: a partial last tile and idle waves after it, every epilogue
    # operand, both prologues, the 1536-long staged row
    ('int4', 64, 576, 'silu_mul', (49160,), 0, True, True),
    ('int4', 128, 1536, 'rmsnorm', (32768,), 0, False, False),
]


def make_case(case, seed):
    fmt, group, K, prologue, sizes, rank, residual, bias = case
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(K, generator=g).half()
    x2 = torch.randn(K, generator=g).half() if prologue == 'silu_mul' else None
    gamma = (1 + 0.1 * torch.randn(K, generator=g)).half() if prologue == 'rmsnorm' else None
    problems = []
    for n in sizes:
        w = torch.randn(n, K, generator=g) * 0.02
        pr = dict(N=n, w=w.half())
        if fmt != 'fp16':
            pr['packed'] = quantize_weight(w, format=fmt, group_size=group)
        if rank:
            pr['down'] = (torch.randn(rank, K, generator=g) * 0.01).half()
            pr['up'] = (torch.randn(n, rank, generator=g) * 0.01).half()
        if residual:
            pr['residual'] = torch.randn(n, generator=g).half()
        if bias:
            pr['bias'] = (0.1 * torch.randn(n, generator=g)).half()
        problems.append(pr)
    return x, x2, gamma, problems


def expected(case, x, x2, gamma, problems):
    fmt, group, K, prologue = case[:4]
    xp = prologue_cpu(prologue, x, x2, gamma)[None].numpy()
    outs = []
    for pr in problems:
        n = pr['N']
        down = pr['down'].numpy() if 'down' in pr else None
        up = pr['up'].numpy() if 'up' in pr else None
        b = pr['bias'].numpy() if 'bias' in pr else None
        if fmt == 'fp16':
            y = lo.dense_linear(xp, pr['w'].numpy())
            if b is not None:
                y = (y.astype(np.float64) + b.astype(np.float64)).astype(np.float16)
            if down is not None:
                z = lo.dense_linear(xp, down)
                y = (y.astype(np.float64) + lo.dense_linear(z, up).astype(np.float64)).astype(np.float16)
        else:
            q = pr['packed']
            y = lo.linear(xp, fmt, (n, K), q.group_size, q.data, q.scales, bias=b, down=down, up=up)
        if 'residual' in pr:
            y = (pr['residual'].numpy().astype(np.float64) + y.astype(np.float64)).astype(np.float16)
        outs.append(torch.from_numpy(y[0]))
    return outs


def device_problems(case, problems, device, in_place):
    fmt = case[0]
    out = []
    for pr in problems:
        if fmt == 'fp16':
            codes, scales = pr['w'].to(device), None
        else:
            codes, scales = pr['packed'].device_tensors(device)
        d = dict(codes=codes, scales=scales, N=pr['N'])
        if 'residual' in pr:
            res = pr['residual'].to(device)
            d['residual'] = res
            d['y'] = res if in_place else torch.full((pr['N'],), float('nan'), dtype=torch.float16, device=device)
        else:
            d['y'] = torch.full((pr['N'],), float('nan'), dtype=torch.float16, device=device)
        for key in ('down', 'up', 'bias'):
            if key in pr:
                d[key] = pr[key].to(device)
        out.append(d)
    return out


@pytest.mark.parametrize('shared_z', [True, False], ids=['shared-z', 'own-z'])
@pytest.mark.parametrize('index', range(len(CASES)))
def test_fused_linear_matches_oracle(device, index, shared_z):
    """Both correction modes: z in dedicated workgroups (workspace) or in every workgroup."""
    case = CASES[index]
    fmt, group, K, prologue, sizes, rank = case[:6]
    if not shared_z and not rank:
        pytest.skip('no correction: the two modes are one launch')
    announce('fused linear', case, 'shared z' if shared_z else 'own z')
    x, x2, gamma, problems = make_case(case, 100 + index)
    want = expected(case, x, x2, gamma, problems)
    for in_place in (False, True):
        dev = device_problems(case, problems, device, in_place)
        call = lb.PreparedFused(x.to(device), dev, format=fmt, K=K,
                                group_size=K if group is None or fmt == 'fp16' else group, prologue=prologue,
                                x2=None if x2 is None else x2.to(device),
                                gamma=None if gamma is None else gamma.to(device), eps=1e-5, shared_z=shared_z)
        call.run()
        torch.cuda.synchronize()
        got = [d['y'].cpu() for d in dev]
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.isfinite(a).all(), (i, in_place)
            err = rel_l2(a, b)
            assert err <= 1e-3, (i, in_place, err)
        tiles = sum((n + 15) // 16 for n in sizes)
        if shared_z and rank:
            assert call.counters() == [tiles, 0]   # every tile workgroup counted once, no timed-out wait
        if not in_place:  # further calls on the same buffers give the same bits
            for _ in range(3):
                call.run()
            torch.cuda.synchronize()
            for d, a in zip(dev, got):
                assert torch.equal(d['y'].cpu(), a)
            if shared_z and rank:
                assert call.counters() == [4 * tiles, 0]


def test_shared_z_equals_own_z_bit_for_bit(device):
    """The shared z is the same fp16 value each workgroup would compute (same prologue
    arithmetic), so both modes give identical outputs on the decode shapes."""
    announce('shared z vs own z')
    for index in range(4):
        case = CASES[index]
        fmt, group, K, prologue = case[:4]
        x, x2, gamma, problems = make_case(case, 300 + index)
        outs = []
        for shared_z in (True, False):
            dev = device_problems(case, problems, device, False)
            lb.PreparedFused(x.to(device), dev, format=fmt, K=K, group_size=K, prologue=prologue,
                             x2=None if x2 is None else x2.to(device), gamma=None if gamma is None else gamma.to(device),
                             eps=1e-5, shared_z=shared_z).run()
            torch.cuda.synchronize()
            outs.append([d['y'].cpu() for d in dev])
        for a, b in zip(*outs):
            assert torch.equal(a, b), case


def test_fused_linear_agrees_with_lb_linear(device):
    """Same W8 + correction projection through lb_linear (prologue done on the CPU) and fused."""
    announce('fused vs lb_linear')
    case = CASES[0]
    x, _, gamma, problems = make_case(case, 7)
    xp = prologue_cpu('rmsnorm', x, gamma=gamma).to(device)[None]
    dev = device_problems(case, problems, device, False)
    lb.PreparedFused(x.to(device), dev, format='int8', K=576, group_size=576, prologue='rmsnorm',
                     gamma=gamma.to(device)).run()
    for d in dev:
        ref = lb.linear(xp, d['codes'], d['scales'], format='int8', N=d['N'], K=576, group_size=576,
                        down=d['down'], up=d['up'], rank=d['down'].shape[0])
        torch.cuda.synchronize()
        assert rel_l2(d['y'].cpu(), ref[0].cpu()) <= 1e-3


def test_fused_linear_rejects_bad_arguments(device):
    x = torch.zeros(576, dtype=torch.float16, device=device)
    w = quantize_weight(torch.randn(64, 576), format='int8')
    codes, scales = w.device_tensors(device)
    y = torch.zeros(64, dtype=torch.float16, device=device)
    up5 = torch.zeros(64, 5, dtype=torch.float16, device=device)
    down5 = torch.zeros(5, 576, dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match='up_ld'):
        lb.fused_linear(x, [dict(codes=codes, scales=scales, N=64, y=y, down=down5, up=up5)], format='int8', K=576,
                        group_size=576)
    with pytest.raises(ValueError, match='overlaps'):
        lb.fused_linear(x, [dict(codes=codes, scales=scales, N=64, y=x[:64])], format='int8', K=576, group_size=576)
    with pytest.raises(ValueError, match='K='):
        lb.fused_linear(torch.zeros(1600, dtype=torch.float16, device=device),
                        [dict(codes=codes, scales=scales, N=64, y=y)], format='int8', K=1600, group_size=1600)


def attention_case(pos, cap, seed):
    g = torch.Generator().manual_seed(seed)
    keys = (torch.randn(1, 3, cap, 64, generator=g) * 0.7).half()
    values = torch.randn(1, 3, cap, 64, generator=g).half()
    q = (torch.randn(576, generator=g) * 0.7).half()
    k = (torch.randn(192, generator=g) * 0.7).half()
    v = torch.randn(192, generator=g).half()
    cos, sin = so.rope_tables(10000.0, cap)
    return keys, values, q, k, v, cos, sin


@pytest.mark.parametrize('split', [True, False], ids=['split', 'whole'])
@pytest.mark.parametrize('pos', [0, 1, 2, 3, 37, 47, 48, 255, 383])
def test_decode_attention_matches_oracle(device, pos, split):
    announce('decode attention', pos, split)
    cap = 384
    keys, values, q, k, v, cos, sin = attention_case(pos, cap, pos)
    c, s = cos[pos:pos + 1][None, None], sin[pos:pos + 1][None, None]
    qr = so.OracleLayer._rotate(q.view(1, 1, 9, 64).transpose(1, 2), c, s)
    kr = so.OracleLayer._rotate(k.view(1, 1, 3, 64).transpose(1, 2), c, s)
    ks = torch.cat((keys[:, :, :pos], kr), dim=2)
    vs = torch.cat((values[:, :, :pos], v.view(1, 1, 3, 64).transpose(1, 2)), dim=2)
    want = so.OracleLayer._attend(qr, ks, vs, torch.zeros(1, pos + 1)).reshape(576)
    dk, dv = keys.to(device), values.to(device)
    out = torch.full((576,), float('nan'), dtype=torch.float16, device=device)
    position = torch.tensor([pos], dtype=torch.int64, device=device)
    call = lb.PreparedAttention(q.to(device), k.to(device), v.to(device), cos.to(device), sin.to(device), position,
                                dk, dv, out, heads=9, kv_heads=3, split=split)
    call.run()
    torch.cuda.synchronize()
    assert rel_l2(out.cpu(), want) <= 1e-3
    if split:
        assert call.counters() == [36, 0]      # every output workgroup counted once, no timed-out wait
        first = out.cpu().clone()
        dk[:, :, pos] = keys[:, :, pos].to(device)   # undo the append, run twice more on the same workspace
        dv[:, :, pos] = values[:, :, pos].to(device)
        call.run()
        call.run()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), first) and call.counters() == [108, 0]
    assert torch.equal(dk[:, :, pos].cpu(), kr[:, :, 0])
    assert torch.equal(dv[:, :, pos].cpu(), v.view(3, 64)[None])
    others = [i for i in range(cap) if i != pos]
    assert torch.equal(dk[:, :, others].cpu(), keys[:, :, others])
    assert torch.equal(dv[:, :, others].cpu(), values[:, :, others])


@pytest.mark.parametrize('split', [True, False], ids=['split', 'whole'])
@pytest.mark.parametrize('pos,cap,poison', [(100, 384, True), (383, 384, False), (700, 1024, True), (1023, 1024, False),
                                            (4095, 4096, True), (10, 16, True)])
def test_decode_attention_masks_slots_past_the_position(device, pos, cap, poison, split):
    """Slots past the position may hold anything (here NaN / Inf when `poison`): the kernel loads the
    first 512 slots before it reads the position, and must select them away; capacities above 512
    take further load rounds."""
    announce('decode attention mask', pos, cap, poison)
    keys, values, q, k, v, cos, sin = attention_case(pos, cap, pos + cap)
    if poison:
        keys[:, :, pos + 1:] = float('nan')
        values[:, :, pos + 1::2] = float('inf')
        values[:, :, pos + 2::2] = float('nan')
    c, s = cos[pos:pos + 1][None, None], sin[pos:pos + 1][None, None]
    qr = so.OracleLayer._rotate(q.view(1, 1, 9, 64).transpose(1, 2), c, s)
    kr = so.OracleLayer._rotate(k.view(1, 1, 3, 64).transpose(1, 2), c, s)
    ks = torch.cat((keys[:, :, :pos], kr), dim=2)
    vs = torch.cat((values[:, :, :pos], v.view(1, 1, 3, 64).transpose(1, 2)), dim=2)
    want = so.OracleLayer._attend(qr, ks, vs, torch.zeros(1, pos + 1)).reshape(576)
    dk, dv = keys.to(device), values.to(device)
    out = torch.full((576,), float('nan'), dtype=torch.float16, device=device)
    position = torch.tensor([pos], dtype=torch.int64, device=device)
    lb.PreparedAttention(q.to(device), k.to(device), v.to(device), cos.to(device), sin.to(device), position, dk, dv,
                         out, heads=9, kv_heads=3, split=split).run()
    torch.cuda.synchronize()
    got = out.cpu()
    assert bool(torch.isfinite(got).all())
    assert rel_l2(got, want) <= 1e-3


def test_decode_attention_past_the_capacity_leaves_the_cache_and_gives_nan(device):
    """A position outside the cache (full, or negative) reads and writes no slot, and the output is
    NaN everywhere: a caller past the capacity sees it instead of stale values."""
    announce('decode attention past capacity')
    cap = 16
    keys, values, q, k, v, cos, sin = attention_case(0, cap, 3)
    dk, dv = keys.to(device), values.to(device)
    for split in (True, False):
        for pos in (cap, cap + 5, -1):
            out = torch.full((576,), 7.0, dtype=torch.float16, device=device)
            position = torch.tensor([pos], dtype=torch.int64, device=device)
            lb.PreparedAttention(q.to(device), k.to(device), v.to(device), cos.to(device), sin.to(device), position,
                                 dk, dv, out, heads=9, kv_heads=3, split=split).run()
            torch.cuda.synchronize()
            assert torch.equal(dk.cpu(), keys) and torch.equal(dv.cpu(), values)
            assert bool(torch.isnan(out.cpu()).all()), (pos, split)


def test_argmax_next_order_position_and_embedding(device):
    announce('argmax next')
    vocab, hidden = 1003, 64
    g = torch.Generator().manual_seed(11)
    emb = torch.randn(vocab, hidden, generator=g).half().to(device)
    logits = torch.randn(vocab, generator=g).half()
    logits[700] = logits[300] = 9.0           # tie: the first index wins (torch.argmax)
    logits[1001] = float('nan')               # never chosen
    assert int(logits[:1001].float().argmax()) == 300
    tokens = torch.full((10,), -1, dtype=torch.int64, device=device)
    token = torch.zeros(1, dtype=torch.int64, device=device)
    position = torch.tensor([5], dtype=torch.int64, device=device)
    h = torch.zeros(hidden, dtype=torch.float16, device=device)
    call = lb.PreparedArgmax(logits.to(device), emb, h, tokens, token, position, limit=10)
    call.run()
    torch.cuda.synchronize()
    assert int(token) == 300 and int(position) == 6 and int(tokens[5]) == 300
    assert torch.equal(h, emb[300])
    position.fill_(10)                        # at the limit: token and h still update, nothing else
    call.run()
    torch.cuda.synchronize()
    assert int(position) == 10 and int((tokens >= 0).sum()) == 1
    ninf = torch.full((vocab,), float('-inf'), dtype=torch.float16, device=device)
    lb.PreparedArgmax(ninf, emb, h, tokens, token, position, limit=10).run()
    torch.cuda.synchronize()
    assert int(token) == 0 and torch.equal(h, emb[0])
