"""GPU parity of lb_head_next (final RMSNorm -> head -> greedy token in one launch) against the
two calls it replaces, lb_fused_linear + lb_argmax_next, and against torch.argmax order on its own
logits.

Where lb_fused_linear runs the same four-tiles-per-workgroup kernel (heads from 32768 rows) the
logits must be equal bit for bit; for shorter heads lb_fused_linear may add a row's K slices in
another order, so there the logits agree within rel-L2 1e-3 and the token is checked against the
logits lb_head_next wrote.  Token, recorded token, position and next embedding are exact.  The
planted cases (equal rows, a NaN row, an infinite logit, nothing but -inf/NaN) follow the
semantics of argmax_next (include/lowbit_decode_hip.h): first index of the largest logit, NaN never
chosen, token 0 when no logit is above -inf.
"""
import ctypes

import pytest
import torch

import lowbit_hip as lb
from conftest import announce
from torch_npu_lowbit import quantize_weight

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


def normed_cpu(h, gamma):
    f = h.float()
    return ((f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half() * gamma).half()


def argmax_cpu(logits):
    """First index of the largest logit; NaN never chosen; 0 when no logit is above -inf."""
    v = logits.float().cpu().clone()
    v[torch.isnan(v)] = float('-inf')
    if not bool((v > float('-inf')).any()):
        return 0
    return int(torch.nonzero(v == v.max())[0])


class Pair:
    """The same head run as lb_head_next and as lb_fused_linear + lb_argmax_next, each on its own
    copies of the state (h, logits, tokens, token, position)."""

    def __init__(self, device, fmt, head_codes, scales, group, embedding, gamma, limit=16):
        vocab, hidden = embedding.shape
        self.vocab, self.hidden, self.embedding = vocab, hidden, embedding
        self.state = {}
        for side in ('next', 'two'):
            st = dict(h=torch.zeros(hidden, dtype=torch.float16, device=device),
                      logits=torch.zeros(vocab, dtype=torch.float16, device=device),
                      tokens=torch.full((limit,), -1, dtype=torch.int64, device=device),
                      token=torch.zeros(1, dtype=torch.int64, device=device),
                      position=torch.zeros(1, dtype=torch.int64, device=device))
            problem = dict(codes=head_codes, scales=scales, N=vocab, y=st['logits'])
            if side == 'next':
                st['call'] = lb.PreparedHeadNext(st['h'], problem, embedding, st['tokens'], st['token'],
                                                 st['position'], format=fmt, K=hidden, group_size=group,
                                                 gamma=gamma, limit=limit)
            else:
                st['calls'] = [lb.PreparedFused(st['h'], [problem], format=fmt, K=hidden, group_size=group,
                                                prologue='rmsnorm', gamma=gamma),
                               lb.PreparedArgmax(st['logits'], embedding, st['h'], st['tokens'], st['token'],
                                                 st['position'], limit=limit)]
            self.state[side] = st

    def set(self, h, position):
        for st in self.state.values():
            st['h'].copy_(h)
            st['position'].fill_(position)

    def run(self):
        self.state['next']['call'].run()
        for call in self.state['two']['calls']:
            call.run()
        torch.cuda.synchronize()

    def counters(self):
        """The whole lb_head_next workspace: maximum words and counters, zero after every call."""
        return self.state['next']['call'].workspace.cpu()


def random_head(device, fmt, vocab, hidden, seed, group=64):
    g = torch.Generator().manual_seed(seed)
    emb = (torch.randn(vocab, hidden, generator=g) * 0.02).half()
    gamma = (1.0 + 0.1 * torch.randn(hidden, generator=g)).half()
    if fmt == 'fp16':
        return emb.to(device), None, hidden, emb.to(device), gamma.to(device), g
    q = quantize_weight(emb.float(), format=fmt, group_size=group)
    codes, scales = q.device_tensors(device)
    return codes, scales, group, emb.to(device), gamma.to(device), g


# (format, vocab, hidden): the config-4 tied head, its INT4 g64 form, a head with a partial last
# group of workgroups and a partial last workgroup, a short head, an INT4 head on the 1536 row.
CASES = [('fp16', 49152, 576), ('int4', 49152, 576), ('fp16', 70001, 576), ('fp16', 1003, 64),
         ('int4', 33000, 1536)]


@pytest.mark.parametrize('fmt,vocab,hidden', CASES)
def test_head_next_matches_head_then_argmax(device, fmt, vocab, hidden):
    announce('head next', fmt, vocab, hidden)
    codes, scales, group, emb, gamma, g = random_head(device, fmt, vocab, hidden, seed=vocab % 97)
    pair = Pair(device, fmt, codes, scales, group, emb, gamma)
    exact = vocab >= 32768
    for step in range(6):
        h = torch.randn(hidden, generator=g).half().to(device)
        pair.set(h, position=step)
        pair.run()
        a, b = pair.state['next'], pair.state['two']
        if exact:
            assert torch.equal(a['logits'], b['logits']), step
        else:
            assert rel_l2(a['logits'], b['logits']) <= 1e-3
        t = argmax_cpu(a['logits'])
        assert int(a['token']) == t
        if exact:
            assert int(b['token']) == t
        assert int(a['position']) == step + 1 and int(a['tokens'][step]) == t
        assert torch.equal(a['h'], emb[t])
        assert bool((pair.counters() == 0).all())
    if exact:
        assert torch.equal(pair.state['next']['tokens'], pair.state['two']['tokens'])


def planted(device, vocab, hidden, rows):
    """An fp16 head whose rows `rows` (dict row -> kind) give chosen logits for a fixed h."""
    g = torch.Generator().manual_seed(7)
    h = torch.randn(hidden, generator=g).half()
    gamma = torch.ones(hidden).half()
    n = normed_cpu(h, gamma).float()
    emb = (torch.randn(vocab, hidden, generator=g) * 0.02).half()
    for r, kind in rows.items():
        if kind == 'big':              # logit about 8: above every random row
            emb[r] = (n * (8.0 / float(n.square().sum()))).half()
        elif kind == 'nan':            # +inf + -inf
            emb[r] = 0
            emb[r, 0] = float('inf') if n[0] > 0 else float('-inf')
            emb[r, 1] = float('-inf') if n[1] > 0 else float('inf')
        elif kind == 'inf':
            emb[r] = 0
            emb[r, 0] = float('inf') if n[0] > 0 else float('-inf')
        elif kind == 'ninf':
            emb[r] = 0
            emb[r, 0] = float('-inf') if n[0] > 0 else float('inf')
    return h.to(device), gamma.to(device), emb.to(device)


@pytest.mark.parametrize('vocab', [4096, 49152])
@pytest.mark.parametrize('kind', ['tie', 'inf', 'nan_only'])
def test_head_next_planted_logits(device, vocab, kind):
    announce('head next planted', kind, vocab)
    hidden = 64
    if kind == 'tie':      # equal largest logits at 300 and vocab - 5: the first wins; a NaN row loses
        rows = {vocab - 5: 'big', 300: 'big', 1001: 'nan'}
        want = 300
    elif kind == 'inf':    # +inf beats every finite logit; the first of two
        rows = {vocab - 70: 'inf', vocab - 3: 'inf', 5: 'big'}
        want = vocab - 70
    else:                  # nothing above -inf (rows of NaN and of -inf): token 0
        rows = {}
        want = 0
    h, gamma, emb = planted(device, vocab, hidden, rows)
    if kind == 'nan_only':
        n = normed_cpu(h.cpu(), gamma.cpu()).float()
        inf = float('inf')
        e = torch.zeros(vocab, hidden, dtype=torch.float16)
        e[:, 0] = inf if n[0] > 0 else -inf
        e[:, 1] = -inf if n[1] > 0 else inf
        e[::3, 1] = 0
        e[::3, 0] = -inf if n[0] > 0 else inf
        emb = e.to(device)
    pair = Pair(device, 'fp16', emb, None, hidden, emb, gamma)
    for step in range(2):
        pair.set(h, position=step)
        pair.run()
        a, b = pair.state['next'], pair.state['two']
        assert argmax_cpu(a['logits']) == want
        assert int(a['token']) == want and int(b['token']) == want
        assert int(a['tokens'][step]) == want and int(a['position']) == step + 1
        assert torch.equal(a['h'], emb[want])
        assert bool((pair.counters() == 0).all())


def test_head_next_position_outside_limit(device):
    """At or past the limit, and at a negative position, only token and h_next change."""
    announce('head next limit')
    codes, scales, group, emb, gamma, g = random_head(device, 'fp16', 4096, 64, seed=3)
    pair = Pair(device, 'fp16', codes, scales, group, emb, gamma, limit=4)
    st = pair.state['next']
    for pos in (4, 9, -1):
        h = torch.randn(64, generator=g).half().to(device)
        pair.set(h, position=pos)
        pair.run()
        t = argmax_cpu(st['logits'])
        assert int(st['token']) == t and int(st['position']) == pos
        assert bool((st['tokens'] == -1).all())
        assert torch.equal(st['h'], emb[t])


def test_head_next_graph_replays(device):
    """lb_head_next captured in a HIP graph: every replay (with eager work and synchronisations
    between them) equals the eager two-call result for its input, and the counters stay zero."""
    announce('head next graph')
    codes, scales, group, emb, gamma, g = random_head(device, 'fp16', 49152, 576, seed=13)
    pair = Pair(device, 'fp16', codes, scales, group, emb, gamma)
    a, b = pair.state['next'], pair.state['two']
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        a['call'].run()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        a['call'].run()
    for step in range(5):
        h = torch.randn(576, generator=g).half().to(device)
        pair.set(h, position=step)
        graph.replay()
        for call in b['calls']:
            call.run()
        torch.cuda.synchronize()
        assert torch.equal(a['logits'], b['logits']), step
        assert int(a['token']) == int(b['token']) and int(a['position']) == step + 1
        assert torch.equal(a['h'], b['h'])
        assert bool((pair.counters() == 0).all())


def test_head_next_decoder_equals_two_call_decoder(device):
    """A 4-layer graph decoder with lb_head_next gives the same tokens and bit-identical logits
    at every step as the same decoder with lb_fused_linear + lb_argmax_next."""
    announce('head next decoder')
    import smollm_random
    from torch_npu_smollm import GraphDecoder
    stack, io, _, _ = smollm_random.build(seed=25, layers=4, rank=32, theta=10000.0, capacity=96,
                                          std=0.05, qk_std=0.02, embed_std=0.05)
    io = io.to(device)
    ids = smollm_random.prompt(seed=25, length=40)
    runs = []
    for head_next in (True, False):
        h, caches = stack.prefill(io.embed_tokens(ids.to(device)))
        first = int(io.logits(h[:, -1:])[0, 0].float().argmax())
        decoder = GraphDecoder(stack, io, head_next=head_next)
        assert (decoder.head_next is not None) == head_next
        decoder.load(caches, first)
        tokens, logits = [], []
        for _ in range(12):
            tokens += decoder.generate(1)
            logits.append(decoder.logits.view(-1).clone())
        assert decoder.timeouts() == 0
        runs.append((tokens, torch.stack(logits)))
    assert runs[0][0] == runs[1][0]
    assert len(set(runs[0][0])) >= 3
    assert torch.equal(runs[0][1], runs[1][1])
