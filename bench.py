"""Benchmark of the MI355X low-bit linear path (one JSON line on stdout).

Headline workload: INT4 group-wise dequant-GEMV at M=1 over
every SmolLM-135M linear shape -- q/o 576x576, k/v 192x576, gate/up 1536x576,
down 576x1536, lm_head 49152x576.  The reference requires K % group == 0, so K=576
shapes use group 64 and K=1536 uses group 128.  One step = one pass over the eight
linears, each reading a distinct weight replica from a pool larger than the 256 MB
MALL, so the bandwidth is HBM bandwidth.  The pass is issued as the SmolLM decode step
issues it: q|k|v and gate|up share their input row and run as one grouped launch each,
o, down and lm_head as one launch each (5 launches).  Launches are replayed from HIP
graphs so host launch cost is not in the timed region; inputs are resident in HBM.

Also reported: the pass with one launch per shape (8 launches), at M=4 and M=16,
per-launch GB/s, config 1 (W8 per-row 1536x576 + rank-32 correction at M=1), the config-5
roofline sweep (INT4 at M = 1, 8, 32 and W8 per-row at M = 1), prefill GEMM TFLOP/s on the
config-3 and config-5 cells with hipBLASLt fp16 (no dequantization) beside the M = 512 cells, the
config-4 decode leg, and the CPU baseline (the reference's CPU path: fp32 torch matmul on
pre-dequantized weights) timed on this host.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 32] [--quick] [--no-cpu]
       python bench.py --profile-kernel   (dominant kernel + a copy kernel, for rocprofv3 --pmc)
       python bench.py --decode-only      (config-4 decode leg alone, for rocprofv3 --kernel-trace)
       python bench.py --profile-gemm     (prefill GEMMs + hipBLASLt fp16 of the same shapes, for --pmc)
       python bench.py --profile-llama 14336x4096  (one config-5 INT4 GEMV at M=1 + a copy, for rocprofv3)
       python bench.py --profile-multirow (multi-row GEMVs and a split-K GEMM, for rocprofv3 --kernel-trace)
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / 'torch-intel-npu_amd'):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = 'dequant-GEMV HBM GB/s (% of peak) at M=1; decode tokens/sec SmolLM-135M W8'
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
POOL_BYTES = 1.1 * 2 ** 30

# (name, N, K, group) -- config 2 shapes with the group substitution for K=576.
SMOL_SHAPES = [('q_proj', 576, 576, 64), ('k_proj', 192, 576, 64), ('v_proj', 192, 576, 64),
               ('o_proj', 576, 576, 64), ('gate_proj', 1536, 576, 64), ('up_proj', 1536, 576, 64),
               ('down_proj', 576, 1536, 128), ('lm_head', 49152, 576, 64)]
LLAMA_SHAPES = [('4096x4096', 4096, 4096, 128), ('1024x4096', 1024, 4096, 128),
                ('14336x4096', 14336, 4096, 128), ('4096x14336', 4096, 14336, 128),
                ('128256x4096', 128256, 4096, 128)]


def log(*parts):
    print('[bench]', *parts, file=sys.stderr, flush=True)


def algorithmic_bytes(fmt, m, n, k, group):
    code = n * k if fmt == 'int8' else n * k // 2
    return code + 2 * n * (k // group) + 2 * m * k + 2 * m * n + (32 if fmt == 'nf4' else 0)


def make_weight(fmt, n, k, group, seed):
    from torch_npu_lowbit import quantize_weight
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    return quantize_weight(w, format=fmt, group_size=group)


class Linear:
    """A packed weight replicated `copies` times on the device, plus fixed x / y buffers."""

    def __init__(self, packed, m, copies, device, seed):
        import lowbit_hip
        self.packed = packed
        self.fmt = packed.format
        self.n, self.k = packed.shape
        self.group = packed.group_size
        self.m = m
        codes, scales = packed.device_tensors(device)
        self.replicas = [(codes.clone(), scales.clone()) for _ in range(copies)]
        g = torch.Generator().manual_seed(seed)
        self.x = torch.randn(m, self.k, generator=g).half().to(device)
        self.y = torch.empty(m, self.n, dtype=torch.float16, device=device)
        self.calls = [lowbit_hip.PreparedLinear(self.x, c, s, format=self.fmt, N=self.n, K=self.k,
                                                group_size=self.group, out=self.y) for c, s in self.replicas]
        self.bytes = algorithmic_bytes(self.fmt, m, self.n, self.k, self.group)
        self.flops = 2 * m * self.n * self.k


def copies_for(bytes_per_copy, cap=64):
    return int(max(2, min(cap, np.ceil(POOL_BYTES / bytes_per_copy))))


def capture(fns, stream):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for fn in fns:
            fn()
    return graph


def time_graphs(graphs, count, stream):
    """Replay graphs[i % len] for i < count between two events on `stream`; returns ms."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for i in range(count):
            graphs[i % len(graphs)].replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


PASSES_PER_GRAPH = 16


def time_passes(pass_fns, copies, steps, warmup, stream):
    """Time exactly `steps` passes (ms).  Passes are recorded PASSES_PER_GRAPH to a graph (pass t of
    graph i reads replica (i * PASSES_PER_GRAPH + t) mod copies), so one graph launch is shared by
    several passes, as in a decode loop captured whole; a remainder uses one-pass graphs."""
    per = PASSES_PER_GRAPH
    full = [capture([fn for t in range(per) for fn in pass_fns(i * per + t)], stream)
            for i in range((copies + per - 1) // per)]
    single = [capture(pass_fns(r), stream) for r in range(min(copies, steps % per))]
    time_graphs(full, max(1, warmup // per), stream)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for i in range(steps // per):
            full[i % len(full)].replay()
        for i in range(steps % per):
            single[i % len(single)].replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


def kernel_time_us(linear, stream, replays=8):
    """Average duration of one launch of `linear`, over a graph of all its replicas."""
    for call in linear.calls[:2]:
        call.run()
    graph = capture([c.run for c in linear.calls], stream)
    time_graphs([graph], 2, stream)
    ms = time_graphs([graph], replays, stream)
    return 1000.0 * ms / (replays * len(linear.calls))


# Launch groups of the decode step: projections that read the same activation row run as one
# lb_fused_linear launch (q|k|v, gate|up), exactly as the SmolLM decode step issues them.
DECODE_GROUPS = [('qkv', ('q_proj', 'k_proj', 'v_proj')), ('o_proj', ('o_proj',)), ('gate_up', ('gate_proj', 'up_proj')),
                 ('down_proj', ('down_proj',)), ('lm_head', ('lm_head',))]


class Group:
    """Replicated weights of projections sharing one input row, run as one fused launch per replica."""

    def __init__(self, linears, device):
        import lowbit_hip
        self.linears = linears
        self.bytes = sum(lin.bytes for lin in linears) - 2 * linears[0].k * (len(linears) - 1)  # x read once
        first = linears[0]
        x = first.x.view(-1)
        self.ys = [torch.empty(lin.n, dtype=torch.float16, device=device) for lin in linears]
        self.calls = []
        for r in range(len(first.replicas)):
            problems = [dict(codes=lin.replicas[r][0], scales=lin.replicas[r][1], N=lin.n, y=y)
                        for lin, y in zip(linears, self.ys)]
            self.calls.append(lowbit_hip.PreparedFused(x, problems, format=first.fmt, K=first.k,
                                                       group_size=first.group))


def smol_pass(m, device, stream, steps, warmup, grouped=False, group=None):
    """One pass over the eight config-2 linears: per shape (8 launches) or, for M=1, in the decode
    step's launch groups (5 launches).  `group` replaces every shape's group size (32: the SmolLM
    default the survey's config-2 row also asks for)."""
    linears = []
    shapes = [(name, n, k, group or g) for name, n, k, g in SMOL_SHAPES]
    total = sum(algorithmic_bytes('int4', m, n, k, g) for _, n, k, g in shapes)
    copies = copies_for(total)
    for i, (name, n, k, g) in enumerate(shapes):
        linears.append(Linear(make_weight('int4', n, k, g, 100 + i), m, copies, device, 200 + i))
    by_name = {name: lin for (name, *_), lin in zip(shapes, linears)}
    if grouped:
        units = [(label, Group([by_name[n] for n in names], device) if len(names) > 1 else by_name[names[0]])
                 for label, names in DECODE_GROUPS]
        total = sum(u.bytes for _, u in units)
    else:
        units = [(name, lin) for (name, *_), lin in zip(shapes, linears)]
    for _, unit in units:
        unit.calls[0].run()
    ms = time_passes(lambda r: [unit.calls[r % copies].run for _, unit in units], copies, steps, warmup, stream)
    per_kernel = {}
    for name, unit in units:
        us = kernel_time_us(unit, stream)
        per_kernel[name] = dict(us=round(us, 3), gbs=round(unit.bytes / us / 1e3, 1))
    return dict(ms_per_step=ms / steps, bytes_per_step=total, copies=copies, launches=len(units),
                gbs=total / (ms / steps) / 1e6, per_kernel=per_kernel, linears=linears)


# Config 3 (NF4 g64, SmolLM-360M MLP) and config 5 (INT4 g128, Llama-3-8B) prefill cells, plus the
# Llama gate/up shape at M = 512 where the M=512 MFMA target is quoted.
GEMM_SPECS = ([('nf4', m, n, k, 64, name) for m in (128, 512, 2048)
               for name, n, k in (('smol360m_gate', 2560, 960), ('smol360m_down', 960, 2560))]
              + [('int4', m, n, k, g, name) for m in (256, 1024) for name, n, k, g in LLAMA_SHAPES]
              + [('int4', 512, 14336, 4096, 128, '14336x4096'), ('nf4', 512, 14336, 4096, 128, '14336x4096'),
                 ('int8', 256, 576, 576, 576, 'smol135m_q_prefill')])
# The cells the reference publishes (1024 x 1024; NPU times in ms, context only: its calls are bound by
# one synchronous graph submission each), as (fmt, M, N, K, group, name, reference ms, source).
REF_SPECS = [
    ('int4', 1, 1024, 1024, 1024, 'ref_1024sq_per_channel', 0.530, 'research/results/lowbit/REPORT.md:56'),
    ('nf4', 1, 1024, 1024, 1024, 'ref_1024sq_per_channel', 0.428, 'research/results/lowbit/REPORT.md:56'),
    ('int4', 1, 1024, 1024, 128, 'ref_1024sq_g128', 0.369, 'research/results/lowbit-group/REPORT.md:54'),
    ('nf4', 1, 1024, 1024, 128, 'ref_1024sq_g128', 0.349, 'research/results/lowbit-group/REPORT.md:57'),
    ('int4', 128, 1024, 1024, 1024, 'ref_1024sq_per_channel', None, 'research/results/lowbit/REPORT.md:58 (CPU only)'),
    ('nf4', 128, 1024, 1024, 1024, 'ref_1024sq_per_channel', None, 'research/results/lowbit/REPORT.md:58 (CPU only)'),
    ('int4', 128, 1024, 1024, 128, 'ref_1024sq_g128', 0.547, 'research/results/lowbit-group/REPORT.md:55'),
    ('nf4', 128, 1024, 1024, 128, 'ref_1024sq_g128', 0.485, 'research/results/lowbit-group/REPORT.md:58'),
    ('int8', 1, 1024, 1024, 1024, 'ref_w8a16_1024sq', 0.2119, 'research/results/throughput-20261005/REPORT.md:24'),
    ('int8', 512, 1024, 1024, 1024, 'ref_w8a16_1024sq', 0.4436, 'research/results/throughput-20261005/REPORT.md:27'),
    ('int8', 1024, 1024, 1024, 1024, 'ref_w8a16_1024sq', 0.6308, 'research/results/throughput-20261005/REPORT.md:28'),
]
# hipBLASLt fp16 (torch.matmul, no dequantization) on the M = 512 cells: the vendor rate on these shapes.
VENDOR_SPECS = [(512, 2560, 960, 'smol360m_gate'), (512, 960, 2560, 'smol360m_down'),
                (512, 14336, 4096, '14336x4096'), (1024, 14336, 4096, '14336x4096')]


def sweep_row(lin, stream, fmt, m, n, k, g, name):
    us = float(np.median([kernel_time_us(lin, stream, replays=4) for _ in range(3)]))  # median of 3 timed graphs
    row = dict(fmt=fmt, M=m, N=n, K=k, group=g, shape=name, us=round(us, 2),
               gbs=round(lin.bytes / us / 1e3, 1), tflops=round(lin.flops / us / 1e6, 2))
    row['hbm_frac' if m <= 32 else 'mfma_frac'] = round(
        row['gbs'] / HBM_PEAK_GBS if m <= 32 else row['tflops'] / FP16_MFMA_PEAK_TFLOPS, 4)
    log('sweep', json.dumps(row))
    return row


def sweep(device, stream, quick):
    """Config-5 GEMVs (INT4 and NF4 at M = 1, 8, 32; W8 per-row at M = 1), the prefill cells of configs 3
    and 5, the 1024 x 1024 cells the reference publishes (with its NPU time beside ours), and hipBLASLt
    fp16 on the M = 512 cells.  One packed weight per (format, shape) serves every M."""
    specs = [('int4', m, n, k, g, name) for m in ((1, 32) if quick else (1, 8, 32)) for name, n, k, g in LLAMA_SHAPES]
    specs += [('int8', 1, n, k, k, name) for name, n, k, _ in LLAMA_SHAPES]
    if not quick:
        specs += [('nf4', m, n, k, g, name) for m in (1, 8, 32) for name, n, k, g in LLAMA_SHAPES]
    specs += GEMM_SPECS[:4] if quick else GEMM_SPECS
    reference = {}
    for fmt, m, n, k, g, name, ms, src in ([] if quick else REF_SPECS):
        reference[len(specs)] = dict(reference_npu_ms=ms, reference_source='/root/reference/npunlock-probe/' + src)
        specs.append((fmt, m, n, k, g, name))
    order = sorted(range(len(specs)), key=lambda i: (specs[i][0], specs[i][2], specs[i][3]))
    rows, packed = [None] * len(specs), {}
    for i in order:
        fmt, m, n, k, g, name = specs[i]
        key = (fmt, n, k, g)
        if key not in packed:
            packed.clear()
            torch.cuda.empty_cache()
            packed[key] = make_weight(fmt, n, k, g, 300 + len(rows) + i)
        bytes_w = algorithmic_bytes(fmt, 0, n, k, g)
        lin = Linear(packed[key], m, copies_for(bytes_w, cap=32), device, 400 + i)
        rows[i] = sweep_row(lin, stream, fmt, m, n, k, g, name)
        if i in reference:
            rows[i].update(reference[i])
            if reference[i]['reference_npu_ms']:
                rows[i]['speedup_vs_reference_npu'] = round(1e3 * reference[i]['reference_npu_ms'] / rows[i]['us'], 1)
        del lin
        torch.cuda.empty_cache()
    for m, n, k, name in ([] if quick else VENDOR_SPECS):
        a = torch.randn(m, k, device=device, dtype=torch.float16)
        b = [torch.randn(n, k, device=device, dtype=torch.float16) for _ in range(copies_for(2 * n * k, cap=16))]
        for w in b[:2]:
            torch.matmul(a, w.t())
        graph = capture([lambda w=w: torch.matmul(a, w.t()) for w in b], stream)
        time_graphs([graph], 2, stream)
        us = float(np.median([1000.0 * time_graphs([graph], 4, stream) / (4 * len(b)) for _ in range(3)]))
        row = dict(fmt='fp16 hipBLASLt (torch.matmul, no dequantization)', M=m, N=n, K=k, shape=name,
                   us=round(us, 2), tflops=round(2 * m * n * k / us / 1e6, 2))
        row['mfma_frac'] = round(row['tflops'] / FP16_MFMA_PEAK_TFLOPS, 4)
        log('sweep', json.dumps(row))
        rows.append(row)
        del a, b, graph
        torch.cuda.empty_cache()
    return rows


def config1_leg(device, stream):
    """Config 1: W8A16 576->1536 + rank-32 correction at M=1, seed 0.
    Draw order W [1536,576]*0.02 fp32, x [1,576] fp16, U [1536,32]*0.01 fp16, V [32,576]*0.01 fp16;
    y = x.(q*s)^T + fp16(fp16(x.V^T).U^T) through one lb_linear (the fused one-row kernel)."""
    import lowbit_hip
    from torch_npu_lowbit import quantize_weight
    g = torch.Generator().manual_seed(0)
    w = torch.randn(1536, 576, generator=g) * 0.02
    x = torch.randn(1, 576, generator=g).half().to(device)
    up = (torch.randn(1536, 32, generator=g) * 0.01).half()
    down = (torch.randn(32, 576, generator=g) * 0.01).half()
    packed = quantize_weight(w, format='int8')
    n, k, r = 1536, 576, 32
    total = algorithmic_bytes('int8', 1, n, k, k) + 2 * r * (n + k)
    copies = copies_for(total)
    codes, scales = packed.device_tensors(device)
    reps = [(codes.clone(), scales.clone(), down.to(device), up.to(device)) for _ in range(copies)]
    y = torch.empty(1, n, dtype=torch.float16, device=device)
    calls = [lowbit_hip.PreparedLinear(x, c, s, format='int8', N=n, K=k, group_size=k, out=y, down=d, up=u, rank=r)
             for c, s, d, u in reps]
    unit = type('Unit', (), {})()
    unit.calls = calls
    for call in calls[:2]:
        call.run()
    us = float(np.median([kernel_time_us(unit, stream, replays=8) for _ in range(3)]))
    row = dict(shape='gate_proj 1536x576', fmt='int8 per-row + rank-32 correction', M=1, us=round(us, 3),
               algorithmic_bytes=total, gbs=round(total / us / 1e3, 1), replicas=copies)
    row['hbm_frac'] = round(row['gbs'] / HBM_PEAK_GBS, 4)
    log('config1', json.dumps(row))
    return row


def cpu_leg(budget_s):
    from oracle import cpu_baseline
    problems = []
    for i, (name, n, k, g) in enumerate(SMOL_SHAPES):
        packed = make_weight('int4', n, k, g, 100 + i)
        x = torch.randn(1, k, generator=torch.Generator().manual_seed(200 + i)).half().numpy()
        problems.append((x, 'int4', (n, k), g, packed.data, packed.scales))
    cpu = cpu_baseline.CpuPass(problems)
    pre, deq, rounds = cpu_baseline.time_pass(cpu, budget_s=budget_s)
    total = sum(algorithmic_bytes('int4', 1, n, k, g) for _, n, k, g in SMOL_SHAPES)
    return dict(value=round(total / pre / 1e9, 3), unit='GB/s', cores=cpu.threads, kind='port',
                sample=(f'{rounds} interleaved rounds (median) of one M=1 pass over the 8 SmolLM-135M '
                        f'INT4 shapes: fp32 torch CPU matmul on pre-dequantized weights, fp16 out '
                        f'(reference timing method, torch_npu_lowbit_demo.py:65,71); the dequant-inclusive '
                        f'variant adds the fp16 PackedWeight.dequantize() per call; host {cpu_baseline.cpu_model()}'),
                ms_per_pass=round(pre * 1e3, 3), dequant_inclusive_ms_per_pass=round(deq * 1e3, 3),
                dequant_inclusive_gbs=round(total / deq / 1e9, 3))


DECODE_TOKENS_PER_GRAPH = 8


def decode_leg(device, steps, cpu_steps):
    """Config 4: 30-layer random-init SmolLM-135M, W8 per-row + rank-32 corrections, theta 1e4,
    256-token prompt, then greedy decode with the fp16 KV cache (GraphDecoder replays)."""
    import smollm_random
    from torch_npu_smollm import GraphDecoder
    stack, io, _, _ = smollm_random.build(seed=0, layers=30, rank=32, theta=10000.0, capacity=384)
    io = io.to(device)
    ids = smollm_random.prompt(seed=0, length=256).to(device)
    out = {}
    with torch.no_grad():
        for _ in range(2):  # warm (device copies of weights, allocator)
            h, caches = stack.prefill(io.embed_tokens(ids))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        h, caches = stack.prefill(io.embed_tokens(ids))
        first = int(io.logits(h[:, -1:])[0, 0].float().argmax())
        out['prefill_ms'] = round((time.perf_counter() - t0) * 1e3, 3)
        out['prefill_tokens_per_s'] = round(256 / (time.perf_counter() - t0), 1)
        # eager decode (one Python-driven step per token)
        x = io.embed_tokens(torch.tensor([[first]], device=device))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eager_caches = caches
        for _ in range(8):
            h2, eager_caches = stack.decode(x, eager_caches)
            x = io.embed_tokens(io.logits(h2)[0, 0].float().argmax().view(1, 1))
        torch.cuda.synchronize()
        out['eager_decode_tokens_per_s'] = round(8 / (time.perf_counter() - t0), 1)
        decoder = GraphDecoder(stack, io)
        decoder.load(caches, first)
        per_graph = DECODE_TOKENS_PER_GRAPH if steps % DECODE_TOKENS_PER_GRAPH == 0 else 1
        decoder.capture(tokens=per_graph)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps // per_graph):
            decoder.graph.replay()
        stop.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(stop)
        # A hand-over wait that gave up ends its launch early with stale words: such a run's time
        # is not a decode rate, so it is reported as the failure it is, without tokens/s.
        timeouts = decoder.timeouts()
        out.update(decode_steps=steps, tokens_per_graph=per_graph, decode_timeouts=timeouts,
                   first_tokens=decoder.tokens[256:256 + 8].tolist())
        if timeouts:
            out['decode_error'] = f'{timeouts} hand-over wait(s) timed out: tokens/s not reported'
        else:
            out.update(decode_ms_per_token=round(ms / steps, 4), decode_tokens_per_s=round(steps * 1000.0 / ms, 1))
    if cpu_steps:
        from oracle import smollm_oracle as so
        packed = lambda l: {n: (q.format, q.shape, q.group_size, q.data, q.scales) for n, q in l._packed.items()}
        layers = [so.OracleLayer(l._weights, packed(l), {n: c.tensors() for n, c in l._corrections.items()},
                                 theta=10000.0, capacity=384) for l in stack.layers]
        model = so.OracleModel(layers, io.embedding.cpu(), io.norm.cpu())
        t0 = time.perf_counter()
        x, kv = model.prefill(ids.cpu())
        prefill_s = time.perf_counter() - t0
        h = model.embed(torch.tensor([[first]]))
        t0 = time.perf_counter()
        pos = 256
        for _ in range(cpu_steps):
            new = []
            for layer, (k, v) in zip(model.layers, kv):
                h, k, v = layer.decode(h, k, v, pos)
                new.append((k, v))
            kv, pos = new, pos + 1
            h = model.embed(model.logits(h)[:, 0].float().argmax(-1).view(1, 1))
        dt = time.perf_counter() - t0
        out['cpu_baseline'] = dict(decode_tokens_per_s=round(cpu_steps / dt, 2), prefill_s=round(prefill_s, 2),
                                   cores=torch.get_num_threads(), kind='port',
                                   sample=f'oracle staged decoder on the host: 256-token prefill + {cpu_steps} greedy steps')
    return out


def profile_kernel(device, stream, shape=None):
    """One M=1 INT4 GEMV over its replica pool (default: the dominant kernel, the config-2 lm_head),
    then a known-size copy (the PMC calibration kernel)."""
    name, n, k, g = shape or SMOL_SHAPES[-1]
    lin = Linear(make_weight('int4', n, k, g, 107), 1, copies_for(algorithmic_bytes('int4', 0, n, k, g)),
                 device, 207)
    for _ in range(4):
        for call in lin.calls:
            call.run()
    src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps(dict(profile=f'{name} {n}x{k} int4 g{g} M=1', launches=4 * len(lin.calls),
                          algorithmic_bytes=lin.bytes, copy_bytes=src.numel())), flush=True)


GEMM_PROFILE_SHAPES = [('int4', 1024, 14336, 4096, 128), ('nf4', 512, 2560, 960, 64), ('int4', 512, 14336, 4096, 128)]


def profile_gemm(device, stream):
    """Prefill GEMMs alone (configs 5 and 3), 20 launches each, then hipBLASLt fp16 matmuls of the
    same shapes (torch.matmul) as the reference rate; for rocprofv3 --pmc (MFMA busy cycles)."""
    for i, (fmt, m, n, k, g) in enumerate(GEMM_PROFILE_SHAPES):
        lin = Linear(make_weight(fmt, n, k, g, 500 + i), m, 2, device, 600 + i)
        for _ in range(10):
            for call in lin.calls:
                call.run()
        torch.cuda.synchronize()
        a = torch.randn(m, k, device=device, dtype=torch.float16)
        b = torch.randn(n, k, device=device, dtype=torch.float16)
        for _ in range(20):
            torch.matmul(a, b.t())
        torch.cuda.synchronize()
        print(json.dumps(dict(profile='gemm', fmt=fmt, M=m, N=n, K=k, group=g, launches=20,
                              flops_per_launch=2 * m * n * k)), flush=True)


def profile_linears(device, specs, launches=16):
    """Each `fmt:M:N:K:group` spec (group 0: per row) alone on its default dispatch, `launches`
    launches over its replica pool, then a 256 MiB copy (the PMC calibration kernel); for
    rocprofv3 --kernel-trace and --pmc FETCH_SIZE / WRITE_SIZE."""
    for i, spec in enumerate(specs):
        fmt, m, n, k, g = spec.split(':')
        m, n, k, g = int(m), int(n), int(k), int(g)
        g = g or k
        wb = algorithmic_bytes(fmt, 0, n, k, g)
        lin = Linear(make_weight(fmt, n, k, g, 900 + i), m, copies_for(wb, cap=16), device, 950 + i)
        for r in range(launches):
            lin.calls[r % len(lin.calls)].run()
        torch.cuda.synchronize()
        print(json.dumps(dict(profile='linear', fmt=fmt, M=m, N=n, K=k, group=g, launches=launches,
                              algorithmic_bytes=lin.bytes, flops_per_launch=2 * m * n * k)), flush=True)
        del lin
        torch.cuda.empty_cache()
    src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps(dict(profile='copy', copy_bytes=src.numel(), launches=4)), flush=True)


MULTIROW_PROFILE_SHAPES = [('int4', 8, 4096, 4096, 128), ('int4', 16, 128256, 4096, 128),
                           ('int4', 32, 128256, 4096, 128), ('nf4', 512, 960, 2560, 64)]


def profile_multirow(device, stream):
    """The multi-row GEMV paths and a split-K prefill GEMM on their default dispatch, 16 launches
    each over the replica pool (for rocprofv3 --kernel-trace): one-tile rows (config 5 at M=8),
    streaming rows (M=16), K-outer streaming rows (M=32), split-K NF4 down projection (M=512)."""
    for i, (fmt, m, n, k, g) in enumerate(MULTIROW_PROFILE_SHAPES):
        wb = algorithmic_bytes(fmt, 0, n, k, g)
        lin = Linear(make_weight(fmt, n, k, g, 700 + i), m, copies_for(wb, cap=16), device, 800 + i)
        for r in range(16):
            lin.calls[r % len(lin.calls)].run()
        torch.cuda.synchronize()
        print(json.dumps(dict(profile='multirow', fmt=fmt, M=m, N=n, K=k, group=g, launches=16,
                              algorithmic_bytes=lin.bytes, flops_per_launch=2 * m * n * k)), flush=True)
        del lin
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=256)
    ap.add_argument('--warmup', type=int, default=32)
    ap.add_argument('--quick', action='store_true', help='shorter sweep')
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--no-sweep', action='store_true')
    ap.add_argument('--cpu-seconds', type=float, default=15.0)
    ap.add_argument('--profile-kernel', action='store_true')
    ap.add_argument('--no-decode', action='store_true')
    ap.add_argument('--decode-steps', type=int, default=128)
    ap.add_argument('--decode-only', action='store_true', help='only the config-4 decode leg (for tracing)')
    ap.add_argument('--profile-gemm', action='store_true', help='prefill GEMMs alone (for rocprofv3 --pmc)')
    ap.add_argument('--profile-multirow', action='store_true',
                    help='multi-row GEMV paths and a split-K prefill GEMM alone (for rocprofv3 --kernel-trace)')
    ap.add_argument('--profile-pass', action='store_true',
                    help='only the config-2 M=1 pass in its decode launch groups (for rocprofv3 --kernel-trace)')
    ap.add_argument('--profile-linear', nargs='+', metavar='FMT:M:N:K:GROUP',
                    help='these linears alone on their default dispatch (group 0: per row), then a copy, '
                         'for rocprofv3')
    ap.add_argument('--profile-llama', choices=[s[0] for s in LLAMA_SHAPES],
                    help='one config-5 INT4 g128 GEMV at M=1 (its default kernel) alone, then a copy, for rocprofv3')
    args = ap.parse_args()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(json.dumps(dict(error='single-GPU build: the low-bit linear path is measured on one MI355X; '
                                    'sharding it over several GPUs is designed but not built', n_gpus=args.gpus)))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps(dict(error='no ROCm device visible')))
        sys.exit(1)
    import lowbit_hip
    lowbit_hip.library()
    device = torch.device('cuda:0')
    stream = torch.cuda.Stream(device)
    torch.manual_seed(0)
    if args.profile_kernel:
        profile_kernel(device, stream)
        return
    if args.profile_gemm:
        profile_gemm(device, stream)
        return
    if args.profile_llama:
        profile_kernel(device, stream, next(s for s in LLAMA_SHAPES if s[0] == args.profile_llama))
        return
    if args.profile_linear:
        profile_linears(device, args.profile_linear)
        return
    if args.profile_multirow:
        profile_multirow(device, stream)
        return
    if args.profile_pass:
        one = smol_pass(1, device, stream, args.steps, args.warmup, grouped=True)
        del one['linears']
        print(json.dumps(dict(config2_pass_m1=one)), flush=True)
        return
    if args.decode_only:
        decode = decode_leg(device, args.decode_steps, 0)
        print(json.dumps(dict(decode_smollm135m_w8_rank32=decode)), flush=True)
        return

    t0 = time.time()
    log('config-2 pass, M=1 (decode launch groups)')
    head = smol_pass(1, device, stream, args.steps, args.warmup, grouped=True)
    log(f"M=1: {head['gbs']:.1f} GB/s per pass, {head['ms_per_step'] * 1e3:.2f} us/step")
    dominant = head['per_kernel']['lm_head']
    lm = head['linears'][-1]
    del head['linears']
    torch.cuda.empty_cache()
    log('config-2 pass, M=1 (one launch per shape)')
    flat = smol_pass(1, device, stream, max(32, args.steps // 4), 8)
    del flat['linears']
    others = {'M=1 per shape': dict(gbs=round(flat['gbs'], 1), us_per_step=round(flat['ms_per_step'] * 1e3, 2),
                                    launches=flat['launches'], per_kernel=flat['per_kernel'])}
    torch.cuda.empty_cache()
    log('config-2 pass, M=1, group 32 (decode launch groups)')
    g32 = smol_pass(1, device, stream, max(32, args.steps // 4), 8, grouped=True, group=32)
    del g32['linears']
    others['M=1 g32'] = dict(gbs=round(g32['gbs'], 1), us_per_step=round(g32['ms_per_step'] * 1e3, 2),
                             launches=g32['launches'], per_kernel=g32['per_kernel'])
    torch.cuda.empty_cache()
    for m in (4, 16):
        log(f'config-2 pass, M={m}')
        r = smol_pass(m, device, stream, max(32, args.steps // 4), 8)
        del r['linears']
        others[f'M={m}'] = dict(gbs=round(r['gbs'], 1), us_per_step=round(r['ms_per_step'] * 1e3, 2),
                                per_kernel=r['per_kernel'])
        torch.cuda.empty_cache()
    config1 = config1_leg(device, stream)
    rows = [] if args.no_sweep else sweep(device, stream, args.quick)
    cpu = None if args.no_cpu else cpu_leg(args.cpu_seconds)
    decode = None
    if not args.no_decode:
        log('config-4 decode')
        decode = decode_leg(device, args.decode_steps, 0 if args.no_cpu else 6)
        log('decode', json.dumps(decode))
    achieved = lm.bytes / dominant['us'] / 1e3
    result = {
        'metric': METRIC,
        'value': round(head['gbs'], 1),
        'unit': 'GB/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(head['ms_per_step'], 5),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'int4 codes -> fp16 weights, fp32 accumulate',
        'data': 'synthetic: seeded N(0,0.02) weights quantized by quantize_weight, N(0,1) fp16 activations',
        'config': {
            'workload': 'configs[1]: INT4 group-wise dequant-GEMV, M=1, all SmolLM-135M linear shapes '
                        '(q,k,v,o 576/192x576 g64; gate,up 1536x576 g64; down 576x1536 g128; lm_head 49152x576 g64)',
            'step': ('one pass over the 8 linears in the decode step\'s 5 launches (q|k|v and gate|up share their '
                     'input row and run as one lb_fused_linear each; o, down, lm_head one lb_linear each), '
                     'replayed from a HIP graph'),
            'weight_pool_bytes': int(head['bytes_per_step'] * head['copies']),
            'replicas': head['copies'],
            'hbm_frac_of_pass': round(head['gbs'] / HBM_PEAK_GBS, 4),
        },
        'roofline': {
            'kernel': 'pack_gemv_kernel<INT4, scaled, 4 loads per wave> (one-row lb_linear, 3 rows per '
                      'wave-wide load) lm_head 49152x576 g64, M=1',
            'profile': 'profiles/pack_gemv_int4_lm_head_49152x576_m1.md',
            'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
            'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': traffic_per_launch(),
            'algorithmic_bytes_per_launch': lm.bytes, 'avg_launch_us': dominant['us'],
        },
        'cpu_baseline': cpu,
        'config1_w8_rank32_m1': config1,
        'per_launch_M1': head['per_kernel'],
        'decode_smollm135m_w8_rank32': decode,
        'passes': others,
        'sweep': rows,
        'wall_s': round(time.time() - t0, 1),
    }
    print(json.dumps(result), flush=True)


def traffic_per_launch():
    """HBM bytes per dominant-kernel launch from the committed rocprofv3 --pmc summary, if any."""
    path = ROOT / 'profiles' / 'traffic_lm_head_int4_m1.json'
    if path.exists():
        try:
            return json.loads(path.read_text()).get('traffic_bytes_per_launch')
        except (OSError, ValueError):
            return None
    return None


if __name__ == '__main__':
    main()
