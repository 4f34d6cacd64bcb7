"""CPU baseline of the low-bit linear path -- TEST/BENCH INFRASTRUCTURE ONLY.

Times the reference's CPU path as the reference timed its CPU column
(torch_npu_lowbit_demo.py:65,71): fp32 torch CPU matmul on pre-dequantized weights,
fp16 output.  A dequant-inclusive variant adds the reference's host dequantization per call:
the package's PackedWeight.dequantize(), the numpy fp16 restatement of reference
torch_npu_lowbit.py:67-75 (fp16 codes times fp16 scales, one fp16 rounding).  Protocol (demo :62-71): warmups, then the median
of interleaved A/B rounds.
"""
import os
import statistics
import time

import numpy as np
import torch

from oracle import lowbit_oracle as o


class CpuPass:
    """One pass of linears [(x fp16 [M,K], fmt, (N,K), group, data, scales)] on the host CPU."""

    def __init__(self, problems, threads=None):
        self.threads = threads or os.cpu_count()
        torch.set_num_threads(self.threads)
        self.problems = problems
        self.weights = [torch.from_numpy(o.dequantize(fmt, shape, g, data, scales).astype(np.float32))
                        for (_, fmt, shape, g, data, scales) in problems]
        self.inputs = [torch.from_numpy(np.asarray(x, np.float16)).float() for (x, *_) in problems]
        from torch_npu_lowbit import PackedWeight
        self.packed = [PackedWeight(tuple(shape), fmt, g, bytes(data), bytes(scales))
                       for (_, fmt, shape, g, data, scales) in problems]

    def run_predequantized(self):
        return [(x @ w.T).half() for x, w in zip(self.inputs, self.weights)]

    def run_with_dequant(self):
        out = []
        for x, packed in zip(self.inputs, self.packed):
            w = torch.from_numpy(packed.dequantize()).float()
            out.append((x @ w.T).half())
        return out


def time_pass(cpu, *, warmup=3, rounds=31, budget_s=20.0):
    """Median seconds per pass for (pre-dequantized, dequant-inclusive), interleaved ABBA."""
    for _ in range(warmup):
        cpu.run_predequantized()
        cpu.run_with_dequant()
    a, b = [], []
    start = time.perf_counter()
    for i in range(rounds):
        order = (cpu.run_predequantized, cpu.run_with_dequant) if i % 2 == 0 else \
            (cpu.run_with_dequant, cpu.run_predequantized)
        for fn in order:
            t0 = time.perf_counter()
            fn()
            (a if fn == cpu.run_predequantized else b).append(time.perf_counter() - t0)
        if time.perf_counter() - start > budget_s and i >= 4:
            break
    return statistics.median(a), statistics.median(b), len(a)


def cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'
