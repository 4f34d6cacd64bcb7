"""CPU oracle for the low-bit linear path -- TEST INFRASTRUCTURE ONLY.

A plain restatement (numpy / torch CPU) of the reference's CPU-visible algorithm:
packing, quantizer, dequantizer, staged fp16 linear + low-rank correction, and the
staged SmolLM decoder reference.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker or the timed CPU baseline.
The product (torch-intel-npu_amd/) never imports it.

Pinning status of each function is recorded in the module docstrings; every function
cites the reference file:line it restates.
"""
