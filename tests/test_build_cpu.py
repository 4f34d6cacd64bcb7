"""Build checks of liblowbit_hip.so's gfx950 code objects (CPU only: reads the metadata notes of this
repository's own build with the ROCm LLVM tools).

Kernel scratch memory: a struct or array the compiler cannot keep in registers lands in per-lane
scratch (private segment), which costs a memory round trip per access on the decode path's
latency chain; a one-row GEMV regressed by 1.5 us that way.  Every kernel must keep at most a few
bytes of it (the compiler reserves an unused 20-byte slot in two stacked decode kernels).
"""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / 'torch-intel-npu_amd' / 'liblowbit_hip.so'
LLVM = Path('/opt/rocm/llvm/bin')
MAGIC = b'__CLANG_OFFLOAD_BUNDLE__'
SCRATCH_LIMIT = 32  # bytes per lane


def _kernel_metadata(tmp_path):
    if not LIB.exists():
        pytest.skip('library not built')
    for tool in ('llvm-objcopy', 'clang-offload-bundler', 'llvm-readelf'):
        if not (LLVM / tool).exists():
            pytest.skip(f'{tool} not found')
    fat = tmp_path / 'fatbin.bin'
    subprocess.run([str(LLVM / 'llvm-objcopy'), f'--dump-section=.hip_fatbin={fat}', str(LIB), str(tmp_path / 'x.so')],
                   check=True, capture_output=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)] + [len(data)]
    kernels = {}
    for i, (a, b) in enumerate(zip(starts, starts[1:])):
        part = tmp_path / f'bundle{i}.bin'
        part.write_bytes(data[a:b])
        obj = tmp_path / f'gfx950_{i}.o'
        subprocess.run([str(LLVM / 'clang-offload-bundler'), '--type=o', '--targets=hipv4-amdgcn-amd-amdhsa--gfx950',
                        f'--input={part}', f'--output={obj}', '--unbundle'], check=True, capture_output=True)
        notes = subprocess.run([str(LLVM / 'llvm-readelf'), '--notes', str(obj)], check=True, capture_output=True,
                               text=True).stdout
        name = None
        for line in notes.splitlines():
            m = re.match(r'\s*\.name:\s+(\S+)', line)
            if m:
                name = m.group(1)
            m = re.match(r'\s*\.private_segment_fixed_size:\s+(\d+)', line)
            if m and name:
                kernels[name] = int(m.group(1))
    return kernels


def test_library_kernels_keep_no_scratch(tmp_path):
    kernels = _kernel_metadata(tmp_path)
    assert len(kernels) > 50  # both translation units' code objects were read
    heavy = {k: v for k, v in kernels.items() if v > SCRATCH_LIMIT}
    assert not heavy, f'kernels with more than {SCRATCH_LIMIT} scratch bytes per lane: {heavy}'
    for family in ('fused_gemv_kernel', 'decode_layer_kernel', 'rows_gemv_kernel', 'gemm4_kernel'):
        assert any(family in k for k in kernels), family
