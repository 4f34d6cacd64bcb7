"""Build liblowbit_hip.so (gfx950) in-tree with hipcc.

Usage: python torch-intel-npu_amd/build.py   (or __graft_entry__.build()).
Every call recompiles; the output lands next to this file so it travels with the tree.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / 'csrc'
LIBRARY = HERE / 'liblowbit_hip.so'
SOURCES = [CSRC / 'lowbit_abi.hip', CSRC / 'decode_abi.hip']
HEADERS = [CSRC / 'lb_common.h', CSRC / 'lb_kernels.h', CSRC / 'lb_decode.h', CSRC / 'abi_util.h',
           CSRC / 'lb_gemm.h', CSRC / 'lb_variants.h', CSRC / 'fused_launch.h', CSRC / 'lb_stream.h', CSRC / 'lb_layer.h',
           CSRC / 'lb_line.h',
           HERE.parent / 'include' / 'lowbit_hip.h', HERE.parent / 'include' / 'lowbit_decode_hip.h']
ARCH = 'gfx950'


def hipcc():
    for candidate in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError('hipcc not found; the low-bit HIP library cannot be built')


def command(output=LIBRARY, defines=()):
    return [hipcc(), f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared',
            *(f'-D{d}' for d in defines),
            # Packed fp32 VALU forms are kept out of the generated code on purpose.
            '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
            # Leading scalar kernel arguments (up to 14 dwords) arrive preloaded in registers.
            '-mllvm', '-amdgpu-kernarg-preload-count=14',
            '-Wall', '-Wno-unused-function', '-Wno-unused-variable',
            '-o', str(output), *map(str, SOURCES)]


def build(verbose=False, output=LIBRARY, defines=()):
    """Compile to `output` (default: the in-tree library); `defines` are extra -D macros."""
    output = Path(output)
    tmp = output.with_name(output.name + '.tmp')
    cmd = command(tmp, defines)
    if verbose:
        print(' '.join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    messages = [line for line in (result.stdout + result.stderr).splitlines() if noise not in line]
    if result.returncode != 0:
        raise RuntimeError('hipcc failed:\n' + '\n'.join(messages))
    if verbose and messages:
        print('\n'.join(messages), flush=True)
    os.replace(tmp, output)
    return output


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
