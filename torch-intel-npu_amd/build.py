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
SOURCES = [CSRC / 'lowbit_abi.hip', CSRC / 'decode_abi.hip', CSRC / 'wide_abi.hip']
HEADERS = [CSRC / 'lb_common.h', CSRC / 'lb_kernels.h', CSRC / 'lb_decode.h', CSRC / 'abi_util.h',
           CSRC / 'lb_gemm.h', CSRC / 'lb_variants.h', CSRC / 'fused_launch.h', CSRC / 'lb_stream.h', CSRC / 'lb_layer.h',
           CSRC / 'lb_line.h', CSRC / 'lb_wide.h',
           HERE.parent / 'include' / 'lowbit_hip.h', HERE.parent / 'include' / 'lowbit_decode_hip.h']
ARCH = 'gfx950'


def hipcc():
    for candidate in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError('hipcc not found; the low-bit HIP library cannot be built')


def compile_command(source, obj, defines=()):
    return [hipcc(), f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-c',
            *(f'-D{d}' for d in defines),
            # Packed fp32 VALU forms are kept out of the generated code on purpose.
            '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
            # Leading scalar kernel arguments (up to 14 dwords) arrive preloaded in registers.
            '-mllvm', '-amdgpu-kernarg-preload-count=14',
            '-Wall', '-Wno-unused-function', '-Wno-unused-variable',
            '-o', str(obj), str(source)]


def link_command(objects, output):
    return [hipcc(), f'--offload-arch={ARCH}', '-shared', '-o', str(output), *map(str, objects)]


def _run(commands, verbose):
    """Run the commands concurrently; raise with the compiler's messages if any fails."""
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    procs = []
    for cmd in commands:
        if verbose:
            print(' '.join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
    failed = []
    for proc in procs:
        out, _ = proc.communicate()
        messages = [line for line in out.splitlines() if noise not in line]
        if proc.returncode != 0:
            failed.append('\n'.join(messages))
        elif verbose and messages:
            print('\n'.join(messages), flush=True)
    if failed:
        raise RuntimeError('hipcc failed:\n' + '\n'.join(failed))


def build(verbose=False, output=LIBRARY, defines=()):
    """Compile to `output` (default: the in-tree library); `defines` are extra -D macros.  The
    sources compile concurrently to objects beside the output, which are then linked."""
    output = Path(output)
    tmp = output.with_name(output.name + '.tmp')
    objects = [output.with_name(f'{output.stem}.{src.stem}.o') for src in SOURCES]
    try:
        _run([compile_command(src, obj, defines) for src, obj in zip(SOURCES, objects)], verbose)
        _run([link_command(objects, tmp)], verbose)
    finally:
        for obj in objects:
            obj.unlink(missing_ok=True)
    os.replace(tmp, output)
    return output


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
