"""A hand-over wait that gives up is an error, not a silent wrong result.

The one-launch decode kernels (lb_decode_stack, lb_decode_layer) and the shared-z fused GEMV hand
data between workgroups through tagged workspace words, with bounded waits; a wait that gives up
sets the workspace's timeout word.  Here the host presets that word before a decode step, the
condition a timed-out wait leaves: every wait of the stacked and per-layer kernels then gives up at
its 64th poll, so every kernel still ends normally (the shared-z waits find their words and end as
usual).  GraphDecoder.generate() must raise RuntimeError, and the library must then refuse every
later call (LB_DEVICE_FAILED), as the reference's failed context does
(npunlock-probe/torch-device/backend.cpp:280-292).

The failed state is process-wide and sticky, so each case runs in a child process.
"""
import subprocess
import sys
from pathlib import Path

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

CHILD = r'''
import sys
sys.path[:0] = sys.argv[1:3]
mode = sys.argv[3]
import torch
import lowbit_hip
import smollm_random
from torch_npu_smollm import GraphDecoder

print('[child] case', mode, flush=True)
device = torch.device('cuda:0')
stack, io, _, _ = smollm_random.build(seed=5, layers=2, rank=32, theta=10000.0, capacity=64)
io = io.to(device)
ids = smollm_random.prompt(seed=5, length=16)
h, caches = stack.prefill(io.embed_tokens(ids.to(device)))
decoder = GraphDecoder(stack, io, layer=mode != 'fused', stack_kernel=mode == 'stack')
assert decoder.stack_kernel == (mode == 'stack') and decoder.layer_kernel == (mode != 'fused')
decoder.load(caches, 7)
healthy = decoder.generate(2)
assert decoder.timeouts() == 0 and not lowbit_hip.failed()
waiting = list(decoder._waiting_calls())
assert waiting, 'no call of this mode waits on a workspace'
call = waiting[-1]
word = call.workspace[call._timeout_offset:call._timeout_offset + 4].view(torch.int32)
word.fill_(1)          # the word a timed-out wait leaves
torch.cuda.synchronize()
try:
    decoder.generate(1)
except RuntimeError as error:
    assert 'hand-over wait' in str(error), error
    print('[child] generate raised:', str(error)[:120], flush=True)
else:
    raise AssertionError('generate() returned despite a timed-out wait')
assert lowbit_hip.failed()
try:
    decoder.step()     # every later call is refused before launch
except RuntimeError as error:
    assert 'LB_DEVICE_FAILED' in str(error), error
else:
    raise AssertionError('the failed library accepted a launch')
x = torch.zeros(1, 64, dtype=torch.float16, device=device)
codes = torch.zeros(64 * 32, dtype=torch.uint8, device=device)
scales = torch.ones(64 * 2, dtype=torch.float16, device=device)
try:
    lowbit_hip.linear(x, codes, scales, format='int4', N=64, K=64, group_size=32)
except RuntimeError as error:
    assert 'LB_DEVICE_FAILED' in str(error), error
else:
    raise AssertionError('the failed library accepted lb_linear')
print('ok', flush=True)
'''


@pytest.mark.parametrize('mode', ['stack', 'layer', 'fused'])
def test_timed_out_wait_raises_and_fails_the_library(device, mode):
    announce('timeout word preset by the host', mode)
    root = Path(__file__).resolve().parents[1]
    out = subprocess.run([sys.executable, '-u', '-c', CHILD, str(root), str(root / 'torch-intel-npu_amd'), mode],
                         capture_output=True, text=True, timeout=180)
    print(out.stdout[-2000:], out.stderr[-2000:], flush=True)
    assert out.returncode == 0 and out.stdout.strip().endswith('ok'), out.stdout + out.stderr
    import lowbit_hip
    assert not lowbit_hip.failed()  # this process is untouched
