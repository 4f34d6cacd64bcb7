"""Host-only checks of the C-ABI: the library loads, exports every declared entry point,
and rejects bad arguments before touching the device (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest

import lowbit_hip

HEADER = Path(__file__).resolve().parents[1] / 'include' / 'lowbit_hip.h'


def declared_functions():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r'\b(lb_[a-z_]+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    lib = lowbit_hip.library()
    names = declared_functions()
    assert set(names) == set(lowbit_hip.EXPORTS), names
    for name in names:
        assert hasattr(lib, name), name
    assert lib.lb_abi_version() == lowbit_hip.ABI_VERSION
    assert lowbit_hip.status_name(1) == 'LB_INVALID_ARGUMENT'
    assert lowbit_hip.status_name(10) == 'LB_DEVICE_FAILED'


def test_struct_layout_matches_header():
    # struct_size is checked by the library: a wrong Python mirror is rejected as too small.
    assert ctypes.sizeof(lowbit_hip.LinearArgs) == 8 + 8 * 4 + 8 * 2 + 8 * 2 + 8 * 2 + 8 + 8 * 3 + 8 + 8 + 8 + 8


def args(**over):
    a = lowbit_hip.LinearArgs()
    a.struct_size = ctypes.sizeof(a)
    a.format, a.M, a.N, a.K, a.group_size = 1, 1, 64, 128, 32
    a.codes, a.scales, a.x, a.y = 0x10000, 0x20000, 0x30000, 0x40000
    a.ldx, a.ldy = 128, 64
    for key, value in over.items():
        setattr(a, key, value)
    return a


def workspace(a):
    size = ctypes.c_size_t(0)
    status = lowbit_hip.library().lb_workspace_bytes(ctypes.byref(a), ctypes.byref(size))
    return status, size.value, lowbit_hip.library().lb_last_error().decode()


@pytest.mark.parametrize('over,needle', [
    (dict(struct_size=8), 'struct_size'),
    (dict(format=9), 'format'),
    (dict(M=0), 'positive'),
    (dict(group_size=48), 'group_size'),
    (dict(group_size=0), 'group_size'),
    (dict(codes=0), 'non-NULL'),
    (dict(ldx=64), 'ldx'),
    (dict(rank=3), 'correction'),
    (dict(rank=500), 'rank'),
    (dict(y=0x30000), 'overlaps x'),
    (dict(y=0x10010), 'overlaps codes'),
    (dict(flags=3), 'at most one'),
    (dict(M=40, flags=1), 'FORCE_GEMV'),
    (dict(x=0x30001), 'aligned'),
])
def test_argument_errors_are_reported_before_launch(over, needle):
    status, _, message = workspace(args(**over))
    assert status == lowbit_hip.INVALID_ARGUMENT, message
    assert needle in message


def test_forced_fast_path_on_unaligned_shape_is_unsupported():
    status, _, message = workspace(args(K=48, group_size=48, ldx=48, flags=lowbit_hip.FLAG_FORCE_GEMV))
    assert status == lowbit_hip.UNSUPPORTED and 'K % 32' in message


def test_workspace_sizes():
    status, size, _ = workspace(args())
    assert status == 0 and size == 0
    # correction on the decode path needs z = M x rank fp16
    status, size, _ = workspace(args(rank=32, down=0x50000, up=0x60000, up_ld=32))
    assert status == 0 and size == 256
    # split-K decode of a tall K needs fp32 partials
    status, size, _ = workspace(args(N=1024, K=14336, ldx=14336, ldy=1024, group_size=128,
                                     x=0x1000000, y=0x2000000, scales=0x3000000, codes=0x4000000))
    assert status == 0 and size > 0 and size % (1024 * 4) == 0  # fp32 split-K partials [splits, M, N]
    # prefill with correction needs z and the fp16 delta
    status, size, _ = workspace(args(M=256, rank=32, down=0x5000000, up=0x6000000, up_ld=32,
                                     x=0x1000000, y=0x2000000))
    assert status == 0 and size == 256 * 32 * 2 + 256 * 64 * 2


def test_missing_workspace_is_rejected_by_lb_linear():
    a = args(N=1024, K=14336, ldx=14336, ldy=1024, group_size=128, x=0x1000000, y=0x2000000,
             scales=0x3000000, codes=0x4000000)
    status = lowbit_hip.library().lb_linear(ctypes.byref(a), None)
    assert status == lowbit_hip.INVALID_ARGUMENT
    assert 'workspace' in lowbit_hip.library().lb_last_error().decode()


def test_unpack_and_dequantize_argument_errors():
    lib = lowbit_hip.library()
    assert lib.lb_unpack_codes(7, 2, 2, 0x1000, 0x2000, None) == lowbit_hip.INVALID_ARGUMENT
    assert lib.lb_unpack_codes(1, 0, 2, 0x1000, 0x2000, None) == lowbit_hip.INVALID_ARGUMENT
    assert lib.lb_unpack_codes(1, 4, 4, 0x1000, 0x1004, None) == lowbit_hip.INVALID_ARGUMENT  # overlap
    assert lib.lb_dequantize(1, 4, 6, 4, 0x1000, 0x2000, 0x3000, None) == lowbit_hip.INVALID_ARGUMENT
    assert lib.lb_dequantize(3, 4, 8, 4, 0x1000, 0x2000, 0x3000, None) == lowbit_hip.INVALID_ARGUMENT
