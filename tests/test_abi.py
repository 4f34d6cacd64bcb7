"""Host-only checks of the C-ABI: the library loads, exports every declared entry point,
and rejects bad arguments before touching the device (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import lowbit_hip

HEADERS = sorted((Path(__file__).resolve().parents[1] / 'include').glob('*.h'))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r'/\*.*?\*/', '', header.read_text(), flags=re.S)
        names |= set(re.findall(r'\b(lb_[a-z_]+)\s*\(', text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = lowbit_hip.library()
    names = declared_functions()
    assert len(HEADERS) == 2
    assert set(names) == set(lowbit_hip.EXPORTS) | set(lowbit_hip.DECODE_EXPORTS), names
    for name in names:
        assert hasattr(lib, name), name
    assert lib.lb_abi_version() == lowbit_hip.ABI_VERSION
    assert lowbit_hip.status_name(1) == 'LB_INVALID_ARGUMENT'
    assert lowbit_hip.status_name(10) == 'LB_DEVICE_FAILED'


def test_struct_layout_matches_header():
    # struct_size is checked by the library: a wrong Python mirror is rejected as too small.
    assert ctypes.sizeof(lowbit_hip.LinearArgs) == 8 + 8 * 4 + 8 * 2 + 8 * 2 + 8 * 2 + 8 + 8 * 3 + 8 + 8 + 8 + 8 + 8
    assert ctypes.sizeof(lowbit_hip.FusedProblem) == 10 * 8
    assert ctypes.sizeof(lowbit_hip.FusedLinearArgs) == 8 + 8 + 8 + 8 + 3 * 8 + 8 + 3 * 80 + 16
    assert ctypes.sizeof(lowbit_hip.DecodeAttentionArgs) == 8 + 4 * 8 + 9 * 8 + 8 + 16


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
    # one row with K <= 1536: the single-tile kernel computes z inside each workgroup
    status, size, _ = workspace(args(rank=32, down=0x50000, up=0x60000, up_ld=32))
    assert status == 0 and size == 0
    # the split decode GEMV (forced, or M > 1) stages z = M x rank fp16 in the workspace
    status, size, _ = workspace(args(rank=32, down=0x50000, up=0x60000, up_ld=32, flags=lowbit_hip.FLAG_FORCE_GEMV))
    assert status == 0 and size == 256
    status, size, _ = workspace(args(M=2, rank=32, down=0x50000, up=0x60000, up_ld=32))
    assert status == 0 and size == 256
    # an unaligned U keeps one row on the split GEMV, with its z buffer
    status, size, _ = workspace(args(rank=32, down=0x50000, up=0x60002, up_ld=32))
    assert status == 0 and size == 256
    # split-K decode of a tall K (the forced split GEMV) needs fp32 partials
    status, size, _ = workspace(args(N=1024, K=14336, ldx=14336, ldy=1024, group_size=128,
                                     x=0x1000000, y=0x2000000, scales=0x3000000, codes=0x4000000,
                                     flags=lowbit_hip.FLAG_FORCE_GEMV))
    assert status == 0 and size > 0 and size % (1024 * 4) == 0  # fp32 split-K partials [splits, M, N]
    # prefill with correction needs z and the fp16 delta
    status, size, _ = workspace(args(M=256, rank=32, down=0x5000000, up=0x6000000, up_ld=32,
                                     x=0x1000000, y=0x2000000))
    assert status == 0 and size == 256 * 32 * 2 + 256 * 64 * 2
    # a prefill GEMM of few 64 x 64 tiles splits K: fp32 partials [splits, M, N] (960 x 2560 at
    # M = 512: 120 tiles, 40 k steps -> 4 slices)
    status, size, _ = workspace(args(format=2, M=512, N=960, K=2560, group_size=64, ldx=2560, ldy=960,
                                     x=0x1000000, y=0x2000000, scales=0x3000000, codes=0x4000000))
    assert status == 0 and size == 4 * 512 * 960 * 4
    # enough tiles: no split, no workspace
    status, size, _ = workspace(args(format=2, M=512, N=2560, K=960, group_size=64, ldx=960, ldy=2560,
                                     x=0x1000000, y=0x2000000, scales=0x3000000, codes=0x4000000))
    assert status == 0 and size == 0


def test_prefill_tile_plan_workspace():
    """The planner's tile choice shows in the workspace: split grids need fp32 partials."""
    big = dict(x=0x10000000, y=0x20000000, scales=0x30000000, codes=0x40000000)
    # 128 x 128 grid of 128 tiles over 32 k steps: two slices give 256 workgroups
    status, size, _ = workspace(args(M=512, N=4096, K=2048, group_size=128, ldx=2048, ldy=4096, **big))
    assert status == 0 and size == 2 * 512 * 4096 * 4
    # 64 tiles over 64 k steps: four slices
    status, size, _ = workspace(args(M=256, N=4096, K=4096, group_size=128, ldx=4096, ldy=4096, **big))
    assert status == 0 and size == 4 * 256 * 4096 * 4
    # 224 tiles of 256 x 128 fill the CUs in one round: no split
    status, size, _ = workspace(args(M=512, N=14336, K=4096, group_size=128, ldx=4096, ldy=14336, **big))
    assert status == 0 and size == 0
    # 168 tiles of 256 x 256: no split
    status, size, _ = workspace(args(M=768, N=14336, K=4096, group_size=128, ldx=4096, ldy=14336, **big))
    assert status == 0 and size == 0


def test_missing_workspace_is_rejected_by_lb_linear():
    a = args(N=1024, K=14336, ldx=14336, ldy=1024, group_size=128, x=0x1000000, y=0x2000000,
             scales=0x3000000, codes=0x4000000, flags=lowbit_hip.FLAG_FORCE_GEMV)
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


def fused(**over):
    a = lowbit_hip.FusedLinearArgs()
    a.struct_size = ctypes.sizeof(a)
    a.format, a.K, a.group_size, a.prologue, a.count = 0, 576, 576, 1, 1
    a.x, a.gamma, a.eps = 0x10000, 0x20000, 1e-5
    p = a.problems[0]
    p.codes, p.scales, p.N, p.y = 0x100000, 0x30000, 64, 0x40000
    for key, value in over.items():
        target = p if key.startswith('p_') else a
        setattr(target, key[2:] if key.startswith('p_') else key, value)
    return a


@pytest.mark.parametrize('over,needle', [
    (dict(struct_size=16), 'struct_size'),
    (dict(format=7), 'format'),
    (dict(K=600), 'multiple of 32'),
    (dict(K=2048), 'multiple of 32'),
    (dict(format=1, group_size=48), 'group_size'),
    (dict(prologue=5), 'prologue'),
    (dict(count=0), 'count'),
    (dict(count=4), 'count'),
    (dict(x=0x10008), 'x must be'),
    (dict(gamma=0), 'gamma'),
    (dict(prologue=2), 'x2'),
    (dict(p_N=0), 'N='),
    (dict(p_codes=0x100008), 'codes'),
    (dict(p_rank=33), 'rank'),
    (dict(p_rank=8, p_down=0x50000, p_up=0x60000, p_up_ld=12), 'up_ld'),
    (dict(p_y=0x10010), 'overlaps x'),
    (dict(p_y=0x100010), 'overlaps codes'),
    (dict(p_residual=0x40002), 'overlaps residual'),
])
def test_fused_linear_argument_errors(over, needle):
    lib = lowbit_hip.library()
    status = lib.lb_fused_linear(ctypes.byref(fused(**over)), None)
    message = lib.lb_last_error().decode()
    assert status == lowbit_hip.INVALID_ARGUMENT, message
    assert needle in message


def test_fused_linear_outputs_may_not_overlap_each_other():
    a = fused(count=2)
    p = a.problems[1]
    p.codes, p.scales, p.N, p.y = 0x200000, 0x70000, 64, 0x40040
    lib = lowbit_hip.library()
    assert lib.lb_fused_linear(ctypes.byref(a), None) == lowbit_hip.INVALID_ARGUMENT
    assert 'outputs of problems 0 and 1' in lib.lb_last_error().decode()


def attention(**over):
    a = lowbit_hip.DecodeAttentionArgs()
    a.struct_size = ctypes.sizeof(a)
    a.heads, a.kv_heads, a.head_dim, a.capacity = 9, 3, 64, 64
    a.q, a.k, a.v, a.cos, a.sin, a.position = 0x10000, 0x11000, 0x12000, 0x20000, 0x30000, 0x40000
    a.keys, a.values, a.out, a.scale = 0x100000, 0x200000, 0x50000, 0.125
    for key, value in over.items():
        setattr(a, key, value)
    return a


@pytest.mark.parametrize('over,needle,status', [
    (dict(head_dim=128), 'head_dim', lowbit_hip.UNSUPPORTED),
    (dict(kv_heads=4), 'multiple of kv_heads', lowbit_hip.INVALID_ARGUMENT),
    (dict(capacity=5000), 'capacity', lowbit_hip.INVALID_ARGUMENT),
    (dict(keys=0), 'NULL', lowbit_hip.INVALID_ARGUMENT),
    (dict(keys=0x100008), 'misaligned', lowbit_hip.INVALID_ARGUMENT),
    (dict(values=0x100000 + 3 * 64 * 128 - 16), 'keys overlap values', lowbit_hip.INVALID_ARGUMENT),
    (dict(out=0x10040), 'overlaps q', lowbit_hip.INVALID_ARGUMENT),
    (dict(scale=float('inf')), 'scale', lowbit_hip.INVALID_ARGUMENT),
])
def test_decode_attention_argument_errors(over, needle, status):
    lib = lowbit_hip.library()
    assert lib.lb_decode_attention(ctypes.byref(attention(**over)), None) == status
    assert needle in lib.lb_last_error().decode()


def test_argmax_next_argument_errors():
    lib = lowbit_hip.library()
    ok = (0x10000, 1000, 0x100000, 64, 0x20000, 0x30000, 0x31000, 0x32000, 8)
    for index, value in ((0, 0), (1, 0), (3, 12), (4, 0x20008), (5, 0x30004), (8, -1), (4, 0x100000 + 640)):
        bad = list(ok)
        bad[index] = value
        assert lib.lb_argmax_next(*bad, None) == lowbit_hip.INVALID_ARGUMENT, (index, value)


def head_next_args(**over):
    """A valid lb_head_next head: fp16 [1000, 64] tied rows, RMSNorm, its workspace."""
    a = lowbit_hip.FusedLinearArgs()
    a.struct_size = ctypes.sizeof(a)
    a.format, a.K, a.group_size, a.prologue, a.count = 3, 64, 64, 1, 1
    a.x, a.gamma, a.eps = 0x10000, 0x11000, 1e-5
    q = a.problems[0]
    q.codes, q.N, q.y = 0x100000, 1000, 0x20000
    a.workspace, a.workspace_bytes = 0x40000, lowbit_hip.head_next_workspace_bytes(1000)
    for key, value in over.items():
        target = q if key in ('codes', 'scales', 'N', 'y', 'bias', 'residual', 'rank') else a
        setattr(target, key, value)
    return a


HEAD_NEXT_OK = dict(embedding=0x100000, h_next=0x12000, tokens=0x30000, token=0x31000, position=0x32000, limit=8)


@pytest.mark.parametrize('over,call_over,needle,status', [
    (dict(count=2), {}, 'one problem', lowbit_hip.INVALID_ARGUMENT),
    (dict(prologue=0), {}, 'RMSNorm', lowbit_hip.INVALID_ARGUMENT),
    (dict(bias=0x50000), {}, 'no correction, bias or residual', lowbit_hip.INVALID_ARGUMENT),
    (dict(format=0, scales=0x60000), {}, 'fp16 or int4', lowbit_hip.UNSUPPORTED),
    (dict(K=1024, group_size=1024, x=0x200000, gamma=0x210000), dict(embedding=0x1000000, h_next=0x220000),
     'K <= 640', lowbit_hip.UNSUPPORTED),
    (dict(workspace_bytes=16), {}, 'workspace', lowbit_hip.INVALID_ARGUMENT),
    (dict(workspace=0x40008), {}, 'workspace', lowbit_hip.INVALID_ARGUMENT),
    (dict(struct_size=ctypes.sizeof(lowbit_hip.FusedLinearArgs) - 16), {}, 'struct_size', lowbit_hip.INVALID_ARGUMENT),
    ({}, dict(embedding=0), 'NULL', lowbit_hip.INVALID_ARGUMENT),
    ({}, dict(h_next=0x12008), 'alignment', lowbit_hip.INVALID_ARGUMENT),
    ({}, dict(limit=-1), 'limit', lowbit_hip.INVALID_ARGUMENT),
    ({}, dict(h_next=0x20000), 'h_next overlaps', lowbit_hip.INVALID_ARGUMENT),      # the logits
    ({}, dict(h_next=0x11000), 'h_next overlaps gamma', lowbit_hip.INVALID_ARGUMENT),
    ({}, dict(token=0x30008), 'tokens overlaps token', lowbit_hip.INVALID_ARGUMENT),
    ({}, dict(position=0x40010), 'overlaps workspace', lowbit_hip.INVALID_ARGUMENT),
])
def test_head_next_argument_errors(over, call_over, needle, status):
    lib = lowbit_hip.library()
    call = dict(HEAD_NEXT_OK, **call_over)
    got = lib.lb_head_next(ctypes.byref(head_next_args(**over)), call['embedding'], call['h_next'], call['tokens'],
                           call['token'], call['position'], call['limit'], None)
    assert got == status, lib.lb_last_error().decode()
    assert needle in lib.lb_last_error().decode()


def test_head_next_workspace_size_matches_header():
    """LB_HEAD_NEXT_WORKSPACE_BYTES as the Python helper computes it (the header macro is the ABI)."""
    import re
    from pathlib import Path
    text = (Path(__file__).resolve().parents[1] / 'include' / 'lowbit_decode_hip.h').read_text()
    assert re.search(r'#define LB_HEAD_NEXT_WORKGROUPS\(vocab\) \(\(\(size_t\)\(vocab\) \+ 63u\) / 64u\)', text)
    assert '#define LB_HEAD_NEXT_WORKSPACE_BYTES(vocab) (16u * ((LB_HEAD_NEXT_WORKGROUPS(vocab) + 7u) / 8u + 1u))' in text
    for vocab, want in ((1, 32), (512, 32), (513, 48), (49152, 16 * 97), (70001, 16 * 138)):
        assert lowbit_hip.head_next_workspace_bytes(vocab) == want, vocab


W8 = dict(format=0, group_size=128, K=128, flags=lowbit_hip.FLAG_W8A8, activation_scale=1 / 128)


@pytest.mark.parametrize('over,status,needle', [
    (dict(flags=0x100), lowbit_hip.INVALID_ARGUMENT, 'unknown flags'),
    # compact groups (reference QuantizedLinear: at most 32 groups, packed weights only)
    (dict(K=4096, ldx=4096, group_size=32, flags=lowbit_hip.FLAG_COMPACT_GROUPS), lowbit_hip.INVALID_ARGUMENT,
     'at most 32 groups'),
    (dict(format=3, flags=lowbit_hip.FLAG_COMPACT_GROUPS), lowbit_hip.INVALID_ARGUMENT, 'packed'),
    (dict(flags=lowbit_hip.FLAG_COMPACT_GROUPS, rank=4, down=0x50000, up=0x60000, up_ld=4), lowbit_hip.UNSUPPORTED,
     'correction'),
    # W8A8 (reference _activation_scale, torch_npu_lowbit.py:155-166)
    (dict(W8, format=1), lowbit_hip.INVALID_ARGUMENT, 'per-channel int8'),
    (dict(W8, group_size=64), lowbit_hip.INVALID_ARGUMENT, 'per-channel int8'),
    (dict(W8, flags=lowbit_hip.FLAG_W8A8 | lowbit_hip.FLAG_COMPACT_GROUPS), lowbit_hip.INVALID_ARGUMENT,
     'no compact groups'),
    (dict(W8, activation_scale=3 / 256), lowbit_hip.INVALID_ARGUMENT, 'power of two'),
    (dict(W8, activation_scale=512.0), lowbit_hip.INVALID_ARGUMENT, 'power of two'),
    (dict(W8, activation_scale=2.0 ** -25), lowbit_hip.INVALID_ARGUMENT, 'power of two'),
    (dict(W8, activation_scale=float('inf')), lowbit_hip.INVALID_ARGUMENT, 'power of two'),
    (dict(W8, rank=4, down=0x50000, up=0x60000, up_ld=4), lowbit_hip.UNSUPPORTED, 'correction'),
    (dict(W8, K=131136, ldx=131136, group_size=131136, N=1, ldy=1, codes=0x1000000, scales=0x2000000, x=0x3000000,
          y=0x4000000), lowbit_hip.UNSUPPORTED, 'K <='),
    (dict(W8, K=96, ldx=96, group_size=96, flags=lowbit_hip.FLAG_W8A8 | lowbit_hip.FLAG_FORCE_GEMV),
     lowbit_hip.UNSUPPORTED, 'K % 64'),
])
def test_variant_argument_errors(over, status, needle):
    got, _, message = workspace(args(**over))
    assert got == status, message
    assert needle in message


S = lowbit_hip.FLAG_FORCE_STREAM


@pytest.mark.parametrize('over,status,needle', [
    (dict(flags=S | lowbit_hip.FLAG_FORCE_GEMV), lowbit_hip.INVALID_ARGUMENT, 'at most one'),
    (dict(flags=S, M=2), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),        # two rows need groups >= 64
    (dict(flags=S, M=33, group_size=128, ldy=64), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),  # at most 32 rows
    (dict(flags=S, M=9, group_size=64), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),  # 9..16 rows: >= 128
    (dict(flags=S, M=2, K=8192, ldx=8192, group_size=128, N=1, ldy=1), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),
    (dict(flags=S, format=2), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),   # nf4
    (dict(flags=S, format=3), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),   # fp16
    (dict(flags=S, rank=4, down=0x50000, up=0x60000, up_ld=8), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),
    (dict(flags=S | lowbit_hip.FLAG_COMPACT_GROUPS), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),
    (dict(flags=S, K=192, ldx=192, group_size=96), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),  # 96 spans 1.33 pieces
    (dict(flags=S, K=768, ldx=768, group_size=384), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),  # not a power of two
    (dict(flags=S, format=0, K=128, group_size=8, ldx=128), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),  # group < 16
    (dict(flags=S, K=32768, ldx=32768, group_size=128, N=1, ldy=1), lowbit_hip.UNSUPPORTED, 'FORCE_STREAM'),
])
def test_force_stream_argument_errors(over, status, needle):
    got, _, message = workspace(args(**over))
    assert got == status, message
    assert needle in message


@pytest.mark.parametrize('over,needle', [
    (dict(K=4096 + 256, ldx=4352), 'LB_FLAG_FORCE_WIDE'),
    (dict(K=4096, ldx=4096, group_size=64), 'LB_FLAG_FORCE_WIDE'),
    (dict(K=4096, ldx=4096, format=2), 'LB_FLAG_FORCE_WIDE'),
    (dict(K=4096, ldx=4096, M=33), 'LB_FLAG_FORCE_WIDE'),
    (dict(K=4096, ldx=4096, rank=8, down=0x50000, up=0x60000, up_ld=8), 'LB_FLAG_FORCE_WIDE'),
])
def test_force_wide_argument_errors(over, needle):
    status, _, message = workspace(args(flags=lowbit_hip.FLAG_FORCE_WIDE, x=0x1000000, y=0x2000000, scales=0x3000000,
                                        codes=0x4000000, **over))
    assert status == lowbit_hip.UNSUPPORTED and needle in message, message


def test_force_wide_workspace_holds_the_slices():
    """One K slice needs no workspace; several need their fp32 partials [slices, M, N]."""
    far = dict(x=0x1000000, y=0x8000000, scales=0x10000000, codes=0x20000000)
    status, size, _ = workspace(args(M=32, N=65536, K=4096, ldx=4096, ldy=65536, group_size=128,
                                     flags=lowbit_hip.FLAG_FORCE_WIDE, **far))
    assert status == 0 and size == 0
    status, size, _ = workspace(args(M=32, N=4096, K=4096, ldx=4096, ldy=4096, group_size=128,
                                     flags=lowbit_hip.FLAG_FORCE_WIDE, **far))
    slices = size // (32 * 4096 * 4)
    assert status == 0 and size == slices * 32 * 4096 * 4 and slices in (2, 4, 8)   # few row blocks: split K
    status, size, _ = workspace(args(M=24, N=14336, K=4096, ldx=4096, ldy=14336, group_size=128, **far))
    slices = size // (24 * 14336 * 4)
    assert status == 0 and size == slices * 24 * 14336 * 4 and slices in (2, 4, 8)   # the default at 17..32 rows


@pytest.mark.parametrize('fmt,m,n,k,slices', [
    ('int4', 16, 14336, 4096, 4),    # 9..16 rows, INT4 / NF4, slices the kernel adds: wide_rows_kernel, 4 x 1024
    ('nf4', 9, 14336, 4096, 4),
    ('int4', 8, 14336, 4096, 0),     # 8 rows: tile_rows_kernel, 4096 codes staged whole
    ('int8', 16, 14336, 4096, 2),    # INT8: tile_rows_kernel, 2 x 2048
    ('int4', 16, 4096, 14336, 7),    # 14 wide slices, more than the kernel adds: tile_rows_kernel, 7 x 2048
    ('int4', 16, 8192, 4096, 2),     # 8 wide slices: tile_rows_kernel, 2 x 2048
])
def test_nine_to_sixteen_rows_take_wide_only_where_it_adds_its_slices(fmt, m, n, k, slices):
    """The default dispatch of 9..16 rows over 16..64 MB: the workspace holds the chosen kernel's
    fp32 partials [slices, M, N] (none for rows staged whole), which names the kernel."""
    far = dict(x=0x1000000, y=0x8000000, scales=0x10000000, codes=0x20000000)
    group = k if fmt == 'int8' else 128
    code = {'int8': 0, 'int4': 1, 'nf4': 2}[fmt]
    status, size, _ = workspace(args(M=m, N=n, K=k, ldx=k, ldy=n, group_size=group, format=code, **far))
    assert status == 0 and size == slices * m * n * 4


@pytest.mark.parametrize('m,n,k,group,fmt,slices', [
    (8, 4096, 14336, 128, 1, 4),     # 4 x 3584 codes (up to 8 rows: 4096 staged)
    (2, 576, 12288, 32, 1, 3),       # 3 x 4096
    (16, 1024, 14336, 128, 1, 7),    # 7 x 2048 (beyond 8 rows: 2048 staged)
    (12, 600, 4096, 128, 2, 2),      # NF4, 2 x 2048
    (8, 1030, 8192, 8192, 0, 2),     # per-row INT8: any slice length
    (8, 4096, 4096, 128, 1, 1),      # staged whole: no workspace
    (8, 1024, 4096, 128, 1, 4),      # fits, but 64 tiles: 4 x 1024 codes give 256 tile slices
    (4, 1000, 2048, 64, 1, 2),       # 63 tiles: 2 x 1024 (no smaller slice)
    (8, 576, 1536, 128, 1, 1),       # 36 tiles, but no slice of >= 1024 codes
])
def test_tile_rows_k_slices_take_their_partials(m, n, k, group, fmt, slices):
    """2..16 rows over rows longer than tile_rows_kernel stages whole: equal K slices of whole
    512-code steps and scale groups, each writing fp32 partials [slices, M, N] into the workspace."""
    far = dict(x=0x1000000, y=0x8000000, scales=0x10000000, codes=0x20000000)
    status, size, message = workspace(args(M=m, N=n, K=k, ldx=k, ldy=n, group_size=group, format=fmt, **far))
    want = 0 if slices == 1 else -(-slices * m * n * 4 // 256) * 256
    assert status == 0 and size == want, (size, want, message)


def test_zeroed_workspace_flag_reserves_its_bytes():
    """LB_FLAG_ZEROED_WORKSPACE: every plan puts its scratch after LB_ZEROED_WORKSPACE_BYTES reserved
    bytes (the counters), so a call that needed none needs exactly those; the header and the Python
    constants agree; lb_linear_noalloc ignores the flag (its refusal of oversized calls is unchanged)."""
    text = (Path(__file__).resolve().parents[1] / 'include' / 'lowbit_hip.h').read_text()
    assert f'#define LB_FLAG_ZEROED_WORKSPACE 0x{lowbit_hip.FLAG_ZEROED_WORKSPACE:x}u' in text
    assert f'#define LB_ZEROED_WORKSPACE_BYTES {lowbit_hip.ZEROED_WORKSPACE_BYTES}u' in text
    Z, R = lowbit_hip.FLAG_ZEROED_WORKSPACE, lowbit_hip.ZEROED_WORKSPACE_BYTES
    far = dict(x=0x1000000, y=0x8000000, scales=0x10000000, codes=0x20000000)
    cases = [dict(),                                                                     # one-row GEMV: no scratch
             dict(M=32, N=4096, K=4096, ldx=4096, ldy=4096, group_size=128, **far),      # wide, K slices
             dict(M=24, N=14336, K=4096, ldx=4096, ldy=14336, group_size=128, **far),
             dict(M=256, N=512, K=8192, ldx=8192, ldy=512, group_size=128, **far),       # GEMM
             dict(W8, **far),                                                            # W8A8 activations
             dict(K=1024, ldx=1024, group_size=128, flags=lowbit_hip.FLAG_COMPACT_GROUPS, **far)]
    for over in cases:
        base = args(**over)
        status, plain, message = workspace(base)
        assert status == 0, message
        flagged = args(**over)
        flagged.flags |= Z
        status, size, message = workspace(flagged)
        assert status == 0 and size == R + plain, (over, plain, size, message)
    lib = lowbit_hip.library()
    big = args(M=64, N=8200, K=1024, group_size=32, ldx=1024, ldy=8200, x=0x10000000, y=0x20000000,
               scales=0x30000000, codes=0x40000000, flags=lowbit_hip.FLAG_COMPACT_GROUPS | Z)
    assert lib.lb_linear_noalloc(ctypes.byref(big), None) == lowbit_hip.INVALID_ARGUMENT
    assert 'scratch' in lib.lb_last_error().decode()


@pytest.mark.parametrize('over', [dict(), dict(group_size=64), dict(group_size=128), dict(K=4096, ldx=4096, group_size=4096),
                                  dict(format=0, group_size=16), dict(format=0, K=576, ldx=576, group_size=576),
                                  dict(M=8, group_size=64), dict(M=16, group_size=128), dict(M=3, format=0, group_size=64),
                                  dict(M=17, group_size=128), dict(M=32, group_size=32), dict(M=24, format=0, group_size=16)])
def test_force_stream_accepts_and_needs_no_workspace(over):
    status, size, message = workspace(args(flags=S, **over))
    assert (status, size) == (0, 0), message


def test_variant_workspace_sizes():
    # compact: fp16 pieces [groups, M, N]; one group is the default graph (no workspace at M=1)
    status, size, message = workspace(args(M=3, flags=lowbit_hip.FLAG_COMPACT_GROUPS))
    assert status == 0, message
    assert size == (128 // 32) * 3 * 64 * 2
    status, size, _ = workspace(args(group_size=128, flags=lowbit_hip.FLAG_COMPACT_GROUPS))
    assert (status, size) == (0, 0)
    # W8A8 with K % 64 == 0: the quantized activations int8 [M, K], 256-byte rounded
    status, size, message = workspace(args(M=5, **W8))
    assert status == 0, message
    assert size == 5 * 128 + 128  # 640 rounded up to 768
    # W8A8 on the generic path (K not a multiple of 64) quantizes as it reads: no workspace
    status, size, _ = workspace(args(M=5, **dict(W8, K=96, ldx=96, group_size=96)))
    assert (status, size) == (0, 0)


# --- operand checks of the Python binding (before any launch; no GPU needed) ----------------------------

def _operands(**over):
    n, k, g = 8, 64, 32
    base = dict(x=torch.zeros(2, k, dtype=torch.float16), codes=torch.zeros(n * k // 2, dtype=torch.uint8),
                scales=torch.zeros(n, k // g, dtype=torch.float16), format='int4', N=n, K=k, group_size=g,
                y=torch.zeros(2, n, dtype=torch.float16), bias=torch.zeros(n, dtype=torch.float16),
                down=torch.zeros(4, k, dtype=torch.float16), up=torch.zeros(n, 4, dtype=torch.float16), rank=4)
    base.update(over)
    return base


@pytest.mark.parametrize('over, needle', [
    (dict(codes=torch.zeros(8 * 64 // 2, dtype=torch.float32)), 'codes'),
    (dict(codes=torch.zeros(8 * 64 // 2 - 1, dtype=torch.uint8)), 'codes'),
    (dict(codes=torch.zeros(8 * 64, dtype=torch.uint8)[::2]), 'codes'),
    (dict(scales=torch.zeros(8, 2, dtype=torch.float32)), 'scales'),
    (dict(scales=torch.zeros(2, 8, dtype=torch.float16).t()), 'scales'),
    (dict(scales=torch.zeros(8, 1, dtype=torch.float16)), 'scales'),
    (dict(scales=None), 'scales'),
    (dict(bias=torch.zeros(8, dtype=torch.float32)), 'bias'),
    (dict(bias=torch.zeros(16, dtype=torch.float16)[::2]), 'bias'),
    (dict(down=torch.zeros(4, 32, dtype=torch.float16)), 'down'),
    (dict(up=torch.zeros(8, 2, dtype=torch.float16)), 'up'),
    (dict(up=torch.zeros(8, 4, dtype=torch.float32)), 'up'),
    (dict(y=torch.zeros(2, 9, dtype=torch.float16)), 'out'),
    (dict(y=torch.zeros(8, 2, dtype=torch.float16).t()), 'out'),
    (dict(x=torch.zeros(2, 64, dtype=torch.float32)), 'x'),
    (dict(group_size=48), 'group_size'),
    (dict(rank=0), 'rank'),
    (dict(format='fp16'), 'codes'),
    (dict(format='int5'), 'format'),
    (dict(N=True), 'N'),
])
def test_operand_checks_raise_value_error(over, needle):
    import lowbit_hip
    with pytest.raises(ValueError, match=needle):
        lowbit_hip.check_operands(**_operands(**over))


def test_operand_checks_require_the_device():
    """Well-formed host tensors still fail: every operand must sit on x's ROCm device."""
    import lowbit_hip
    with pytest.raises(ValueError, match='ROCm device'):
        lowbit_hip.check_operands(**_operands())
    with pytest.raises(ValueError, match='ROCm device'):
        lowbit_hip.linear(torch.zeros(1, 64, dtype=torch.float16), torch.zeros(256, dtype=torch.uint8),
                          torch.zeros(8, 2, dtype=torch.float16), format='int4', N=8, K=64, group_size=32)


def test_noalloc_entry_refuses_workspace_and_oversized_calls():
    """lb_linear_noalloc checks everything on the host before touching a device: a caller
    workspace is refused, and so is a call needing more than the library's scratch."""
    lib = lowbit_hip.library()
    a = args(N=1024, K=14336, ldx=14336, ldy=1024, group_size=128, x=0x1000000, y=0x2000000,
             scales=0x3000000, codes=0x4000000, flags=lowbit_hip.FLAG_FORCE_GEMV, workspace=0x8000000,
             workspace_bytes=1 << 20)
    assert lib.lb_linear_noalloc(ctypes.byref(a), None) == lowbit_hip.INVALID_ARGUMENT
    assert 'workspace' in lib.lb_last_error().decode()
    big = args(M=64, N=8200, K=1024, group_size=32, ldx=1024, ldy=8200, x=0x10000000, y=0x20000000,
               scales=0x30000000, codes=0x40000000, flags=lowbit_hip.FLAG_COMPACT_GROUPS)
    status, need, _ = workspace(big)
    assert status == 0 and need > lowbit_hip.NOALLOC_SCRATCH_BYTES
    assert lib.lb_linear_noalloc(ctypes.byref(big), None) == lowbit_hip.INVALID_ARGUMENT
    assert 'scratch' in lib.lb_last_error().decode()
    assert lib.lb_linear_noalloc(None, None) == lowbit_hip.INVALID_ARGUMENT


def test_decode_check_and_release_argument_errors():
    """lb_decode_check and lb_decode_stack_release reject bad arguments before any device call;
    the timeout offsets match the header's workspace layouts."""
    lib = lowbit_hip.library()
    word = ctypes.c_uint32(7)
    for ws, offset in ((None, 8), (0x10010, 8), (0x10000, 6)):
        assert lib.lb_decode_check(ws, offset, None, ctypes.byref(word)) == lowbit_hip.INVALID_ARGUMENT
        assert '256-byte aligned' in lib.lb_last_error().decode()
        assert word.value == 0
    assert lib.lb_decode_stack_release(0x10000) == lowbit_hip.INVALID_ARGUMENT
    assert 'not prepared' in lib.lb_last_error().decode()
    assert lib.lb_decode_stack_release(None) == lowbit_hip.INVALID_ARGUMENT
    assert lowbit_hip.FUSED_TIMEOUT_OFFSET == 392 < lowbit_hip.FUSED_WORKSPACE_BYTES
    assert lowbit_hip.DECODE_TIMEOUT_OFFSET == 8
    assert lowbit_hip.attention_timeout_offset(9, 384) == 9 * 8 * 128 + 8
    header = (HEADERS[0].parent / 'lowbit_decode_hip.h').read_text()
    assert '#define LB_FUSED_TIMEOUT_OFFSET 392u' in header and '#define LB_DECODE_TIMEOUT_OFFSET 8u' in header


def test_failed_state_refuses_every_enqueueing_entry():
    """After a reported device failure the library refuses work (reference backend.cpp:58-60,
    280-292).  Forced from the host in a child process: the state lasts until the process ends."""
    import subprocess
    import sys
    code = r'''
import ctypes, sys
sys.path[:0] = sys.argv[1:]
import lowbit_hip
lib = lowbit_hip.library()
assert lib.lb_failed() == 0 and not lowbit_hip.failed()
a = lowbit_hip.LinearArgs(); a.struct_size = ctypes.sizeof(a)
a.format, a.M, a.N, a.K, a.group_size = 1, 1, 64, 128, 32
a.codes, a.scales, a.x, a.y, a.ldx, a.ldy = 0x10000, 0x20000, 0x30000, 0x40000, 128, 64
lowbit_hip.mark_failed('forced by the test')
assert lib.lb_failed() == 1 and lowbit_hip.failed()
calls = [('lb_linear', lambda: lib.lb_linear(ctypes.byref(a), None)),
         ('lb_linear_noalloc', lambda: lib.lb_linear_noalloc(ctypes.byref(a), None)),
         ('lb_unpack_codes', lambda: lib.lb_unpack_codes(1, 64, 128, 0x10000, 0x50000, None)),
         ('lb_dequantize', lambda: lib.lb_dequantize(1, 64, 128, 32, 0x10000, 0x20000, 0x50000, None)),
         ('lb_fused_linear', lambda: lib.lb_fused_linear(ctypes.byref(lowbit_hip.FusedLinearArgs()), None)),
         ('lb_decode_attention', lambda: lib.lb_decode_attention(ctypes.byref(lowbit_hip.DecodeAttentionArgs()), None)),
         ('lb_argmax_next', lambda: lib.lb_argmax_next(0x1, 16, 0x2, 8, 0x3, 0x4, 0x5, 0x6, 4, None)),
         ('lb_head_next', lambda: lib.lb_head_next(ctypes.byref(lowbit_hip.FusedLinearArgs()), 0x1, 0x2, 0x3, 0x4, 0x5,
                                                   4, None))]
for name, call in calls:
    assert call() == lowbit_hip.DEVICE_FAILED, name
    message = lib.lb_last_error().decode()
    assert 'restart the process' in message and 'forced by the test' in message, message
size = ctypes.c_size_t(0)
assert lib.lb_workspace_bytes(ctypes.byref(a), ctypes.byref(size)) == 0   # host-only queries still answer
try:
    import torch
    lowbit_hip.check_operands  # the Python wrappers raise RuntimeError from the status
    lowbit_hip._check(lowbit_hip.DEVICE_FAILED, 'lb_linear')
except RuntimeError as error:
    assert 'LB_DEVICE_FAILED' in str(error)
else:
    raise AssertionError('no RuntimeError')
print('ok')
'''
    root = Path(__file__).resolve().parents[1]
    out = subprocess.run([sys.executable, '-c', code, str(root), str(root / 'torch-intel-npu_amd')],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip().endswith('ok'), out.stdout + out.stderr
    assert not lowbit_hip.failed()   # this process is untouched
