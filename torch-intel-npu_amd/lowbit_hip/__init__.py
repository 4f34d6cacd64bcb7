"""ctypes binding of liblowbit_hip.so (the gfx950 low-bit linear C-ABI).

PyTorch-ROCm supplies device memory and the current HIP stream; every computation
runs in the HIP library.  There is no CPU or PyTorch fallback: if the library is
missing or fails to load, the first call raises.

The wrappers follow the reference's error split (torch_npu_lowbit.py:343-352,
torch_intel_npu.py:516-521): contract violations raise ValueError before any
launch, native failures raise RuntimeError carrying lb_last_error().
"""
import ctypes
import os
from pathlib import Path

import torch

LIBRARY_PATH = Path(os.environ.get('LOWBIT_HIP_LIBRARY', Path(__file__).resolve().parent.parent / 'liblowbit_hip.so'))

ABI_VERSION = 6
OK, INVALID_ARGUMENT, OUT_OF_MEMORY, UNSUPPORTED, DEVICE_FAILED, INTERNAL = 0, 1, 2, 5, 10, 12
FORMATS = {'int8': 0, 'int4': 1, 'nf4': 2, 'fp16': 3}
FLAG_FORCE_GEMV, FLAG_FORCE_GEMM, FLAG_FORCE_GENERIC, FLAG_FORCE_STREAM, FLAG_FORCE_WIDE = 0x1, 0x2, 0x4, 0x20, 0x40
FLAG_COMPACT_GROUPS, FLAG_W8A8 = 0x8, 0x10
# LB_FLAG_ZEROED_WORKSPACE / LB_ZEROED_WORKSPACE_BYTES: the workspace starts with that many zero bytes
# the library keeps zero (its counters); the wrappers set it on the workspaces they allocate.
FLAG_ZEROED_WORKSPACE, ZEROED_WORKSPACE_BYTES = 0x80, 4096
EXPORTS = ('lb_abi_version', 'lb_status_name', 'lb_last_error', 'lb_failed', 'lb_mark_failed',
           'lb_workspace_bytes', 'lb_linear', 'lb_linear_noalloc', 'lb_unpack_codes', 'lb_dequantize')
NOALLOC_SCRATCH_BYTES = 32 << 20   # LB_NOALLOC_SCRATCH_BYTES
DECODE_EXPORTS = ('lb_fused_linear', 'lb_decode_attention', 'lb_argmax_next', 'lb_head_next', 'lb_decode_layer',
                  'lb_decode_stack_prepare', 'lb_decode_stack', 'lb_decode_stack_release', 'lb_decode_check')
PROLOGUES = {'none': 0, 'rmsnorm': 1, 'silu_mul': 2}
MAX_PROBLEMS, MAX_RANK, MAX_FUSED_K = 3, 32, 1536
def attention_workspace_bytes(heads, capacity):
    """LB_ATTN_WORKSPACE_BYTES: tagged score words [heads][ceil(capacity / 48) * 16], launch count, timeout."""
    return heads * ((capacity + 47) // 48) * 128 + 16


FUSED_WORKSPACE_BYTES = 512  # LB_FUSED_WORKSPACE_BYTES: tagged z words [3][12] u64, launch count u64, timeout u32
FUSED_TIMEOUT_OFFSET = 392   # LB_FUSED_TIMEOUT_OFFSET
DECODE_TIMEOUT_OFFSET = 8    # LB_DECODE_TIMEOUT_OFFSET (lb_decode_layer / lb_decode_stack workspaces)


def head_next_workspace_bytes(vocab):
    """LB_HEAD_NEXT_WORKSPACE_BYTES: room for a maximum word and a counter (u64) per group of 8
    workgroups of 64 rows, and one pair for the total."""
    wgs = (vocab + 63) // 64
    return 16 * ((wgs + 7) // 8 + 1)


def attention_timeout_offset(heads, capacity):
    """LB_ATTN_TIMEOUT_OFFSET: the timeout word of a split-attention workspace."""
    return attention_workspace_bytes(heads, capacity) - 8


class LinearArgs(ctypes.Structure):
    """Mirror of lb_linear_args (include/lowbit_hip.h)."""
    _fields_ = [('struct_size', ctypes.c_uint32), ('format', ctypes.c_uint32),
                ('M', ctypes.c_int64), ('N', ctypes.c_int64), ('K', ctypes.c_int64),
                ('group_size', ctypes.c_int64),
                ('codes', ctypes.c_void_p), ('scales', ctypes.c_void_p),
                ('x', ctypes.c_void_p), ('ldx', ctypes.c_int64),
                ('y', ctypes.c_void_p), ('ldy', ctypes.c_int64),
                ('bias', ctypes.c_void_p),
                ('rank', ctypes.c_int64), ('down', ctypes.c_void_p), ('up', ctypes.c_void_p),
                ('up_ld', ctypes.c_int64),
                ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_size_t),
                ('flags', ctypes.c_uint32), ('reserved', ctypes.c_uint32),
                ('activation_scale', ctypes.c_float), ('reserved2', ctypes.c_uint32)]


class FusedProblem(ctypes.Structure):
    """Mirror of lb_fused_problem (include/lowbit_decode_hip.h)."""
    _fields_ = [('codes', ctypes.c_void_p), ('scales', ctypes.c_void_p), ('N', ctypes.c_int64),
                ('y', ctypes.c_void_p), ('bias', ctypes.c_void_p), ('residual', ctypes.c_void_p),
                ('rank', ctypes.c_int64), ('down', ctypes.c_void_p), ('up', ctypes.c_void_p),
                ('up_ld', ctypes.c_int64)]


class FusedLinearArgs(ctypes.Structure):
    """Mirror of lb_fused_linear_args."""
    _fields_ = [('struct_size', ctypes.c_uint32), ('format', ctypes.c_uint32),
                ('K', ctypes.c_int64), ('group_size', ctypes.c_int64),
                ('prologue', ctypes.c_uint32), ('count', ctypes.c_uint32),
                ('x', ctypes.c_void_p), ('x2', ctypes.c_void_p), ('gamma', ctypes.c_void_p),
                ('eps', ctypes.c_float), ('reserved', ctypes.c_uint32),
                ('problems', FusedProblem * 3),
                ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_size_t)]


class DecodeAttentionArgs(ctypes.Structure):
    """Mirror of lb_decode_attention_args."""
    _fields_ = [('struct_size', ctypes.c_uint32), ('reserved', ctypes.c_uint32),
                ('heads', ctypes.c_int64), ('kv_heads', ctypes.c_int64), ('head_dim', ctypes.c_int64),
                ('capacity', ctypes.c_int64),
                ('q', ctypes.c_void_p), ('k', ctypes.c_void_p), ('v', ctypes.c_void_p),
                ('cos', ctypes.c_void_p), ('sin', ctypes.c_void_p), ('position', ctypes.c_void_p),
                ('keys', ctypes.c_void_p), ('values', ctypes.c_void_p), ('out', ctypes.c_void_p),
                ('scale', ctypes.c_float), ('reserved2', ctypes.c_uint32),
                ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_size_t)]


class DecodeLayerArgs(ctypes.Structure):
    """Mirror of lb_decode_layer_args."""
    _fields_ = [('struct_size', ctypes.c_uint32), ('format', ctypes.c_uint32),
                ('group_size', ctypes.c_int64), ('hidden', ctypes.c_int64), ('intermediate', ctypes.c_int64),
                ('h', ctypes.c_void_p), ('norm1', ctypes.c_void_p), ('norm2', ctypes.c_void_p),
                ('eps', ctypes.c_float), ('reserved', ctypes.c_uint32),
                ('proj', FusedProblem * 7),
                ('heads', ctypes.c_int64), ('kv_heads', ctypes.c_int64), ('capacity', ctypes.c_int64),
                ('cos', ctypes.c_void_p), ('sin', ctypes.c_void_p), ('position', ctypes.c_void_p),
                ('keys', ctypes.c_void_p), ('values', ctypes.c_void_p),
                ('scale', ctypes.c_float), ('reserved2', ctypes.c_uint32),
                ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_size_t)]


def layer_words(hidden, intermediate, kv_heads):
    """LB_DECODE_LAYER_WORDS: words of one layer's region of a decode-layer workspace."""
    return (224 + (hidden + 128 * kv_heads) // 2 + 3 * hidden // 2 + intermediate + 31) // 32 * 32


def layer_workspace_bytes(hidden, intermediate, kv_heads):
    """LB_DECODE_LAYER_WORKSPACE_BYTES."""
    return 8 * (8 + layer_words(hidden, intermediate, kv_heads))


STACK_MAX_LAYERS = 64


def stack_workspace_bytes(hidden, intermediate, kv_heads, layers):
    """LB_DECODE_STACK_WORKSPACE_BYTES."""
    return 8 * (8 + layers * layer_words(hidden, intermediate, kv_heads))


def stack_table_bytes(layers):
    """LB_DECODE_STACK_TABLE_BYTES."""
    return 256 * layers


class DecodeStackLayer(ctypes.Structure):
    """Mirror of lb_decode_stack_layer."""
    _fields_ = [('norm1', ctypes.c_void_p), ('norm2', ctypes.c_void_p), ('proj', FusedProblem * 7),
                ('keys', ctypes.c_void_p), ('values', ctypes.c_void_p)]


class DecodeStackArgs(ctypes.Structure):
    """Mirror of lb_decode_stack_args."""
    _fields_ = [('struct_size', ctypes.c_uint32), ('format', ctypes.c_uint32),
                ('group_size', ctypes.c_int64), ('hidden', ctypes.c_int64), ('intermediate', ctypes.c_int64),
                ('layers', ctypes.c_int64), ('layer', ctypes.POINTER(DecodeStackLayer)),
                ('h', ctypes.c_void_p), ('eps', ctypes.c_float), ('reserved', ctypes.c_uint32),
                ('heads', ctypes.c_int64), ('kv_heads', ctypes.c_int64), ('capacity', ctypes.c_int64),
                ('cos', ctypes.c_void_p), ('sin', ctypes.c_void_p), ('position', ctypes.c_void_p),
                ('scale', ctypes.c_float), ('reserved2', ctypes.c_uint32),
                ('table', ctypes.c_void_p), ('table_bytes', ctypes.c_size_t),
                ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_size_t)]


_lib = None


def library():
    """Load (once) and return the ctypes handle; raises if the HIP library is absent."""
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            raise RuntimeError(f'{LIBRARY_PATH} is missing: build it with __graft_entry__.build() '
                               'or torch-intel-npu_amd/build.py (no CPU fallback exists)')
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        lib.lb_abi_version.restype = ctypes.c_int
        lib.lb_status_name.restype = ctypes.c_char_p
        lib.lb_status_name.argtypes = [ctypes.c_int]
        lib.lb_last_error.restype = ctypes.c_char_p
        lib.lb_failed.restype = ctypes.c_int
        lib.lb_failed.argtypes = []
        lib.lb_mark_failed.restype = None
        lib.lb_mark_failed.argtypes = [ctypes.c_char_p]
        lib.lb_workspace_bytes.restype = ctypes.c_int
        lib.lb_workspace_bytes.argtypes = [ctypes.POINTER(LinearArgs), ctypes.POINTER(ctypes.c_size_t)]
        lib.lb_linear.restype = ctypes.c_int
        lib.lb_linear.argtypes = [ctypes.POINTER(LinearArgs), ctypes.c_void_p]
        lib.lb_linear_noalloc.restype = ctypes.c_int
        lib.lb_linear_noalloc.argtypes = [ctypes.POINTER(LinearArgs), ctypes.c_void_p]
        lib.lb_unpack_codes.restype = ctypes.c_int
        lib.lb_unpack_codes.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p]
        lib.lb_dequantize.restype = ctypes.c_int
        lib.lb_dequantize.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.lb_fused_linear.restype = ctypes.c_int
        lib.lb_fused_linear.argtypes = [ctypes.POINTER(FusedLinearArgs), ctypes.c_void_p]
        lib.lb_decode_attention.restype = ctypes.c_int
        lib.lb_decode_attention.argtypes = [ctypes.POINTER(DecodeAttentionArgs), ctypes.c_void_p]
        lib.lb_decode_layer.restype = ctypes.c_int
        lib.lb_decode_layer.argtypes = [ctypes.POINTER(DecodeLayerArgs), ctypes.c_void_p]
        for name in ('lb_decode_stack_prepare', 'lb_decode_stack'):
            getattr(lib, name).restype = ctypes.c_int
            getattr(lib, name).argtypes = [ctypes.POINTER(DecodeStackArgs), ctypes.c_void_p]
        lib.lb_decode_stack_release.restype = ctypes.c_int
        lib.lb_decode_stack_release.argtypes = [ctypes.c_void_p]
        lib.lb_decode_check.restype = ctypes.c_int
        lib.lb_decode_check.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                        ctypes.POINTER(ctypes.c_uint32)]
        lib.lb_argmax_next.restype = ctypes.c_int
        lib.lb_argmax_next.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_void_p]
        lib.lb_head_next.restype = ctypes.c_int
        lib.lb_head_next.argtypes = [ctypes.POINTER(FusedLinearArgs), ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                     ctypes.c_void_p]
        if lib.lb_abi_version() != ABI_VERSION:
            raise RuntimeError(f'liblowbit_hip ABI {lib.lb_abi_version()} != expected {ABI_VERSION}')
        _lib = lib
    return _lib


def status_name(status):
    return library().lb_status_name(status).decode()


def _check(status, what):
    if status != OK:
        message = library().lb_last_error().decode()
        error = ValueError if status == INVALID_ARGUMENT else RuntimeError
        raise error(f'{what} failed with {status_name(status)}: {message}')


def failed():
    """True once the library refuses work after a device failure (restart the process)."""
    return bool(library().lb_failed())


def mark_failed(reason):
    """Put the library in its failed state: every later call raises RuntimeError (LB_DEVICE_FAILED)."""
    library().lb_mark_failed(str(reason).encode()[:200])


def synchronize(device=None):
    """torch.cuda.synchronize; a device error found there marks the library failed, then re-raises
    (the library itself never waits on the device, so this is where an asynchronous fault shows)."""
    try:
        torch.cuda.synchronize(device)
    except RuntimeError as error:
        mark_failed(f'synchronisation failed: {error}')
        raise


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _device_tensor(t, name, dtype=None):
    if not isinstance(t, torch.Tensor) or t.device.type != 'cuda':
        raise ValueError(f'{name} must be a ROCm device tensor')
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f'{name} must be {dtype}')
    return t


def _code_bytes(format, N, K):
    return N * K * 2 if format == 'fp16' else N * K if format == 'int8' else (N * K + 1) // 2


def check_operands(x, codes, scales, *, format, N, K, group_size, y=None, bias=None, down=None, up=None, rank=0):
    """Every operand of one lb_linear call, before anything reaches the library: dtype, size and
    layout first (so a wrong operand is named whatever its device), then the device -- all on
    x's ROCm device.  The C side checks only pointers and alignment, so a host tensor or a
    strided view caught here would otherwise be read as device memory of the wrong layout."""
    if format not in FORMATS:
        raise ValueError(f'unknown format {format!r}')
    for name, value in (('N', N), ('K', K), ('group_size', group_size), ('rank', rank)):
        if isinstance(value, bool) or not hasattr(value, '__index__') or value < (0 if name == 'rank' else 1):
            raise ValueError(f'{name} must be a positive integer')
    if K % group_size:
        raise ValueError('group_size must divide K')
    if not isinstance(x, torch.Tensor) or x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != K:
        raise ValueError('x must be fp16 [M, K]')
    operands = [('x', x)]
    code_types = (torch.float16,) if format == 'fp16' else (torch.uint8, torch.int8)
    if not isinstance(codes, torch.Tensor) or codes.dtype not in code_types:
        raise ValueError(f'codes must be a {" or ".join(map(str, code_types))} tensor for format {format}')
    if not codes.is_contiguous() or codes.numel() * codes.element_size() < _code_bytes(format, N, K):
        raise ValueError(f'codes must be contiguous with the packed bytes of a {N}x{K} {format} weight')
    operands.append(('codes', codes))
    if format == 'fp16':
        if scales is not None:
            raise ValueError('fp16 weights take no scales')
    else:
        if not isinstance(scales, torch.Tensor) or scales.dtype != torch.float16:
            raise ValueError('scales must be an fp16 tensor')
        if not scales.is_contiguous() or scales.numel() < N * (K // group_size):
            raise ValueError(f'scales must be contiguous fp16 [N, K/group_size] = [{N}, {K // group_size}]')
        operands.append(('scales', scales))
    if y is not None:
        if (not isinstance(y, torch.Tensor) or y.dtype != torch.float16 or tuple(y.shape) != (x.shape[0], N)
                or (N > 1 and y.stride(1) != 1)):
            raise ValueError(f'out must be fp16 [M, N] = [{x.shape[0]}, {N}] with unit column stride')
        operands.append(('out', y))
    if bias is not None:
        if (not isinstance(bias, torch.Tensor) or bias.dtype != torch.float16 or not bias.is_contiguous()
                or bias.numel() != N):
            raise ValueError(f'bias must be contiguous fp16 [{N}]')
        operands.append(('bias', bias))
    if rank:
        if (not isinstance(down, torch.Tensor) or down.dtype != torch.float16 or down.ndim != 2
                or tuple(down.shape) != (rank, K)):
            raise ValueError(f'down must be fp16 [rank, K] = [{rank}, {K}]')
        if (not isinstance(up, torch.Tensor) or up.dtype != torch.float16 or up.ndim != 2
                or up.shape[0] != N or up.shape[1] < rank):
            raise ValueError(f'up must be fp16 [N, >= rank] = [{N}, >= {rank}]')
        operands += [('down', down), ('up', up)]
    elif down is not None or up is not None:
        raise ValueError('down/up need rank > 0')
    if x.device.type != 'cuda':
        raise ValueError('x must be a ROCm device tensor')
    for name, t in operands:
        if t.device != x.device:
            raise ValueError(f'{name} must be on {x.device} with x (found {t.device})')


def make_args(x, codes, scales, *, format, N, K, group_size, y, bias=None, down=None, up=None, rank=0,
              flags=0, activation_scale=None):
    """Fill an lb_linear_args for device tensors; x and y are 2-D views with unit column stride."""
    args = LinearArgs()
    args.struct_size = ctypes.sizeof(LinearArgs)
    args.format = FORMATS[format]
    args.M, args.N, args.K = x.shape[0], N, K
    args.group_size = group_size
    args.codes, args.scales = _ptr(codes), _ptr(scales)
    args.x, args.ldx = _ptr(x), x.stride(0) if x.shape[0] > 1 else K
    args.y, args.ldy = _ptr(y), y.stride(0) if y.shape[0] > 1 else N
    args.bias = _ptr(bias)
    args.rank = rank
    if rank:
        args.down, args.up = _ptr(down), _ptr(up)
        args.up_ld = up.stride(0)
    args.flags = flags
    if activation_scale is not None:
        args.flags |= FLAG_W8A8
        args.activation_scale = activation_scale
    return args


def workspace_bytes(args):
    size = ctypes.c_size_t(0)
    _check(library().lb_workspace_bytes(ctypes.byref(args), ctypes.byref(size)), 'lb_workspace_bytes')
    return size.value


def linear(x, codes, scales, *, format, N, K, group_size, bias=None, down=None, up=None, rank=0, flags=0,
           out=None, workspace=None, activation_scale=None):
    """y[M,N] fp16 = x . dequant(W)^T (+bias) (+fp16(fp16(x.V^T).U^T)) on the current stream.

    x: fp16 [M,K] cuda (unit column stride).  codes: uint8 (or fp16 for format='fp16').
    scales: fp16 [N, K/group_size].  down: fp16 [rank,K] (row stride K); up: fp16 [N, >=rank].
    flags may add FLAG_COMPACT_GROUPS; activation_scale (a power of two) selects W8A8.
    """
    check_operands(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=out, bias=bias,
                   down=down, up=up, rank=rank)
    if K > 1 and x.stride(1) != 1:
        x = x.contiguous()
    if rank:
        if down.stride(-1) != 1 or down.stride(0) != K:
            down = down.contiguous()
        if up.stride(-1) != 1:
            up = up.contiguous()
    M = x.shape[0]
    y = torch.empty((M, N), dtype=torch.float16, device=x.device) if out is None else out
    args = make_args(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=y, bias=bias,
                     down=down, up=up, rank=rank, flags=flags, activation_scale=activation_scale)
    need = workspace_bytes(args)
    if need:
        if workspace is None or workspace.numel() < need:
            workspace = zeroed_workspace(args, x.device)
        args.workspace, args.workspace_bytes = _ptr(workspace), workspace.numel()
    _check(library().lb_linear(ctypes.byref(args), _stream(x.device)), 'lb_linear')
    return y


def zeroed_workspace(args, device):
    """A workspace allocated zeroed for `args`, with FLAG_ZEROED_WORKSPACE added to args.flags (the
    library keeps its first ZEROED_WORKSPACE_BYTES zero across the calls that use it)."""
    args.flags |= FLAG_ZEROED_WORKSPACE
    return torch.zeros(workspace_bytes(args), dtype=torch.uint8, device=device)


def linear_noalloc(x, codes, scales, *, out, format, N, K, group_size, bias=None, down=None, up=None, rank=0,
                   flags=0, activation_scale=None):
    """lb_linear_noalloc: the same product as linear() into the caller's `out`, with no device
    allocation by the library or by this wrapper (the scratch is the library's per-GPU array of
    NOALLOC_SCRATCH_BYTES).  Operands must already have the layouts the call needs (no copies
    are made); a call needing more scratch raises ValueError.  Calls overlapping on one GPU race."""
    check_operands(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=out, bias=bias,
                   down=down, up=up, rank=rank)
    if out is None:
        raise ValueError('linear_noalloc writes into a caller-provided out')
    if K > 1 and x.stride(1) != 1:
        raise ValueError('linear_noalloc needs x with unit column stride')
    if rank and (down.stride(-1) != 1 or down.stride(0) != K or up.stride(-1) != 1):
        raise ValueError('linear_noalloc needs row-major down [rank, K] and up with unit column stride')
    args = make_args(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=out, bias=bias,
                     down=down, up=up, rank=rank, flags=flags, activation_scale=activation_scale)
    _check(library().lb_linear_noalloc(ctypes.byref(args), _stream(x.device)), 'lb_linear_noalloc')
    return out


def unpack_codes(codes, *, format, N, K):
    """Bit-exact decoded integers int8 [N,K]: int8 value, int4 ((c^8)-8), nf4 code index."""
    _device_tensor(codes, 'codes', torch.uint8)
    out = torch.empty((N, K), dtype=torch.int8, device=codes.device)
    _check(library().lb_unpack_codes(FORMATS[format], N, K, _ptr(codes), _ptr(out), _stream(codes.device)),
           'lb_unpack_codes')
    return out


def dequantize(codes, scales, *, format, N, K, group_size):
    """fp16 [N,K] = fp16(q*s), bit-identical to PackedWeight.dequantize()."""
    _device_tensor(codes, 'codes', torch.uint8)
    _device_tensor(scales, 'scales', torch.float16)
    out = torch.empty((N, K), dtype=torch.float16, device=codes.device)
    _check(library().lb_dequantize(FORMATS[format], N, K, group_size, _ptr(codes), _ptr(scales), _ptr(out),
                                   _stream(codes.device)), 'lb_dequantize')
    return out


class PreparedLinear:
    """A fixed lb_linear call (shapes, buffers and workspace bound once) for hot loops.

    Holds references to every tensor it points at, so the device memory stays alive.
    run() enqueues on the current stream of the output's device (or `stream`), so it can be
    captured into a HIP graph with torch.cuda.graph.
    """

    def __init__(self, x, codes, scales, *, format, N, K, group_size, out, bias=None, down=None, up=None,
                 rank=0, flags=0, workspace=None, activation_scale=None):
        check_operands(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=out, bias=bias,
                       down=down, up=up, rank=rank)
        if K > 1 and x.stride(1) != 1:
            raise ValueError('PreparedLinear needs x [M, K] with unit column stride')
        if rank:
            if down.stride(-1) != 1 or down.stride(0) != K:
                down = down.contiguous()
            if up.stride(-1) != 1:
                up = up.contiguous()
        self._keep = [x, codes, scales, out, bias, down, up]
        self.args = make_args(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=out,
                              bias=bias, down=down, up=up, rank=rank, flags=flags,
                              activation_scale=activation_scale)
        need = workspace_bytes(self.args)
        if need:
            if workspace is None or workspace.numel() < need:
                workspace = zeroed_workspace(self.args, x.device)
                need = workspace.numel()
            self.args.workspace, self.args.workspace_bytes = _ptr(workspace), workspace.numel()
            self._keep.append(workspace)
        self.workspace = workspace if need else None
        self.workspace_bytes = need
        self.out = out
        self._ref = ctypes.byref(self.args)
        self._fn = library().lb_linear
        self._device = x.device

    def run(self, stream=None):
        handle = torch.cuda.current_stream(self._device).cuda_stream if stream is None else stream
        status = self._fn(self._ref, ctypes.c_void_p(handle))
        if status != OK:
            _check(status, 'lb_linear')
        return self.out


# ---------------------------------------------------------------- decode-step entry points
def _row(t, name, count, dtype=torch.float16):
    """A contiguous device row of at least `count` elements (views into larger buffers are fine)."""
    _device_tensor(t, name, dtype)
    if not t.is_contiguous() or t.numel() < count:
        raise ValueError(f'{name} must be contiguous with at least {count} elements')
    return t


def check_workspace(workspace, timeout_offset, what='lb_decode_check', stream=None):
    """lb_decode_check: synchronise the stream, then read the workspace's timeout word.  Nonzero
    means a bounded hand-over wait of a call on it gave up, so its outputs are not valid: the
    library enters its failed state (every later call raises) and this raises RuntimeError, as the
    reference's failed context does (npunlock-probe/torch-device/backend.cpp:280-292)."""
    handle = torch.cuda.current_stream(workspace.device).cuda_stream if stream is None else stream
    word = ctypes.c_uint32(0)
    status = library().lb_decode_check(_ptr(workspace), timeout_offset, ctypes.c_void_p(handle), ctypes.byref(word))
    if status != OK:
        _check(status, what)


class _Prepared:
    """A fixed call of one decode-step entry point; run() enqueues it on the current stream.
    Calls with a hand-over workspace (`workspace`, timeout word at `_timeout_offset`) are checked by
    check() after a synchronisation."""

    workspace = None
    _timeout_offset = None

    def _bind(self, fn, what, args, device, keep):
        self.args, self._keep, self._device, self._what = args, keep, device, what
        self._fn = getattr(library(), fn)
        self._ref = ctypes.byref(args)

    def run(self, stream=None):
        handle = torch.cuda.current_stream(self._device).cuda_stream if stream is None else stream
        status = self._fn(self._ref, ctypes.c_void_p(handle))
        if status != OK:
            _check(status, self._what)

    def check(self, stream=None):
        """Raise RuntimeError (and leave the library failed) if a bounded wait of any run() so far
        gave up; synchronises the stream.  Calls without a workspace have no waits to check."""
        if self.workspace is not None:
            check_workspace(self.workspace, self._timeout_offset, f'{self._what} (workspace check)', stream)


class PreparedFused(_Prepared):
    """One lb_fused_linear call: up to three linears sharing the activation row `x` (K fp16).

    problems: sequence of dicts with keys codes, scales (None for fp16), N, y (fp16 row of N),
    and optionally bias, residual (may be y itself), down [rank,K], up [N,rank] (rank = down rows).
    prologue: 'none', 'rmsnorm' (gamma, eps) or 'silu_mul' (x = gate row, x2 = up row).
    shared_z (default): with corrections, each z = fp16(x'.V^T) is computed once per call by
    dedicated workgroups into a zeroed FUSED_WORKSPACE_BYTES workspace owned by this call;
    False: every workgroup computes z itself (no workspace).
    """

    def __init__(self, x, problems, *, format, K, group_size, prologue='none', x2=None, gamma=None, eps=1e-5,
                 shared_z=True):
        if prologue not in PROLOGUES:
            raise ValueError(f'unknown prologue {prologue!r}')
        if not 1 <= len(problems) <= MAX_PROBLEMS:
            raise ValueError(f'1..{MAX_PROBLEMS} problems per fused call')
        a = FusedLinearArgs()
        a.struct_size = ctypes.sizeof(FusedLinearArgs)
        a.format = FORMATS[format]
        a.K, a.group_size = K, group_size
        a.prologue, a.count = PROLOGUES[prologue], len(problems)
        keep = [_row(x, 'x', K)]
        a.x = _ptr(x)
        if prologue == 'silu_mul':
            keep.append(_row(x2, 'x2', K))
            a.x2 = _ptr(x2)
        if prologue == 'rmsnorm':
            keep.append(_row(gamma, 'gamma', K))
            a.gamma = _ptr(gamma)
        a.eps = eps
        for i, pr in enumerate(problems):
            q = a.problems[i]
            n = pr['N']
            q.N = n
            q.codes = _ptr(pr['codes'])
            q.scales = _ptr(pr.get('scales'))
            q.y = _ptr(_row(pr['y'], 'y', n))
            q.bias = _ptr(pr.get('bias'))
            q.residual = _ptr(pr.get('residual'))
            down, up = pr.get('down'), pr.get('up')
            if down is not None:
                q.rank = down.shape[0]
                q.down, q.up, q.up_ld = _ptr(down.contiguous()), _ptr(up), up.stride(0)
                keep += [down, up]
            keep += [pr['codes'], pr.get('scales'), pr['y'], pr.get('bias'), pr.get('residual')]
        self.workspace = None
        if shared_z and any(pr.get('down') is not None for pr in problems):
            self.workspace = torch.zeros(FUSED_WORKSPACE_BYTES, dtype=torch.uint8, device=x.device)
            a.workspace, a.workspace_bytes = _ptr(self.workspace), FUSED_WORKSPACE_BYTES
            self._timeout_offset = FUSED_TIMEOUT_OFFSET
            keep.append(self.workspace)
        self._bind('lb_fused_linear', 'lb_fused_linear', a, x.device, keep)
        self.outputs = [pr['y'] for pr in problems]

    def counters(self):
        """(tile workgroups counted over all calls so far, timeout word) of the workspace."""
        if self.workspace is None:
            return None
        return [int(self.workspace[384:392].view(torch.int64)), int(self.workspace[392:396].view(torch.int32))]


def fused_linear(x, problems, **options):
    """Run one lb_fused_linear on the current stream; returns the problems' y tensors."""
    call = PreparedFused(x, problems, **options)
    call.run()
    return call.outputs


class PreparedAttention(_Prepared):
    """lb_decode_attention for one token: q [heads*64], k, v [kv_heads*64], position int64 [1].
    split (heads / kv_heads <= 3): scores computed once per 48 positions by dedicated workgroups,
    through a zeroed workspace owned by this call; False (default): every output workgroup computes
    the whole score row (no workspace), the faster form at the SmolLM cache sizes."""

    def __init__(self, q, k, v, cos, sin, position, keys, values, out, *, heads, kv_heads, scale=0.125,
                 split=False):
        capacity = keys.shape[-2]
        a = DecodeAttentionArgs()
        a.struct_size = ctypes.sizeof(DecodeAttentionArgs)
        a.heads, a.kv_heads, a.head_dim, a.capacity = heads, kv_heads, 64, capacity
        rows = ((q, 'q', heads * 64), (k, 'k', kv_heads * 64), (v, 'v', kv_heads * 64),
                (cos, 'cos', capacity * 64), (sin, 'sin', capacity * 64), (keys, 'keys', kv_heads * capacity * 64),
                (values, 'values', kv_heads * capacity * 64), (out, 'out', heads * 64))
        for t, name, count in rows:
            _row(t, name, count)
        _row(position, 'position', 1, torch.int64)
        a.q, a.k, a.v, a.cos, a.sin = _ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin)
        a.position, a.keys, a.values, a.out = _ptr(position), _ptr(keys), _ptr(values), _ptr(out)
        a.scale = scale
        keep = [q, k, v, cos, sin, position, keys, values, out]
        self.workspace = None
        if split and heads // kv_heads <= 3:
            size = attention_workspace_bytes(heads, capacity)
            self.workspace = torch.zeros(size, dtype=torch.uint8, device=q.device)
            a.workspace, a.workspace_bytes = _ptr(self.workspace), size
            self._timeout_offset = attention_timeout_offset(heads, capacity)
            keep.append(self.workspace)
        self._bind('lb_decode_attention', 'lb_decode_attention', a, q.device, keep)
        self.out = out

    def counters(self):
        """(output workgroups counted over all calls so far, timeout word) of the split workspace."""
        if self.workspace is None:
            return None
        tail = self.workspace[-16:]
        return [int(tail[:8].view(torch.int64)), int(tail[8:12].view(torch.int32))]


class PreparedArgmax:
    """lb_argmax_next: greedy token of `logits`, recorded at tokens[position], position += 1,
    h_next = embedding[token]."""

    def __init__(self, logits, embedding, h_next, tokens, token, position, *, limit):
        vocab, hidden = embedding.shape
        _row(logits, 'logits', vocab)
        _row(embedding, 'embedding', vocab * hidden)
        _row(h_next, 'h_next', hidden)
        for t, name in ((tokens, 'tokens'), (token, 'token'), (position, 'position')):
            _row(t, name, 1, torch.int64)
        if tokens.numel() < limit:
            raise ValueError('tokens must hold `limit` entries')
        self._keep = [logits, embedding, h_next, tokens, token, position]
        self._call = (_ptr(logits), vocab, _ptr(embedding), hidden, _ptr(h_next), _ptr(tokens), _ptr(token),
                      _ptr(position), limit)
        self._fn = library().lb_argmax_next
        self._device = logits.device

    def run(self, stream=None):
        handle = torch.cuda.current_stream(self._device).cuda_stream if stream is None else stream
        status = self._fn(*self._call, ctypes.c_void_p(handle))
        if status != OK:
            _check(status, 'lb_argmax_next')


class PreparedHeadNext:
    """lb_head_next: final RMSNorm -> head -> greedy token in one launch, the result of
    PreparedFused(h, [head], prologue='rmsnorm') followed by PreparedArgmax on its logits, with
    h_next = h.  head: dict(codes, scales (None for fp16), N = vocab, y = logits); format 'fp16'
    (K <= 640) or 'int4'.  Owns a zeroed workspace (every run leaves it zero again)."""

    FORMATS = ('fp16', 'int4')

    def __init__(self, h, head, embedding, tokens, token, position, *, format, K, group_size, gamma, eps=1e-5,
                 limit):
        if format not in self.FORMATS or (format == 'fp16' and K > 640):
            raise ValueError('lb_head_next takes fp16 heads of K <= 640 and int4 heads')
        vocab = head['N']
        if embedding.shape != (vocab, K):
            raise ValueError('embedding must be [N, K]')
        for t, name in ((tokens, 'tokens'), (token, 'token'), (position, 'position')):
            _row(t, name, 1, torch.int64)
        if tokens.numel() < limit:
            raise ValueError('tokens must hold `limit` entries')
        _row(embedding, 'embedding', vocab * K)
        self._fused = PreparedFused(h, [head], format=format, K=K, group_size=group_size, prologue='rmsnorm',
                                    gamma=gamma, eps=eps, shared_z=False)
        size = head_next_workspace_bytes(vocab)
        self.workspace = torch.zeros(size, dtype=torch.uint8, device=h.device)
        self._fused.args.workspace, self._fused.args.workspace_bytes = _ptr(self.workspace), size
        self._keep = [embedding, tokens, token, position, self.workspace]
        self._call = (_ptr(embedding), _ptr(h), _ptr(tokens), _ptr(token), _ptr(position), limit)
        self._fn = library().lb_head_next
        self._device = h.device

    def run(self, stream=None):
        handle = torch.cuda.current_stream(self._device).cuda_stream if stream is None else stream
        status = self._fn(self._fused._ref, *self._call, ctypes.c_void_p(handle))
        if status != OK:
            _check(status, 'lb_head_next')


def _fill_projections(proj, projections, keep):
    """The seven lb_fused_problem entries of a layer (U padded to a row stride of 8 where needed)."""
    for i, pr in enumerate(projections):
        q = proj[i]
        q.N = pr['N']
        q.codes, q.scales = _ptr(pr['codes']), _ptr(pr.get('scales'))
        keep += [pr['codes'], pr.get('scales')]
        down, up = pr.get('down'), pr.get('up')
        if down is not None:
            down = down.contiguous()
            if up.stride(-1) != 1 or up.stride(0) % 8:
                padded = torch.zeros((up.shape[0], (up.shape[1] + 7) // 8 * 8), dtype=up.dtype, device=up.device)
                padded[:, :up.shape[1]] = up
                up = padded
            q.rank = down.shape[0]
            q.down, q.up, q.up_ld = _ptr(down), _ptr(up), up.stride(0)
            keep += [down, up]


class PreparedLayer(_Prepared):
    """lb_decode_layer: one decoder layer for one token in one launch.

    h: fp16 [hidden] residual row (input, replaced by the output).  projections: seven dicts
    (q, k, v, o, gate, up, down) with codes, scales (None for fp16), N, and optionally down [rank, K]
    and up [N, rank].  group_size 0 means int8 per row.  cos/sin [capacity, 64], position int64 [1],
    keys/values [kv_heads, capacity, 64].  The call owns a zeroed workspace.
    """

    def __init__(self, h, projections, *, format, group_size, hidden, intermediate, norm1, norm2, eps, heads,
                 kv_heads, cos, sin, position, keys, values, scale=0.125):
        if len(projections) != 7:
            raise ValueError('seven projections: q, k, v, o, gate, up, down')
        capacity = keys.shape[-2]
        a = DecodeLayerArgs()
        a.struct_size = ctypes.sizeof(DecodeLayerArgs)
        a.format = FORMATS[format]
        a.group_size, a.hidden, a.intermediate = group_size, hidden, intermediate
        keep = [_row(h, 'h', hidden), _row(norm1, 'norm1', hidden), _row(norm2, 'norm2', hidden)]
        a.h, a.norm1, a.norm2, a.eps = _ptr(h), _ptr(norm1), _ptr(norm2), eps
        _fill_projections(a.proj, projections, keep)
        for t, name, count in ((cos, 'cos', capacity * 64), (sin, 'sin', capacity * 64),
                               (keys, 'keys', kv_heads * capacity * 64), (values, 'values', kv_heads * capacity * 64)):
            keep.append(_row(t, name, count))
        keep.append(_row(position, 'position', 1, torch.int64))
        a.heads, a.kv_heads, a.capacity = heads, kv_heads, capacity
        a.cos, a.sin, a.position, a.keys, a.values, a.scale = (_ptr(cos), _ptr(sin), _ptr(position), _ptr(keys),
                                                               _ptr(values), scale)
        size = layer_workspace_bytes(hidden, intermediate, kv_heads)
        self.workspace = torch.zeros(size, dtype=torch.uint8, device=h.device)
        a.workspace, a.workspace_bytes = _ptr(self.workspace), size
        self._timeout_offset = DECODE_TIMEOUT_OFFSET
        keep.append(self.workspace)
        self._bind('lb_decode_layer', 'lb_decode_layer', a, h.device, keep)
        self.out = h

    def counters(self):
        """(workgroups counted over all calls so far, timeout word) of the workspace."""
        return [int(self.workspace[:8].view(torch.int64)), int(self.workspace[8:12].view(torch.int32))]


class PreparedStack(_Prepared):
    """lb_decode_stack: every layer of a decoder stack for one token in one launch.

    layers: sequence of dicts with norm1, norm2, keys, values and projections (the seven dicts of
    PreparedLayer); the other arguments as PreparedLayer.  The call owns a zeroed workspace and the
    device layer table, written once here by lb_decode_stack_prepare.
    """

    def __init__(self, h, layers, *, format, group_size, hidden, intermediate, eps, heads, kv_heads, cos, sin,
                 position, scale=0.125):
        if not 1 <= len(layers) <= STACK_MAX_LAYERS:
            raise ValueError(f'1..{STACK_MAX_LAYERS} layers per stack')
        keys0 = layers[0]['keys']
        capacity = keys0.shape[-2]
        a = DecodeStackArgs()
        a.struct_size = ctypes.sizeof(DecodeStackArgs)
        a.format = FORMATS[format]
        a.group_size, a.hidden, a.intermediate, a.layers = group_size, hidden, intermediate, len(layers)
        keep = [_row(h, 'h', hidden)]
        self._rows = (DecodeStackLayer * len(layers))()
        for row, layer in zip(self._rows, layers):
            if len(layer['projections']) != 7:
                raise ValueError('seven projections per layer: q, k, v, o, gate, up, down')
            keep += [_row(layer['norm1'], 'norm1', hidden), _row(layer['norm2'], 'norm2', hidden),
                     _row(layer['keys'], 'keys', kv_heads * capacity * 64),
                     _row(layer['values'], 'values', kv_heads * capacity * 64)]
            row.norm1, row.norm2 = _ptr(layer['norm1']), _ptr(layer['norm2'])
            row.keys, row.values = _ptr(layer['keys']), _ptr(layer['values'])
            _fill_projections(row.proj, layer['projections'], keep)
        a.layer = self._rows
        a.h, a.eps = _ptr(h), eps
        for t, name in ((cos, 'cos'), (sin, 'sin')):
            keep.append(_row(t, name, capacity * 64))
        keep.append(_row(position, 'position', 1, torch.int64))
        a.heads, a.kv_heads, a.capacity = heads, kv_heads, capacity
        a.cos, a.sin, a.position, a.scale = _ptr(cos), _ptr(sin), _ptr(position), scale
        self.table = torch.zeros(stack_table_bytes(len(layers)), dtype=torch.uint8, device=h.device)
        a.table, a.table_bytes = _ptr(self.table), self.table.numel()
        size = stack_workspace_bytes(hidden, intermediate, kv_heads, len(layers))
        self.workspace = torch.zeros(size, dtype=torch.uint8, device=h.device)
        a.workspace, a.workspace_bytes = _ptr(self.workspace), size
        self._timeout_offset = DECODE_TIMEOUT_OFFSET
        keep += [self.table, self.workspace]
        self._bind('lb_decode_stack', 'lb_decode_stack', a, h.device, keep)
        handle = torch.cuda.current_stream(h.device).cuda_stream
        _check(library().lb_decode_stack_prepare(self._ref, ctypes.c_void_p(handle)), 'lb_decode_stack_prepare')
        self._prepared = True
        self.out = h

    def release(self):
        """Forget the prepared table (lb_decode_stack_release); run() then raises ValueError.  Done
        by the garbage collector too, before the table's memory returns to the allocator."""
        if getattr(self, '_prepared', False):
            self._prepared = False
            _check(library().lb_decode_stack_release(_ptr(self.table)), 'lb_decode_stack_release')

    def __del__(self):
        try:
            self.release()
        except Exception:  # interpreter shutdown: the library may already be gone
            pass

    def counters(self):
        """(workgroups counted over all calls so far, timeout word) of the workspace."""
        return [int(self.workspace[:8].view(torch.int64)), int(self.workspace[8:12].view(torch.int32))]
