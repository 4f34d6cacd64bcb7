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

ABI_VERSION = 1
OK, INVALID_ARGUMENT, OUT_OF_MEMORY, UNSUPPORTED, DEVICE_FAILED, INTERNAL = 0, 1, 2, 5, 10, 12
FORMATS = {'int8': 0, 'int4': 1, 'nf4': 2, 'fp16': 3}
FLAG_FORCE_GEMV, FLAG_FORCE_GEMM, FLAG_FORCE_GENERIC = 0x1, 0x2, 0x4
EXPORTS = ('lb_abi_version', 'lb_status_name', 'lb_last_error', 'lb_workspace_bytes', 'lb_linear',
           'lb_unpack_codes', 'lb_dequantize')


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
                ('flags', ctypes.c_uint32), ('reserved', ctypes.c_uint32)]


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
        lib.lb_workspace_bytes.restype = ctypes.c_int
        lib.lb_workspace_bytes.argtypes = [ctypes.POINTER(LinearArgs), ctypes.POINTER(ctypes.c_size_t)]
        lib.lb_linear.restype = ctypes.c_int
        lib.lb_linear.argtypes = [ctypes.POINTER(LinearArgs), ctypes.c_void_p]
        lib.lb_unpack_codes.restype = ctypes.c_int
        lib.lb_unpack_codes.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p]
        lib.lb_dequantize.restype = ctypes.c_int
        lib.lb_dequantize.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
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


def make_args(x, codes, scales, *, format, N, K, group_size, y, bias=None, down=None, up=None, rank=0,
              flags=0):
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
    return args


def workspace_bytes(args):
    size = ctypes.c_size_t(0)
    _check(library().lb_workspace_bytes(ctypes.byref(args), ctypes.byref(size)), 'lb_workspace_bytes')
    return size.value


def linear(x, codes, scales, *, format, N, K, group_size, bias=None, down=None, up=None, rank=0, flags=0,
           out=None, workspace=None):
    """y[M,N] fp16 = x . dequant(W)^T (+bias) (+fp16(fp16(x.V^T).U^T)) on the current stream.

    x: fp16 [M,K] cuda (unit column stride).  codes: uint8 (or fp16 for format='fp16').
    scales: fp16 [N, K/group_size].  down: fp16 [rank,K] (row stride K); up: fp16 [N, >=rank].
    """
    _device_tensor(x, 'x', torch.float16)
    if x.ndim != 2 or x.shape[1] != K:
        raise ValueError('x must be [M, K]')
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
                     down=down, up=up, rank=rank, flags=flags)
    need = workspace_bytes(args)
    if need:
        if workspace is None or workspace.numel() < need:
            workspace = torch.zeros(need, dtype=torch.uint8, device=x.device)
        args.workspace, args.workspace_bytes = _ptr(workspace), workspace.numel()
    _check(library().lb_linear(ctypes.byref(args), _stream(x.device)), 'lb_linear')
    return y


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
                 rank=0, flags=0, workspace=None):
        _device_tensor(x, 'x', torch.float16)
        _device_tensor(out, 'out', torch.float16)
        if x.ndim != 2 or x.shape[1] != K or (K > 1 and x.stride(1) != 1):
            raise ValueError('PreparedLinear needs x [M, K] with unit column stride')
        if out.shape != (x.shape[0], N) or (N > 1 and out.stride(1) != 1):
            raise ValueError('PreparedLinear needs out [M, N] with unit column stride')
        self._keep = [x, codes, scales, out, bias, down, up]
        self.args = make_args(x, codes, scales, format=format, N=N, K=K, group_size=group_size, y=out,
                              bias=bias, down=down, up=up, rank=rank, flags=flags)
        need = workspace_bytes(self.args)
        if need:
            if workspace is None or workspace.numel() < need:
                workspace = torch.zeros(need, dtype=torch.uint8, device=x.device)
            self.args.workspace, self.args.workspace_bytes = _ptr(workspace), workspace.numel()
            self._keep.append(workspace)
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
