"""CPU oracle of the low-bit weight format and linear -- TEST INFRASTRUCTURE ONLY.

Restates, in numpy (fp64 where the reference leaves the accumulation order to a BLAS),
the reference's CPU semantics from LCS-Official/torch-intel-npu:

  NF4                  torch_npu_lowbit.py:17-21
  pack / unpack        torch_npu_lowbit.py:24-30, 69-73
  dequantize           torch_npu_lowbit.py:67-75
  quantize             torch_npu_lowbit.py:78-105
  staged linear        torch_npu_smollm.py:150-165 (W8 exact q*s, 4-bit fp16(q*s),
                       correction z=fp16(x.V^T), d=fp16(z.U^T), y=fp16(y+d));
                       bias staging torch_npu_lowbit.py:262-266
  rounding budget      torch_npu_lowbit_demo.py:88-95
  compact_linear       torch_npu_lowbit.py:235-256 (per-group fp16 products, balanced fp16
                       add tree), bias :262-266
  w8a8_linear          torch_npu_int8_demo.py:34-51 (linear_reference with an activation
                       scale: the DPU's zero-point-128 weight grid), graph :224-231

Pinning (what checks each function, see tests/test_oracle.py):
  pack/unpack   reference known answers (test_torch_npu_lowbit.py:36,41;
                npunlock/tests/python/test_python_api.py:23-36) + round trip.
  dequantize    reference known answers (test_torch_npu_lowbit.py:37-40, 91-93, 56-58)
                + brute force over every (code, fp16 scale) pair against an fp32
                multiply-and-round computed by a different route.
  quantize      closed-form tie cases (exact NF4 midpoints, k+0.5 halves), invariants
                (|q| <= limit, s >= 2^-24, zero rows), reconstruction error bound.
  linear        textbook fp64 matmul of decoded weights, identity-input bit-exact case,
                zero-factor correction leaves output unchanged, linearity.
  compact_linear  one group equals linear; the reference's edge cases (all codes in two
                groups with identity input bit-exact, zero weights, overflowing fp16
                partials); the pairing order against an explicitly written tree on pieces
                chosen so that sequential and other pairings round differently.
  w8a8_linear   the reference's exact cases (all 256 weight codes, activation ties and
                clipping, large-integer accumulation with cancellation, scale boundaries,
                zero weights), a pure-Python integer brute force on small shapes, and the
                quantization error bound against the unquantized product.
"""
import numpy as np

# Published NormalFloat4 codebook (the reference's fp32 literals).
NF4_F32 = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)
LIMITS = {'int4': 7, 'nf4': 1, 'int8': 127}
FP16_MAX = 65504.0


def pack(codes):
    """uint8 codes 0..15 (any shape, flattened row-major) -> bytes, element 2i low nibble."""
    flat = np.asarray(codes, dtype=np.uint8).reshape(-1)
    if flat.size % 2:
        flat = np.concatenate([flat, np.zeros(1, np.uint8)])
    lo, hi = flat[0::2].astype(np.uint16), flat[1::2].astype(np.uint16)
    return (lo + 16 * hi).astype(np.uint8).tobytes()


def nibbles(data, count):
    """Flat nibble codes 0..15 of the first `count` elements of packed 4-bit data."""
    raw = np.frombuffer(data, dtype=np.uint8)
    out = np.empty(2 * raw.size, dtype=np.uint8)
    out[0::2] = raw % 16
    out[1::2] = raw // 16
    return out[:count]


def unpack(fmt, data, count):
    """Decoded integers as the HIP unpack reports them: int8 value, int4 (c^8)-8, nf4 index c."""
    if fmt == 'int8':
        return np.frombuffer(data, dtype=np.int8)[:count].astype(np.int16)
    c = nibbles(data, count).astype(np.int16)
    if fmt == 'int4':
        return np.where(c >= 8, c - 16, c)  # two's complement nibble == (c ^ 8) - 8
    return c


def code_values(fmt, data, count):
    """q as exact fp64: int8/int4 integers, nf4 the fp16-rounded codebook entry."""
    ints = unpack(fmt, data, count)
    if fmt == 'nf4':
        return NF4_F32.astype(np.float16).astype(np.float64)[ints]
    return ints.astype(np.float64)


def scales_of(scales_bytes, n, groups):
    return np.frombuffer(scales_bytes, dtype=np.float16).reshape(n, groups)


def exact_weight(fmt, shape, group, data, scales_bytes):
    """W[n,k] = q * s in fp64 (exact: 11-bit scale times <=8-bit code)."""
    n, k = shape
    q = code_values(fmt, data, n * k).reshape(n, k // group, group)
    s = scales_of(scales_bytes, n, k // group).astype(np.float64)[:, :, None]
    return (q * s).reshape(n, k)


def dequantize(fmt, shape, group, data, scales_bytes):
    """fp16(q * s) with a single rounding of the exact product (fp64 -> fp16 is RNE)."""
    with np.errstate(over='ignore'):  # |q*s| > 65504 becomes inf, as in the reference
        return exact_weight(fmt, shape, group, data, scales_bytes).astype(np.float16)


def quantize(weight, fmt, group=None):
    """Symmetric per-(row, group) quantizer -> (data bytes, fp16 scale bytes).

    weight: float array [N, K] (converted to fp32 first, as weight.float() does).
    Raises ValueError where the reference raises.
    """
    w = np.asarray(weight, dtype=np.float32)
    n, k = w.shape
    g = k if group is None else group
    if fmt not in LIMITS or not 1 <= g <= k or k % g:
        raise ValueError('bad format/group')
    if not np.isfinite(w).all():
        raise ValueError('nonfinite weights')
    blocks = w.reshape(n, k // g, g)
    limit = np.float32(LIMITS[fmt])
    raw_scale = np.abs(blocks).max(axis=2) / limit            # fp32
    if (raw_scale > np.float32(FP16_MAX)).any():
        raise ValueError('scale overflows fp16')
    scale16 = np.where(raw_scale < np.float32(2.0 ** -24), np.float32(2.0 ** -24), raw_scale).astype(np.float16)
    u = blocks / scale16.astype(np.float32)[:, :, None]       # fp32 division by the rounded scale
    if fmt == 'nf4':
        mids = ((NF4_F32[:-1] + NF4_F32[1:]) / np.float32(2)).astype(np.float32)
        codes = (u[..., None] > mids).sum(axis=-1).astype(np.uint8)   # ties go to the lower code
        data = pack(codes)
    else:
        q = np.clip(np.rint(u), -LIMITS[fmt], LIMITS[fmt]).astype(np.int8)  # rint: half to even
        data = q.tobytes() if fmt == 'int8' else pack((q.astype(np.int16) % 16).astype(np.uint8))
    return data, scale16.tobytes()


def _f16(v):
    return np.asarray(v, dtype=np.float64).astype(np.float16)


def linear(x, fmt, shape, group, data, scales_bytes, *, bias=None, down=None, up=None):
    """Staged fp16 reference linear; x fp16 [M,K]; returns fp16 [M,N].

    int8 with per-row scales: fp16(x . (q*s)^T) with exact q*s (torch_npu_smollm.py:153-157).
    Every other case multiplies by the fp16-dequantized weight (torch_npu_smollm.py:159,
    torch_npu_lowbit_demo.py:38).  Accumulation is fp64 here (the reference: CPU BLAS fp32/fp64).
    """
    n, k = shape
    x64 = np.asarray(x, dtype=np.float16).astype(np.float64)
    if fmt == 'int8' and group == k:
        w = exact_weight(fmt, shape, group, data, scales_bytes)
    else:
        w = dequantize(fmt, shape, group, data, scales_bytes).astype(np.float64)
    y = _f16(x64 @ w.T)
    if bias is not None:
        y = _f16(y.astype(np.float64) + np.asarray(bias, np.float16).astype(np.float64))
    if down is not None:
        v = np.asarray(down, np.float16).astype(np.float64)
        u = np.asarray(up, np.float16).astype(np.float64)
        z = _f16(x64 @ v.T)
        d = _f16(z.astype(np.float64) @ u.T)
        y = _f16(y.astype(np.float64) + d.astype(np.float64))
    return y


def dense_linear(x, w):
    """fp16(x . w^T) for fp16 x, w with fp64 accumulation."""
    return _f16(np.asarray(x, np.float16).astype(np.float64) @ np.asarray(w, np.float16).astype(np.float64).T)


def ideal(x, fmt, shape, group, data, scales_bytes):
    """x . (q*s)^T in fp64 with exact weights: the reference performance gate's 'ideal'."""
    return np.asarray(x, np.float16).astype(np.float64) @ exact_weight(fmt, shape, group, data, scales_bytes).T


def rounding_budget(x, fmt, shape, group, data, scales_bytes):
    """Per-output tolerance |x| . |W_exact - W_f16|^T + 2 eps16 |ideal| + 2e-4 (demo :91-93)."""
    exact = exact_weight(fmt, shape, group, data, scales_bytes)
    rounded = exact.astype(np.float16).astype(np.float64)
    x64 = np.abs(np.asarray(x, np.float16).astype(np.float64))
    eps16 = float(np.finfo(np.float16).eps)
    return x64 @ np.abs(exact - rounded).T + 2 * eps16 * np.abs(ideal(x, fmt, shape, group, data, scales_bytes)) + 2e-4


def rel_l2(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    denom = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (denom if denom else 1.0))


def _tree_sum(pieces):
    """Balanced fp16 addition: neighbours pair up (0+1, 2+3, ...); an odd last piece moves up."""
    with np.errstate(over='ignore', invalid='ignore'):
        while len(pieces) > 1:
            pieces = [_f16(pieces[i].astype(np.float64) + pieces[i + 1].astype(np.float64)) if i + 1 < len(pieces)
                      else pieces[i] for i in range(0, len(pieces), 2)]
    return pieces[0]


def compact_linear(x, fmt, shape, group, data, scales_bytes, *, bias=None):
    """compact_groups: y = tree(fp16(x_g . fp16(q s)_g^T) for each group g), then fp16(y + b).

    With one group the reference builds the default graph (torch_npu_lowbit.py:235 tests
    `groups > 1`), so that case is `linear`.  A partial that overflows fp16 stays +-inf
    (the reference records this as a known limitation of compact graphs).
    """
    n, k = shape
    groups = k // group
    if groups == 1:
        return linear(x, fmt, shape, group, data, scales_bytes, bias=bias)
    x64 = np.asarray(x, dtype=np.float16).astype(np.float64)
    w = dequantize(fmt, shape, group, data, scales_bytes).astype(np.float64)
    with np.errstate(over='ignore', invalid='ignore'):
        pieces = [_f16(x64[:, g * group:(g + 1) * group] @ w[:, g * group:(g + 1) * group].T) for g in range(groups)]
        y = _tree_sum(pieces)
        if bias is not None:
            y = _f16(y.astype(np.float64) + np.asarray(bias, np.float16).astype(np.float64))
    return y


def w8a8_weight_steps(scales_bytes):
    """Per-row weight step of the W8A8 grid: (fp16(127 s) - fp16(-128 s)) / 255 in fp64."""
    s = np.frombuffer(scales_bytes, dtype=np.float16).astype(np.float64)
    with np.errstate(over='ignore'):
        low = (-128 * s).astype(np.float16).astype(np.float64)
        high = (127 * s).astype(np.float16).astype(np.float64)
    return (high - low) / 255


def quantize_activations(x, activation_scale):
    """clip(rint(x / s_x), -128, 127) as int64 (s_x a power of two, so x / s_x is exact)."""
    return np.clip(np.rint(np.asarray(x, np.float16).astype(np.float64) / activation_scale), -128, 127).astype(np.int64)


def w8a8_linear(x, shape, data, scales_bytes, activation_scale, *, bias=None):
    """W8A8 linear: y = fp16((sum_k qx qw) * s_x * step_n), fp16(y + b) with a bias.

    qx = clip(rint(x / s_x), -128, 127); qw the stored int8 codes (per-row scales); the integer
    sum is exact and the scaling one fp64 product, in the reference's order
    (torch_npu_int8_demo.py:41-51).
    """
    n, k = shape
    qx = quantize_activations(x, activation_scale)
    qw = np.frombuffer(data, dtype=np.int8).reshape(n, k).astype(np.int64)
    acc = qx @ qw.T
    with np.errstate(over='ignore', invalid='ignore'):
        y = _f16(acc.astype(np.float64) * activation_scale * w8a8_weight_steps(scales_bytes)[None, :])
        if bias is not None:
            y = _f16(y.astype(np.float64) + np.asarray(bias, np.float16).astype(np.float64))
    return y
