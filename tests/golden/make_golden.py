"""Write the committed golden fixtures under tests/golden/.

known_answers.json  literal vectors transcribed from the reference's own tests
                    (file:line in each entry); no reference code is imported or run.
linear_small.npz    oracle outputs on small seeded problems, so GPU parity tests and
                    later oracle edits are checked against frozen vectors.

Run: python tests/golden/make_golden.py
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import lowbit_oracle as o  # noqa: E402


def known_answers():
    return {
        'pack_arange16': {
            'source': 'test_torch_npu_lowbit.py:36',
            'codes': list(range(16)), 'packed_hex': '1032547698badcfe'},
        'pack_odd3': {
            'source': 'test_torch_npu_lowbit.py:41',
            'codes': [0, 1, 2], 'packed_hex': '1002'},
        'int4_all_codes_scale1': {
            'source': 'test_torch_npu_lowbit.py:37-40 (np.arange(-8,8)[(codes+8)%16])',
            'packed_hex': '1032547698badcfe', 'values': [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]},
        'nf4_all_codes_scale1_f16_bits': {
            'source': 'test_torch_npu_lowbit.py:39 (NF4.astype(np.float16)); table torch_npu_lowbit.py:17-20',
            'packed_hex': '1032547698badcfe',
            # the codebook's decimal literals as written in torch_npu_lowbit.py:17-20
            'literals': ['-1.', '-.6961928009986877', '-.5250730514526367', '-.39491748809814453',
                         '-.28444138169288635', '-.18477343022823334', '-.09105003625154495', '0.',
                         '.07958029955625534', '.16093020141124725', '.24611230194568634', '.33791524171829224',
                         '.44070982933044434', '.5626170039176941', '.7229568362236023', '1.'],
            # fp16 bit patterns of float32(literal) rounded to nearest even.
            'bits': [0xbc00, 0xb992, 0xb833, 0xb652, 0xb48d, 0xb1ea, 0xadd4, 0x0000,
                     0x2d18, 0x3126, 0x33e0, 0x3568, 0x370d, 0x3880, 0x39c9, 0x3c00]},
        'int8_codec_eighth': {
            'source': 'test_torch_npu_lowbit.py:91-93 (codes -128..127, scale 0.125, exact)',
            'codes': list(range(-128, 128)), 'scale': 0.125},
        'odd_padding_rejected': {
            'source': 'test_torch_npu_lowbit.py:63-64; npunlock/tests/python/test_python_api.py:25-36',
            'valid': [{'shape': [1, 3], 'packed_hex': 'f007'}],
            'invalid': [{'shape': [1, 3], 'packed_hex': '10f2'}, {'shape': [1, 3], 'packed_hex': 'f0f7'},
                        {'shape': [1, 3], 'packed_hex': 'f0'}, {'shape': [1, 3], 'packed_hex': ''}]},
        'identity_input_exact': {
            'source': 'torch_npu_lowbit_demo.py:124-128 (all 16 codes x scale {0.125,1,16}, eye(16) input, bit-exact)',
            'scales': [0.125, 1.0, 16.0]},
    }


def linear_fixtures(rng):
    cases = {}
    specs = [
        # name, fmt, M, N, K, group, rank, bias
        ('int8_row_c1', 'int8', 1, 96, 64, None, 8, False),
        ('int8_row_m3', 'int8', 3, 40, 96, None, 0, True),
        ('int4_g32', 'int4', 2, 48, 64, 32, 0, False),
        ('int4_g64_bias', 'int4', 5, 24, 128, 64, 0, True),
        ('nf4_g32', 'nf4', 4, 32, 96, 32, 0, False),
        ('int4_odd', 'int4', 3, 13, 17, None, 0, False),
        ('nf4_g3', 'nf4', 2, 5, 9, 3, 0, False),
        ('int8_g32', 'int8', 2, 16, 64, 32, 4, False),
    ]
    for name, fmt, m, n, k, group, rank, bias in specs:
        g = k if group is None else group
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
        data, scales = o.quantize(w, fmt, g)
        x = rng.standard_normal((m, k)).astype(np.float16)
        b = (rng.standard_normal(n) * 0.1).astype(np.float16) if bias else None
        down = (rng.standard_normal((rank, k)) * 0.01).astype(np.float16) if rank else None
        up = (rng.standard_normal((n, rank)) * 0.01).astype(np.float16) if rank else None
        y = o.linear(x, fmt, (n, k), g, data, scales, bias=b, down=down, up=up)
        entry = dict(fmt=np.array(fmt), shape=np.array([m, n, k, g, rank]), weight=w, x=x,
                     data=np.frombuffer(data, np.uint8), scales=np.frombuffer(scales, np.float16), y=y)
        if bias:
            entry['bias'] = b
        if rank:
            entry['down'], entry['up'] = down, up
        for key, value in entry.items():
            cases[f'{name}/{key}'] = value
    return cases


def main():
    (HERE / 'known_answers.json').write_text(json.dumps(known_answers(), indent=1) + '\n')
    rng = np.random.default_rng(20261201)
    np.savez_compressed(HERE / 'linear_small.npz', **linear_fixtures(rng))
    print('wrote', HERE / 'known_answers.json', HERE / 'linear_small.npz')


if __name__ == '__main__':
    main()
