#!/usr/bin/env python3
"""Write ``weight_quant_kat.json``: the reference's known-answer vectors as data.

Every case restates literal inputs and expected outputs that the reference's
own tests hold (file:line given per case), or a vector derived by hand in the
comment next to it.  Nothing here imports or runs the reference; the values
are typed from the test sources and from the arithmetic in the comments.

Run: ``python tests/golden/make_golden.py`` (rewrites the JSON next to it).
"""
from __future__ import annotations

import json
import struct
from pathlib import Path


def i32(word: int) -> int:
    """Reinterpret an unsigned 32-bit pattern as a signed int32 value."""
    return struct.unpack('<i', struct.pack('<I', word & 0xFFFFFFFF))[0]


def f16_bits(value: float) -> int:
    return struct.unpack('<H', struct.pack('<e', value))[0]


CASES = {
    # tests/test_weight_quant_backend.py:7-11 - LSB nibble first, both axes.
    'kat_unpack': {
        'source': 'tests/test_weight_quant_backend.py:7-11',
        'packed': [[i32(0x76543210)]],
        'bits': 4, 'length': 8,
        'expected_axis1': [[0, 1, 2, 3, 4, 5, 6, 7]],
        'expected_axis0': [[0], [1], [2], [3], [4], [5], [6], [7]],
    },
    # tests/test_weight_quant_backend.py:14-25 - group zero point and scale.
    'kat_group_decode': {
        'source': 'tests/test_weight_quant_backend.py:14-25',
        'name': 'mlp.up_proj.weight', 'group_size': 4,
        'weight_packed': [[i32(0x76543210)], [i32(0x76543210)]],
        'weight_shape': [2, 8],
        'weight_scale': [[1.0, 2.0], [3.0, 4.0]],
        'weight_zero_point': [[0x10, 0x32]],
        'expected': [[0, 1, 2, 3, 4, 6, 8, 10], [-3, 0, 3, 6, 4, 8, 12, 16]],
    },
    # tests/test_weight_quant_backend.py:28-32 - no zero point means z = 8.
    'kat_symmetric': {
        'source': 'tests/test_weight_quant_backend.py:28-32',
        'name': 'self_attn.q_proj.weight', 'group_size': 4,
        'weight_packed': [[i32(0x76543210)]],
        'weight_shape': [1, 8],
        'weight_scale': [[1.0, 1.0]],
        'expected': [[-8, -7, -6, -5, -4, -3, -2, -1]],
    },
    # tests/test_weight_quant_backend.py:33-35 - INT8 channel scale.
    'kat_int8_channel': {
        'source': 'tests/test_weight_quant_backend.py:33-35',
        'name': 'self_attn.q_proj.weight',
        'weight': [[1, -2], [3, -4]],
        'weight_scale': [[0.5], [2.0]],
        'expected': [[0.5, -1.0], [6.0, -8.0]],
    },
    # tests/test_weight_quant_backend.py:38-45 - sampled rows equal full decode.
    # Scales are fp16(arange(1,17)/10); stored here as fp16 bit patterns.
    'kat_sampled_rows': {
        'source': 'tests/test_weight_quant_backend.py:38-45',
        'name': 'mlp.up_proj.weight',
        'packed_word': i32(0x76543210), 'packed_shape': [8, 32],
        'weight_shape': [8, 256],
        'weight_scale_f16_bits': [[f16_bits(v / 10) for v in (2 * r + 1, 2 * r + 2)] for r in range(8)],
        'weight_zero_point': [[i32(0x76543210), i32(0x01234567)]],
        'rows': [0, 3, 7],
    },
    # tests/test_weight_quant_backend.py:48-66 - row-split dispatch.
    'kat_row_dispatch': {
        'source': 'tests/test_weight_quant_backend.py:48-66',
        'max_rows': 16, 'x_shape': [2, 12, 4], 'n': 8,
        'expected_widths': [16, 8], 'expected_calls': 1, 'expected_gemm_calls': 2,
    },
    # tests/test_quantization.py:43-62 - zero row gets scale 1, tiny row a
    # finite positive scale.  Hand derivation of the full expected vectors:
    #   row 0: absmax 0 -> scale 1, q = 0.
    #   row 1: absmax 1e-10, 1e-10/127 underflows fp16 -> smallest subnormal
    #          2**-24 (bits 0x0001); 1e-10 / 2**-24 = 0.0017 -> q = 0.
    #   row 2: absmax 1 -> 1/127 = 0.0078740 -> fp16 0.0078735 (bits 0x2008);
    #          q = rint([1, -0.5, 0.25, 0] / 0.0078735) = [127, -64, 32, 0].
    'kat_int8_zero_tiny_rows': {
        'source': 'tests/test_quantization.py:43-62 (+ hand-derived q/scale)',
        'weight': [[0.0, 0.0, 0.0, 0.0], [1e-10, -1e-10, 0.0, 1e-10], [1.0, -0.5, 0.25, 0.0]],
        'row_block_size': 1,
        'expected_q': [[0, 0, 0, 0], [0, 0, 0, 0], [127, -64, 32, 0]],
        'expected_scale_f16_bits': [f16_bits(1.0), 0x0001, 0x2008],
    },
    # Hand-derived: absmax 127 -> scale exactly 1.0, so q = rint(w) and the
    # ties check round-half-even (half-away-from-zero would give 3,4,-3,1,2).
    'kat_int8_half_even': {
        'source': 'hand-derived (quantization.py:280 uses torch.round = half-to-even)',
        'weight': [[127.0, 2.5, 3.5, -2.5, 0.5, 1.5]],
        'expected_q': [[127, 2, 4, -2, 0, 2]],
        'expected_scale_f16_bits': [f16_bits(1.0)],
    },
    # Hand-derived: the *stored* fp16 scale (0.0078735) divides the row, not
    # the fp32 1/127.  0.49998/0.0078735 = 63.501 -> 64, but
    # 0.49998/0.0078740 = 63.497 -> 63 (quantization.py:279-280).
    'kat_int8_stored_scale': {
        'source': 'hand-derived (quantization.py:266,279-280)',
        'weight': [[1.0, 0.49998]],
        'expected_q': [[127, 64]],
        'expected_scale_f16_bits': [0x2008],
    },
    # Hand-derived: absmax = 1.4*127*2**-24; absmax/127 = 1.4*2**-24 rounds to
    # the subnormal 2**-24, so absmax/scale = 177.8 -> clamp to 127; the
    # second element -0.5*absmax -> -88.9 -> -89 (quantization.py:280-281).
    'kat_int8_clamp': {
        'source': 'hand-derived (quantization.py:281 clamp to [-127, 127])',
        'weight': [[1.4 * 127 * 2.0 ** -24, -0.5 * 1.4 * 127 * 2.0 ** -24]],
        'expected_q': [[127, -89]],
        'expected_scale_f16_bits': [0x0001],
    },
}


def main() -> None:
    out = Path(__file__).with_name('weight_quant_kat.json')
    out.write_text(json.dumps(CASES, indent=1) + '\n')
    print('wrote', out)


if __name__ == '__main__':
    main()
