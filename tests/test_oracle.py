"""Pins the CPU oracle (``oracle/``) before anything is compared against it.

Each check is independent of the oracle's own formulas: the reference's
known-answer vectors (``tests/golden/weight_quant_kat.json``), scalar
brute-force re-derivations with Python ints/floats and ``struct`` fp16
rounding, hand-derived INT8 vectors, and the reference's quantizer invariants.
"""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import qdq, synth, tile_layout

KAT = json.loads((Path(__file__).parent / 'golden' / 'weight_quant_kat.json').read_text())


def f16(value: float) -> np.float16:
    """Round a Python float to fp16 (IEEE round-to-nearest-even via struct)."""
    return np.frombuffer(struct.pack('<e', value), dtype=np.float16)[0]


# --------------------------------------------------------------------------- unpack / pack

def test_unpack_kat_both_axes():
    c = KAT['kat_unpack']
    packed = np.array(c['packed'], dtype=np.int32)
    assert qdq.unpack_unsigned(packed, 4, 1, 8).tolist() == c['expected_axis1']
    assert qdq.unpack_unsigned(packed, 4, 0, 8).tolist() == c['expected_axis0']


def test_unpack_matches_unsigned_scalar_extraction():
    rng = np.random.default_rng(1)
    words = rng.integers(0, 2**32, size=(5, 3), dtype=np.uint64)
    packed = words.astype(np.uint32).view(np.int32)
    got = qdq.unpack_unsigned(packed, 4, 1, 24)
    for r in range(5):
        for c in range(24):
            assert got[r, c] == (int(words[r, c // 8]) >> (4 * (c % 8))) & 0xF
    got0 = qdq.unpack_unsigned(packed, 4, 0, 40)
    for r in range(40):
        for c in range(3):
            assert got0[r, c] == (int(words[r // 8, c]) >> (4 * (r % 8))) & 0xF


def test_pack_is_inverse_and_reproduces_kat_words():
    assert qdq.pack_unsigned(np.arange(8).reshape(1, 8), 4, 1).tolist() == KAT['kat_unpack']['packed']
    # zero points of rows (0, 1) for groups (0, 1) are (0, 1) and (2, 3): words 0x10, 0x32
    assert qdq.pack_unsigned(np.array([[0, 2], [1, 3]]), 4, 0).tolist() == KAT['kat_group_decode']['weight_zero_point']
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, size=(16, 64))
    assert np.array_equal(qdq.unpack_unsigned(qdq.pack_unsigned(codes, 4, 1), 4, 1, 64), codes)
    assert np.array_equal(qdq.unpack_unsigned(qdq.pack_unsigned(codes, 4, 0), 4, 0, 16), codes)


# --------------------------------------------------------------------------- decode

def _kat_weights(c, prefix):
    w = {f'{prefix}.weight_packed': np.array(c['weight_packed'], dtype=np.int32),
         f'{prefix}.weight_shape': np.array(c['weight_shape']),
         f'{prefix}.weight_scale': np.array(c['weight_scale'], dtype=np.float32)}
    if 'weight_zero_point' in c:
        w[f'{prefix}.weight_zero_point'] = np.array(c['weight_zero_point'], dtype=np.int32)
    return w


def test_group_zero_point_and_scale_kat():
    c = KAT['kat_group_decode']
    got = qdq.decode_weight(_kat_weights(c, 'mlp.up_proj'), c['name'], group_size=c['group_size'])
    assert got.dtype == np.float16 and got.tolist() == c['expected']


def test_symmetric_bias_kat():
    c = KAT['kat_symmetric']
    got = qdq.decode_weight(_kat_weights(c, 'self_attn.q_proj'), c['name'], group_size=c['group_size'])
    assert got.tolist() == c['expected']


def test_int8_channel_kat():
    c = KAT['kat_int8_channel']
    w = {c['name']: np.array(c['weight'], dtype=np.int8),
         'self_attn.q_proj.weight_scale': np.array(c['weight_scale'], dtype=np.float32)}
    assert qdq.decode_weight(w, c['name']).tolist() == c['expected']
    q, s = w[c['name']], w['self_attn.q_proj.weight_scale'].reshape(-1)
    assert qdq.dequantize_linear_weight(q, s).tolist() == c['expected']


def test_sampled_rows_kat():
    c = KAT['kat_sampled_rows']
    scale = np.array(c['weight_scale_f16_bits'], dtype=np.uint16).view(np.float16)
    w = {'mlp.up_proj.weight_packed': np.full(c['packed_shape'], c['packed_word'], dtype=np.int32),
         'mlp.up_proj.weight_shape': np.array(c['weight_shape']),
         'mlp.up_proj.weight_scale': scale,
         'mlp.up_proj.weight_zero_point': np.array(c['weight_zero_point'], dtype=np.int32)}
    rows = np.array(c['rows'])
    assert np.array_equal(qdq.decode_rows(w, c['name'], rows), qdq.decode_weight(w, c['name'])[rows])


@pytest.mark.parametrize('use_gidx', [False, True])
@pytest.mark.parametrize('symmetric', [False, True])
def test_decode_matches_scalar_brute_force(use_gidx, symmetric):
    rng = np.random.default_rng(3)
    n, k, g = 16, 256, 64
    codes = rng.integers(0, 16, size=(n, k))
    zeros = rng.integers(0, 16, size=(n, k // g))
    scale = (rng.random((n, k // g)) * 0.01 + 1e-3).astype(np.float16)
    gidx = rng.permutation(np.repeat(np.arange(k // g), g)) if use_gidx else None
    w = {'p.weight_packed': qdq.pack_unsigned(codes, 4, 1), 'p.weight_shape': np.array([n, k]),
         'p.weight_scale': scale}
    if not symmetric:
        w['p.weight_zero_point'] = qdq.pack_unsigned(zeros, 4, 0)
    if use_gidx:
        w['p.weight_g_idx'] = gidx.astype(np.int32)
    got = qdq.decode_weight(w, 'p.weight', group_size=g)
    for r in range(n):
        for c in range(k):
            grp = int(gidx[c]) if use_gidx else c // g
            z = 8 if symmetric else int(zeros[r, grp])
            want = f16((int(codes[r, c]) - z) * float(scale[r, grp]))
            assert got[r, c] == want or (math.isnan(want) and math.isnan(got[r, c]))


# --------------------------------------------------------------------------- INT8 quantizer

@pytest.mark.parametrize('case', ['kat_int8_zero_tiny_rows', 'kat_int8_half_even', 'kat_int8_stored_scale',
                                  'kat_int8_clamp'])
def test_int8_quantizer_known_answers(case):
    c = KAT[case]
    q, s = qdq.quantize_linear_weight(np.array(c['weight'], dtype=np.float32),
                                      row_block_size=c.get('row_block_size', 256))
    assert q.tolist() == c['expected_q']
    assert s.view(np.uint16).tolist() == c['expected_scale_f16_bits']


def test_int8_quantizer_invariants():
    # tests/test_quantization.py:21-40 with a numpy draw: rows scaled 0.02 .. 2.
    rng = np.random.default_rng(7)
    w = rng.standard_normal((9, 37)).astype(np.float32) * np.linspace(0.02, 2.0, 9, dtype=np.float32)[:, None]
    qb, sb = qdq.quantize_linear_weight(w, row_block_size=2)
    qu, su = qdq.quantize_linear_weight(w, row_block_size=9)
    assert np.array_equal(qb, qu) and np.array_equal(sb, su)
    assert qb.min() >= -127 and qb.max() <= 127
    recon = qdq.dequantize_linear_weight(qb, sb).astype(np.float32)
    assert np.all(np.abs(w - recon).max(axis=1) <= sb.astype(np.float32) * 0.6 + 2e-6)
    assert np.all(np.abs(qb).max(axis=1) >= 126)   # the row absmax lands near the top code


def test_int8_quantizer_errors():
    with pytest.raises(ValueError):
        qdq.quantize_linear_weight(np.zeros(4, dtype=np.float32))
    with pytest.raises(TypeError):
        qdq.quantize_linear_weight(np.zeros((2, 2), dtype=np.int32))
    with pytest.raises(ValueError):
        qdq.quantize_linear_weight(np.zeros((0, 2), dtype=np.float32))
    with pytest.raises(ValueError):
        qdq.quantize_linear_weight(np.array([[1.0, np.nan]], dtype=np.float32))
    with pytest.raises(OverflowError):
        qdq.quantize_linear_weight(np.array([[1e7 * 127, 1.0]], dtype=np.float32))
    with pytest.raises(ValueError):
        qdq.quantize_linear_weight(np.ones((2, 2), dtype=np.float32), row_block_size=0)


# --------------------------------------------------------------------------- linear + metrics

def test_linear_fp32_matches_float64_brute_force():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 7)).astype(np.float16)
    w = (rng.standard_normal((5, 7)) * 0.3).astype(np.float16)
    b = rng.standard_normal(5).astype(np.float16)
    got = qdq.linear_fp32(x, w, b)
    assert got.shape == (3, 5)
    for m in range(3):
        for n in range(5):
            ref = sum(float(x[m, j]) * float(w[n, j]) for j in range(7)) + float(b[n])
            # fp32 vs fp64 accumulation may differ by one fp16 ulp after rounding
            assert abs(float(got[m, n]) - float(f16(ref))) <= 2.0 ** -10 * max(abs(ref), 2.0 ** -14)


def test_parity_metrics_closed_form():
    m = qdq.parity_metrics(np.array([1.0, 2.0, 3.0]), np.array([1.0, 2.0, 4.0]))
    assert m['max_abs'] == 1.0 and m['ref_inf'] == 4.0
    assert m['mean_rel'] == pytest.approx(1 / 7)
    assert m['relative_l2'] == pytest.approx(1 / math.sqrt(21))
    assert m['cosine'] == pytest.approx(17 / math.sqrt(14 * 21))
    assert not qdq.parity_ok(m)
    assert qdq.parity_ok(qdq.parity_metrics(np.array([1.0, 2.0]), np.array([1.0, 2.0])))


# --------------------------------------------------------------------------- tile layout model

def test_nibble_order_gives_consecutive_pairs_under_the_kernel_masks():
    rng = np.random.default_rng(5)
    src = rng.integers(0, 2**32, size=64, dtype=np.uint64).astype(np.uint32)
    tile = tile_layout.permute_nibbles(src)
    for s, t in zip(src.tolist(), tile.tolist()):
        e = [(s >> (4 * j)) & 0xF for j in range(8)]
        lo = [t & 0x000F000F, (t & 0x00F000F0) >> 4, (t >> 8) & 0x000F000F, ((t >> 8) & 0x00F000F0) >> 4]
        for p, v in enumerate(lo):
            assert (v & 0xFFFF, v >> 16) == (e[2 * p], e[2 * p + 1])
    assert np.array_equal(tile_layout.unpermute_nibbles(tile), src)


@pytest.mark.parametrize('n,k,g,sym', [(16, 256, 128, False), (24, 512, 256, False), (40, 384, 128, True)])
def test_w4_tile_round_trip_and_dequant(n, k, g, sym):
    weights, _ = synth.w4_case(n, k, 1, seed=11, group_size=g, symmetric=sym, name='p.weight')
    packed, scale = weights['p.weight_packed'], weights['p.weight_scale']
    zero = weights.get('p.weight_zero_point')
    tiles, meta = tile_layout.w4_repack(packed, scale, zero, n, k, g)
    assert tiles.nbytes == (-(-n // 16) * 16) * k // 2
    p2, s2, z2 = tile_layout.w4_unpack(tiles, meta, n, k, g)
    assert np.array_equal(p2, packed) and np.array_equal(s2.view(np.uint16), scale.view(np.uint16))
    if zero is None:
        assert np.all(z2.view(np.uint32) == tile_layout.SYMMETRIC_ZERO_WORD)
    else:
        assert np.array_equal(z2, zero)
    assert np.array_equal(tile_layout.w4_dequant(tiles, meta, n, k, g).view(np.uint16),
                          qdq.decode_weight(weights, 'p.weight', group_size=g).view(np.uint16))


@pytest.mark.parametrize('n,k', [(16, 128), (40, 384), (1000, 256)])
def test_w8_tile_layout_round_trip_and_lane_products(n, k):
    """The INT8 tile model: unpack(repack(q)) == q, rows past n are zero, and
    summing, per (tile, block, piece, lane), the lane's 16 bytes times x at
    the k the INT8 kernels pair them with (128b + 64p + 16*(l//16) + j, row
    16t + l%16) gives q @ x exactly: every weight meets its own x once."""
    rng = np.random.default_rng(n + k)
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    x = rng.integers(-1000, 1000, k).astype(np.int64)
    t = tile_layout.w8_repack(q)
    assert t.shape == (-(-n // 16), k // 128, 2, 64, 16) and t.dtype == np.int8
    assert np.array_equal(tile_layout.w8_unpack(t, n, k), q)
    y = np.zeros(t.shape[0] * 16, dtype=np.int64)
    j = np.arange(16)
    for tt in range(t.shape[0]):
        for b in range(k // 128):
            for p in range(2):
                for lane in range(64):
                    y[16 * tt + lane % 16] += t[tt, b, p, lane].astype(np.int64) @ x[128 * b + 64 * p + 16 * (lane // 16) + j]
    assert np.array_equal(y[:n], q.astype(np.int64) @ x)
    assert not y[n:].any()


def test_awq_synthetic_quantizer_is_valid_and_close():
    n, k = 32, 512
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    t = synth.awq_quantize(w)
    assert t['weight_packed'].shape == (n, k // 8) and t['weight_packed'].dtype == np.int32
    assert t['weight_scale'].shape == (n, k // 128) and np.all(t['weight_scale'] > 0)
    assert t['weight_zero_point'].shape == (n // 8, k // 128)
    dec = qdq.decode_weight(synth.prefixed(t, 'a.weight'), 'a.weight').astype(np.float32)
    s = np.repeat(t['weight_scale'].astype(np.float32), 128, axis=1)
    # round-to-nearest: half a step, plus the fp16 rounding of the decoded value
    w32 = w.astype(np.float32)
    assert np.all(np.abs(dec - w32) <= s * 0.5 + np.abs(w32) * 2.0 ** -10 + 1e-7)


# ------------------------------------------------------------------- W8A8
def test_w8a8_activation_quantizer_known_answers():
    """Hand-derived: at absmax 127 the scale is exactly 1, so x / scale = x
    and the ties 62.5 / -2.5 / 0.5 show round-half-even (62, -2, 0; half-away
    would give 63, -3, 1); a zero row takes the 1e-12 floor (q = 0, scale
    bits of fp32(1e-12) / 127); the scale of absmax 1 is the fp32 quotient
    1/127, not its fp16 rounding."""
    x = np.array([[127.0, 62.5, -2.5, 0.5, -127.0, 3.0, 0.0, 1.0],
                  [0.0] * 8,
                  [1.0, -0.5, 0.25, 0.0, 0.0, 0.0, 0.0, 0.0]], dtype=np.float16)
    q, s = qdq.quantize_activations_per_token(x)
    assert q.dtype == np.int8 and s.dtype == np.float32
    assert q[0].tolist() == [127, 62, -2, 0, -127, 3, 0, 1]
    assert s[0] == np.float32(1.0)
    assert q[1].tolist() == [0] * 8 and s[1] == np.float32(np.float32(1e-12) / np.float32(127))
    assert s[2] == np.float32(1.0) / np.float32(127) and s[2] != np.float32(np.float16(1.0 / 127))
    assert q[2].tolist() == [127, -64, 32, 0, 0, 0, 0, 0]   # -63.5 -> -64 and 31.75 -> 32


def test_w8a8_activation_quantizer_matches_reference_torch_expression():
    """The reference's own torch lines (backend.py:258-260) on the CPU."""
    import torch
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((7, 96)) * rng.choice([0.01, 1.0, 30.0], size=(7, 1))).astype(np.float16)
    x[3] = 0
    t = torch.from_numpy(x).float()
    scale = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / 127
    q_ref = t.div(scale).round().clamp(-127, 127)
    q, s = qdq.quantize_activations_per_token(x)
    assert np.array_equal(q.astype(np.float32), q_ref.numpy())
    assert np.array_equal(s, scale.numpy()[:, 0])


def test_reference_w8a8_linear_matches_reference_torch_lines():
    """backend.py:257-263 on the CPU: decode the channel-INT8 weight, fake
    quantize x, F.linear (fp32 accumulation)."""
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, 64)).astype(np.float16)
    qw = rng.integers(-127, 128, (12, 64)).astype(np.int8)
    ws = (rng.random(12) * 0.01 + 1e-3).astype(np.float16)
    t = torch.from_numpy(x).float()
    scale = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / 127
    xq = (t.div(scale).round().clamp(-127, 127) * scale).half()
    w = (torch.from_numpy(qw).float() * torch.from_numpy(ws).float()[:, None]).half()
    expected = F.linear(xq.float(), w.float()).half().numpy()
    assert np.array_equal(qdq.reference_w8a8_linear(x, qw, ws), expected)


def test_w8a8_scaled_int_gemm_brute_force():
    """Python-integer dot products, then the fp32 scaling left to right."""
    rng = np.random.default_rng(7)
    qx = rng.integers(-127, 128, (3, 40)).astype(np.int8)
    qw = rng.integers(-127, 128, (5, 40)).astype(np.int8)
    xs = (rng.random(3) * 0.1).astype(np.float32)
    wsc = (rng.random(5) * 0.01).astype(np.float32)
    bias = rng.standard_normal(5).astype(np.float16)
    got = qdq.w8a8_linear_int(qx, xs, qw, wsc, bias)
    for m in range(3):
        for n in range(5):
            acc = sum(int(qx[m, k]) * int(qw[n, k]) for k in range(40))
            r = np.float32(np.float32(np.float32(acc) * xs[m]) * wsc[n]) + np.float32(bias[n])
            assert got[m, n] == np.float16(np.float32(r))
    # the largest magnitude a Qwen3 shape produces still fits int32
    assert 127 * 127 * 17408 < 2 ** 31


# ------------------------------------------------------------------- torch-CPU restatement (bench baseline)

def _torch_weights(weights):
    import torch
    return {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in weights.items()}


@pytest.mark.parametrize('sym', [False, True])
def test_torch_qdq_decode_is_bit_identical_to_the_numpy_oracle(sym):
    from oracle import qdq_torch
    weights, x = synth.w4_case(48, 512, 3, seed=11, symmetric=sym, name='p.weight')
    got = qdq_torch.decode_weight(_torch_weights(weights), 'p.weight').numpy()
    assert np.array_equal(got.view(np.uint16), qdq.decode_weight(weights, 'p.weight').view(np.uint16))
    y = qdq_torch.qdq_linear(_torch_weights({'x': x})['x'], _torch_weights(weights), 'p.weight').numpy()
    assert qdq.parity_ok(qdq.parity_metrics(y, qdq.qdq_linear(x, weights, 'p.weight')))
    assert np.abs(y.astype(np.float32) - qdq.qdq_linear(x, weights, 'p.weight').astype(np.float32)).max() <= \
        2 ** -10 * np.abs(y).max()


def test_torch_qdq_int8_matches_the_numpy_oracle():
    import torch
    from oracle import qdq_torch
    _, q, s, x = synth.int8_case(40, 256, 2, seed=12)
    ct = {'p.weight': torch.from_numpy(q), 'p.weight_scale': torch.from_numpy(s).reshape(-1, 1)}
    assert np.array_equal(qdq_torch.decode_weight(ct, 'p.weight').numpy().view(np.uint16),
                          qdq.dequantize_linear_weight(q, s).view(np.uint16))
    y = qdq_torch.int8_qdq_linear(torch.from_numpy(x), torch.from_numpy(q), torch.from_numpy(s)).numpy()
    assert qdq.parity_ok(qdq.parity_metrics(y, qdq.int8_weight_only_linear(x, q, s)))
    # the KAT of test_weight_quant_backend.py:33-35 through the torch decode
    kat = {'p.weight': torch.tensor([[2, -3]], dtype=torch.int8), 'p.weight_scale': torch.tensor([[0.5]]).half()}
    assert qdq_torch.decode_weight(kat, 'p.weight').tolist() == [[1.0, -1.5]]


def test_torch_unpack_matches_kat_words():
    import torch
    from oracle import qdq_torch
    word = torch.tensor([[0x76543210]], dtype=torch.int32)
    assert qdq_torch.unpack_unsigned(word, 4, 1, 8).tolist() == [[0, 1, 2, 3, 4, 5, 6, 7]]
    assert qdq_torch.unpack_unsigned(word, 4, 0, 8).t().tolist() == [[0, 1, 2, 3, 4, 5, 6, 7]]
    neg = torch.tensor([[-1]], dtype=torch.int32)     # sign bits must not leak into the top field
    assert qdq_torch.unpack_unsigned(neg, 4, 1, 8).tolist() == [[15] * 8]
