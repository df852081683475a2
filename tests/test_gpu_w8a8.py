"""GPU parity of the W8A8 path (``int8_gemm``) through the C ABI.

Bars: the activation quantizer bit-exact against ``oracle.qdq.
quantize_activations_per_token`` (codes and fp32 scales); the scaled INT8
linear bit-exact against ``oracle.qdq.w8a8_linear_int`` (integer accumulation
is exact and the fp32 rescale is done in the same order); the backend end to
end within the reference harness's bar against ``reference_w8a8``
(``validate_weight_quant_kernels.py:44-76``: cosine >= 0.9999, rel-L2 <=
0.02) plus ``oracle.qdq.parity_ok``.
"""
import numpy as np
import pytest
import torch

from oracle import qdq
from ondeviceinfer_amd import _native
from ondeviceinfer_amd.weight_quantization import backend as wq

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize('m,k,scale', [(1, 5120, 1.0), (5, 64, 0.01), (300, 5120, 30.0), (3, 17408, 1.0)])
def test_w8a8_quantize_bit_exact(m, k, scale):
    print(f'[w8a8_quantize] m={m} k={k}', flush=True)
    rng = np.random.default_rng(m + k)
    x = (rng.standard_normal((m, k)) * scale).astype(np.float16)
    if m > 2:
        x[1] = 0                                    # zero row: the 1e-12 floor
        x[2, :8] = [127.0, 62.5, -2.5, 0.5, -127.0, 3.0, 0.0, 1.0]   # half-even ties at scale 1
        x[2, 8:] = 0
    qx, sx = _native.w8a8_quantize(dev(x))
    q_ref, s_ref = qdq.quantize_activations_per_token(x)
    assert np.array_equal(host(qx), q_ref)
    assert np.array_equal(host(sx), s_ref)


def test_scaled_int8_quant_harness_surface():
    """``backend.ops.scaled_int8_quant(x)`` as the reference's kernel harness
    calls it (``validate_weight_quant_kernels.py:51``): ``(qx, scale [M, 1],
    None)``, bit-exact against the oracle's per-token quantizer."""
    x = (np.random.default_rng(11).standard_normal((32, 5120)) * 0.1).astype(np.float16)
    qx, sx, azp = wq.CompressedLinearBackend('int8_gemm').ops.scaled_int8_quant(dev(x))
    q_ref, s_ref = qdq.quantize_activations_per_token(x)
    assert azp is None and qx.dtype == torch.int8 and tuple(sx.shape) == (32, 1) and sx.dtype == torch.float32
    assert np.array_equal(host(qx), q_ref) and np.array_equal(host(sx).reshape(-1), s_ref)


@pytest.mark.parametrize('m,n,k,with_bias', [
    (1, 5120, 5120, False),      # decode, q/o shape
    (1, 1024, 17408, True),      # decode, long k
    (2, 1000, 192, False),       # ragged n, 3 k-steps
    (16, 64, 64, True),          # largest decode batch, one k-step
    (17, 80, 256, False),        # smallest GEMM batch, ragged m and n
    (65, 1000, 5120, True),
    (300, 520, 192, False),      # GEMM batch with k/64 not a multiple of the chunk -> decode kernel per 16 rows
    (256, 5120, 5120, False),    # GEMM, 128-row x tiles, one weight tile per wave
    (200, 17408, 128, True),     # GEMM, 32-row x tiles, four weight tiles per wave
])
def test_w8a8_linear_bit_exact(m, n, k, with_bias):
    print(f'[w8a8_linear] m={m} n={n} k={k} bias={with_bias}', flush=True)
    rng = np.random.default_rng(m * 7 + n + k)
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    xs = (rng.random(m) * 0.05 + 1e-4).astype(np.float32)
    wsc = (rng.random(n) * 0.002 + 1e-5).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float16) if with_bias else None
    y = _native.w8a8_linear(dev(qx), dev(xs), dev(qw), dev(wsc), None if bias is None else dev(bias))
    expected = qdq.w8a8_linear_int(qx, xs, qw, wsc, bias)
    got = host(y)
    assert np.array_equal(got.view(np.uint16), expected.view(np.uint16)), \
        np.argwhere(got.view(np.uint16) != expected.view(np.uint16))[:5]


def test_w8a8_linear_prefill_sampled_rows_bit_exact():
    """configs[2]-sized batch (M = 4096, 5120 -> 5120: 128-row x tiles, four
    weight tiles per wave), checked bit for bit on 48 sampled rows."""
    rng = np.random.default_rng(4096)
    m, n, k = 4096, 5120, 5120
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    xs = (rng.random(m) * 0.05 + 1e-4).astype(np.float32)
    wsc = (rng.random(n) * 0.002 + 1e-5).astype(np.float32)
    y = host(_native.w8a8_linear(dev(qx), dev(xs), dev(qw), dev(wsc)))
    rows = np.sort(rng.choice(m, 48, replace=False))
    expected = qdq.w8a8_linear_int(qx[rows], xs[rows], qw, wsc)
    assert np.array_equal(y[rows].view(np.uint16), expected.view(np.uint16))


def test_w8a8_linear_rejects_unsupported_k():
    qx = torch.zeros(1, 96, dtype=torch.int8, device='cuda')
    qw = torch.zeros(16, 96, dtype=torch.int8, device='cuda')
    one = torch.ones(1, device='cuda')
    with pytest.raises(Exception, match='k % 64'):
        _native.w8a8_linear(qx, one, qw, torch.ones(16, device='cuda'))


@pytest.mark.parametrize('m', [1, 4, 32, 256])
def test_int8_gemm_backend_matches_reference_w8a8(m):
    """The reference harness at layer shape 5120 -> 5120 (channel INT8 with
    fp16 scales, x ~ 0.1 N(0, 1)), both backends through the same dict."""
    print(f'[int8_gemm backend] m={m}', flush=True)
    rng = np.random.default_rng(m)
    w = (rng.standard_normal((5120, 5120)) * 0.02).astype(np.float32)
    qw, ws = qdq.quantize_linear_weight(w)
    layer = {'self_attn.o_proj.weight': dev(qw), 'self_attn.o_proj.weight_scale': dev(ws.reshape(-1, 1))}
    ref_layer = dict(layer)
    fused, reference = wq.CompressedLinearBackend('int8_gemm'), wq.CompressedLinearBackend('reference_w8a8')
    fused.prepare(layer, 'self_attn.o_proj.weight')
    x = (rng.standard_normal((m, 5120)) * 0.1).astype(np.float16)
    got = host(fused.linear(dev(x), layer, 'self_attn.o_proj.weight'))
    want = host(reference.linear(dev(x), ref_layer, 'self_attn.o_proj.weight'))
    oracle = qdq.reference_w8a8_linear(x, qw, ws)
    metrics = qdq.parity_metrics(got, want)
    assert metrics['cosine'] >= 0.9999 and metrics['relative_l2'] <= 0.02, metrics
    assert qdq.parity_ok(qdq.parity_metrics(got, oracle))
    assert (fused.calls, fused.gemm_calls, fused.activation_quantize_calls) == (1, 1, 1)
    assert reference.explicit_dequant_bytes == 5120 * 5120 * 2


def test_int8_gemm_backend_repeatable():
    rng = np.random.default_rng(11)
    qw = rng.integers(-127, 128, (1024, 5120)).astype(np.int8)
    layer = {'mlp.up_proj.weight': dev(qw), 'mlp.up_proj.weight_scale': dev(np.full((1024, 1), 1e-3, np.float16))}
    b = wq.CompressedLinearBackend('int8_gemm')
    b.prepare(layer, 'mlp.up_proj.weight')
    x = dev((rng.standard_normal((3, 5120))).astype(np.float16))
    first = host(b.linear(x, layer, 'mlp.up_proj.weight'))
    for _ in range(3):
        assert np.array_equal(host(b.linear(x, layer, 'mlp.up_proj.weight')), first)
