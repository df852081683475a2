"""Prefill W4A16 GEMM with the MLP's elementwise op in its epilogue
(wq_w4a16_linear_epilogue): bit-identical to the plain GEMM followed by
wq_silu_mul / the fp16 residual add, and within the parity bar of the oracle
(oracle.qdq decode + fp32-accumulated linear, oracle.qwen3.swiglu) on sampled
rows.  Shapes cover each epilogue grid (256-wide slices of 128-row tiles,
128-wide slices of 64-row tiles, 64-wide slices for the residual) and
partial last slices, where a wave's gate tiles run past the gate half."""
import numpy as np
import pytest
import torch

from oracle import qdq, qwen3, synth
from ondeviceinfer_amd import _native
from ondeviceinfer_amd.weight_quantization import backend as wq

pytestmark = pytest.mark.gpu


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _gate_up(n_half, k, seed, device):
    """Fused [gate | up] prepared weight plus the two parts' weight dicts."""
    wg, _ = synth.w4_case(n_half, k, 1, seed=seed, name='mlp.gate_proj.weight')
    wu, _ = synth.w4_case(n_half, k, 1, seed=seed + 1, name='mlp.up_proj.weight')
    layer = {name: _dev(v, device) for name, v in {**wg, **wu}.items()}
    backend = wq.CompressedLinearBackend('marlin', group_size=128)
    backend.prepare(layer, 'mlp.gate_proj.weight')
    backend.prepare(layer, 'mlp.up_proj.weight')
    backend.fuse_projections(layer)
    return backend, layer, wg, wu


def _rows(m):
    picks = {0, 1, 15, 63, 64, 127, 128, m // 2, m - 65, m - 1}
    return np.array(sorted(r for r in picks if 0 <= r < m))


@pytest.mark.parametrize('m,n_half,k', [
    (4096, 17408, 5120),    # Qwen3-14B gate_up at the 4K prompt: 256-wide slices of 128-row tiles
    (4096, 17456, 1024),    # 1091 tiles per half: the last slice's gate tiles run into the up half
    (300, 17408, 5120),     # 128-wide slices of 64-row tiles, partial last row block
    (4096, 1040, 512),      # 65 tiles per half on the 128-wide grid
    (65, 17408, 1024),      # the smallest row count the epilogue takes
])
def test_silu_epilogue_equals_gemm_then_silu_mul(gpu, m, n_half, k):
    print(f'[epilogue silu] m={m} n_half={n_half} k={k}', flush=True)
    _, layer, wg, wu = _gate_up(n_half, k, seed=m + n_half, device=gpu)
    p = layer['mlp.gate_up_proj._prepared']
    assert _native.w4a16_epilogue_supported(m, 2 * n_half, k, 128, _native.EPI_SILU_MUL)
    rng = np.random.default_rng(m)
    x = _dev(rng.standard_normal((m, k), dtype=np.float32).astype(np.float16), gpu)
    fused = _native.w4a16_linear_epilogue(x, p.tiles, p.meta, 2 * n_half, 128, _native.EPI_SILU_MUL)
    plain = _native.silu_mul(_native.w4a16_linear(x, p.tiles, p.meta, 2 * n_half, 128))
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))
    rows = _rows(m)
    xs = x[torch.from_numpy(rows).to(gpu)].cpu().numpy()
    ref = qwen3.swiglu(qdq.qdq_linear(xs, wg, 'mlp.gate_proj.weight'), qdq.qdq_linear(xs, wu, 'mlp.up_proj.weight'))
    got = fused.cpu().numpy()[rows]
    metrics = qdq.parity_metrics(got, ref)
    assert qdq.parity_ok(metrics), metrics


@pytest.mark.parametrize('m,n,k', [
    (4096, 5120, 17408),    # Qwen3-14B down at the 4K prompt
    (1024, 5120, 5120),     # 128-wide slices of 64-row tiles
    (2560, 1024, 1024),     # 64-wide slices (one tile per wave)
    (4096, 1000, 256),      # n not a multiple of 16: partial last tile
])
def test_residual_epilogue_equals_gemm_then_add(gpu, m, n, k):
    print(f'[epilogue residual] m={m} n={n} k={k}', flush=True)
    weights, _ = synth.w4_case(n, k, 1, seed=n + k, name='mlp.down_proj.weight')
    layer = {name: _dev(v, gpu) for name, v in weights.items()}
    wq.CompressedLinearBackend('marlin', group_size=128).prepare(layer, 'mlp.down_proj.weight')
    p = layer['mlp.down_proj._prepared']
    assert _native.w4a16_epilogue_supported(m, n, k, 128, _native.EPI_RESIDUAL)
    rng = np.random.default_rng(k)
    x = _dev(rng.standard_normal((m, k), dtype=np.float32).astype(np.float16), gpu)
    res = _dev((rng.standard_normal((m, n), dtype=np.float32) * 4).astype(np.float16), gpu)
    fused = _native.w4a16_linear_epilogue(x, p.tiles, p.meta, n, 128, _native.EPI_RESIDUAL, res)
    plain = res + _native.w4a16_linear(x, p.tiles, p.meta, n, 128)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))
    # In place (out aliases the residual) gives the same bits.
    inplace = res.clone()
    _native.w4a16_linear_epilogue(x, p.tiles, p.meta, n, 128, _native.EPI_RESIDUAL, inplace, out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(inplace.view(torch.int16), plain.view(torch.int16))
    rows = _rows(m)
    xs = x[torch.from_numpy(rows).to(gpu)].cpu().numpy()
    ref = (qdq.qdq_linear(xs, weights, 'mlp.down_proj.weight').astype(np.float32)
           + res.cpu().numpy()[rows].astype(np.float32)).astype(np.float16)
    metrics = qdq.parity_metrics(fused.cpu().numpy()[rows], ref)
    assert qdq.parity_ok(metrics), metrics


def _int8_weight(n, k, seed, device):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s = (rng.random(n) * 2e-3 + 1e-4).astype(np.float16)
    return q, s, _native.w8_repack(_dev(q, device)), _dev(s, device)


@pytest.mark.parametrize('m,n_half,k', [
    (4096, 17408, 5120),    # the INT8 model's fused gate_up at the 4K prompt
    (300, 17408, 5120),     # 128-wide slices of 64-row tiles
    (4096, 1040, 512),      # partial last slice
])
def test_int8_silu_epilogue_equals_gemm_then_silu_mul(gpu, m, n_half, k):
    print(f'[int8 epilogue silu] m={m} n_half={n_half} k={k}', flush=True)
    q, s, tiles, scale = _int8_weight(2 * n_half, k, m + k, gpu)
    assert _native.w8a16_epilogue_supported(m, 2 * n_half, k, _native.EPI_SILU_MUL)
    x = torch.randn(m, k, dtype=torch.float16, device=gpu)
    fused = _native.w8a16_linear_epilogue(x, tiles, scale, _native.EPI_SILU_MUL)
    plain = _native.silu_mul(_native.w8a16_linear(x, tiles, scale))
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))
    rows = _rows(m)
    xs = x[torch.from_numpy(rows).to(gpu)].cpu().numpy()
    ref = qwen3.swiglu(qdq.int8_weight_only_linear(xs, q[:n_half], s[:n_half]),
                       qdq.int8_weight_only_linear(xs, q[n_half:], s[n_half:]))
    metrics = qdq.parity_metrics(fused.cpu().numpy()[rows], ref)
    assert qdq.parity_ok(metrics), metrics


@pytest.mark.parametrize('m,n,k', [(4096, 5120, 17408), (2560, 1024, 1024)])
def test_int8_residual_epilogue_equals_gemm_then_add(gpu, m, n, k):
    print(f'[int8 epilogue residual] m={m} n={n} k={k}', flush=True)
    q, s, tiles, scale = _int8_weight(n, k, n + k, gpu)
    assert _native.w8a16_epilogue_supported(m, n, k, _native.EPI_RESIDUAL)
    x = torch.randn(m, k, dtype=torch.float16, device=gpu)
    res = torch.randn(m, n, dtype=torch.float16, device=gpu) * 4
    fused = _native.w8a16_linear_epilogue(x, tiles, scale, _native.EPI_RESIDUAL, res)
    plain = res + _native.w8a16_linear(x, tiles, scale)
    inplace = res.clone()
    _native.w8a16_linear_epilogue(x, tiles, scale, _native.EPI_RESIDUAL, inplace, out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(inplace.view(torch.int16), plain.view(torch.int16))
    assert not _native.w8a16_epilogue_supported(64, n, k, _native.EPI_RESIDUAL)


def test_epilogue_rejects_decode_rows_and_backend_falls_back(gpu):
    backend, layer, wg, wu = _gate_up(17408, 512, seed=3, device=gpu)
    p = layer['mlp.gate_up_proj._prepared']
    n = 2 * 17408
    assert not _native.w4a16_epilogue_supported(64, n, 512, 128, _native.EPI_SILU_MUL)
    assert not _native.w4a16_epilogue_supported(4096, 2040, 512, 128, _native.EPI_SILU_MUL)   # n % 32
    assert not _native.w4a16_epilogue_supported(200, 1024, 1024, 128, _native.EPI_RESIDUAL)    # deep-ring grid
    x = torch.randn(64, 512, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match='epilogue'):
        _native.w4a16_linear_epilogue(x, p.tiles, p.meta, n, 128, _native.EPI_SILU_MUL)
    # The backend returns None for such rows (the model then runs the two steps).
    assert backend.linear_epilogue(x, layer, 'mlp.gate_up_proj.weight', _native.EPI_SILU_MUL) is None
    # With row chunks (marlin_max_rows_per_call) every chunk must take the epilogue.
    x = torch.randn(300, 512, dtype=torch.float16, device=gpu)
    backend.marlin_max_rows_per_call = 128
    assert backend.linear_epilogue(x, layer, 'mlp.gate_up_proj.weight', _native.EPI_SILU_MUL) is None
    backend.marlin_max_rows_per_call = 150
    chunked = backend.linear_epilogue(x, layer, 'mlp.gate_up_proj.weight', _native.EPI_SILU_MUL)
    whole = _native.silu_mul(_native.w4a16_linear(x, p.tiles, p.meta, n, 128))
    torch.cuda.synchronize()
    assert torch.equal(chunked.view(torch.int16), whole.view(torch.int16))
