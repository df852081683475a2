"""The prefill GEMM block loops on odd numbers of 128-k blocks, where the loop
unrolled over two weight-register sets ends on a run-out step (its loads read
past the end of every buffer and its math is skipped): W4A16 on each grid
launch_gemm_auto picks (64-row tiles, two tiles per wave, four tiles per wave
on 128-row tiles, the deep ring), W8A16 over INT8 tiles and row-major INT8,
and the W8A8 GEMM's one-tile grids, against the CPU oracle on ragged M and N.

Bars: ``oracle.qdq.parity_ok`` for the fp16 paths; W8A8 bit for bit
(integer products summed exactly, one fp32 scale step, as in
test_gpu_w8a8.py)."""
import numpy as np
import pytest
import torch

from oracle import qdq, synth
from ondeviceinfer_amd import _native
from ondeviceinfer_amd.weight_quantization import backend as wq

pytestmark = pytest.mark.gpu


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check_parity(actual, expected, label):
    m = qdq.parity_metrics(actual, expected)
    print(label, {k: (round(v, 8) if isinstance(v, float) else v) for k, v in m.items()}, flush=True)
    assert qdq.parity_ok(m), (label, m)


# (n, k, m): k = 384 / 640 / 5248 are 3 / 5 / 41 blocks.  Grids: n = 1000 at
# m = 65 and 200 the deep ring (41 blocks also split in four k ranges of 10,
# 10, 10 and 11 through the workspace), at m = 1600 one tile per wave on
# 64-row tiles;
# n = 16400 (1025 tiles) at m = 300 two tiles per wave on 64-row tiles, at
# m = 1100 four tiles per wave on 128-row tiles.
W4_CASES = [(1000, 384, 65), (1000, 5248, 200), (1000, 640, 1600), (16400, 384, 300), (16400, 640, 1100)]


@pytest.mark.parametrize('n,k,m', W4_CASES)
def test_w4a16_gemm_odd_block_counts(gpu, n, k, m):
    name = 'p.weight'
    weights, x = synth.w4_case(n, k, m, seed=n + k + m, name=name)
    layer = {key: dev(v, gpu) for key, v in weights.items()}
    backend = wq.CompressedLinearBackend('marlin')
    backend.prepare(layer, name)
    print(f'[w4 gemm odd blocks] n={n} k={k} m={m}', flush=True)
    y = host(backend.linear(dev(x, gpu), layer, name))
    rows = np.sort(np.random.default_rng(k + m).choice(m, size=min(m, 48), replace=False))
    check_parity(y[rows], qdq.qdq_linear(x[rows], weights, name), f'w4 n={n} k={k} m={m}')
    # The rows of a shorter call equal the same rows of this one bit for bit
    # (every grid sums each output in the same k order).
    y_short = host(backend.linear(dev(x[:70], gpu), layer, name))
    assert np.array_equal(y_short.view(np.uint16), y[:70].view(np.uint16))


def test_w4a16_gemm_long_k_split_on_a_wider_grid(gpu):
    """k = 8320 (65 blocks, at least 64: a long chain) on the deep ring's
    464 workgroups (16 n slices x 29 row blocks at m = 900), above the 384
    to which short chains split: four k splits of 16 or 17 blocks."""
    n, k, m = 1000, 8320, 900
    assert _native.w4a16_workspace_size(m, n, k, 128) > 0
    assert _native.w4a16_workspace_size(m, n, 5120, 128) == 0     # a short chain on the same grid
    name = 'p.weight'
    weights, x = synth.w4_case(n, k, m, seed=7, name=name)
    layer = {key: dev(v, gpu) for key, v in weights.items()}
    backend = wq.CompressedLinearBackend('marlin')
    backend.prepare(layer, name)
    print(f'[w4 gemm long-k split] n={n} k={k} m={m}', flush=True)
    y = host(backend.linear(dev(x, gpu), layer, name))
    rows = np.sort(np.random.default_rng(m).choice(m, size=48, replace=False))
    check_parity(y[rows], qdq.qdq_linear(x[rows], weights, name), f'w4 long-k n={n} k={k} m={m}')


def test_w4a16_down_shape_splits_k_at_m256(gpu):
    """The down projection's shape (17408 -> 5120, 136 blocks) at M = 256:
    640 deep-ring workgroups in two k splits of 68 blocks, against the oracle
    on 48 rows, and against the whole-k call (a workspace too small for the
    split) to the same bar; the split's counters are back at zero."""
    n, k, m = 5120, 17408, 256
    nbytes = _native.w4a16_workspace_size(m, n, k, 128)
    assert nbytes == 16384 + 640 * 2 * 8192
    name = 'mlp.down_proj.weight'
    weights, x = synth.w4_case(n, k, m, seed=11, name=name)
    layer = {key: dev(v, gpu) for key, v in weights.items()}
    wq.CompressedLinearBackend('marlin').prepare(layer, name)
    prep = layer['mlp.down_proj._prepared']
    xd = dev(x, gpu)
    print(f'[w4 gemm down shape split] n={n} k={k} m={m}', flush=True)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    split = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=ws))
    whole = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128,
                                      workspace=torch.zeros(16, dtype=torch.uint8, device=gpu)))
    rows = np.sort(np.random.default_rng(m).choice(m, size=48, replace=False))
    check_parity(split[rows], qdq.qdq_linear(x[rows], weights, name), 'down shape, two k splits')
    check_parity(split, whole.astype(np.float32), 'down shape, split against whole k')
    assert torch.count_nonzero(ws[:16384]).item() == 0


@pytest.mark.parametrize('n,k,m', [(1000, 384, 200), (1040, 640, 300), (5120, 640, 1100)])
def test_w8a16_gemm_odd_block_counts(gpu, n, k, m):
    _, q, s, x = synth.int8_case(n, k, m, seed=n + k + m)
    qd, sd, xd = dev(q, gpu), dev(s, gpu), dev(x, gpu)
    print(f'[w8a16 gemm odd blocks] n={n} k={k} m={m}', flush=True)
    y_rm = _native.w8a16_linear(xd, qd, sd)
    y_t = _native.w8a16_linear(xd, _native.w8_repack(qd), sd)
    assert torch.equal(y_rm, y_t), f'tiled != row-major n={n} k={k} m={m}'
    rows = np.sort(np.random.default_rng(k).choice(m, size=48, replace=False))
    ref = qdq.linear_fp32(x[rows], qdq.dequantize_linear_weight(q, s))
    check_parity(host(y_t)[rows], ref, f'w8a16 n={n} k={k} m={m}')


# One-tile W8A8 grids (at most one round of workgroups): 32-row tiles below
# m = 256, 128-row tiles from there; 3 and 5 blocks, ragged m and n.
@pytest.mark.parametrize('m,n,k', [(100, 1000, 384), (33, 520, 640), (300, 520, 640), (257, 1000, 384)])
def test_w8a8_one_tile_gemm_odd_block_counts(gpu, m, n, k):
    print(f'[w8a8 one-tile odd blocks] m={m} n={n} k={k}', flush=True)
    rng = np.random.default_rng(m * 3 + n + k)
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    xs = (rng.random(m) * 0.05 + 1e-4).astype(np.float32)
    wsc = (rng.random(n) * 0.002 + 1e-5).astype(np.float32)
    expected = qdq.w8a8_linear_int(qx, xs, qw, wsc, None)
    for w in (dev(qw, gpu), _native.w8_repack(dev(qw, gpu))):
        got = host(_native.w8a8_linear(dev(qx, gpu), dev(xs, gpu), w, dev(wsc, gpu)))
        assert np.array_equal(got.view(np.uint16), expected.view(np.uint16)), \
            np.argwhere(got.view(np.uint16) != expected.view(np.uint16))[:5]
