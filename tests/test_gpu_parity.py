"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars: repack/unpack/decode/quantize bit-exact; linear outputs within
max|d| <= 1e-2 * ||y_ref||_inf, mean|d|/mean|y_ref| <= 2e-3 (fp32
accumulation), cosine >= 0.9999 and rel-L2 <= 0.02 (``oracle.qdq.parity_ok``).
The benchmark configs' full shapes are checked whole at M=1 and on sampled activation rows
at M=4096 (the oracle restricted to those rows is the same computation).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import qdq, synth, tile_layout
from ondeviceinfer_amd import _native
from ondeviceinfer_amd import quantization as q8
from ondeviceinfer_amd.quantized_model import int8_weight_only_linear
from ondeviceinfer_amd.weight_quantization import backend as wq

pytestmark = pytest.mark.gpu
KAT = json.loads((Path(__file__).parent / 'golden' / 'weight_quant_kat.json').read_text())


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def check_parity(actual, expected, label):
    m = qdq.parity_metrics(actual, expected)
    print(label, {k: (round(v, 8) if isinstance(v, float) else v) for k, v in m.items()}, flush=True)
    assert qdq.parity_ok(m), (label, m)


def prepared_w4(weights, name, device, group_size=128):
    layer = {k: dev(v, device) for k, v in weights.items()}
    backend = wq.CompressedLinearBackend('marlin', group_size=group_size)
    backend.prepare(layer, name)
    return backend, layer


# ------------------------------------------------------------------ layout / decode, bit-exact

@pytest.mark.parametrize('n,k,g,sym', [(16, 256, 128, False), (1000, 1024, 128, False), (24, 512, 256, True),
                                       (5120, 5120, 128, False)])
def test_repack_is_the_tile_layout_and_round_trips(gpu, n, k, g, sym):
    weights, _ = synth.w4_case(n, k, 1, seed=n, group_size=g, symmetric=sym, name='p.weight')
    packed, scale, zero = weights['p.weight_packed'], weights['p.weight_scale'], weights.get('p.weight_zero_point')
    tiles, meta = _native.w4_repack(dev(packed, gpu), dev(scale, gpu), None if zero is None else dev(zero, gpu),
                                    n, k, g)
    ref_tiles, ref_meta = tile_layout.w4_repack(packed, scale, zero, n, k, g)
    assert np.array_equal(host(tiles), ref_tiles.view(np.uint8).ravel())
    assert np.array_equal(host(meta), ref_meta.ravel())
    p2, s2, z2 = _native.w4_unpack(tiles, meta, n, k, g)
    assert np.array_equal(host(p2), packed)
    assert np.array_equal(bits(host(s2)), bits(scale))
    if zero is None:
        assert np.all(host(z2).view(np.uint32) == tile_layout.SYMMETRIC_ZERO_WORD)
    else:
        assert np.array_equal(host(z2), zero)
    # the kernels' own unpack arithmetic reproduces the reference decode bit for bit
    deq = _native.w4_dequant(tiles, meta, n, k, g)
    assert np.array_equal(bits(host(deq)), bits(qdq.decode_weight(weights, 'p.weight', group_size=g)))


def test_decode_known_answers_on_gpu(gpu):
    c = KAT['kat_group_decode']
    w = {'mlp.up_proj.weight_packed': torch.tensor(c['weight_packed'], dtype=torch.int32, device=gpu),
         'mlp.up_proj.weight_shape': torch.tensor(c['weight_shape']),
         'mlp.up_proj.weight_scale': torch.tensor(c['weight_scale'], device=gpu),
         'mlp.up_proj.weight_zero_point': torch.tensor(c['weight_zero_point'], dtype=torch.int32, device=gpu)}
    assert host(wq.decode_weight(w, c['name'], group_size=c['group_size'])).tolist() == c['expected']
    c = KAT['kat_symmetric']
    w = {'self_attn.q_proj.weight_packed': torch.tensor(c['weight_packed'], dtype=torch.int32, device=gpu),
         'self_attn.q_proj.weight_shape': torch.tensor(c['weight_shape']),
         'self_attn.q_proj.weight_scale': torch.tensor(c['weight_scale'], device=gpu)}
    assert host(wq.decode_weight(w, c['name'], group_size=c['group_size'])).tolist() == c['expected']
    c = KAT['kat_int8_channel']
    w = {c['name']: torch.tensor(c['weight'], dtype=torch.int8, device=gpu),
         'self_attn.q_proj.weight_scale': torch.tensor(c['weight_scale'], device=gpu)}
    assert host(wq.decode_weight(w, c['name'])).tolist() == c['expected']


@pytest.mark.parametrize('use_gidx', [False, True])
@pytest.mark.parametrize('sym', [False, True])
def test_decode_random_bit_exact(gpu, use_gidx, sym):
    n, k, g = 64, 1024, 128
    weights, _ = synth.w4_case(n, k, 1, seed=5, group_size=g, symmetric=sym, name='p.weight')
    if use_gidx:
        weights['p.weight_g_idx'] = np.random.default_rng(1).permutation(np.arange(k) // g).astype(np.int32)
    got = wq.decode_weight({kk: dev(v, gpu) for kk, v in weights.items()}, 'p.weight', group_size=g)
    assert np.array_equal(bits(host(got)), bits(qdq.decode_weight(weights, 'p.weight', group_size=g)))


def test_decode_rows_matches_oracle(gpu):
    """decode_rows (``wq_w4_decode_rows``): the reference KAT
    (``test_weight_quant_backend.py:38-45``), sampled rows of a 151936-row
    LM-head-sized weight, the symmetric format and INT8 channel rows, each
    bit-exact against ``oracle.qdq.decode_rows``."""
    c = KAT['kat_sampled_rows']
    scale = np.array(c['weight_scale_f16_bits'], dtype=np.uint16).view(np.float16)
    w = {'mlp.up_proj.weight_packed': np.full(c['packed_shape'], c['packed_word'], dtype=np.int32),
         'mlp.up_proj.weight_shape': np.array(c['weight_shape']),
         'mlp.up_proj.weight_scale': scale,
         'mlp.up_proj.weight_zero_point': np.array(c['weight_zero_point'], dtype=np.int32)}
    rows = np.array(c['rows'])
    got = wq.decode_rows({k: dev(v, gpu) for k, v in w.items()}, c['name'], dev(rows, gpu))
    assert np.array_equal(bits(host(got)), bits(qdq.decode_rows(w, c['name'], rows)))
    for sym in (False, True):
        weights, _ = synth.w4_case(151936, 256, 1, seed=5, symmetric=sym, name='lm_head.weight')
        rows = np.sort(np.random.default_rng(6).choice(151936, size=333, replace=False))
        rows[0], rows[-1] = 0, 151935
        got = wq.decode_rows({k: dev(v, gpu) for k, v in weights.items()}, 'lm_head.weight', dev(rows, gpu))
        assert got.shape == (333, 256)
        assert np.array_equal(bits(host(got)), bits(qdq.decode_rows(weights, 'lm_head.weight', rows))), sym
    _, q, s8, _ = synth.int8_case(40, 256, 1, seed=7)
    w8 = {'p.weight': q, 'p.weight_scale': s8.reshape(-1, 1)}
    rows = np.array([39, 0, 17, 17])
    got = wq.decode_rows({k: dev(v, gpu) for k, v in w8.items()}, 'p.weight', dev(rows, gpu))
    assert np.array_equal(bits(host(got)), bits(qdq.decode_rows(w8, 'p.weight', rows)))
    with pytest.raises(IndexError):
        wq.decode_rows({k: dev(v, gpu) for k, v in weights.items()}, 'lm_head.weight',
                       torch.tensor([151936], device=gpu))


# ------------------------------------------------------------------ W4A16 linear

@pytest.mark.parametrize('m', [1, 2, 15, 16, 17, 33, 64, 65, 128, 300])
@pytest.mark.parametrize('n,k', [(16, 128), (1000, 1024), (1024, 5120)])
def test_w4a16_linear_parity_small(gpu, m, n, k):
    name = 'mlp.up_proj.weight'
    weights, x = synth.w4_case(n, k, m, seed=m * 7 + n, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    y = backend.linear(dev(x, gpu), layer, name)
    check_parity(host(y), qdq.qdq_linear(x, weights, name), f'w4 m={m} n={n} k={k}')


@pytest.mark.parametrize('m', [5, 9, 16, 17, 40, 64])
def test_w4a16_skinny_four_tiles_per_wave(gpu, m):
    """M = 5 .. 64 over 1025 tiles (four tiles per wave from 1024 on, the last
    group partial): every output against the oracle."""
    name = 'mlp.gate_up_proj.weight'
    weights, x = synth.w4_case(16400, 1024, m, seed=m + 100, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    y = backend.linear(dev(x, gpu), layer, name)
    check_parity(host(y), qdq.qdq_linear(x, weights, name), f'w4 skinny m={m} n=16400')


@pytest.mark.parametrize('m,g,sym', [(5, 128, False), (8, 256, False), (16, 128, True), (33, 128, False),
                                     (64, 256, True)])
def test_w4a16_skinny_load_ring_long_k(gpu, m, g, sym):
    """The skinny load ring on a narrow, long-K shape (66 blocks over the
    waves of a k-split, 63 tiles, the last one partial): groups of 128 and
    256, symmetric and with zero points, M = 5 .. 64; every output against
    the oracle."""
    name = 'p.weight'
    weights, x = synth.w4_case(1000, 8448, m, seed=m + g, group_size=g, symmetric=sym, name=name)
    backend, layer = prepared_w4(weights, name, gpu, group_size=g)
    y = backend.linear(dev(x, gpu), layer, name)
    check_parity(host(y), qdq.qdq_linear(x, weights, name, group_size=g), f'w4 ring m={m} g={g} sym={sym}')


@pytest.mark.parametrize('n,k,g,sym', [(32776, 640, 128, False),    # 2049 tiles, one per wave; 5 blocks
                                       (65544, 768, 128, True),     # 4097 tiles, two per wave, the last alone
                                       (32768, 2048, 256, False),   # groups of 256
                                       (32768, 128, 128, False)])   # a single block: the ring runs out at once
def test_w4a16_deep_ring_wide_n(gpu, n, k, g, sym):
    """The deep-ring GEMM (wide N, 16 < M <= 64): every output against the
    oracle at M = 17, 31, 32, 33, 50 and 64, and bit-identical to the same
    rows of an M = 65 call, which runs the prefill GEMM."""
    name = 'p.weight'
    weights, x = synth.w4_case(n, k, 65, seed=k + n % 11, group_size=g, symmetric=sym, name=name)
    backend, layer = prepared_w4(weights, name, gpu, group_size=g)
    w = qdq.decode_weight(weights, name, group_size=g)
    y65 = host(backend.linear(dev(x, gpu), layer, name))
    for m in (17, 31, 32, 33, 50, 64):
        y = host(backend.linear(dev(x[:m], gpu), layer, name))
        check_parity(y, qdq.linear_fp32(x[:m], w), f'w4 deep n={n} k={k} g={g} m={m}')
        assert np.array_equal(bits(y), bits(y65[:m])), f'deep ring vs prefill GEMM m={m}'


@pytest.mark.parametrize('n,k', [(1000, 128), (1000, 384), (1000, 5248), (1000, 8448), (16400, 640)])
def test_w4a16_decode_uneven_wave_splits(gpu, n, k):
    """Decode plans with uneven work: one block (one wave), 3 blocks over 3
    waves, 41 blocks over 12 waves (5 waves take an extra block), 66 blocks
    over 4 k-splits of 16 / 17 blocks, and 5 blocks over 4 waves on a wide N."""
    name = 'p.weight'
    for m in (1, 3):
        weights, x = synth.w4_case(n, k, m, seed=k + m, name=name)
        backend, layer = prepared_w4(weights, name, gpu)
        y = backend.linear(dev(x, gpu), layer, name)
        check_parity(host(y), qdq.qdq_linear(x, weights, name), f'w4 n={n} k={k} m={m}')


def test_w4a16_group_256_and_symmetric(gpu):
    for g, sym in ((256, False), (128, True)):
        weights, x = synth.w4_case(256, 2048, 3, seed=g, group_size=g, symmetric=sym, name='p.weight')
        backend, layer = prepared_w4(weights, 'p.weight', gpu, group_size=g)
        y = backend.linear(dev(x, gpu), layer, 'p.weight')
        check_parity(host(y), qdq.qdq_linear(x, weights, 'p.weight', group_size=g), f'w4 g={g} sym={sym}')


@pytest.mark.parametrize('k,n', [(5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120), (5120, 7168),
                                 (5120, 34816)])
def test_w4a16_decode_full_shapes(gpu, k, n):
    """configs 2 and 4: the Qwen3-14B projection shapes at M=1, whole output."""
    name = 'mlp.up_proj.weight'
    weights, x = synth.w4_case(n, k, 1, seed=0, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    y = backend.linear(dev(x, gpu), layer, name)
    check_parity(host(y), qdq.qdq_linear(x, weights, name), f'w4 decode {k}->{n}')


@pytest.mark.parametrize('k,n', [(5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120)])
def test_w4a16_prefill_full_shapes_sampled_rows(gpu, k, n):
    """config 3: M=4096 on the full weight; 48 activation rows checked whole."""
    name = 'mlp.up_proj.weight'
    weights, _ = synth.w4_case(n, k, 1, seed=1, name=name)
    x = np.random.default_rng(2).standard_normal((4096, k), dtype=np.float32).astype(np.float16)
    backend, layer = prepared_w4(weights, name, gpu)
    y = host(backend.linear(dev(x, gpu), layer, name))
    rows = np.random.default_rng(3).choice(4096, size=48, replace=False)
    rows.sort()
    check_parity(y[rows], qdq.qdq_linear(x[rows], weights, name), f'w4 prefill {k}->{n} rows')
    assert np.isfinite(y).all()


@pytest.mark.parametrize('k,n', [(5120, 1024), (17408, 5120), (5120, 7168)])
def test_w4a16_prefill_grids_agree_across_m(gpu, k, n):
    """Every prefill-GEMM grid that keeps each tile's k range in one
    workgroup (128- or 64-wide n slices of 128-, 64- or 32-row tiles, plain
    or deep ring, chosen by the grid size; from 4096 rows on, row blocks owned
    per XCD) sums each output in the same order, so the rows of an M-row call
    equal the same rows of a 4096-row call bit for bit.  The smallest grids
    split the deep ring's k range when a workspace is given (their rows then
    differ by the fp32 summation order): those calls are checked against the
    oracle, and their no-workspace form bit for bit.  48 rows of the
    4096-row call against the oracle."""
    name = 'mlp.up_proj.weight'
    weights, _ = synth.w4_case(n, k, 1, seed=5, name=name)
    x = np.random.default_rng(6).standard_normal((4096, k), dtype=np.float32).astype(np.float16)
    backend, layer = prepared_w4(weights, name, gpu)
    prep = layer['mlp.up_proj._prepared']
    xd = dev(x, gpu)
    y_full = host(backend.linear(xd, layer, name))
    tiny = torch.zeros(16, dtype=torch.uint8, device=gpu)
    for m in (65, 96, 128, 300, 512, 1024, 2048):
        y = host(backend.linear(xd[:m], layer, name))
        if _native.w4a16_workspace_size(m, n, k, 128) > 0:
            check_parity(y, qdq.qdq_linear(x[:m], weights, name), f'w4 prefill split {k}->{n} m={m}')
            y = host(_native.w4a16_linear(xd[:m], prep.tiles, prep.meta, n, 128, workspace=tiny))
        assert np.array_equal(bits(y), bits(y_full[:m])), f'{k}->{n} m={m} differs from the 4096-row call'
    rows = np.sort(np.random.default_rng(7).choice(4096, size=48, replace=False))
    check_parity(y_full[rows], qdq.qdq_linear(x[rows], weights, name), f'w4 prefill {k}->{n} m=4096 rows')


CONFIG4_M = (1, 8, 32, 128, 512)


@pytest.mark.parametrize('name,n,ncols', [('self_attn.qkv_proj.weight', 7168, None),
                                          ('mlp.gate_up_proj.weight', 34816, 4096),
                                          ('lm_head.weight', 151936, 4096)])
def test_w4a16_config4_batch_sweep(gpu, name, n, ncols):
    """config 4: fused QKV 5120->7168, gate_up 5120->34816 and lm_head 5120->151936 at
    M in {1, 8, 32, 128, 512} (GEMV, skinny and GEMM paths); every output column of
    QKV, 4096 sampled columns of the wider two."""
    k = 5120
    weights, x = synth.w4_case(n, k, max(CONFIG4_M), seed=9 + n % 7, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    cols = np.arange(n) if ncols is None else np.sort(np.random.default_rng(4).choice(n, size=ncols, replace=False))
    w_cols = qdq.decode_rows(weights, name, cols)
    for m in CONFIG4_M:
        y = host(backend.linear(dev(x[:m], gpu), layer, name))
        assert y.shape == (m, n)
        check_parity(y[:, cols], qdq.linear_fp32(x[:m], w_cols), f'w4 {name} {k}->{n} m={m}')


def test_bitwise_repeatability_of_the_decoder_linears(gpu):
    """The reference harness's determinism check (``validate_weight_quant_kernels.py:49-70``):
    each of the 7 Qwen3-14B decoder linears at M in {1, 4, 32, 256}, 20 repeated calls
    on the same input compared bit for bit with the first (decode GEMV with its
    k-split reduction, skinny kernels, GEMM)."""
    from ondeviceinfer_amd.weight_quantization.synthetic import awq_quantize
    shapes = {'self_attn.q_proj.weight': (5120, 5120), 'self_attn.k_proj.weight': (1024, 5120),
              'self_attn.v_proj.weight': (1024, 5120), 'self_attn.o_proj.weight': (5120, 5120),
              'mlp.gate_proj.weight': (17408, 5120), 'mlp.up_proj.weight': (17408, 5120),
              'mlp.down_proj.weight': (5120, 17408)}
    gen = torch.Generator(device=gpu).manual_seed(0)
    backend = wq.CompressedLinearBackend('marlin')
    changes = {}
    for name, (n, k) in shapes.items():
        w = (torch.randn(n, k, generator=gen, device=gpu) * 0.02).half()
        layer = {f"{name.removesuffix('.weight')}.{key}": v.to(gpu) for key, v in awq_quantize(w).items()}
        backend.prepare(layer, name)
        for m in (1, 4, 32, 256):
            x = torch.randn(m, k, generator=gen, device=gpu).half()
            first = backend.linear(x, layer, name).clone()
            changes[(name, m)] = sum(int(not torch.equal(backend.linear(x, layer, name), first)) for _ in range(20))
            assert torch.isfinite(first).all()
    print('bitwise changes over 20 repeats:', changes, flush=True)
    assert not any(changes.values()), changes


def test_w4a16_repeat_calls_are_bitwise_identical(gpu):
    name = 'mlp.down_proj.weight'
    weights, x = synth.w4_case(5120, 17408, 4, seed=3, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    for m in (1, 4):
        xd = dev(x[:m], gpu)
        first = backend.linear(xd, layer, name).clone()
        for _ in range(5):
            assert torch.equal(backend.linear(xd, layer, name), first)


def test_w4a16_split_k_workspace_contract(gpu):
    """Tiles split over several workgroups need the workspace; without one the
    same result comes from one workgroup per tile."""
    name = 'mlp.down_proj.weight'
    weights, x = synth.w4_case(1024, 17408, 2, seed=12, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    prep = layer['mlp.down_proj._prepared']
    need = _native.w4a16_workspace_size(1, 1024, 17408, 128)
    assert need > 0 and prep.workspace is not None and prep.workspace.numel() >= need
    expected = qdq.qdq_linear(x, weights, name)
    xd = dev(x, gpu)
    with_ws = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, 1024, 128, workspace=prep.workspace))
    tiny = torch.zeros(16, dtype=torch.uint8, device=gpu)
    without = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, 1024, 128, workspace=tiny))
    check_parity(with_ws, expected, 'split with workspace')
    check_parity(without, expected, 'split fallback')
    counters = prep.workspace[:((1024 // 16) * 4 + 255) // 256 * 256]
    assert torch.count_nonzero(counters).item() == 0      # per-tile counters re-armed


def test_default_workspaces_of_different_layouts_do_not_mix(gpu):
    """Split linears of different tile counts called without a workspace,
    interleaved: each layout's counters must not land on another's partials."""
    cases = []
    for n, seed in ((1024, 21), (5120, 22)):
        name = 'mlp.down_proj.weight'
        weights, x = synth.w4_case(n, 17408, 1, seed=seed, name=name)
        _, layer = prepared_w4(weights, name, gpu)
        prep = layer['mlp.down_proj._prepared']
        assert _native.w4a16_workspace_size(1, n, 17408, 128) > 0
        cases.append((n, prep, dev(x, gpu), qdq.qdq_linear(x, weights, name)))
    for rep in range(2):
        for n, prep, xd, expected in cases:
            got = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128))
            check_parity(got, expected, f'default workspace n={n} call {rep}')


def test_w4a16_graph_replays_match_eager(gpu):
    """HIP-graph capture of decode GEMVs (split and unsplit shapes), replayed
    several times with eager work in between; every replay equals eager."""
    cases = []
    for i, (k, n) in enumerate(((17408, 5120), (5120, 1024), (5120, 5120))):
        name = f'l{i}.weight'
        weights, x = synth.w4_case(n, k, 1, seed=30 + i, name=name)
        backend, layer = prepared_w4(weights, name, gpu)
        cases.append((backend, layer, name, dev(x, gpu), torch.empty(1, n, dtype=torch.float16, device=gpu)))
    eager = [b.linear(x, l, nm).clone() for b, l, nm, x, _ in cases]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for b, l, nm, x, out in cases:
            b.ops.w4a16_linear(x, l[nm.removesuffix('.weight') + '._prepared'], out)
    for _ in range(4):
        for _, _, _, _, out in cases:
            out.fill_(float('nan'))
        graph.replay()
        torch.cuda.synchronize()
        for (_, _, _, _, out), ref in zip(cases, eager):
            assert torch.equal(out, ref)
        torch.cuda.synchronize()


def test_backend_shapes_counters_and_row_split(gpu, monkeypatch):
    name = 'self_attn.o_proj.weight'
    weights, x = synth.w4_case(512, 1024, 24, seed=8, name=name)
    backend, layer = prepared_w4(weights, name, gpu)
    assert 'self_attn.o_proj.weight_packed' not in layer and 'self_attn.o_proj._prepared' in layer
    x3 = dev(x.reshape(2, 12, 1024), gpu)
    y = backend.linear(x3, layer, name)
    assert y.shape == (2, 12, 512) and backend.calls == 1 and backend.gemm_calls == 1
    backend.marlin_max_rows_per_call = 16
    y2 = backend.linear(x3, layer, name)
    assert backend.gemm_calls == 3 and backend.fallback_count == 0
    check_parity(host(y2).reshape(24, 512), qdq.qdq_linear(x, weights, name), 'row split')
    assert backend.linear(dev(x[:0], gpu), layer, name).shape == (0, 512)


def test_reference_int4_backend_matches_oracle(gpu):
    name = 'mlp.gate_proj.weight'
    weights, x = synth.w4_case(256, 1024, 5, seed=2, name=name)
    layer = {k: dev(v, gpu) for k, v in weights.items()}
    ref = wq.CompressedLinearBackend('reference_int4')
    y = ref.linear(dev(x, gpu), layer, name)
    assert ref.explicit_dequant_bytes == 256 * 1024 * 2
    check_parity(host(y), qdq.qdq_linear(x, weights, name), 'reference_int4')


def test_w4a16_rejects_unsupported_shapes(gpu):
    weights, _ = synth.w4_case(16, 256, 1, name='p.weight')
    layer = {k: dev(v, gpu) for k, v in weights.items()}
    with pytest.raises(ValueError):
        wq.CompressedLinearBackend('marlin', group_size=64).prepare(layer, 'p.weight')
    layer['p.weight_g_idx'] = torch.zeros(256, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError, match='G-index'):
        wq.CompressedLinearBackend('marlin').prepare(layer, 'p.weight')


@pytest.mark.parametrize('fmt', ['w4', 'w8'])
def test_prefill_gemm_activations_beyond_2gib(gpu, fmt):
    """x of 65601 x 17408 fp16 (2.28 GB, past 2^31 bytes): the GEMM addresses it through
    per-workgroup buffer bases with 32-bit offsets; rows at the start, the middle and the
    end, including the partial last 128-row block, checked against the oracle."""
    m, k, n = 65601, 17408, 64
    rows = np.array([0, 1, 127, 128, 32767, 40000, 65535, 65536, 65599, 65600])
    x = torch.randn(m, k, device=gpu, dtype=torch.float16)
    xr = host(x[torch.from_numpy(rows).to(gpu)])
    if fmt == 'w4':
        name = 'mlp.down_proj.weight'
        weights, _ = synth.w4_case(n, k, 1, seed=21, name=name)
        backend, layer = prepared_w4(weights, name, gpu)
        y = host(backend.linear(x, layer, name))
        expected = qdq.qdq_linear(xr, weights, name)
    else:
        _, q, s, _ = synth.int8_case(n, k, 1, seed=22)
        y = host(_native.w8a16_linear(x, dev(q, gpu), dev(s, gpu)))
        expected = int8_ref(xr, q, s)
    del x
    check_parity(y[rows], expected, f'{fmt} prefill m={m} k={k} n={n} rows')
    assert np.isfinite(y).all()


@pytest.mark.parametrize('fmt', ['w4', 'w8'])
@pytest.mark.parametrize('k', [1 << 23, (1 << 23) + 128])
def test_prefill_gemm_at_the_largest_k(gpu, fmt, k):
    """k = 2^23, the largest the prefill GEMM takes (row 127 of a 128-row x tile
    then sits just under the 2^31-byte buffer range), and one block more, which
    goes to the skinny / any-shape kernels; m = 300 selects the 128-row tiles.
    Sampled rows include rows 64..127 of a tile, the ones a too-small range
    would read as zeros."""
    m, n = 300, 16
    rows = np.array([0, 63, 64, 100, 127, 128, 191, 192, 255, 256, 299])
    x = torch.randn(m, k, device=gpu, dtype=torch.float16)
    xr = host(x[torch.from_numpy(rows).to(gpu)])
    if fmt == 'w4':
        name = 'mlp.down_proj.weight'
        weights, _ = synth.w4_case(n, k, 1, seed=41, name=name)
        backend, layer = prepared_w4(weights, name, gpu)
        y = host(backend.linear(x, layer, name))
        expected = qdq.qdq_linear(xr, weights, name)
    else:
        _, q, s, _ = synth.int8_case(n, k, 1, seed=42)
        y = host(_native.w8a16_linear(x, dev(q, gpu), dev(s, gpu)))
        expected = int8_ref(xr, q, s)
    del x
    check_parity(y[rows], expected, f'{fmt} m={m} k={k} rows')


@pytest.mark.parametrize('fmt', ['w4', 'w8'])
def test_linear_with_k_beyond_gemm_offsets(gpu, fmt):
    """k = 2^24 + 128 (past the prefill GEMM's largest k) at m = 66: W4
    runs the skinny kernels 64 rows at a time (the 2-row tail included), W8
    the any-shape kernel; sampled rows against the oracle."""
    m, k, n = 66, (1 << 24) + 128, 16
    rows = np.array([0, 1, 63, 64, 65])
    x = torch.randn(m, k, device=gpu, dtype=torch.float16)
    xr = host(x[torch.from_numpy(rows).to(gpu)])
    if fmt == 'w4':
        name = 'mlp.down_proj.weight'
        weights, _ = synth.w4_case(n, k, 1, seed=31, name=name)
        backend, layer = prepared_w4(weights, name, gpu)
        y = host(backend.linear(x, layer, name))
        expected = qdq.qdq_linear(xr, weights, name)
    else:
        _, q, s, _ = synth.int8_case(n, k, 1, seed=32)
        y = host(_native.w8a16_linear(x, dev(q, gpu), dev(s, gpu)))
        expected = int8_ref(xr, q, s)
    del x
    check_parity(y[rows], expected, f'{fmt} m={m} k={k} rows')


# ------------------------------------------------------------------ INT8 (W8A16)

def int8_ref(x, q, s, bias=None):
    return qdq.linear_fp32(x, qdq.dequantize_linear_weight(q, s), bias)


@pytest.mark.parametrize('m', [1, 3, 16, 40, 64, 65, 200])
@pytest.mark.parametrize('n,k', [(40, 256), (1000, 1024), (5120, 5120)])
def test_w8a16_linear_parity(gpu, m, n, k):
    _, q, s, x = synth.int8_case(n, k, m, seed=m + n)
    y = _native.w8a16_linear(dev(x, gpu), dev(q, gpu), dev(s, gpu))
    check_parity(host(y), int8_ref(x, q, s), f'w8 m={m} n={n} k={k}')


@pytest.mark.parametrize('m', [1, 4])
def test_w8a16_down_shape_split(gpu, m):
    _, q, s, x = synth.int8_case(5120, 17408, m, seed=40 + m)
    y = _native.w8a16_linear(dev(x, gpu), dev(q, gpu), dev(s, gpu))
    check_parity(host(y), int8_ref(x, q, s), f'w8 down m={m}')


def test_w8a16_config1_and_bias_and_generic_shapes(gpu):
    w, q, s, x = synth.int8_case(5120, 5120, 1, seed=0)          # config 1
    y = _native.w8a16_linear(dev(x, gpu), dev(q, gpu), dev(s, gpu))
    check_parity(host(y), int8_ref(x, q, s), 'w8 config1')
    rng = np.random.default_rng(19)
    for m, n, k in ((6, 11, 13), (2, 33, 200), (300, 24, 96)):    # k % 128 != 0 -> one-wave-per-output kernel
        _, q, s, x = synth.int8_case(n, k, m, seed=n)
        b = rng.standard_normal(n).astype(np.float16)
        y = _native.w8a16_linear(dev(x, gpu), dev(q, gpu), dev(s, gpu), bias=dev(b, gpu))
        check_parity(host(y), int8_ref(x, q, s, b), f'w8 generic m={m} n={n} k={k}')


def test_int8_quantizer_bit_exact(gpu):
    for case in ('kat_int8_zero_tiny_rows', 'kat_int8_half_even', 'kat_int8_stored_scale', 'kat_int8_clamp'):
        c = KAT[case]
        got = q8.quantize_linear_weight(torch.tensor(c['weight'], device=gpu))
        assert host(got.qweight).tolist() == c['expected_q'], case
        assert host(got.scale).view(np.uint16).tolist() == c['expected_scale_f16_bits'], case
    w = (np.random.default_rng(0).standard_normal((5120, 5120), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    got = q8.quantize_linear_weight(dev(w, gpu))
    qr, sr = qdq.quantize_linear_weight(w)
    assert np.array_equal(host(got.qweight), qr)
    assert np.array_equal(bits(host(got.scale)), bits(sr))
    with pytest.raises(ValueError, match='NaN'):
        q8.quantize_linear_weight(torch.tensor([[1.0, float('nan')]], device=gpu))
    with pytest.raises(OverflowError):
        q8.quantize_linear_weight(torch.tensor([[1e7 * 127, 1.0]], device=gpu))


def test_int8_modules_match_reference_semantics(gpu):
    torch.manual_seed(19)
    weight = torch.randn(11, 13, device=gpu) * 0.2
    qw = q8.quantize_linear_weight(weight)
    x = torch.randn(2, 3, 13, device=gpu, dtype=torch.float16)
    bias = torch.randn(11, device=gpu, dtype=torch.float16)
    scratch = q8.FP16DequantScratch.allocate(weight.numel(), device=gpu)
    deq = qw.dequantize(scratch).clone()
    assert deq.data_ptr() != scratch.buffer.data_ptr()
    assert qw.dequantize(scratch).data_ptr() == scratch.buffer.data_ptr()
    assert np.array_equal(bits(host(deq)), bits(qdq.dequantize_linear_weight(host(qw.qweight), host(qw.scale))))
    actual = q8.quantized_linear(x, qw, scratch, bias=bias)
    expected = qdq.linear_fp32(host(x), host(deq), host(bias))
    check_parity(host(actual), expected, 'quantized_linear')
    assert torch.allclose(actual, torch.nn.functional.linear(x, weight.half(), bias), atol=2e-2, rtol=2e-2)
    # the INT8 v1 runtime linear (quantized_model.py:76-121)
    _, q, s, xx = synth.int8_case(1024, 5120, 1, seed=4)
    weights = {'mlp.down_proj.qweight': dev(q, gpu), 'mlp.down_proj.scale': dev(s, gpu)}
    y = int8_weight_only_linear(dev(xx.reshape(1, 1, 5120), gpu), weights, 'mlp.down_proj.weight',
                                torch.empty(1024 * 5120, dtype=torch.float16, device=gpu))
    assert y.shape == (1, 1, 1024)
    check_parity(host(y).reshape(1, 1024), int8_ref(xx, q, s), 'int8_weight_only_linear')


def test_w8a16_backend(gpu):
    name = 'mlp.up_proj.weight'
    _, q, s, x = synth.int8_case(256, 1024, 7, seed=6)
    layer = {name: dev(q, gpu), 'mlp.up_proj.weight_scale': dev(s.reshape(-1, 1), gpu)}
    backend = wq.CompressedLinearBackend('w8a16')
    backend.prepare(layer, name)
    y = backend.linear(dev(x, gpu), layer, name)
    check_parity(host(y), int8_ref(x, q, s), 'w8a16 backend')
