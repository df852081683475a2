"""GPU parity of the small-batch W4A16 kernel (wq_batch.hip: 12 <= M <= 32 on
narrow N, activations shared in LDS, k split over workgroups) against the
CPU oracle, through the backend and the C ABI.

Bars as in test_gpu_parity.py (``oracle.qdq.parity_ok``).  The k split
changes the fp32 summation order relative to the skinny kernels, so the two
paths are compared with the oracle, not with each other bit for bit; the
batch path itself must be bitwise repeatable (its partials are added in split
order, not arrival order)."""
import numpy as np
import pytest
import torch

from oracle import qdq, synth
from ondeviceinfer_amd import _native
from ondeviceinfer_amd.weight_quantization import backend as wq

pytestmark = pytest.mark.gpu

BATCH_M = (8, 12, 16, 17, 24, 32)   # 8 runs the skinny kernels, the rest the batch kernel


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check_parity(actual, expected, label):
    m = qdq.parity_metrics(actual, expected)
    print(label, {k: (round(v, 8) if isinstance(v, float) else v) for k, v in m.items()}, flush=True)
    assert qdq.parity_ok(m), (label, m)


def prepared(n, k, m, seed, gpu, group_size=128, symmetric=False):
    name = 'self_attn.qkv_proj.weight'
    weights, x = synth.w4_case(n, k, m, seed=seed, group_size=group_size, symmetric=symmetric, name=name)
    layer = {key: dev(v, gpu) for key, v in weights.items()}
    backend = wq.CompressedLinearBackend('marlin', group_size=group_size)
    backend.prepare(layer, name)
    return backend, layer, name, weights, x


# (n, k, group, symmetric): the fused QKV and q/o shapes (4 splits of 10 blocks), k/v
# (8 tiles: one workgroup per split), a partial last tile group (1000 rows = 63 tiles,
# one split of 8 blocks), group 256 with two splits of 10 blocks, and the gate / up
# projection (136 tile groups x 4 splits, about two rounds of workgroups).
SHAPES = [(7168, 5120, 128, False), (5120, 5120, 128, False), (1024, 5120, 128, True), (1000, 1024, 128, False),
          (2048, 2560, 256, False), (17408, 5120, 128, False)]


@pytest.mark.parametrize('n,k,g,sym', SHAPES)
def test_batch_kernel_matches_oracle(gpu, n, k, g, sym):
    backend, layer, name, weights, x = prepared(n, k, max(BATCH_M), 40 + n % 13, gpu, g, sym)
    w32 = qdq.decode_weight(weights, name, group_size=g).astype(np.float32)
    for m in BATCH_M:
        y = host(backend.linear(dev(x[:m], gpu), layer, name))
        assert y.shape == (m, n)
        expected = (x[:m].astype(np.float32) @ w32.T).astype(np.float16)
        check_parity(y, expected, f'batch n={n} k={k} g={g} m={m}')


def test_batch_plans_use_the_workspace_and_fall_back_without_it(gpu):
    """The split plans need a workspace; with none (or too small) the same
    linear runs the skinny kernels, also within the bar.  The counters are
    back at zero after the calls."""
    n, k, m = 7168, 5120, 32
    assert _native.w4a16_workspace_size(m, n, k, 128) > 0
    assert _native.w4a16_workspace_size(m, 17408, k, 128) > 0    # gate / up (1088 tiles)
    assert _native.w4a16_workspace_size(m, 34816, k, 128) == 0   # the fused gate_up keeps the ring kernels
    assert _native.w4a16_workspace_size(33, n, k, 128) == 0      # beyond M = 32
    assert _native.w4a16_workspace_size(11, n, k, 128) == 0      # below M = 12 (skinny kernels)
    assert _native.w4a16_workspace_size(12, n, k, 128) > 0
    _, layer, name, weights, x = prepared(n, k, m, 7, gpu)
    prep = layer['self_attn.qkv_proj._prepared']
    expected = qdq.qdq_linear(x, weights, name)
    xd = dev(x, gpu)
    ws = torch.zeros(_native.w4a16_workspace_size(m, n, k, 128), dtype=torch.uint8, device=gpu)
    with_ws = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=ws))
    tiny = torch.zeros(16, dtype=torch.uint8, device=gpu)
    without = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=tiny))
    check_parity(with_ws, expected, 'batch with workspace')
    check_parity(without, expected, 'skinny fallback')
    assert torch.count_nonzero(ws[:512]).item() == 0   # per-group counters re-armed
    assert not np.array_equal(with_ws.view(np.uint16), np.zeros_like(with_ws.view(np.uint16)))


def test_batch_kernel_is_bitwise_repeatable_and_graph_safe(gpu):
    """20 repeats equal the first call bit for bit; a captured graph of two
    batch linears of different shapes (sharing the default workspace),
    replayed with eager work in between, equals the eager calls."""
    cases = []
    for i, (n, k) in enumerate(((7168, 5120), (1024, 5120))):
        backend, layer, name, _, x = prepared(n, k, 24, 60 + i, gpu)
        cases.append((backend, layer, name, dev(x, gpu)))
    eager = []
    for backend, layer, name, xd in cases:
        first = backend.linear(xd, layer, name).clone()
        for _ in range(20):
            assert torch.equal(backend.linear(xd, layer, name), first)
        eager.append(first)
    outs = [torch.empty_like(e) for e in eager]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for (backend, layer, name, xd), o in zip(cases, outs):
            o.copy_(backend.linear(xd, layer, name))
    torch.cuda.current_stream().wait_stream(stream)
    for rep in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f'replay {rep}'
        backend, layer, name, xd = cases[0]
        assert torch.equal(backend.linear(xd, layer, name), eager[0])   # eager call between replays


# ------------------------------------------------------------------ deep-ring GEMM k split

@pytest.mark.parametrize('n,k', [(7168, 5120), (5120, 5120), (1024, 5120), (5120, 17408), (1000, 2048)])
def test_deep_ring_split_matches_oracle(gpu, n, k):
    """The smallest prefill grids (deep ring on 32-row tiles) split their k
    range over workgroups when a workspace is given: every output against
    the oracle, 20 repeats bit for bit, the counters back at zero, and the
    no-workspace form (whole k range per workgroup) also within the bar."""
    name = 'self_attn.q_proj.weight'
    weights, x = synth.w4_case(n, k, 300, seed=70 + n % 11, name=name)
    layer = {key: dev(v, gpu) for key, v in weights.items()}
    backend = wq.CompressedLinearBackend('marlin')
    backend.prepare(layer, name)
    prep = layer['self_attn.q_proj._prepared']
    w32 = qdq.decode_weight(weights, name).astype(np.float32)
    for m in (65, 128, 300):
        need = _native.w4a16_workspace_size(m, n, k, 128)
        xd = dev(x[:m], gpu)
        expected = (x[:m].astype(np.float32) @ w32.T).astype(np.float16)
        if need == 0:
            check_parity(host(backend.linear(xd, layer, name)), expected, f'deep n={n} k={k} m={m} (no split)')
            continue
        ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
        first = _native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=ws).clone()
        check_parity(host(first), expected, f'deep split n={n} k={k} m={m}')
        for _ in range(20):
            assert torch.equal(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=ws), first)
        assert torch.count_nonzero(ws[:16384]).item() == 0
        tiny = torch.zeros(16, dtype=torch.uint8, device=gpu)
        whole = host(_native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=tiny))
        check_parity(whole, expected, f'deep whole-k n={n} k={k} m={m}')


def test_split_kernels_share_one_workspace(gpu):
    """One buffer serving the decode GEMV's split (m = 1, 17408 -> 5120), the
    small-batch kernel (m = 24) and the deep-ring split (m = 128), called in
    turn twice: each result equals its own-workspace call bit for bit."""
    cases = []
    for i, (n, k, m) in enumerate(((5120, 17408, 1), (7168, 5120, 24), (7168, 5120, 128), (1024, 5120, 96))):
        name = 'mlp.down_proj.weight'
        weights, x = synth.w4_case(n, k, m, seed=90 + i, name=name)
        layer = {key: dev(v, gpu) for key, v in weights.items()}
        wq.CompressedLinearBackend('marlin').prepare(layer, name)
        prep = layer['mlp.down_proj._prepared']
        xd = dev(x, gpu)
        own = torch.zeros(max(_native.w4a16_workspace_size(m, n, k, 128), 16), dtype=torch.uint8, device=gpu)
        ref = _native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=own).clone()
        cases.append((n, k, m, prep, xd, ref))
    need = max(_native.w4a16_workspace_size(m, n, k, 128) for n, k, m, *_ in cases)
    assert need > 0
    shared = torch.zeros(need, dtype=torch.uint8, device=gpu)
    for rep in range(2):
        for n, k, m, prep, xd, ref in cases:
            got = _native.w4a16_linear(xd, prep.tiles, prep.meta, n, 128, workspace=shared)
            assert torch.equal(got, ref), f'n={n} k={k} m={m} call {rep}'
