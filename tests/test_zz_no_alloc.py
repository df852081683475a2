"""wq_w4a16_linear_noalloc (scratch in a library-owned device array) against
wq_w4a16_linear with a caller workspace: bit-identical outputs, two calls in a
row with the second on a smaller input, called through the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import synth
from ondeviceinfer_amd import _native
from ondeviceinfer_amd.weight_quantization.backend import CompressedLinearBackend

pytestmark = pytest.mark.gpu


def _prepared(n, k, seed, gpu):
    name = 'mlp.down_proj.weight'
    weights, _ = synth.w4_case(n, k, 1, seed=seed, name=name)
    layer = {key: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for key, v in weights.items()}
    CompressedLinearBackend('marlin').prepare(layer, name)
    return layer['mlp.down_proj._prepared']


def _with_workspace(x, p, n):
    lib = _native.load()
    m, k = x.shape
    ws_bytes = _native.w4a16_workspace_size(m, n, k, 128)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    y = torch.empty(m, n, dtype=torch.float16, device=x.device)
    rc = lib.wq_w4a16_linear(x.data_ptr(), m, k, p.tiles.data_ptr(), p.meta.data_ptr(), n, 128, y.data_ptr(),
                             ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.wq_last_error()
    return y, ws_bytes


def _noalloc(x, p, n):
    lib = _native.load()
    m, k = x.shape
    y = torch.full((m, n), float('nan'), dtype=torch.float16, device=x.device)
    rc = lib.wq_w4a16_linear_noalloc(x.data_ptr(), m, k, p.tiles.data_ptr(), p.meta.data_ptr(), n, 128,
                                     y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.wq_last_error()
    return y


def test_noalloc_matches_workspace_entry_point(gpu):
    # (n, k, m): the first two use the decode GEMV's k-split scratch (320 and
    # 64 tiles, 4 splits), the second smaller than the first; then a non-split
    # decode shape and a skinny M, which use no scratch; a GEMM M on the deep
    # ring's k split and a small-batch M, which use it again.
    cases = [(5120, 17408, 1), (1024, 8448, 1), (1024, 8448, 4), (5120, 5120, 1), (1024, 8448, 33),
             (1024, 8448, 100), (7168, 5120, 24)]
    gen = torch.Generator(device=gpu).manual_seed(0)
    for idx, (n, k, m) in enumerate(cases):
        print(f'noalloc case {idx}: n={n} k={k} m={m}', flush=True)
        p = _prepared(n, k, idx, gpu)
        x = torch.randn(m, k, generator=gen, device=gpu).half()
        expected, ws_bytes = _with_workspace(x, p, n)
        if idx < 3 or idx >= 5:
            assert ws_bytes > 0   # these shapes exercise the scratch
        got = _noalloc(x, p, n)
        torch.cuda.synchronize()
        assert torch.isfinite(expected).all()
        assert torch.equal(got, expected), f'case {idx}'


def test_noalloc_rejects_bad_shapes_on_the_host(gpu):
    lib = _native.load()
    rc = lib.wq_w4a16_linear_noalloc(None, 1, 200, 1, 1, 16, 128, None, None)
    assert rc == _native.WQ_ERR_UNSUPPORTED
    assert rc != 0 and b'group' in lib.wq_last_error()
    rc = lib.wq_w4a16_linear_noalloc(None, 1, 256, None, None, 16, 128, None, None)
    assert rc == _native.WQ_ERR_INVALID_ARGUMENT


def test_noalloc_under_graph_capture(gpu):
    """After one eager call on the device (the scratch set-up), calls captured
    in a HIP graph record only the linear: several replays on the k-split
    shapes, with eager work and synchronizations between them, each equal bit
    for bit to wq_w4a16_linear with a caller workspace."""
    gen = torch.Generator(device=gpu).manual_seed(1)
    shapes = [(5120, 17408), (1024, 8448)]
    preps = [_prepared(n, k, 10 + i, gpu) for i, (n, k) in enumerate(shapes)]
    xs = [torch.randn(1, k, generator=gen, device=gpu).half() for _, k in shapes]
    ys = [torch.empty(1, n, dtype=torch.float16, device=gpu) for n, _ in shapes]
    lib = _native.load()
    _noalloc(xs[0], preps[0], shapes[0][0])          # eager set-up call (already done if earlier tests ran)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for (n, k), p, x, y in zip(shapes, preps, xs, ys):
                rc = lib.wq_w4a16_linear_noalloc(x.data_ptr(), 1, k, p.tiles.data_ptr(), p.meta.data_ptr(), n, 128,
                                                 y.data_ptr(), stream.cuda_stream)
                assert rc == 0, lib.wq_last_error()
    for rep in range(4):
        print(f'noalloc graph replay {rep}', flush=True)
        for x in xs:                                   # new inputs, written eagerly between replays
            x.copy_(torch.randn(x.shape, generator=gen, device=gpu).half())
        for y in ys:
            y.fill_(float('nan'))
        graph.replay()
        torch.cuda.synchronize()
        for (n, k), p, x, y in zip(shapes, preps, xs, ys):
            expected, _ = _with_workspace(x, p, n)
            torch.cuda.synchronize()
            assert torch.equal(y, expected), f'replay {rep} n={n} k={k}'
        # an eager noalloc call between replays shares the same scratch
        assert torch.equal(_noalloc(xs[1], preps[1], shapes[1][0]), _with_workspace(xs[1], preps[1], shapes[1][0])[0])
