#!/usr/bin/env python3
"""Benchmark: W4A16 G=128 decode GEMV over a Qwen3-14B-shaped decoder.

One *step* is one decode token's worth of projection GEMVs at M=1: for each of
the 40 decoder layers, q 5120->5120, k and v 5120->1024, o 5120->5120, gate and
up 5120->17408 and down 17408->5120 (280 launches), every layer with its own
resident weights (6.86 GB of packed uint4 + scales + zero points), so no weight
is served from the 256 MB Infinity Cache.  The 280 launches are captured once
in a HIP graph and the graph is replayed per step.  Inputs are resident in HBM
before the timed region.

``value`` = algorithmic bytes of the step / step time (GB/s).  Algorithmic
bytes per GEMV: ``N*K/2 + N*(K/128)*2 + N*(K/128)/2 + 2*M*K + 2*M*N``.

Also printed in the same JSON line:
* ``roofline``: the dominant kernel's algorithmic bytes per launch / its
  average launch time, measured here with HIP events around a graph of that
  kernel's launches on the stream they run on;
* ``prefill``: the M=4096 W4A16 GEMM (config 3) in TFLOP/s vs dense fp16 MFMA;
* ``copy_ceiling``: a device-to-device copy's GB/s on the same box;
* ``cpu_baseline``: the numpy QDQ oracle (decode + fp32 GEMV) on one decoder
  layer's seven projections, single-threaded, on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'Qwen3-14B AWQ-INT4 decode tok/s at B=1; W4A16 GEMV % of HBM peak'
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
GROUP = 128
HIDDEN, INTER, KV = 5120, 17408, 1024
LAYER_SHAPES = [  # (name, K, N) in decoder order
    ('q_proj', HIDDEN, HIDDEN), ('k_proj', HIDDEN, KV), ('v_proj', HIDDEN, KV), ('o_proj', HIDDEN, HIDDEN),
    ('gate_proj', HIDDEN, INTER), ('up_proj', HIDDEN, INTER), ('down_proj', INTER, HIDDEN),
]


def w4_bytes(m: int, n: int, k: int, g: int = GROUP) -> int:
    return n * k // 2 + n * (k // g) * 2 + n * (k // g) // 2 + 2 * m * k + 2 * m * n


def log(msg: str) -> None:
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def make_layer_weights(torch, native, n_layers: int, device):
    """Random uint4 codes / fp16 scales / zero points, repacked by the HIP repack."""
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    layers = []
    for _ in range(n_layers):
        layer = {}
        for name, k, n in LAYER_SHAPES:
            packed = torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32, device=device, generator=gen)
            scale = (torch.rand((n, k // GROUP), device=device, generator=gen) * 0.008 + 0.002).half()
            zero = torch.randint(-2**31, 2**31 - 1, (n // 8, k // GROUP), dtype=torch.int32, device=device,
                                 generator=gen)
            tiles, meta = native.w4_repack(packed, scale, zero, n, k, GROUP)
            layer[name] = (tiles, meta, n, k)
            del packed, scale, zero
        layers.append(layer)
    torch.cuda.synchronize()
    return layers


def time_graph(torch, graph, reps: int) -> float:
    """Seconds per replay, HIP events on the current stream."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1000.0 / reps


def flat_plan(n: int, k: int) -> tuple[int, int, int]:
    """(split, waves per workgroup, blocks per wave) the library picks for a
    W4 decode GEMV at M <= 4 with the workspace supplied: a restatement of
    plan_flat() in ondeviceinfer_amd/csrc/wq_gemv.hip, used only to name the
    kernel instantiation in the report."""
    ntile, nblk = (n + 15) // 16, k // 128
    split = 4 if ntile < 512 and nblk >= 64 else 1
    if split > nblk:
        split = 1
    per = nblk // split
    ksw = 4 if split > 1 or ntile >= 1024 else 12
    ksw = max(1, min(ksw, per))
    limit = 16 if per // ksw <= 12 else 8
    ksw = min(ksw, limit)
    return split, ksw, per // ksw


def kernel_name_for(native_shape: tuple[int, int, int]) -> str:
    """Kernel the library runs for (M, N, K): M <= 4 goes to the decode GEMV
    gemv_flat_kernel<NB, MM, W4> (NB = k blocks per wave, MM = 1 or 4)."""
    m, n, k = native_shape
    if m > 4:
        return 'w4_skinny_kernel' if m <= 64 else 'wq_gemm_kernel'
    _, _, nb = flat_plan(n, k)
    return f'gemv_flat_kernel<{nb}, {1 if m == 1 else 4}, W4>'


def profiled_traffic(kernel: str, shape: str):
    """HBM bytes per launch of `kernel` at `shape` from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by
    its copy-kernel calibration factor), or None when none was recorded."""
    f = ROOT / 'profiles' / 'decode_gemv_traffic.json'
    if not f.exists():
        return None
    rec = json.loads(f.read_text()).get('kernels', {}).get(f'{kernel} @ {shape}')
    return None if rec is None else int(rec['hbm_bytes_per_launch'])


def cpu_baseline(budget_s: float) -> dict:
    """numpy QDQ oracle on one decoder layer's seven projections (one thread)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import qdq, synth
    cases = []
    for name, k, n in LAYER_SHAPES:
        w, x = synth.w4_case(n, k, 1, seed=0, name=f'{name}.weight')
        cases.append((name, k, n, w, x))
    total_bytes = sum(w4_bytes(1, n, k) for _, k, n, _, _ in cases)
    times = []
    with threadpool_limits(limits=1):
        t_begin = time.perf_counter()
        while True:
            t0 = time.perf_counter()
            for name, _, _, w, x in cases:
                qdq.qdq_linear(x, w, f'{name}.weight')
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_begin > budget_s or len(times) >= 10:
                break
    sec = float(np.median(times))
    return {'value': round(total_bytes / sec / 1e9, 4), 'unit': 'GB/s', 'cores': 1, 'kind': 'port',
            'sample': f'oracle.qdq.qdq_linear (numpy decode_weight + fp32 GEMV, 1 BLAS thread) over one '
                      f'decoder layer\'s 7 W4A16 projections at M=1 ({total_bytes / 1e6:.1f} MB algorithmic), '
                      f'median of {len(times)} passes = {sec:.3f} s/pass',
            'ms_per_layer': round(sec * 1000, 3), 'host_cpu_count': os.cpu_count()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--layers', type=int, default=40)
    ap.add_argument('--cpu-budget', type=float, default=15.0, help='seconds for the CPU baseline sample')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-extras', action='store_true', help='skip prefill / copy / per-kernel sections')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: this build has no multi-GPU path (every box has one GPU); '
              'run with --gpus 1', file=sys.stderr)
        return 2

    import torch
    from ondeviceinfer_amd import _native as native

    if not torch.cuda.is_available():
        print('bench.py needs a GPU', file=sys.stderr)
        return 2
    device = torch.device('cuda:0')
    native.load()
    log(f'device {torch.cuda.get_device_name(0)}; building {args.layers} layers of weights')
    layers = make_layer_weights(torch, native, args.layers, device)

    xs = {HIDDEN: torch.randn(1, HIDDEN, device=device).half(), INTER: torch.randn(1, INTER, device=device).half()}
    outs = {name: torch.empty(1, n, device=device, dtype=torch.float16) for name, _, n in LAYER_SHAPES}

    def step():
        for layer in layers:
            for name, k, n in LAYER_SHAPES:
                tiles, meta, _, _ = layer[name]
                native.w4a16_linear(xs[k], tiles, meta, n, GROUP, out=outs[name])

    step()   # eager warm call (loads code objects)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    log(f'timing {args.steps} steps')
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_per_step = start.elapsed_time(end) / args.steps
    step_bytes = args.layers * sum(w4_bytes(1, n, k) for _, k, n in LAYER_SHAPES)
    value = step_bytes / (ms_per_step / 1000.0) / 1e9

    result = {
        'metric': METRIC, 'value': round(value, 2), 'unit': 'GB/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(ms_per_step, 4), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'fp16', 'data': 'synthetic',
        'config': {'workload': 'configs[1]: W4A16 G=128 decode GEMV, M=1, Qwen3-14B projection shapes '
                               f'(q,k,v,o,gate,up,down) x {args.layers} layers per step, HIP-graph replay',
                   'layers': args.layers, 'launches_per_step': 7 * args.layers,
                   'weight_bytes_resident': step_bytes, 'group_size': GROUP},
        'pct_hbm_peak': round(100.0 * value / HBM_PEAK_GBS, 2),
        'decode_projection_passes_per_s': round(1000.0 / ms_per_step, 2),
        'wall_s_timed': round(wall, 4),
    }

    if not args.no_extras:
        # Per-shape kernel timing: a graph of the `layers` launches of one shape.
        by_shape = []
        for name, k, n in LAYER_SHAPES:
            if name in ('v_proj', 'up_proj'):
                continue   # same shapes as k_proj / gate_proj
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for layer in layers:
                    tiles, meta, _, _ = layer[name]
                    native.w4a16_linear(xs[k], tiles, meta, n, GROUP, out=outs[name])
            per_launch = time_graph(torch, g, 10) / len(layers)
            b = w4_bytes(1, n, k)
            by_shape.append({'shape': f'{k}->{n}', 'kernel': kernel_name_for((1, n, k)), 'bytes': b,
                             'us_per_launch': round(per_launch * 1e6, 3),
                             'gbs': round(b / per_launch / 1e9, 1),
                             'frac': round(b / per_launch / 1e9 / HBM_PEAK_GBS, 4),
                             'launches_per_step': args.layers * (2 if name in ('k_proj', 'gate_proj') else 1)})
            del g
        # dominant kernel = largest total time per step
        for e in by_shape:
            e['us_per_step'] = e['us_per_launch'] * e['launches_per_step']
        kernels = {}
        for e in by_shape:
            agg = kernels.setdefault(e['kernel'], {'bytes': 0, 'us': 0.0, 'launches': 0})
            agg['bytes'] += e['bytes'] * e['launches_per_step']
            agg['us'] += e['us_per_step']
            agg['launches'] += e['launches_per_step']
        dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]['us'])
        achieved = dom['bytes'] / (dom['us'] / 1e6) / 1e9
        dom_shapes = [e['shape'] for e in by_shape if e['kernel'] == dom_name]
        traffic = profiled_traffic(dom_name, dom_shapes[0]) if len(dom_shapes) == 1 else None
        result['roofline'] = {
            'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
            'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': traffic, 'kernel': dom_name,
            'shapes': dom_shapes,
            'avg_launch_us': round(dom['us'] / dom['launches'], 3),
            'algorithmic_bytes_per_launch': dom['bytes'] // dom['launches'],
        }
        result['roofline_by_shape'] = by_shape

        # Prefill GEMM (config 3), M=4096 on the first layer's weights.
        xp = {kk: torch.randn(4096, kk, device=device).half() for kk in (HIDDEN, INTER)}
        prefill = []
        for name, k, n in LAYER_SHAPES:
            if name in ('v_proj', 'up_proj'):
                continue
            tiles, meta, _, _ = layers[0][name]
            yp = torch.empty(4096, n, device=device, dtype=torch.float16)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                native.w4a16_linear(xp[k], tiles, meta, n, GROUP, out=yp)
            sec = time_graph(torch, g, 10)
            tflops = 2 * 4096 * n * k / sec / 1e12
            prefill.append({'shape': f'{k}->{n}', 'M': 4096, 'us': round(sec * 1e6, 1), 'tflops': round(tflops, 1),
                            'frac_fp16_mfma': round(tflops / FP16_MFMA_PEAK_TFLOPS, 4)})
            del g, yp
        result['prefill'] = prefill

        # Copy ceiling: 2 GiB device-to-device copy (read + write bytes).
        src = torch.empty(2**30, dtype=torch.uint16, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(5):
            dst.copy_(src)
        s1.record()
        torch.cuda.synchronize()
        sec = s0.elapsed_time(s1) / 1000.0 / 5
        result['copy_ceiling'] = {'gbs': round(2 * src.numel() * 2 / sec / 1e9, 1), 'bytes_moved': 2 * src.numel() * 2,
                                  'how': 'torch copy_ of 2 GiB, read+write bytes / time'}
        del src, dst

    if not args.no_cpu_baseline:
        log('cpu baseline')
        result['cpu_baseline'] = cpu_baseline(args.cpu_budget)

    print(json.dumps(result), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
