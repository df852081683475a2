#!/usr/bin/env python3
"""Benchmark: Qwen3-14B-shaped AWQ-INT4 (W4A16, G=128) decode on one MI355X.

Headline (the benchmark configs[4], the workload the metric's published number is
quoted on): batch 1, a 4096-token random prompt, greedy decode with the fp16
KV cache resident, random-init weights of the Qwen3-14B architecture (40
layers, hidden 5120, 40/8 heads of 128, SwiGLU 17408, vocab 151936), the
decoder linears drawn as fp16 N(0, 0.02) and quantized to uint4 with fp16
group-128 scales and zero points (asymmetric min-max RTN).  One *step*
is one decode token: a replay of the captured decode-step graph (40 x [QKV
GEMV with the input RMSNorm in its prologue, attention (q/k norm, RoPE, cache
append, GQA) + chunk merge, o GEMV + residual, gate_up GEMV with the
post-attention RMSNorm in its prologue, down GEMV with SiLU*up in its prologue
+ residual], final norm, fp16 LM head with the greedy token).
After the prefill and ``--warmup`` untimed steps, ``--steps`` steps are timed;
``value`` = steps / seconds (tok/s), compared with the reference's published
26.358 tok/s (AWQ-INT4 + Marlin, RTX 3090, same workload).

Also in the same JSON line:
* ``gemv_pass``: the 280 per-projection decode GEMVs of one token
  (q, k, v, o, gate, up, down x 40 layers) replayed as one graph; GB/s of
  algorithmic bytes ``N*K/2 + N*(K/128)*2.5 + 2MK + 2MN``;
* ``roofline``: the dominant kernel of the decode step (largest time per
  token), its algorithmic bytes per launch / its average launch duration
  inside the decode step (torch.profiler device records over 16 decode steps
  run right after the timed ones, on the same model and cache);
  ``one_op_graph_us`` is the same kernel timed in a graph of only its own
  launches; ``traffic`` from the committed rocprofv3 counter summary;
* ``decode_step_kernels``: every kernel of the step, each timed in a graph of
  its own launches (``kernel_us``: device records; ``us_per_launch``: HIP
  events, launch gaps included) and, for the step's kernels, inside the
  step (``in_step_us``);
* ``prefill``: the M=4096 W4A16 GEMM per shape, TFLOP/s, next
  to the vendor library's dense fp16 GEMM (torch.matmul -> hipBLASLt, no
  dequantization) on the same shape for context;
* ``prefill_attention``: the 4096-token prompt's causal GQA attention
  kernel per layer, TFLOP/s, next to torch's fused SDPA for context;
* ``batch_sweep``: fused QKV, fused gate_up and a W4 lm_head at
  M in {1, 8, 32, 128, 512}, GB/s and TFLOP/s per launch;
* ``int8``: configs[0]'s INT8 weight shape on the GPU over a pool of 40
  distinct weights (1.05 GB, past the 256 MB Infinity Cache), streamed as the
  INT8 tiles the prepared linears use: weight-only W8A16 and W8A8
  (``int8_gemm``) decode GB/s, M=4096 W8A16 TFLOP/s and W8A8 TOPS against the
  fp16 / int8 MFMA peaks; the W8A16 pair once more over the row-major weight
  as stored; the vendor library's int8 GEMM (torch._int_mm) at M=4096 for
  context;
* ``int8_e2e``: the INT8 weight-only model (INT8 v1 tensors, the reference's
  first published row) on the same workload, tok/s;
* ``e2e_w4_lm_head``: the headline workload with the optional W4 LM head
  (not the reference's configuration), tok/s;
* ``setup_seconds``: weight generation, the whole-model repack and the
  startup repack of each of layer 0's linears;
* ``copy_ceiling``: a device-to-device copy's GB/s on the same box;
* ``cpu_baseline``: the explicit QDQ path in torch on the host CPU, all
  available threads (oracle/qdq_torch.py), per call on configs[0] and each
  configs[1] shape at M=1 (ms, GB/s), and the tok/s those calls give for the
  40 layers' linears.
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
PUBLISHED_TOKS = 26.358          # the reference's published AWQ INT4 G=128 + vLLM Marlin figure, RTX 3090, same workload
# Peak allocated GiB the reference publishes for the same runs (README.md:31-32).
REFERENCE_PEAK_GIB = {'w4': 9.260, 'int8': 15.517}
HBM_PEAK_GBS = 8000.0
PROFILED_STEPS = 16   # decode steps after the timed ones, under torch.profiler, for in-step kernel durations
FP16_MFMA_PEAK_TFLOPS = 2500.0
INT8_MFMA_PEAK_TOPS = 5000.0      # dense int8 MFMA, MI355X
GROUP = 128
PROMPT = 4096
HIDDEN, INTER, KV, QKV, GATE_UP = 5120, 17408, 1024, 7168, 34816
LINEAR_NAMES = ('self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight',
                'self_attn.o_proj.weight', 'mlp.gate_proj.weight', 'mlp.up_proj.weight', 'mlp.down_proj.weight')
LAYER_SHAPES = [  # (name, K, N) in decoder order
    ('self_attn.q_proj', HIDDEN, HIDDEN), ('self_attn.k_proj', HIDDEN, KV), ('self_attn.v_proj', HIDDEN, KV),
    ('self_attn.o_proj', HIDDEN, HIDDEN), ('mlp.gate_proj', HIDDEN, INTER), ('mlp.up_proj', HIDDEN, INTER),
    ('mlp.down_proj', INTER, HIDDEN),
]


def w4_bytes(m: int, n: int, k: int, g: int = GROUP) -> int:
    return n * k // 2 + n * (k // g) * 2 + n * (k // g) // 2 + 2 * m * k + 2 * m * n


def log(msg: str) -> None:
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def check_step(model, token, cache) -> None:
    """One more decode token after the timed ones (outside the timed region):
    the logits must be finite and the greedy token the graph picked must be
    their argmax; raises otherwise, so a broken step cannot report a rate."""
    import torch
    out = model(token, cache=cache, logits_to_keep=1)
    logits = out.logits.view(-1)
    if not bool(torch.isfinite(logits).all()):
        raise RuntimeError('decode step produced non-finite logits')
    if out.next_token is not None and int(out.next_token.view(-1)[0]) != int(logits.argmax()):
        raise RuntimeError('decode graph token differs from the argmax of its logits')


def kernel_times(torch, graph, reps: int) -> dict:
    """Average device duration (µs) and launches per replay of each kernel
    in `graph`, from torch.profiler's device activity records over `reps`
    replays: the kernel's own execution time, as rocprofv3's kernel trace
    reports it (no launch gaps).  The records can be incomplete when an
    outside profiler (rocprofv3) holds the same tracing interface; see
    kernel_us."""
    from collections import defaultdict
    from torch.profiler import ProfilerActivity, profile
    graph.replay()
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
    per = defaultdict(list)
    for e in prof.events():
        if e.device_type == torch.autograd.DeviceType.CUDA:
            per[e.name].append(e.device_time)
    return {name: {'us': sum(v) / len(v), 'per_replay': len(v) / reps} for name, v in per.items()}


def kernel_us(torch, graph, reps: int, launches: int, event_us: float) -> tuple[float, str]:
    """(µs per launch, source): the kernels' own duration from kernel_times
    when its records cover the graph's `launches` launches per replay and
    agree with the event timing `event_us` (per launch, launch gaps
    included), else `event_us` itself."""
    kt = kernel_times(torch, graph, reps)
    seen = sum(v['per_replay'] for v in kt.values())
    kus = sum(v['us'] * v['per_replay'] for v in kt.values()) / max(launches, 1)
    if kt and abs(seen - launches) < 0.5 and 0.5 * event_us <= kus <= 1.1 * event_us:
        return kus, 'kernel'
    return event_us, 'events'


def step_kernel_times(torch, model, token, cache, steps: int) -> dict:
    """Average device duration (µs) and launches per step of each kernel of
    the decode step, from torch.profiler's device records over `steps`
    decode steps run right after the timed ones on the same model and cache
    (the kernels as the step interleaves them, which is what rocprofv3's
    kernel trace of the timed steps shows)."""
    from collections import defaultdict
    from torch.profiler import ProfilerActivity, profile
    from ondeviceinfer_amd.generation import greedy_token
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(steps):
            token = greedy_token(model(token, cache=cache, logits_to_keep=1))
        torch.cuda.synchronize()
    per = defaultdict(list)
    for e in prof.events():
        if e.device_type == torch.autograd.DeviceType.CUDA:
            per[e.name].append(e.device_time)
    return {name: {'us': sum(v) / len(v), 'per_step': len(v) / steps} for name, v in per.items()}


def step_record_pattern(kernel: str) -> str | None:
    """The mangled-name fragment of a decode-step kernel named as in the
    report (``gemv_flat_kernel<10, 1, W4, RmsNorm>``), as the profiler's
    device records carry it; None for names without one."""
    import re
    m = re.fullmatch(r'gemv_flat_kernel<(\d+), (\d+), (W4|W8)(?:, (RmsNorm|SiluMul))?>', kernel)
    if not m:
        return None
    fmt = {'W4': 0, 'W8': 1}[m.group(3)]
    mode = {None: 0, 'RmsNorm': 1, 'SiluMul': 2}[m.group(4)]
    return f'gemv_flat_kernelILi{m.group(1)}ELi{m.group(2)}ELNS0_4WFmtE{fmt}ELNS0_5XModeE{mode}E'


def in_step_us(step_times: dict, patterns: tuple, launches_per_step: int, own_us: float | None = None) -> float | None:
    """Summed per-launch device time of the kernels whose records contain
    each of `patterns` (one kernel per pattern, each launched
    `launches_per_step` times per step), or None when any is missing or
    launched a different number of times, or when the sum lies outside
    0.5-2x `own_us` (the same kernels timed in a graph of their own
    launches; inside the step they ran 1.0-1.3x that).  Under an outside
    profiler (rocprofv3) the records come back with the right counts but
    durations of about 1 us, which the bound rejects."""
    total = 0.0
    for pat in patterns:
        hits = [v for name, v in step_times.items() if pat in name]
        if len(hits) != 1 or abs(hits[0]['per_step'] - launches_per_step) > 0.01:
            return None
        total += hits[0]['us']
    if own_us is not None and not 0.5 * own_us <= total <= 2.0 * own_us:
        return None
    return total


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


def kernel_name_for(native_shape: tuple[int, int, int], mode: str = 'Plain') -> str:
    """Kernel the library runs for (M, N, K): M <= 4 goes to the decode GEMV
    gemv_flat_kernel<NB, MM, W4[, mode]> (NB = k blocks per wave, MM = 1 or 4;
    mode = the fused x transform of wq_w4a16_decode_fused)."""
    m, n, k = native_shape
    if m > 4:
        return 'w4_skinny_kernel' if m <= 64 else 'wq_gemm_kernel'
    _, _, nb = flat_plan(n, k)
    return f'gemv_flat_kernel<{nb}, {1 if m == 1 else 4}, W4' + ('' if mode == 'Plain' else f', {mode}') + '>'


def profiled_traffic(kernel: str, shape: str):
    """HBM bytes per launch of `kernel` at `shape` from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by
    its copy-kernel calibration factor), or None when none was recorded."""
    f = ROOT / 'profiles' / 'decode_gemv_traffic.json'
    if not f.exists():
        return None
    rec = json.loads(f.read_text()).get('kernels', {}).get(f'{kernel} @ {shape}')
    return None if rec is None else int(rec['hbm_bytes_per_launch'])


def host_threads() -> int:
    """CPU threads this process may use: its affinity set, capped by
    OMP_NUM_THREADS when the launcher sets it (the GPU boxes give each job a
    16-CPU share and say so there)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, 'sched_getaffinity') else (os.cpu_count() or 1)
    omp = os.environ.get('OMP_NUM_THREADS', '')
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in Path('/proc/cpuinfo').read_text().splitlines():
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_baseline(torch, native, device, layers: int) -> dict:
    """The reference's explicit QDQ path on the host CPU with torch
    (oracle/qdq_torch.py: decode_weight + fp32-accumulated F.linear), all
    available threads: configs[0] (INT8 5120x5120 per-channel, M = 1) and each
    configs[1] W4A16 G=128 shape at M = 1; 3 warm-up calls, then the median
    of 10 timed calls per shape.  ``value`` is the tok/s those per-call
    times give for the 7 decoder linears of `layers` layers (the linears
    only: no attention, norms or LM head)."""
    import numpy as np
    from oracle import qdq_torch
    from ondeviceinfer_amd.weight_quantization.synthetic import awq_quantize
    threads = host_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator(device=device).manual_seed(0)
    cpu_gen = torch.Generator().manual_seed(0)

    def timed(fn) -> tuple[float, int]:
        for _ in range(3):
            fn()
        runs = []
        for _ in range(10):
            t0 = time.perf_counter()
            fn()
            runs.append(time.perf_counter() - t0)
        return float(np.median(runs)), len(runs)

    shapes = []
    w = (torch.randn(HIDDEN, HIDDEN, device=device, generator=gen) * 0.02).half()
    q8, s8 = (t.cpu() for t in native.w8_quantize(w))
    x = torch.randn(1, HIDDEN, generator=cpu_gen).half()
    sec, runs = timed(lambda: qdq_torch.int8_qdq_linear(x, q8, s8))
    b = HIDDEN * HIDDEN + 2 * HIDDEN + 2 * HIDDEN + 2 * HIDDEN
    shapes.append({'config': 'configs[0]', 'op': 'INT8 per-channel QDQ linear', 'shape': f'{HIDDEN}->{HIDDEN}', 'M': 1,
                   'ms_per_call': round(sec * 1e3, 3), 'gbs': round(b / sec / 1e9, 2), 'algorithmic_bytes': b,
                   'runs': runs})
    per_shape = {}
    for name, k, n in LAYER_SHAPES:
        if (k, n) in per_shape:
            continue
        w = (torch.randn(n, k, device=device, generator=gen) * 0.02).half()
        weights = {f'p.{key}': v.cpu() for key, v in awq_quantize(w).items()}
        del w
        x = torch.randn(1, k, generator=cpu_gen).half()
        sec, runs = timed(lambda: qdq_torch.qdq_linear(x, weights, 'p.weight'))
        per_shape[(k, n)] = sec
        b = w4_bytes(1, n, k)
        shapes.append({'config': 'configs[1]', 'op': 'W4A16 G=128 QDQ linear', 'shape': f'{k}->{n}', 'M': 1,
                       'ms_per_call': round(sec * 1e3, 3), 'gbs': round(b / sec / 1e9, 2), 'algorithmic_bytes': b,
                       'runs': runs})
    per_token = layers * sum(per_shape[(k, n)] for _, k, n in LAYER_SHAPES)
    return {'value': round(1.0 / per_token, 4), 'unit': 'tok/s', 'cores': threads, 'kind': 'port',
            'sample': f'torch {torch.__version__} on the host CPU ({threads} threads): the explicit QDQ path '
                      '(oracle/qdq_torch.py) at M=1 on configs[0] and each configs[1] shape, median of 10 calls '
                      f'after 3 warm-ups; value = 1 / ({layers} layers x the 7 decoder linears), linears only',
            'shapes': shapes, 'cpu_model': cpu_model(), 'os_cpu_count': os.cpu_count(),
            'omp_num_threads': os.environ.get('OMP_NUM_THREADS')}


def int8_e2e(torch, layers: int, device, steps: int, warmup: int) -> dict:
    """The reference's first published row on this build: the INT8 weight-only
    model (INT8 v1 tensors, linear_backend=None) decoding after a 4096-token
    prompt, B=1, each token one replay of its captured decode graph
    (fused W8A16 GEMVs that read the INT8 weights once)."""
    from ondeviceinfer_amd.config import QWEN3_14B, Qwen3Config
    from ondeviceinfer_amd.quantized_model import QuantizedQwen3ForCausalLM
    from ondeviceinfer_amd.runtime.quantized import QuantizedResidentRuntime
    from ondeviceinfer_amd.weight_quantization.synthetic import random_int8_store
    from ondeviceinfer_amd.generation import greedy_token
    cfg = Qwen3Config.from_dict(dict(QWEN3_14B, num_hidden_layers=layers))
    store = random_int8_store(cfg, seed=0, device=device)
    model = QuantizedQwen3ForCausalLM(store, QuantizedResidentRuntime(store, device=device), device=device)
    log(f'INT8 model bound: {torch.cuda.memory_allocated(device) / 2**30:.3f} GiB allocated')
    prompt = torch.randint(0, cfg.vocab_size, (1, PROMPT), generator=torch.Generator().manual_seed(0)).to(device)
    decoder_bytes = store.decoder_bytes
    # The model holds the weights (as INT8 tiles); drop the store's device
    # copies of the row-major tensors.
    store.layers = [{} for _ in store.layers]
    log(f'INT8 store copies dropped: {torch.cuda.memory_allocated(device) / 2**30:.3f} GiB allocated')
    cache = model.make_resident_cache(batch_size=1, max_seq_len=PROMPT + 2 + warmup + steps)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats(device)
    at_start = torch.cuda.memory_allocated(device)
    t0 = time.perf_counter()
    token = greedy_token(model(prompt, cache=cache, logits_to_keep=1))
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for _ in range(warmup):
        token = greedy_token(model(token, cache=cache, logits_to_keep=1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        token = greedy_token(model(token, cache=cache, logits_to_keep=1))
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    peak = torch.cuda.max_memory_allocated(device)
    check_step(model, token, cache)
    return {'workload': f'INT8 per-channel weight-only Qwen3-14B-shaped decoder ({layers} layers, INT8 v1 tensors), '
                        f'B=1, {PROMPT}-token prompt, greedy decode, fp16 KV resident; decode graph of W8A16 GEMVs',
            'tok_s': round(steps / sec, 2), 'ms_per_token': round(sec * 1e3 / steps, 4), 'steps': steps,
            'prefill_seconds': round(prefill_s, 4), 'decoder_int8_bytes': decoder_bytes,
            'peak_allocated_gib': round(peak / 2**30, 3), 'reference_peak_allocated_gib': REFERENCE_PEAK_GIB['int8'],
            'allocated_at_start_gib': round(at_start / 2**30, 3),
            'checked': 'finite logits and graph token == argmax on the step after the timed ones',
            'vs_reference_int8_explicit_path': round(steps / sec / 5.326, 2)}


def kernel_validation(torch, raw_layers: dict, device) -> dict:
    """The reference's kernel harness (``validate_weight_quant_kernels.py:38-77``)
    on this build, on the bench model's own weights: for every linear of the
    layers in ``raw_layers`` (layer index -> its raw pack-quantized tensors on
    the device) the startup repack time, then at M in {1, 4, 32, 256} with
    x = 0.1 * N(0, 1): the fused linear against torch's fp16 ``F.linear`` on the
    explicitly decoded weight (cosine, rel-L2, max |delta|, worst over 20
    repeats, and ``bitwise_changes`` between repeats), and the per-call time
    (CUDA events, median of 20 after 5 warm-ups) of the fused linear, of that
    fp16 ``F.linear`` and of the explicit-QDQ backend (``reference_int4``:
    decode + ``F.linear`` per call).  Pass: cosine >= 0.9999, rel-L2 <= 0.02,
    finite (the harness's bar)."""
    import statistics
    import torch.nn.functional as F
    from ondeviceinfer_amd.weight_quantization.backend import CompressedLinearBackend, decode_weight

    def per_call_ms(fn, warmups=5, repeats=20):
        for _ in range(warmups):
            fn()
        torch.cuda.synchronize()
        ev = []
        for _ in range(repeats):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            ev.append((a, b))
        torch.cuda.synchronize()
        return statistics.median(a.elapsed_time(b) for a, b in ev)

    gen = torch.Generator(device=device).manual_seed(42)
    rows = []
    for layer_idx, raw in raw_layers.items():
        for name in LINEAR_NAMES:
            prefix = name.removesuffix('.weight')
            weights = {key: v for key, v in raw.items() if key.startswith(prefix + '.')}
            ref_weight = decode_weight(weights, name)
            ref_weights = dict(weights)
            backend, ref_backend = CompressedLinearBackend('marlin'), CompressedLinearBackend('reference_int4')
            torch.cuda.synchronize()
            t = time.perf_counter()
            backend.prepare(weights, name)
            torch.cuda.synchronize()
            repack_ms = (time.perf_counter() - t) * 1e3
            for m in (1, 4, 32, 256):
                x = (torch.randn(m, ref_weight.shape[1], device=device, generator=gen) * 0.1).half()
                expected = F.linear(x, ref_weight).float()
                first = backend.linear(x, weights, name)
                cos, rel, mx, finite, changes = 1.0, 0.0, 0.0, True, 0
                for rep in range(20):
                    y = first if rep == 0 else backend.linear(x, weights, name)
                    d = y.float() - expected
                    cos = min(cos, float(F.cosine_similarity(y.float().flatten(), expected.flatten(), dim=0)))
                    rel = max(rel, float(torch.linalg.vector_norm(d) / torch.linalg.vector_norm(expected).clamp_min(1e-12)))
                    mx = max(mx, float(d.abs().max()))
                    finite = finite and bool(torch.isfinite(y).all())
                    changes += int(rep > 0 and not torch.equal(y, first))
                fused = per_call_ms(lambda: backend.linear(x, weights, name))
                fp16 = per_call_ms(lambda: F.linear(x, ref_weight))
                qdq = per_call_ms(lambda: ref_backend.linear(x, ref_weights, name))
                rows.append([layer_idx, prefix, m, round(cos, 7), round(rel, 6), round(mx, 5), changes, finite,
                             cos >= 0.9999 and rel <= 0.02 and finite, round(fused * 1e3, 2), round(fp16 * 1e3, 2),
                             round(qdq * 1e3, 2), round(repack_ms, 3)])
            del weights, ref_weights, ref_weight, backend, ref_backend
    return {'harness': 'validate_weight_quant_kernels.py:38-77 on the bench weights (layers '
                       f'{sorted(raw_layers)}), 20 correctness repeats, timing median of 20 after 5 warm-ups',
            'columns': ['layer', 'linear', 'm', 'cosine', 'relative_l2', 'max_abs', 'bitwise_changes', 'finite',
                        'passed', 'fused_us', 'fp16_linear_us', 'explicit_qdq_us', 'repack_ms'],
            'rows': rows, 'all_passed': all(r[8] for r in rows),
            'total_bitwise_changes': sum(r[6] for r in rows)}


def build_model(torch, layers: int, device, keep_raw: tuple = ()):
    from ondeviceinfer_amd.config import QWEN3_14B, Qwen3Config
    from ondeviceinfer_amd.quantized_model import QuantizedQwen3ForCausalLM
    from ondeviceinfer_amd.weight_quantization.backend import CompressedLinearBackend, CompressedResidentRuntime
    from ondeviceinfer_amd.weight_quantization.synthetic import random_compressed_store
    cfg = Qwen3Config.from_dict(dict(QWEN3_14B, num_hidden_layers=layers))
    t0 = time.perf_counter()
    store = random_compressed_store(cfg, seed=0, device=device)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # The startup repack per linear (the reference records repack_seconds,
    # validate_weight_quant_kernels.py:46-48): layer 0's seven linears.
    probe = CompressedLinearBackend('marlin')
    repack_ms = {}
    for name in LINEAR_NAMES:
        prefix = name.removesuffix('.weight')
        layer = {k: v for k, v in store.layers[0].items() if k.startswith(prefix + '.')}
        torch.cuda.synchronize()
        t = time.perf_counter()
        probe.prepare(layer, name)
        torch.cuda.synchronize()
        repack_ms[prefix] = round((time.perf_counter() - t) * 1e3, 3)
        del layer
    backend = CompressedLinearBackend('marlin')
    t2 = time.perf_counter()
    runtime = CompressedResidentRuntime(store, backend, device=device, verbose=False)
    model = QuantizedQwen3ForCausalLM(store, runtime, device=device, linear_backend=backend)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    # prepare() keeps only the repacked tiles (backend.py:224-226); drop the
    # store's raw copies as well (but for the layers the kernel report reads).
    raw = {i: store.layers[i] for i in keep_raw}
    store.layers = [{} for _ in store.layers]
    setup = {'random_weights_and_awq_quantize': round(t1 - t0, 2), 'repack_all_layers_and_fuse': round(t3 - t2, 3),
             'repack_ms_per_linear_layer0': repack_ms}
    return cfg, model, runtime, setup, raw


def kernel_sections(torch, native, model, runtime, cfg, args, device, capacity: int, result: dict,
                    step_times: dict | None) -> None:
    """The measurement sections beside the headline: the configs[1] GEMV pass,
    the decode step's kernels (roofline), the M=4096 prefill GEMMs and
    attention, the configs[3] batch sweep, the INT8 kernels and the copy
    ceiling; each adds its key to `result`.  `step_times` (step_kernel_times
    of the headline model) gives each decode-step kernel's duration inside
    the step.  Its buffers are locals, freed on return."""
    layers = [runtime.weights_for(i) for i in range(args.layers)]
    outs, xs = {}, {k: torch.randn(1, k, device=device).half() for k in (HIDDEN, INTER)}

    def linear(x, prepared, out):
        native.w4a16_linear(x, prepared.tiles, prepared.meta, prepared.n, GROUP, out=out,
                            workspace=prepared.workspace)

    # the 280 per-projection GEMVs of one decode token, as one graph.
    for name, k, n in LAYER_SHAPES:
        outs[name] = torch.empty(1, n, device=device, dtype=torch.float16)

    def gemv_pass():
        for w in layers:
            for name, k, n in LAYER_SHAPES:
                linear(xs[k], w[name + '._prepared'], outs[name])

    gemv_pass()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gemv_pass()
    sec = time_graph(torch, g, 10)
    del g
    pass_bytes = args.layers * sum(w4_bytes(1, n, k) for _, k, n in LAYER_SHAPES)
    result['gemv_pass'] = {'workload': 'configs[1]: W4A16 G=128 decode GEMV, M=1, q,k,v,o,gate,up,down x '
                                       f'{args.layers} layers per pass, HIP-graph replay',
                           'gbs': round(pass_bytes / sec / 1e9, 1),
                           'pct_hbm_peak': round(100.0 * pass_bytes / sec / 1e9 / HBM_PEAK_GBS, 2),
                           'us_per_pass': round(sec * 1e6, 1), 'bytes_per_pass': pass_bytes}

    # Kernels of the decode step as the step issues them (fused prologues
    # and epilogues, one weight set per layer), each as a graph of its
    # `layers` launches; then the plain per-projection GEMVs beside them.
    kernels = []
    eps = cfg.rms_norm_eps
    hid = torch.randn(HIDDEN, device=device).half()
    res = torch.randn(HIDDEN, device=device).half()
    gu_in = torch.randn(GATE_UP, device=device).half()
    att_in = torch.randn(HIDDEN, device=device).half()
    norm_w = (1.0 + 0.1 * torch.randn(HIDDEN, device=device)).half()
    sumsq_in = (hid.float() ** 2).view(-1, 16).sum(1).contiguous()   # per-16-row sums, as a producer writes
    sumsq_out = torch.empty(HIDDEN // 16, device=device)
    step_calls = [  # (op, K, N, kernel mode, fused-call keywords)
        ('self_attn.qkv_proj', HIDDEN, QKV, 'RmsNorm',
         dict(x=hid, x_mode=native.X_RMSNORM, norm_weight=norm_w, sumsq_in=sumsq_in, eps=eps)),
        ('self_attn.o_proj', HIDDEN, HIDDEN, 'Plain', dict(x=att_in, residual=res, sumsq_out=sumsq_out)),
        ('mlp.gate_up_proj', HIDDEN, GATE_UP, 'RmsNorm',
         dict(x=hid, x_mode=native.X_RMSNORM, norm_weight=norm_w, sumsq_in=sumsq_in, eps=eps)),
        ('mlp.down_proj', INTER, HIDDEN, 'SiluMul',
         dict(x=gu_in, x_mode=native.X_SILU_MUL, residual=res, sumsq_out=sumsq_out)),
    ]
    for name, k, n, mode, kw in step_calls:
        y = torch.empty(1, n, device=device, dtype=torch.float16)
        extra_kw = {a: v for a, v in kw.items() if a != 'x'}

        def fused_pass():
            for w in layers:
                p = w[name + '._prepared']
                native.w4a16_decode_fused(kw['x'], p.tiles, p.meta, p.n, GROUP, out=y, workspace=p.workspace,
                                          **extra_kw)
        fused_pass()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fused_pass()
        per = time_graph(torch, g, 10) / len(layers)
        kus, src = kernel_us(torch, g, 5, len(layers), per * 1e6)
        b = w4_bytes(1, n, k) + (2 * k if mode == 'SiluMul' else 0) + (2 * n if 'residual' in kw else 0)
        kernels.append({'op': name, 'fusion': mode + (' + residual + sumsq' if 'residual' in kw else ''),
                        'shape': f'{k}->{n}', 'kernel': kernel_name_for((1, n, k), mode), 'bytes': b,
                        'kernel_us': round(kus, 3), 'timing': src, 'us_per_launch': round(per * 1e6, 3),
                        'gbs': round(b / kus / 1e3, 1), 'frac': round(b / kus / 1e3 / HBM_PEAK_GBS, 4),
                        'in_decode_step': True, 'launches_per_token': args.layers})
        del g, y
    for name, k, n in [s for s in LAYER_SHAPES if s[0] in ('self_attn.q_proj', 'self_attn.k_proj',
                                                              'mlp.gate_proj', 'mlp.down_proj')]:
        y = torch.empty(1, n, device=device, dtype=torch.float16)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for w in layers:
                linear(xs[k], w[name + '._prepared'], y)
        per = time_graph(torch, g, 10) / len(layers)
        kus, src = kernel_us(torch, g, 5, len(layers), per * 1e6)
        b = w4_bytes(1, n, k)
        kernels.append({'op': name, 'fusion': 'none (unfused projection)', 'shape': f'{k}->{n}',
                        'kernel': kernel_name_for((1, n, k)), 'bytes': b, 'kernel_us': round(kus, 3), 'timing': src,
                        'us_per_launch': round(per * 1e6, 3), 'gbs': round(b / kus / 1e3, 1),
                        'frac': round(b / kus / 1e3 / HBM_PEAK_GBS, 4), 'in_decode_step': False,
                        'launches_per_token': args.layers})
        del g, y
    # Attention (+ chunk merge) at the decode position of the timed steps,
    # one KV cache per layer as in the step.
    kvh = cfg.num_key_value_heads
    kc = [[torch.randn(kvh, capacity, 128, device=device).half() for _ in range(2)] for _ in range(args.layers)]
    qkv = torch.randn(QKV, device=device).half()
    cos, sin = model.rotary_emb.table(capacity, device)
    pos = torch.tensor([PROMPT + args.warmup], dtype=torch.int32, device=device)
    att_out = torch.empty(HIDDEN, device=device, dtype=torch.float16)
    ws = torch.empty(native.decode_attention_workspace_size(cfg.num_attention_heads, kvh, 128, capacity),
                     dtype=torch.uint8, device=device)
    qn = torch.ones(128, device=device).half()

    def attn_pass():
        for c in kc:
            native.decode_attention(qkv, cfg.num_attention_heads, kvh, qn, qn, eps, cos, sin, pos, c[0], c[1],
                                    128 ** -0.5, out=att_out, workspace=ws)
    attn_pass()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attn_pass()
    per = time_graph(torch, g, 10) / args.layers
    kt = kernel_times(torch, g, 3)
    kus, src = kernel_us(torch, g, 5, 2 * args.layers, per * 1e6 / 2)
    kus *= 2   # the attention launch and its merge launch, per layer
    att_bytes = 2 * kvh * (PROMPT + args.warmup) * 128 * 2 + QKV * 2 + HIDDEN * 2
    kernels.append({'op': 'attention', 'fusion': 'q/k RMSNorm + RoPE + cache append; chunk-merge launch',
                    'shape': f'GQA {cfg.num_attention_heads}/{kvh} x 128, {PROMPT + args.warmup + 1} keys',
                    'kernel': 'decode_attention_kernel + decode_attention_merge_kernel', 'bytes': att_bytes,
                    'kernel_us': round(kus, 3), 'timing': src,
                    'kernels': {n_[:60]: round(v['us'], 3) for n_, v in kt.items()},
                    'us_per_launch': round(per * 1e6, 3), 'gbs': round(att_bytes / kus / 1e3, 1),
                    'frac': round(att_bytes / kus / 1e3 / HBM_PEAK_GBS, 4), 'in_decode_step': True,
                    'launches_per_token': args.layers})
    del g, kc
    # The fp16 LM head with the greedy token (once per token).
    lm_x = torch.randn(HIDDEN, device=device).half()
    lm_logits = torch.empty(cfg.vocab_size, device=device).half()
    lm_tok = torch.zeros(1, dtype=torch.long, device=device)
    lm_ws = torch.zeros(native.lm_head_workspace_size(HIDDEN, cfg.vocab_size), dtype=torch.uint8, device=device)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(4):
            native.lm_head(lm_x, model.lm_head, logits=lm_logits, token=lm_tok, workspace=lm_ws)
    per = time_graph(torch, g, 5) / 4
    kus, src = kernel_us(torch, g, 5, 8, per * 1e6 / 2)
    kus *= 2   # the LM head launch and its pick launch
    lm_b = cfg.vocab_size * HIDDEN * 2 + HIDDEN * 2 + cfg.vocab_size * 2
    kernels.append({'op': 'lm_head', 'fusion': 'fp16 GEMV + greedy token (pick launch)',
                    'shape': f'{HIDDEN}->{cfg.vocab_size}', 'kernel': 'lm_head_kernel<10> + lm_head_pick_kernel',
                    'bytes': lm_b, 'kernel_us': round(kus, 3), 'timing': src, 'us_per_launch': round(per * 1e6, 3),
                    'gbs': round(lm_b / kus / 1e3, 1), 'frac': round(lm_b / kus / 1e3 / HBM_PEAK_GBS, 4),
                    'in_decode_step': True, 'launches_per_token': 1})
    del g
    for e in kernels:
        e['us_per_token'] = round(e['kernel_us'] * e['launches_per_token'], 2)
        if not e['in_decode_step']:
            continue
        # The same kernel inside the decode steps (profiled after the timed ones).
        if e['op'] == 'attention':
            pats = ('decode_attention_kernel', 'decode_attention_merge_kernel')
        elif e['op'] == 'lm_head':
            pats = ('lm_head_kernel', 'lm_head_pick_kernel')
        else:
            pats = (step_record_pattern(e['kernel']),)
        us = in_step_us(step_times, pats, e['launches_per_token'], e['kernel_us']) if step_times and all(pats) else None
        if us is not None:
            e['in_step_us'] = round(us, 3)
            e['in_step_frac'] = round(e['bytes'] / us / 1e3 / HBM_PEAK_GBS, 4)
    step = [e for e in kernels if e['in_decode_step']]
    dom = max(step, key=lambda e: e['us_per_token'])
    # achieved = algorithmic bytes per launch / the kernel's own average
    # duration in the decode steps (torch.profiler device records, as
    # rocprofv3's kernel trace reports it); one_op_graph_us is the same
    # kernel in a graph of only its own launches (one per layer), and
    # graph_us_per_launch adds that graph's launch gaps.
    if 'in_step_us' in dom:
        avg_us, timing = dom['in_step_us'], f'kernel: device records over {PROFILED_STEPS} decode steps'
    else:
        avg_us, timing = dom['kernel_us'], dom['timing'] + ': one-op graph (no usable in-step records)'
    achieved = dom['bytes'] / avg_us / 1e3
    result['roofline'] = {
        'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
        'frac': round(achieved / HBM_PEAK_GBS, 4),
        'traffic': profiled_traffic(dom['kernel'], dom['shape']), 'kernel': dom['kernel'], 'shape': dom['shape'],
        'op': dom['op'], 'avg_launch_us': round(avg_us, 3), 'timing': timing,
        'one_op_graph_us': dom['kernel_us'], 'graph_us_per_launch': dom['us_per_launch'],
        'algorithmic_bytes_per_launch': dom['bytes'],
        # the metric's second half: the configs[1] GEMV pass, % of HBM peak
        'gemv_pass_pct_hbm_peak': result['gemv_pass']['pct_hbm_peak'],
    }
    result['decode_step_kernels'] = kernels

    # prefill GEMM, M=4096 on the first layer's weights.
    xp = {kk: torch.randn(4096, kk, device=device).half() for kk in (HIDDEN, INTER)}
    prefill = []
    for name, k, n in [('self_attn.q_proj', HIDDEN, HIDDEN), ('self_attn.k_proj', HIDDEN, KV),
                       ('mlp.gate_proj', HIDDEN, INTER), ('mlp.down_proj', INTER, HIDDEN),
                       ('self_attn.qkv_proj', HIDDEN, QKV), ('mlp.gate_up_proj', HIDDEN, GATE_UP)]:
        yp = torch.empty(4096, n, device=device, dtype=torch.float16)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            linear(xp[k], layers[0][name + '._prepared'], yp)
        sec = time_graph(torch, g, 10)
        graph_sec = sec
        sec = kernel_us(torch, g, 5, 1, sec * 1e6)[0] / 1e6
        tflops = 2 * 4096 * n * k / sec / 1e12
        # Context, not a target: the vendor library's dense fp16 GEMM
        # (torch.matmul -> hipBLASLt) on the same shape with an fp16
        # weight, no dequantization.
        wt = (torch.randn(k, n, device=device) * 0.02).half()
        gv = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gv):
            torch.matmul(xp[k], wt, out=yp)
        vsec = time_graph(torch, gv, 10)
        vsec = kernel_us(torch, gv, 5, 1, vsec * 1e6)[0] / 1e6
        prefill.append({'op': name, 'shape': f'{k}->{n}', 'M': 4096, 'us': round(sec * 1e6, 1),
                        'graph_us': round(graph_sec * 1e6, 1),
                        'tflops': round(tflops, 1), 'frac_fp16_mfma': round(tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                        'vendor_fp16_gemm_us': round(vsec * 1e6, 1),
                        'vendor_fp16_gemm_tflops': round(2 * 4096 * n * k / vsec / 1e12, 1),
                        'speed_vs_vendor_fp16': round(vsec / sec, 3)})
        del g, gv, yp, wt
    result['prefill'] = prefill

    # The 4096-token prompt's causal GQA attention (wq_prefill_attention:
    # token-major q, cache rows read in place), TFLOP/s over the causal
    # flops 4*T^2*d*H/2, beside torch's fused SDPA on the same tensors (the
    # path it replaces; context, not a target).
    from ondeviceinfer_amd.attention import strided_prefill_attention
    hq, kvh, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    qa = torch.randn(PROMPT, hq, hd, device=device).half()
    ka, va = (torch.randn(kvh, PROMPT, hd, device=device).half() for _ in range(2))
    oa = torch.empty(PROMPT, hq, hd, device=device, dtype=torch.float16)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.prefill_attention(qa, hq, kvh, ka, va, 0, hd ** -0.5, out=oa)
    sec = time_graph(torch, g, 10)
    gs = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gs):
        strided_prefill_attention(qa.transpose(0, 1).unsqueeze(0), ka[None], va[None])
    ssec = time_graph(torch, gs, 10)
    flops = 4 * PROMPT * PROMPT * hd * hq / 2
    result['prefill_attention'] = {
        'op': 'causal GQA flash attention (wq_prefill_attention), one layer',
        'shape': f'T={PROMPT}, {hq}/{kvh} heads x {hd}', 'us': round(sec * 1e6, 1),
        'tflops': round(flops / sec / 1e12, 1), 'frac_fp16_mfma': round(flops / sec / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4),
        'torch_sdpa_us': round(ssec * 1e6, 1), 'torch_sdpa_tflops': round(flops / ssec / 1e12, 1)}
    del g, gs, qa, ka, va, oa

    # fused QKV and gate_up (every layer's weights in one graph,
    # so the 256 MB Infinity Cache cannot serve repeats) and a W4 lm_head
    # 5120->151936 (random tiles, 389 MB), at M in {1, 8, 32, 128, 512}.
    vocab = cfg.vocab_size
    lm_tb, lm_mb = native.w4_repack_size(vocab, HIDDEN, GROUP)
    lm_tiles = torch.randint(0, 256, (lm_tb,), dtype=torch.uint8, device=device)
    lm_meta = torch.randint(0, 256, (lm_mb,), dtype=torch.uint8, device=device)
    lm_meta.view(torch.float16)[:] = 0.001   # finite scales; the zero words take the same bits
    sweep = []
    for name, n, ws_list in [('self_attn.qkv_proj', QKV, None), ('mlp.gate_up_proj', GATE_UP, None),
                             ('lm_head (W4)', vocab, [lm_tiles, lm_meta])]:
        for m in (1, 8, 32, 128, 512):
            xm = torch.randn(m, HIDDEN, device=device).half()
            ym = torch.empty(m, n, device=device, dtype=torch.float16)
            wsz = native.w4a16_workspace_size(m, n, HIDDEN, GROUP)
            wsb = torch.zeros(max(wsz, 1), dtype=torch.uint8, device=device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                if ws_list is None:
                    for w in layers:
                        pr = w[name + '._prepared']
                        native.w4a16_linear(xm, pr.tiles, pr.meta, n, GROUP, out=ym, workspace=wsb)
                else:
                    native.w4a16_linear(xm, ws_list[0], ws_list[1], n, GROUP, out=ym, workspace=wsb)
            launches = len(layers) if ws_list is None else 1
            per = time_graph(torch, g, 5) / launches
            b = w4_bytes(m, n, HIDDEN)
            tf = 2 * m * n * HIDDEN / per / 1e12
            sweep.append({'op': name, 'shape': f'{HIDDEN}->{n}', 'M': m, 'us': round(per * 1e6, 2),
                          'gbs': round(b / per / 1e9, 1), 'frac_hbm': round(b / per / 1e9 / HBM_PEAK_GBS, 4),
                          'tflops': round(tf, 1), 'frac_fp16_mfma': round(tf / FP16_MFMA_PEAK_TFLOPS, 4)})
            del g, xm, ym, wsb
    result['batch_sweep'] = sweep
    del lm_tiles, lm_meta

    # INT8 variants of configs[0] on the GPU over a pool of 40 distinct
    # 5120x5120 weights (N(0, 0.02), per-channel symmetric INT8; 1.05 GB,
    # above the 256 MB Infinity Cache), each case a graph of one launch
    # per weight: weight-only W8A16 decode, W8A8 (int8_gemm) decode and
    # the M=4096 W8A16 / W8A8 prefill GEMMs on the matrix cores, over the
    # INT8 tiles the prepared linears stream (wq_w8_repack), and the
    # W8A16 pair once more over the row-major weight as stored.
    g0 = torch.Generator(device=device).manual_seed(0)
    pool, rowmajor = [], []
    for _ in range(40):
        w8 = (torch.randn(HIDDEN, HIDDEN, device=device, generator=g0) * 0.02).half()
        q8w, s8w = native.w8_quantize(w8)
        pool.append((native.w8_repack(q8w), s8w, s8w.float()))
        rowmajor.append((q8w, s8w, s8w.float()))
    del w8
    int8 = []
    x1 = torch.randn(1, HIDDEN, device=device).half()
    x4k = torch.randn(4096, HIDDEN, device=device).half()
    qx1, sx1 = native.w8a8_quantize(x1)
    qx4k, sx4k = native.w8a8_quantize(x4k)
    y1 = torch.empty(1, HIDDEN, device=device, dtype=torch.float16)
    y4k = torch.empty(4096, HIDDEN, device=device, dtype=torch.float16)
    cases = [
        ('w8a16 decode (configs[0] on the GPU)', 1, 'w8a16', pool,
         lambda q, s, s32: native.w8a16_linear(x1, q, s, out=y1)),
        ('w8a8 int8_gemm decode (quantize + linear)', 1, 'w8a8', pool,
         lambda q, s, s32: native.w8a8_linear(*native.w8a8_quantize(x1), q, s32, out=y1)),
        ('w8a8 linear only, decode', 1, 'w8a8', pool,
         lambda q, s, s32: native.w8a8_linear(qx1, sx1, q, s32, out=y1)),
        ('w8a16 prefill M=4096', 4096, 'w8a16', pool, lambda q, s, s32: native.w8a16_linear(x4k, q, s, out=y4k)),
        ('w8a8 linear only, prefill M=4096', 4096, 'w8a8', pool,
         lambda q, s, s32: native.w8a8_linear(qx4k, sx4k, q, s32, out=y4k)),
        ('w8a16 decode, row-major weight as stored', 1, 'w8a16', rowmajor,
         lambda q, s, s32: native.w8a16_linear(x1, q, s, out=y1)),
        ('w8a16 prefill M=4096, row-major weight as stored', 4096, 'w8a16', rowmajor,
         lambda q, s, s32: native.w8a16_linear(x4k, q, s, out=y4k)),
    ]
    for label, mm, kind, weights, fn in cases:
        fn(*weights[0])
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for q8w, s8w, s32 in weights:
                fn(q8w, s8w, s32)
        sec = time_graph(torch, g, 5) / len(weights)
        w8a8 = kind == 'w8a8'   # int8 x and fp32 scales vs fp16 x and fp16 scales
        b = HIDDEN * HIDDEN + (4 if w8a8 else 2) * HIDDEN + (1 if w8a8 else 2) * mm * HIDDEN + 2 * mm * HIDDEN
        entry = {'op': label, 'shape': f'{HIDDEN}->{HIDDEN}', 'M': mm, 'us': round(sec * 1e6, 2),
                 'weights_rotated': len(pool), 'pool_bytes': len(pool) * HIDDEN * HIDDEN}
        if mm == 1:
            entry.update(gbs=round(b / sec / 1e9, 1), frac_hbm=round(b / sec / 1e9 / HBM_PEAK_GBS, 4),
                         algorithmic_bytes=b)
        else:
            tops = 2 * mm * HIDDEN * HIDDEN / sec / 1e12
            peak = INT8_MFMA_PEAK_TOPS if w8a8 else FP16_MFMA_PEAK_TFLOPS
            entry.update(tops=round(tops, 1), frac_mfma_peak=round(tops / peak, 4),
                         mfma_peak='int8 5.0 POP/s' if w8a8 else 'fp16 2.5 PFLOP/s')
        int8.append(entry)
        del g
    # Context for the W8A8 prefill: the vendor library's int8 GEMM
    # (torch._int_mm -> hipBLASLt, int32 out, no scaling) on the same pool.
    qx4k_t = qx4k.contiguous()
    acc32 = torch.empty(4096, HIDDEN, device=device, dtype=torch.int32)
    wts = [q8w.t().contiguous() for q8w, _, _ in rowmajor[:8]]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for wtq in wts:
            torch._int_mm(qx4k_t, wtq, out=acc32)
    sec = time_graph(torch, g, 5) / len(wts)
    tops = 2 * 4096 * HIDDEN * HIDDEN / sec / 1e12
    int8.append({'op': 'vendor int8 GEMM, M=4096 (torch._int_mm / hipBLASLt, int32 out; context only)',
                 'shape': f'{HIDDEN}->{HIDDEN}', 'M': 4096, 'us': round(sec * 1e6, 2), 'tops': round(tops, 1),
                 'frac_mfma_peak': round(tops / INT8_MFMA_PEAK_TOPS, 4), 'mfma_peak': 'int8 5.0 POP/s'})
    del g, wts, acc32
    result['int8'] = int8
    del pool, rowmajor, x4k, qx4k, y4k

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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=127, help='timed decode tokens')
    ap.add_argument('--warmup', type=int, default=5, help='untimed decode tokens before the timed ones')
    ap.add_argument('--layers', type=int, default=40)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-extras', action='store_true', help='skip the GEMV pass, kernel and prefill sections')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: this build has no multi-GPU path (every box has one GPU); '
              'run with --gpus 1', file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print('need --steps >= 1 and --warmup >= 0', file=sys.stderr)
        return 2

    import torch
    from ondeviceinfer_amd import _native as native
    from ondeviceinfer_amd.generation import greedy_token

    if not torch.cuda.is_available():
        print('bench.py needs a GPU', file=sys.stderr)
        return 2
    device = torch.device('cuda:0')
    torch.manual_seed(0)

    log(f'building a random {args.layers}-layer Qwen3-14B-shaped W4A16 model and repacking it')
    t0 = time.perf_counter()
    report_layers = () if args.no_extras else tuple(sorted({0, args.layers // 2, args.layers - 1}))
    cfg, model, runtime, setup, raw = build_model(torch, args.layers, device, report_layers)
    build_s = time.perf_counter() - t0
    validation = None
    if raw:
        log(f'kernel report in the reference harness\'s shape: layers {list(raw)}, 7 linears, M in 1/4/32/256')
        validation = kernel_validation(torch, raw, device)
        del raw
        torch.cuda.empty_cache()
    capacity = PROMPT + 1 + args.warmup + args.steps + PROFILED_STEPS
    prompt = torch.randint(0, cfg.vocab_size, (1, PROMPT), generator=torch.Generator().manual_seed(0)).to(device)

    def generate(n_untimed: int, n_timed: int, n_profiled: int = 0):
        cache = model.make_resident_cache(batch_size=1, max_seq_len=capacity)
        torch.cuda.synchronize()
        # Peak allocated over prefill + decode with the cache already made,
        # as the reference's harness measures it (benchmark_kv_offload.py:514).
        torch.cuda.reset_peak_memory_stats(device)
        t_p = time.perf_counter()
        out = model(prompt, cache=cache, logits_to_keep=1)
        token = greedy_token(out)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t_p
        for _ in range(n_untimed):
            token = greedy_token(model(token, cache=cache, logits_to_keep=1))
        torch.cuda.synchronize()
        t_d = time.perf_counter()
        for _ in range(n_timed):
            token = greedy_token(model(token, cache=cache, logits_to_keep=1))
        torch.cuda.synchronize()
        decode_s = time.perf_counter() - t_d
        peak = torch.cuda.max_memory_allocated(device)
        check_step(model, token, cache)
        times = step_kernel_times(torch, model, token, cache, n_profiled) if n_profiled else None
        return prefill_s, decode_s, cache, peak, times

    log('warm-up generation (captures the decode-step graph)')
    t0 = time.perf_counter()
    cache = model.make_resident_cache(batch_size=1, max_seq_len=capacity)
    capture_s = time.perf_counter() - t0
    del cache
    generate(2, 0)
    log(f'timed generation: prefill {PROMPT}, {args.warmup} untimed + {args.steps} timed decode tokens')
    prefill_s, decode_s, cache, peak_bytes, step_times = generate(
        args.warmup, args.steps, 0 if args.no_extras else PROFILED_STEPS)
    assert cache.lengths[0] == PROMPT + args.warmup + args.steps + 1 + (0 if args.no_extras else PROFILED_STEPS)
    toks = args.steps / decode_s
    weight_bytes = runtime.resident_storage_bytes
    kv_bytes_per_token = 2 * args.layers * cfg.num_key_value_heads * cfg.head_dim * 2 * (PROMPT + args.warmup)
    lm_bytes = cfg.vocab_size * cfg.hidden_size * 2
    result = {
        'metric': METRIC, 'value': round(toks, 3), 'unit': 'tok/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(decode_s * 1000 / args.steps, 4), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': round(toks / PUBLISHED_TOKS, 3) if args.layers == 40 else None,
        'dtype': 'fp16', 'data': 'synthetic',
        'config': {'workload': f'configs[4]: Qwen3-14B-shaped AWQ-INT4 G=128 decoder ({args.layers} layers), random '
                               f'weights, B=1, {PROMPT}-token random prompt, greedy decode, fp16 KV resident; '
                               'one step = one decode token (graph replay; the LM head picks the greedy token)',
                   'layers': args.layers, 'prompt_tokens': PROMPT, 'group_size': GROUP,
                   'kv_capacity': capacity},
        'prefill_seconds': round(prefill_s, 4),
        'prefill_tok_s': round(PROMPT / prefill_s, 1),
        'bytes_per_token': {'decoder_weights': int(weight_bytes), 'lm_head_fp16': lm_bytes,
                            'kv_cache_read_at_start': kv_bytes_per_token},
        'effective_gbs': round((weight_bytes + lm_bytes + kv_bytes_per_token) * toks / 1e9, 1),
        'setup_seconds': {'build_and_repack': round(build_s, 2), 'graph_capture': round(capture_s, 3), **setup},
        'peak_allocated_gib': round(peak_bytes / 2**30, 3),
        'reference_peak_allocated_gib': REFERENCE_PEAK_GIB['w4'],
    }
    result['pct_hbm_peak_effective'] = round(100.0 * result['effective_gbs'] / HBM_PEAK_GBS, 2)
    del cache

    if not args.no_extras:
        kernel_sections(torch, native, model, runtime, cfg, args, device, capacity, result, step_times)
        result['kernel_validation'] = validation

    if not args.no_extras:
        # The same model with the optional W4 LM head: 0.39 GB of tiles and
        # records per token instead of 1.56 GB of fp16.  Not the reference's
        # configuration (its AWQ recipe keeps lm_head fp16), so not the
        # headline.
        log('W4 LM head variant: quantize the head, capture, decode')
        model.quantize_lm_head()
        generate(2, 0)
        _, dec_w4, cache, peak_w4, _ = generate(args.warmup, args.steps)
        del cache
        tb, mb = native.w4_repack_size(cfg.vocab_size, cfg.hidden_size, GROUP)
        result['e2e_w4_lm_head'] = {
            'workload': 'the headline workload with the LM head quantized to uint4 G=128 (optional; the reference '
                        'keeps it fp16)', 'tok_s': round(args.steps / dec_w4, 3),
            'ms_per_token': round(dec_w4 * 1000 / args.steps, 4), 'lm_head_bytes': tb + mb,
            'peak_allocated_gib': round(peak_w4 / 2**30, 3)}
        torch.cuda.empty_cache()

    # One model per process, as the reference's harness runs them: the W4
    # model's weights and caches are freed before the INT8 model is built.
    del model, runtime
    import gc
    gc.collect()
    torch.cuda.empty_cache()
    log(f'allocated after freeing the W4 model: {torch.cuda.memory_allocated(device) / 2**30:.3f} GiB')
    if not args.no_extras:
        log('INT8 weight-only model: build, prefill and decode')
        result['int8_e2e'] = int8_e2e(torch, args.layers, device, args.steps, args.warmup)
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        log('cpu baseline')
        result['cpu_baseline'] = cpu_baseline(torch, native, device, args.layers)

    # Bulky per-case tables first, the decode summary last: a reader that keeps
    # only the tail of stdout still sees the step's kernels, the GEMV pass, the
    # roofline and the CPU baseline.
    last = ('decode_step_kernels', 'int8_e2e', 'e2e_w4_lm_head', 'prefill_seconds', 'prefill_tok_s',
            'bytes_per_token', 'effective_gbs', 'pct_hbm_peak_effective', 'peak_allocated_gib',
            'reference_peak_allocated_gib', 'gemv_pass', 'roofline', 'cpu_baseline')
    ordered = {k: v for k, v in result.items() if k not in last}
    ordered.update((k, result[k]) for k in last if k in result)
    print(json.dumps(ordered), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
