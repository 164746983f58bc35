"""Per-layer latency of value projection + multi-scale deformable attention on one MI355X.

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50] [--workload rtdetr640-fp16-b1-q300] [--no-cpu]

A step is one ma_deform_attn call (mode='auto', the default) on one batch of synthetic inputs already resident
in HBM. Like the reference's bench (bench/bench.py:40-61) the calls are captured in a HIP graph, so Python launch
overhead is excluded: W warm-up steps (one graph replay), then a graph of EXACTLY K steps replayed 7 times, each
replay bracketed by torch.cuda.synchronize() and timed with events on the replay stream; the best replay gives
the µs per call, as the reference takes the best of 7 replays of its 100-call graph. A replay's fixed cost (about
10-17 µs: the graph launch and the timing events) is inside the timed region, so a short graph reads higher per call
than a long one (about 0.85 µs per call at 20 calls).

Prints diagnostics on stderr and ONE JSON line on stdout: value = µs per layer call (auto mode), with per-mode
times, the roofline of the dominant kernel (algorithmic bytes or flops per launch / its average launch duration,
measured the same way on its own stream), the effective byte rate of the path (algorithmic bytes / time: gathered
rows count every time they are read, L2 hits included) next to the HBM rate the counters measured (bytes that reached
the memory fabric per launch, from the committed rocprofv3 --pmc summary, / the same time), and the CPU baseline
(the oracle's torch restatement of the reference's PyTorch path, float32, on this host's cores, timed on a
bounded sample). For the gather kernels (fused mode, the sampler) the roofline's bound is "l2-gather": the rate at
which all CUs receive randomly chosen rows of the kernel's width from L2 (a buffer of the gathered tensor's size, at
most one XCD's 4 MB L2), measured in the same run by td_probe_gather, with the HBM figures beside it.

Other modes: --table (the reference's sweep), --fit-auto / --holdout (the auto selector), --ceiling (the gather
ceiling over row widths and buffer sizes), --phases (the fused kernel's phase timeline, from the measurement build
libtinydeform_phases.so), --trace-run, --train-run and --pmc-run (short runs for rocprofv3).
"""

import argparse
import json
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, 'tests'))

import marearts_tinydeform_amd as td  # noqa: E402
from marearts_tinydeform_amd import _native  # noqa: E402
from inputs import DINO_LEVELS, LIMIT_LEVELS, RTDETR_LEVELS, workload  # noqa: E402

HBM_PEAK = 8.0e12        # bytes/s, MI355X HBM3E
MFMA_PEAK_16 = 2.5e15    # flop/s, dense fp16/bf16
FUSED_KERNELS = ('fused_vec_kernel',)

WORKLOADS = {
    # name: (B, Q, H, D, C, levels, P, dtype, bias, loc_dist)
    'rtdetr640-fp16-b1-q300': (1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16, True, 'uniform'),
    'rtdetr640-fp16-b1-q100': (1, 100, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16, True, 'uniform'),
    'rtdetr640-fp16-b1-q50': (1, 50, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16, True, 'uniform'),
    'rtdetr640-fp32-b1-q300': (1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float32, True, 'uniform'),
    'rtdetr640-bf16-b8-q300': (8, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.bfloat16, True, 'uniform'),
    'dino4l-fp16-b4-q900': (4, 900, 8, 32, 256, DINO_LEVELS, 4, torch.float16, True, 'outside10'),
    'limit-bf16-c1024-b2-q50': (2, 50, 16, 64, 1024, LIMIT_LEVELS, 16, torch.bfloat16, False, 'uniform'),
    'limit-bf16-c1024-b2-q300': (2, 300, 16, 64, 1024, LIMIT_LEVELS, 16, torch.bfloat16, False, 'uniform'),
    'limit-bf16-c1024-b2-q900': (2, 900, 16, 64, 1024, LIMIT_LEVELS, 16, torch.bfloat16, False, 'uniform'),
    'rtdetr640-fp16-b1-q300-clustered': (1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16, True, 'clustered'),
    # encoder self-attention: every memory token is a query (Q = N = 22223)
    'dino4l-encoder-fp16-b2': (2, 22223, 8, 32, 256, DINO_LEVELS, 4, torch.float16, True, 'encoder'),
}

DTYPE_NAMES = {torch.float16: 'f16', torch.bfloat16: 'bf16', torch.float32: 'f32', torch.float64: 'f64'}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_time_us(fn, steps, warmup, replays=7):
    """µs per call: W warm-up calls (eager on a side stream, then one replay of a W-call graph), then the best of
    `replays` timed replays of a graph of exactly `steps` calls, events recorded on the replay stream (the
    reference's method, bench/bench.py:40-61). Each timed replay carries a fixed cost of 10-17 µs on MI355X
    (two timing events with nothing between them read 4.2 µs; a one-call graph 26.9 µs against 8.0 µs per further
    call at the headline), which a short graph spreads over few calls: about 0.85 µs per call at 20 calls, 0.2 at
    100."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    warm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(warm):
        for _ in range(max(warmup, 1)):
            fn()
    timed = torch.cuda.CUDAGraph()
    with torch.cuda.graph(timed):
        for _ in range(steps):
            fn()
    warm.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float('inf')
    for _ in range(replays):
        torch.cuda.synchronize()
        start.record(cur)
        timed.replay()
        end.record(cur)
        torch.cuda.synchronize()
        best = min(best, start.elapsed_time(end) * 1e3 / steps)
    del warm, timed
    return best


def algorithmic(B, Q, H, D, C, N, L, P, s):
    """Algorithmic bytes / flops per launch of each kernel (element size s)."""
    HD = H * D
    samples = B * Q * H * L * P
    fused = samples * 4 * C * s + samples * 3 * s + HD * C * s + HD * s + B * Q * HD * s
    sample = samples * 4 * D * s + samples * 3 * s + B * Q * HD * s
    gemm_bytes = B * N * C * s + HD * C * s + B * N * HD * s + HD * s
    gemm_flops = 2 * B * N * C * HD
    return {'fused_bytes': fused, 'sample_bytes': sample, 'gemm_bytes': gemm_bytes, 'gemm_flops': gemm_flops}


def layer_times(B, Q, H, D, C, levels, P, dtype, steps, warmup):
    """µs per decoder-layer call (RT-DETR decoder cross-attention: box reference points shared by the levels,
    position embeddings, output_proj) on the same shapes: the fused layer kernel, the layer's project mode, the
    unfused sequence (PyTorch sampling-offset / attention Linear + softmax + reference-point arithmetic, then
    ma_deform_attn and output_proj as separate calls) and the plain PyTorch layer (F.linear + grid_sample)."""
    from inputs import make_layer
    a = make_layer(B, Q, H, D, C, levels, P, ref_dim=4, ref_levels='1', dtype=dtype)
    dev = [t.cuda() if isinstance(t, torch.Tensor) else t for t in a]
    hidden, memory, ref, shapes, starts, ow, ob, aw, ab, vw, vb, o_w, o_b, nh, npt, pos = dev
    shapes_cpu, starts_cpu = a[3], a[4]

    def layer(mode):
        return td.ma_deform_attn_layer(hidden, memory, ref, shapes, starts, ow, ob, aw, ab, vw, vb, o_w, o_b, nh, npt,
                                       position_embeddings=pos, mode=mode)

    def unfused():
        loc, attn = td.layer_locations_reference(hidden, ref, shapes_cpu, ow, ob, aw, ab, nh, npt, pos)
        core = td.ma_deform_attn(memory, vw, vb, shapes, starts, loc, attn)
        return torch.nn.functional.linear(core, o_w, o_b)

    def pytorch():
        return td.ma_deform_attn_layer_reference(hidden, memory, ref, shapes_cpu, starts_cpu, ow, ob, aw, ab, vw, vb,
                                                 o_w, o_b, nh, npt, position_embeddings=pos)

    out = {}
    with torch.inference_mode():
        for mode in ('fused', 'project', 'auto'):
            out[f'layer_{mode}'] = graph_time_us(lambda m=mode: layer(m), steps, warmup)
        out['layer_unfused'] = graph_time_us(unfused, steps, warmup)
        out['layer_pytorch'] = graph_time_us(pytorch, min(steps, 200), min(warmup, 10))
    return out


def train_steps(cpu_args):
    """The training step of the operator and of the PyTorch reference path (F.linear + grid_sample under autograd)
    on the same device, as two callables: the gradients set to None (optimizer.zero_grad's default), the forward, and
    the backward of a fixed random grad_out, with gradients for memory, value_weight, value_bias, the locations and
    the attention weights (so no step accumulates into the previous step's gradients)."""
    dev = [None if t is None else t.cuda() for t in cpu_args]
    ref_args = list(dev)
    ref_args[3], ref_args[4] = cpu_args[3], cpu_args[4]  # the reference reads the level shapes on the host
    leaves = [t.requires_grad_(True) if (i in (0, 1, 2, 5, 6) and t is not None) else t for i, t in enumerate(dev)]
    ref_leaves = [leaves[i] if i in (0, 1, 2, 5, 6) else t for i, t in enumerate(ref_args)]
    B, Q = dev[5].shape[:2]
    go = torch.randn(B, Q, dev[1].shape[0], generator=torch.Generator().manual_seed(1)).to(dev[0].dtype).cuda()

    def zero_grad():
        for t in leaves:
            if t is not None and t.requires_grad:
                t.grad = None

    def ours():
        zero_grad()
        torch.autograd.backward(td.ma_deform_attn_train(*leaves), go)

    def pytorch():
        zero_grad()
        torch.autograd.backward(td.ma_deform_attn_reference(*ref_leaves), go)

    return ours, pytorch


def train_times(cpu_args, steps, warmup):
    """µs per training step (train_steps) of the operator on the library's kernels (ma_deform_attn_train) and of the
    PyTorch reference path, graph-timed."""
    ours, pytorch = train_steps(cpu_args)

    out = {}
    for name, fn, n in (('train_step', ours, steps), ('pytorch_train_step', pytorch, min(steps, 100))):
        try:
            out[name] = graph_time_us(fn, n, min(warmup, 10))
        except RuntimeError as e:  # capture refused: eager steps timed with events
            log(f'  {name}: graph capture failed ({str(e).splitlines()[0][:80]}); timing eager steps')
            torch.cuda.synchronize()
            for _ in range(3):
                fn()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(n):
                fn()
            b.record()
            torch.cuda.synchronize()
            out[name] = a.elapsed_time(b) * 1e3 / n
    return out


def gemm_kernel(M, K, NO, s):
    """Which value-projection kernel td_value_proj launches for an aligned [M, K] x [K, NO] problem (element size
    s), following its size rule: 16-bit with 256 outputs, K = 256 and at least 14000 rows (K = 128: 8000) takes the streaming
    kernel; 16-bit deep K (K >= 512, K % 64 == 0) on a grid of >= 200 tiles of 256 x 128, more than 256 of 128 x 128 or
    from 8000 rows the direct-to-LDS kernels (persistent 256 x 256 tiles from 120 of them when NO % 16 == 0 and the
    sizes stay below 2^31 elements, else 256 x 128 tiles);
    other 16-bit grids take register-operand tiles (32 x 32 to 64 x 64) up to 1100 tiles of 64 x 64 for K <= 256 and
    under 512 for deeper K, larger ones both operands through LDS;
    float32 takes register-operand tiles of 32 x 32 to 64 x 128."""
    tiles_128 = -(-M // 128) * -(-NO // 128)
    if s == 2:
        if NO == 256 and K in (128, 256) and M >= (14000 if K == 256 else 8000):
            return 'gemm_stream_kernel'
        if K >= 512 and K % 64 == 0 and (-(-M // 256) * -(-NO // 128) >= 200 or tiles_128 > 256 or M >= 8000):
            lim = 1 << 31
            if (-(-M // 256) * -(-NO // 256) >= 120 and NO % 16 == 0 and M >= 256 and 256 <= NO <= 8192 and
                    max(M * K, NO * K, M * NO) < lim):
                return 'gemm_dma_persistent_kernel'
            return 'gemm_dma_kernel'
        tiles_64 = -(-M // 64) * -(-NO // 64)
        if K <= 256:
            return 'gemm_mfma_kernel' if tiles_64 <= 1100 else 'gemm_lds_kernel'
        return 'gemm_mfma_kernel' if tiles_64 < 512 else 'gemm_lds_kernel'
    return 'gemm_mfma_kernel'


def cpu_baseline(spec, budget_s):
    """The oracle's torch restatement of the reference's PyTorch path, float32, on this host's cores."""
    from oracle import gridsample
    B, Q, H, D, C, levels, P, _, bias, loc_dist = spec
    args = workload(B, Q, H, D, C, levels, P, torch.float32, bias=bias, loc_dist=loc_dist)
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    with torch.inference_mode():
        for _ in range(3):
            gridsample.deform_attn(*args)
        best, calls, t0 = float('inf'), 0, time.perf_counter()
        while True:
            t = time.perf_counter()
            for _ in range(10):
                gridsample.deform_attn(*args)
            best = min(best, (time.perf_counter() - t) / 10)
            calls += 10
            if calls >= 70 and time.perf_counter() - t0 >= budget_s:
                break
            if time.perf_counter() - t0 >= 3 * budget_s:
                break
    cpu = platform.processor() or platform.machine()
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    cpu = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    return {'value': round(best * 1e6, 1), 'unit': 'µs per layer call', 'cores': threads, 'kind': 'port',
            'sample': f'float32 {B}x{Q} queries, same shapes and seed; best of {calls // 10} x 10 calls '
                      f'({time.perf_counter() - t0:.1f} s) on {cpu}'}


COPY_BYTES = 256 << 20  # plain copy used to scale FETCH_SIZE / WRITE_SIZE to bytes


def measured_traffic(workload_name, kernel):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, each scaled by the plain-copy calibration) from
    the rocprofv3 --pmc summary committed for this workload, or None when there is none."""
    path = os.path.join(ROOT, 'profiles', f'pmc_{workload_name}.json')
    try:
        with open(path) as f:
            k = json.load(f)['kernels'][kernel]
        return int(k['fetch_bytes'] + k['write_bytes'])
    except (OSError, KeyError, ValueError):
        return None


def head_major(dtype, D):
    """Whether td_project_forward projects into the head-major layout (a head row of 64 bytes or less, a multiple
    of 16), so that the kernel legs time the halves the project path runs."""
    row = D * torch.empty((), dtype=dtype).element_size()
    return dtype != torch.float64 and row <= 64 and row % 16 == 0


def project_halves(dev, H, D, dtype):
    """(projection, sampling) callables of the project path: the sampling one takes the projection's output."""
    if head_major(dtype, D):
        return (lambda: _native.value_proj_heads(dev[0], dev[1], dev[2], H),
                lambda v: _native.sample_forward_heads(v, *dev[3:]))
    return (lambda: _native.value_proj(dev[0], dev[1], dev[2]),
            lambda v: _native.sample_forward(v, H, *dev[3:]))


def gather_ceiling(row_bytes, buf_bytes, target_bytes=1 << 30):
    """GB/s at which all CUs together receive randomly chosen rows of `row_bytes` from a buffer of `buf_bytes`:
    td_probe_gather (the gather kernels' 16-byte buffer loads, 8 in flight per lane, row_bytes / 16 lanes per row)
    reading about `target_bytes` per launch, graph-timed like the operator; the best of four occupancies. With the
    memory tensor's size this is the ceiling of the fused kernel's gather phase, whose rows mostly sit in L2 (what
    L2 misses comes from the MALL or HBM, as in the kernel). Rows wider than the probe's widest (1024 bytes, e.g.
    C = 1024 in 16 bits) are probed as 1024-byte rows: the rate is flat from 256-byte rows up."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    row_bytes = min(row_bytes, 1024)
    buf = torch.zeros(max(buf_bytes // 16, row_bytes // 16), 4, dtype=torch.int32, device='cuda')
    best = None
    for waves, per_cu in ((4, 2), (8, 1), (8, 2), (4, 4)):
        wg = cus * per_cu
        sink = torch.zeros(wg, dtype=torch.int32, device='cuda')
        loads = max(8, target_bytes // (wg * waves * 64 * 16) // 8 * 8)
        nbytes = wg * waves * 64 * loads * 16
        t = graph_time_us(lambda: _native.probe_gather(buf, row_bytes, loads, wg, waves, sink), 10, 2)
        rate = nbytes / (t * 1e-6) / 1e9
        if best is None or rate > best['gbps']:
            best = {'gbps': round(rate, 1), 'row_bytes': row_bytes, 'buffer_bytes': buf.numel() * 4,
                    'workgroups': wg, 'waves': waves, 'loads_per_lane': loads, 'us': round(t, 2)}
    del buf
    return best


CEILING_ROWS = (64, 128, 256, 512, 1024)
CEILING_BUFFERS = (('2 MB', 2 << 20), ('RT-DETR 640 memory, fp16 B1 (4.3 MB)', 8400 * 256 * 2),
                   ('RT-DETR 640 memory, bf16 B8 (34.4 MB)', 8 * 8400 * 256 * 2),
                   ('DINO 4-level value, fp16 B4 (45.5 MB)', 4 * 22223 * 256 * 2), ('512 MB', 512 << 20))


def ceiling_table():
    """--ceiling: the gather ceiling for every row width and buffer size of CEILING_ROWS x CEILING_BUFFERS, as a
    markdown table on stdout and one JSON line."""
    rows = []
    log(f'{torch.cuda.get_device_name()} ({torch.cuda.get_device_properties(0).gcnArchName}), '
        f'{torch.cuda.get_device_properties(0).multi_processor_count} CUs')
    for name, nbytes in CEILING_BUFFERS:
        for rb in CEILING_ROWS:
            c = gather_ceiling(rb, nbytes)
            c['buffer'] = name
            rows.append(c)
            log(f'  {name:40s} rows of {rb:5d} B: {c["gbps"]:9.1f} GB/s ({c["workgroups"]} x {c["waves"]} waves)')
    print('| buffer | ' + ' | '.join(f'{r} B rows' for r in CEILING_ROWS) + ' |')
    print('|---|' + '---:|' * len(CEILING_ROWS))
    for name, _ in CEILING_BUFFERS:
        print(f'| {name} | ' + ' | '.join(f'{c["gbps"]:.0f}' for c in rows if c['buffer'] == name) + ' |')
    print(json.dumps({'gather_ceiling_gbps': rows}), flush=True)


ATOMIC_BUFFERS = (('RT-DETR 640 value gradient, B1 (8.6 MB)', 8400 * 256 * 4),
                  ('DINO 4-level value gradient, B4 (91 MB)', 4 * 22223 * 256 * 4))


def atomic_table():
    """--atomic-ceiling: the float-atomic probe (td_probe_atomic) with groups of 16, 32 and 64 lanes (chunks of 64,
    128 and 256 bytes), the chunks chosen at random or in sequence, over buffers the size of the value-gradient
    accumulators, graph-timed (best of 7 replays of 10 launches): lane-group adds and 128-byte lines per second, as a
    markdown table on stdout and one JSON line."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    log(f'{torch.cuda.get_device_name()} ({torch.cuda.get_device_properties(0).gcnArchName}), {cus} CUs')
    rows = []
    for name, nbytes in ATOMIC_BUFFERS:
        buf = torch.zeros(nbytes // 4, dtype=torch.float32, device='cuda')
        for lanes in (16, 32, 64):
            for random in (True, False):
                wg, per = cus * 8, 64
                adds = wg * (256 // lanes) * per
                t = graph_time_us(lambda: _native.probe_atomic(buf, lanes, per, wg, random), 10, 2)
                r = {'buffer': name, 'lanes': lanes, 'bytes': 4 * lanes, 'order': 'random' if random else 'sequential',
                     'g_adds_per_s': round(adds / t / 1e3, 2),
                     'g_lines_per_s': round(adds * lanes * 4 / 128 / t / 1e3, 2), 'us': round(t, 1)}
                rows.append(r)
                log(f'  {name:40s} {lanes:2d} lanes ({4 * lanes:3d} B) {r["order"]:10s}: {r["g_adds_per_s"]:6.2f} G '
                    f'adds/s, {r["g_lines_per_s"]:6.2f} G lines/s')
        del buf
    print('| buffer | lanes per add (bytes) | order | G adds/s | G 128-byte lines/s |')
    print('|---|---:|---|---:|---:|')
    for r in rows:
        print(f'| {r["buffer"]} | {r["lanes"]} ({r["bytes"]}) | {r["order"]} | {r["g_adds_per_s"]:.2f} | '
              f'{r["g_lines_per_s"]:.2f} |')
    print(json.dumps({'atomic_ceiling': rows}), flush=True)


def train_run(cpu_args, steps, warmup):
    """--train-run, for rocprofv3 --kernel-trace: `warmup`, then `steps` eager training steps of the operator
    (train_steps), then the same step graph-timed and, as in --trace-run, a graph of `steps` empty kernels, whose
    traced duration is the tracer's cost per dispatch."""
    ours, _ = train_steps(cpu_args)
    for _ in range(warmup):
        ours()
    torch.cuda.synchronize()
    for _ in range(steps):
        ours()
    torch.cuda.synchronize()
    t = graph_time_us(ours, steps, min(warmup, 10))
    with torch.inference_mode():
        empty = graph_time_us(lambda: _native.probe_empty(1), steps, min(warmup, 10))
    log(f'train run: {steps} eager steps traced; graph-timed {t:.2f} µs per step, empty kernel {empty:.2f} µs per '
        f'launch')
    print(json.dumps({'train_run': {'steps': steps, 'train_step_us': round(t, 3),
                                    'empty_us_per_launch': round(empty, 3)}}), flush=True)


def trace_run(dev, steps, warmup):
    """--trace-run, for rocprofv3 --kernel-trace: a graph of `steps` operator calls (mode auto) and a graph of
    `steps` launches of an empty kernel, each timed as the headline is (best of 7 replays). The empty kernel's
    traced duration is what the tracer reports for a dispatch with no work; the operator's traced duration less
    that is comparable with its graph-timed µs per call, which this run prints."""
    with torch.inference_mode():
        op = graph_time_us(lambda: td.ma_deform_attn(*dev), steps, warmup)
        empty = graph_time_us(lambda: _native.probe_empty(1), steps, warmup)
    log(f'trace run: operator {op:.2f} µs per call, empty kernel {empty:.2f} µs per launch ({steps}-call graphs)')
    print(json.dumps({'trace_run': {'steps': steps, 'operator_us_per_call': round(op, 3),
                                    'empty_us_per_launch': round(empty, 3)}}), flush=True)


# what the phase stamps of libtinydeform_phases.so mark (slot: point), in the order a wavefront passes them
PHASE_POINTS = [(11, 'kernel entry'), (0, 'rows decoded'), (1, 'corner table barrier passed'), (2, 'gather done'),
                (3, 'gather barrier passed'), (4, 'projection set up'), (5, 'projection job start'),
                (6, 'first W chunk done'), (7, 'MFMAs done'), (8, 'partial sums stored'),
                (9, 'projection barrier passed'), (10, 'outputs stored')]
# per-wavefront phases (from slot, to slot, name, which wavefronts: all / gatherers / jobs)
PHASE_SPANS = [(11, 0, 'entry to rows decoded (kernel arguments)', 'all'),
               (0, 1, 'corner table (locations, weights, corners; barrier)', 'all'),
               (1, 2, 'gather of the wavefront\'s rows', 'gatherers'),
               (2, 3, 'wait at the gather barrier', 'all'),
               (3, 5, 'projection set-up', 'jobs'),
               (5, 7, 'projection job (MFMAs)', 'jobs'),
               (7, 8, 'partial sums to LDS', 'jobs'),
               (8, 9, 'wait at the projection barrier', 'all'),
               (9, 10, 'epilogue (K slices summed, bias, stores)', 'all')]


def phases_run(dev, steps, warmup):
    """--phases: the fused kernel's timeline, from libtinydeform_phases.so (td_fused.hip built with
    TD_PHASE_STAMPS: every wavefront of the vector kernel reads the GPU's 100 MHz real-time counter at its phase
    boundaries; the first 1024 workgroups keep theirs). The operator is graph-timed like the headline with the plain
    library and with the instrumented one; the stamps are those of the last call of the last replay, a call that ran
    back to back with the one before it. Prints a markdown summary and one JSON line."""
    import ctypes
    import numpy as np
    path = os.path.join(os.path.dirname(_native.LIB_PATH), 'libtinydeform_phases.so')
    lib = _native.load(path)
    if lib is None:
        raise SystemExit(f'measurement build missing ({_native.load_error}): python -m marearts_tinydeform_amd._build')
    lib.td_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    lib.td_phase_stamps.restype = ctypes.c_int
    B, Q, H, L, P = dev[5].shape[:5]
    C, HD = dev[0].shape[2], dev[1].shape[0]
    plan = _native.fused_plan(dev[0].dtype, B, Q, dev[0].shape[1], C, H, HD // H, L, P)
    if plan[0] != 0:
        raise SystemExit(f'this workload launches the generic fused kernel, which has no stamps: plan {plan}')
    plain = _native.lib
    with torch.inference_mode():
        t_plain = graph_time_us(lambda: td.ma_deform_attn(*dev, mode='fused'), steps, warmup)
        _native.lib = lib
        try:
            t_inst = graph_time_us(lambda: td.ma_deform_attn(*dev, mode='fused'), steps, warmup)
            torch.cuda.synchronize()
            n = 1024 * 12 * 16
            buf = np.zeros(n, dtype=np.uint64)
            if lib.td_phase_stamps(buf.ctypes.data, n) != 0:
                raise SystemExit('td_phase_stamps failed')
        finally:
            _native.lib = plain
    wgs = min(plan[1], 1024)
    st = buf.reshape(1024, 12, 16)[:wgs].astype(np.int64)
    seen = st > 0
    t0 = st[:, :, 11][seen[:, :, 11]].min()
    rel = np.where(seen, (st - t0) * 10, -1)  # ns from the first wavefront's entry
    # the wavefronts that gather rows in every workgroup: the fewest rows a workgroup holds (a slice's, or a full
    # query tile's) times the lanes of a row (16-byte chunks times corner groups), in wavefronts
    rows_min = (B * Q) // plan[4] if plan[4] > 0 else plan[3]
    lanes = C * dev[0].element_size() // 16 * plan[6]
    gatherers = min(plan[2], -(-rows_min * lanes // 64))
    jobs = (rel[:, :, 5] >= 0).any(axis=0)  # the wavefronts that ran a projection job (those stamped at its start)

    def pct(x):
        x = np.asarray(x)
        return {'n': int(x.size), 'p0': float(np.min(x)), 'p50': float(np.median(x)),
                'p90': float(np.percentile(x, 90)), 'max': float(np.max(x))}

    points = []
    for slot, name in PHASE_POINTS:
        v = rel[:, :, slot]
        if (v >= 0).any():
            points.append((name, pct(v[v >= 0])))
    spans = []
    for a, b, name, who in PHASE_SPANS:
        waves = slice(0, gatherers) if who == 'gatherers' else jobs if who == 'jobs' else slice(None)
        x, y = rel[:, waves, a], rel[:, waves, b]
        ok = (x >= 0) & (y >= 0)
        if ok.any():
            spans.append((name, who, pct((y - x)[ok])))
    log(f'phases: {wgs} workgroups x {plan[2]} wavefronts; {t_plain:.2f} µs per call plain, {t_inst:.2f} '
        f'instrumented')
    shape = (f'{plan[4]} slices per head of {rows_min}-{plan[5]} rows' if plan[4] > 0 else
             f'query tiles of {plan[3]} rows')
    print(f'Graph-timed µs per call ({steps}-call graph): {t_plain:.2f} with libtinydeform.so, {t_inst:.2f} with '
          f'the instrumented build. Launch plan: {plan[1]} workgroups of {plan[2]} wavefronts, {shape}, '
          f'{plan[6]} corner groups per row, {plan[7]} loads in flight per lane.')
    print()
    print(f'Points, ns after the first wavefront entered the kernel (every wavefront of the first {wgs} workgroups):')
    print()
    print('| point | wavefronts | p0 | p50 | p90 | max |')
    print('|---|---:|---:|---:|---:|---:|')
    for name, q in points:
        print(f'| {name} | {q["n"]} | {q["p0"]:.0f} | {q["p50"]:.0f} | {q["p90"]:.0f} | {q["max"]:.0f} |')
    print()
    print(f'Phases, ns per wavefront ("gatherers": the first {gatherers} wavefronts, which gather rows in every '
          f'workgroup; "jobs": the wavefronts that ran a projection job; stamped in the first {wgs} workgroups):')
    print()
    print('| phase | wavefronts | n | p0 | p50 | p90 | max |')
    print('|---|---|---:|---:|---:|---:|---:|')
    for name, who, q in spans:
        print(f'| {name} | {who} | {q["n"]} | {q["p0"]:.0f} | {q["p50"]:.0f} | {q["p90"]:.0f} | {q["max"]:.0f} |')
    print(json.dumps({'phases': {'us_per_call': round(t_plain, 3), 'us_per_call_instrumented': round(t_inst, 3),
                                 'plan': list(plan), 'points_ns': dict(points),
                                 'spans_ns': {name: q for name, _, q in spans}}}), flush=True)


def pmc_run(dev, H, steps):
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device='cuda')
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    with torch.inference_mode():
        for _ in range(steps):
            td.ma_deform_attn(*dev, mode='fused')
        torch.cuda.synchronize()
        proj, smp = project_halves(dev, H, dev[1].size(0) // H, dev[0].dtype)
        for _ in range(steps):
            value = proj()
        torch.cuda.synchronize()
        for _ in range(steps):
            smp(value)
        torch.cuda.synchronize()
    log(f'pmc run done: copy of {COPY_BYTES} bytes, {steps} calls of fused / value_proj / sample')


def auto_grid():
    """The shapes the auto selector is fitted on:
      * RT-DETR 640 (the reference's bench grid: 3 dtypes x batch 1/4/8 x 50..900 queries; batch 2 in 16 bits), a
        C = 512 model (batch 1/2/4), DINO 4-level and the C = 1024 / 64-sample limit shape;
      * RT-DETR 640 at 150/450/750 queries and batch 2/3/6 in all three dtypes, uniform and clustered locations;
        C = 512 at those query counts; a five-level map; C = 768 (12 heads of 64);
      * other widths and level layouts: C = 128 (4 heads of 32), C = 320 (10 heads of 32: rows under a wavefront),
        C = 896 (14 heads of 64), one and two levels with 8 and 16 points, in 16 bits and float32; C = 448, 576 and
        704 on DINO 4-level and five-level maps in 16 bits."""
    five = [(100, 100), (50, 50), (25, 25), (13, 13), (7, 7)]
    cases = []
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        for B in (1, 4, 8):
            for Q in (50, 100, 200, 300, 600, 900):
                cases.append(('rtdetr640', B, Q, 8, 32, 256, RTDETR_LEVELS, 4, dt, True, 'uniform'))
        for B in (2, 3, 6):
            for Q in (150, 450, 750):
                for ld in ('uniform', 'clustered'):
                    cases.append(('rtdetr640', B, Q, 8, 32, 256, RTDETR_LEVELS, 4, dt, True, ld))
    for dt in (torch.float16, torch.bfloat16):
        for Q in (100, 300, 600, 900):
            cases.append(('rtdetr640', 2, Q, 8, 32, 256, RTDETR_LEVELS, 4, dt, True, 'uniform'))
        for B in (1, 2, 4):
            for Q in (100, 300, 600, 900):
                cases.append(('c512', B, Q, 8, 64, 512, RTDETR_LEVELS, 4, dt, True, 'uniform'))
        for B in (1, 2, 3, 6):
            for Q in (150, 450, 750):
                cases.append(('c512', B, Q, 8, 64, 512, RTDETR_LEVELS, 4, dt, True, 'uniform'))
        for B, Q in ((1, 300), (4, 300), (4, 900), (8, 900)):
            cases.append(('dino4l', B, Q, 8, 32, 256, DINO_LEVELS, 4, dt, True, 'outside10'))
        for B in (1, 2, 5):
            for Q in (150, 450, 750):
                cases.append(('c768', B, Q, 12, 64, 768, RTDETR_LEVELS, 4, dt, True, 'uniform'))
    for dt in (torch.float32, torch.float16):
        for B in (1, 3):
            for Q in (150, 450, 750):
                cases.append(('five-level', B, Q, 8, 32, 256, five, 4, dt, True, 'uniform'))
    for Q in (50, 300, 900):
        for B in (1, 2):
            cases.append(('limit', B, Q, 16, 64, 1024, LIMIT_LEVELS, 16, torch.bfloat16, False, 'uniform'))
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        for B, Q in ((1, 100), (1, 600), (2, 300), (4, 300), (8, 600)):
            cases.append(('c128', B, Q, 4, 32, 128, RTDETR_LEVELS, 4, dt, True, 'uniform'))
            cases.append(('c320', B, Q, 10, 32, 320, RTDETR_LEVELS, 4, dt, True, 'uniform'))
            cases.append(('one-level-p16', B, Q, 8, 32, 256, [(60, 80)], 16, dt, True, 'uniform'))
            cases.append(('two-level-p8', B, Q, 8, 32, 256, [(64, 64), (32, 32)], 8, dt, True, 'uniform'))
        for B, Q in ((1, 300), (2, 300), (3, 600)):
            cases.append(('c896', B, Q, 14, 64, 896, RTDETR_LEVELS, 4, dt, True, 'uniform'))
    for dt in (torch.float16, torch.bfloat16):
        for C, H, D in ((448, 14, 32), (576, 9, 64), (704, 11, 64)):
            for levels, lname in ((DINO_LEVELS, 'dino4l'), (five, 'five-level')):
                for B, Q in ((1, 200), (2, 400), (4, 800), (6, 200)):
                    cases.append((f'{lname} c{C}', B, Q, H, D, C, levels, 4, dt, True, 'uniform'))
    return cases


cost_features = td.cost_features


def measure_grid(cases):
    """Graph-timed µs of both modes for every case, with the mode the current table picks."""
    rows = []
    with torch.inference_mode():
        for name, B, Q, H, D, C, levels, P, dt, bias, ld in cases:
            dev = [None if t is None else t.cuda() for t in workload(B, Q, H, D, C, levels, P, dt, bias=bias,
                                                                      loc_dist=ld)]
            N, L = dev[0].shape[1], len(levels)
            steps = 100 if B * Q * C < 2_000_000 else 20
            t = {m: graph_time_us(lambda m=m: td.ma_deform_attn(*dev, mode=m), steps, 5) for m in ('fused', 'project')}
            # the project path's halves on their own (the kernels td_project_forward runs)
            proj, smp = project_halves(dev, H, D, dt)
            value = proj()
            t['gemm'] = graph_time_us(proj, steps, 5)
            t['sample'] = graph_time_us(lambda: smp(value), steps, 5)
            del value
            cur = td.choose_mode(dev[0], dev[1], dev[5])
            best = min(t['fused'], t['project'])
            rows.append(dict(case=name, dtype=DTYPE_NAMES[dt], B=B, Q=Q, H=H, D=D, C=C, N=N, L=L, P=P, loc=ld,
                             s=dev[0].element_size(), fused=t['fused'], project=t['project'], gemm=t['gemm'],
                             sample=t['sample'], current_pick=cur, current_loss=round(t[cur] / best, 3)))
            log(f'{name:9s} {DTYPE_NAMES[dt]:4s} B={B} Q={Q:3d} {ld:9s} fused {t["fused"]:8.2f} project '
                f'{t["project"]:8.2f} (gemm {t["gemm"]:7.2f}, sample {t["sample"]:7.2f}) auto picks {cur} '
                f'({t[cur] / best:.3f} of the faster)')
            del dev
            torch.cuda.empty_cache()
    return rows


def holdout_grid():
    """Shapes the auto selector is not fitted on: 250/500/1000 queries, batch 5 and 7, widths 384 (12 heads of 32)
    and 640 (10 heads of 64), four- and five-level maps, uniform and clustered locations, in float16 and bfloat16."""
    four = [(100, 167), (50, 84), (25, 42), (13, 21)]
    five = [(100, 100), (50, 50), (25, 25), (13, 13), (7, 7)]
    cases = []
    for dt in (torch.float16, torch.bfloat16):
        for C, H, D in ((384, 12, 32), (640, 10, 64)):
            for levels, lname in ((four, 'four-level'), (five, 'five-level')):
                for B in (5, 7):
                    for Q in (250, 500, 1000):
                        for ld in ('uniform', 'clustered'):
                            cases.append((f'{lname} c{C}', B, Q, H, D, C, levels, 4, dt, True, ld))
    return cases


def holdout(out_path):
    """Measure both modes over holdout_grid() and report how far the current selector's pick is from the faster
    mode in each case (no refit)."""
    rows = measure_grid(holdout_grid())
    worst = max(r['current_loss'] for r in rows)
    within = sum(r['current_loss'] <= 1.10 for r in rows)
    right = sum(r['current_loss'] <= 1.0 for r in rows)
    log(f'held-out grid: {len(rows)} cases, auto picked the faster mode in {right}, within 10% in {within}; '
        f'worst auto/best {worst:.3f}')
    with open(out_path, 'w') as f:
        json.dump({'rows': rows, 'worst_current': worst, 'current_within_10pct': within, 'faster_picked': right,
                   'cases': len(rows)}, f, indent=1)


def fit_table(rows):
    """FUSED_LIMIT's per-dtype cost lines from measured rows: the fused, GEMM and sampler terms of cost_features each
    fitted to their kernel's time by non-negative least squares on relative error, then project mode's gap (what the
    pair costs beyond its two kernels timed apart: the hand-over, and the sampler reading values the GEMM has just
    written rather than a warm copy) over gap_features, by the same method against the measured project time. One
    table for float32, one shared by float16 and bfloat16."""
    import numpy as np
    from scipy.optimize import nnls
    table = {}
    for fam in (('f32',), ('f16', 'bf16')):
        xs = [r for r in rows if r['dtype'] in fam]
        if not xs:
            continue
        feats = [cost_features(r['B'], r['Q'], r['H'], r['D'], r['C'], r['N'], r['L'], r['P'], r['s']) for r in xs]
        coef = {}
        for i, key in enumerate(('fused', 'gemm', 'sample')):
            F = np.array([f[i] for f in feats])
            t = np.array([r[key] for r in xs])
            coef[key], _ = nnls(F / t[:, None], np.ones(len(xs)))
        pred = np.array([np.dot(coef['gemm'], f[1]) + np.dot(coef['sample'], f[2]) for f in feats])
        tp = np.array([r['project'] for r in xs])
        G = np.array([td.gap_features(r['B'], r['Q'], r['N'], r['H'], r['D'], r['L'], r['P'], r['s']) for r in xs])
        gap, _ = nnls(G / tp[:, None], 1.0 - pred / tp)
        entry = {k: [round(float(c), 4) for c in v] for k, v in coef.items()}
        entry['gap'] = [round(float(c), 4) for c in gap]
        for fd in fam:
            table[fd] = entry
    return table


def score(rows, table):
    """Each row's pick under `table` and its loss (time of the pick / time of the faster mode)."""
    def dot(c, x):
        return sum(a * b for a, b in zip(c, x))
    for r in rows:
        coef = table[r['dtype']]
        ff, fg, fs = cost_features(r['B'], r['Q'], r['H'], r['D'], r['C'], r['N'], r['L'], r['P'], r['s'])
        pf = dot(coef['fused'], ff)
        pp = dot(coef['gemm'], fg) + dot(coef['sample'], fs) + dot(
            coef['gap'], td.gap_features(r['B'], r['Q'], r['N'], r['H'], r['D'], r['L'], r['P'], r['s']))
        r['fitted_pick'] = 'fused' if pf <= pp else 'project'
        r['fitted_loss'] = round(r[r['fitted_pick']] / min(r['fused'], r['project']), 3)
        r['predicted'] = {'fused': round(pf, 2), 'project': round(pp, 2)}
    return rows


def fit_auto(out_path):
    """Measure both modes and the project path's two kernels over auto_grid(), fit the cost lines (fit_table), and
    report every case's loss under the fitted and the current selector."""
    rows = measure_grid(auto_grid())
    table = fit_table(rows)
    score(rows, table)
    worst_fit = max(r['fitted_loss'] for r in rows)
    worst_cur = max(r['current_loss'] for r in rows)
    within = sum(r['fitted_loss'] <= 1.10 for r in rows)
    log(f'fitted table: {json.dumps(table)}')
    log(f'worst auto/best ratio: fitted {worst_fit:.3f} ({within}/{len(rows)} within 10%), current table '
        f'{worst_cur:.3f}')
    with open(out_path, 'w') as f:
        json.dump({'table': table, 'rows': rows, 'worst_fitted': worst_fit, 'worst_current': worst_cur,
                   'fitted_within_10pct': within, 'cases': len(rows)}, f, indent=1)


def table(args):
    """The reference's benchmark table (bench/bench.py:64-121): for every dtype, batch and query count, the PyTorch
    path (F.linear + grid_sample), fused, project and auto, graph-timed µs, with the largest difference of fused and
    project from the PyTorch path. Inputs as the reference's (clustered locations: a centre per query plus 0.05
    randn), generated here on the CPU from a fixed seed. The reference's 'official' column (the Deformable-DETR CUDA
    extension) has no counterpart on this GPU and is left out."""
    levels = [tuple(int(v) for v in s.split('x')) for s in args.levels.split(',')]
    C, H, P = args.channels, args.heads, args.points
    D = C // H
    N = sum(h * w for h, w in levels)
    print(f'{torch.cuda.get_device_name()} ({torch.cuda.get_device_properties(0).gcnArchName}), torch '
          f'{torch.__version__}, tokens {N}, C {C}, heads {H}, levels {len(levels)}, points {P}')
    print('| dtype | batch | queries | pytorch | fused | project | auto (picks) | auto vs pytorch | '
          'max abs diff vs pytorch |')
    print('|---|---:|---:|---:|---:|---:|---:|---:|---:|')
    for name in args.dtype:
        dtype = getattr(torch, name)
        for B in args.batch:
            for Q in args.queries:
                cpu = workload(B, Q, H, D, C, levels, P, dtype, loc_dist='clustered')
                a = [None if t is None else t.cuda() for t in cpu]
                a_ref = a[:3] + [cpu[3], cpu[4]] + a[5:]  # the PyTorch path reads the level sizes on the host
                with torch.inference_mode():
                    ref = td.ma_deform_attn_reference(*a_ref).float()
                    diff = max((td.ma_deform_attn(*a, mode=m).float() - ref).abs().max().item()
                               for m in ('fused', 'project'))
                    t_ref = graph_time_us(lambda: td.ma_deform_attn_reference(*a_ref), 100, 3)
                    t_fus = graph_time_us(lambda: td.ma_deform_attn(*a, mode='fused'), 100, 3)
                    t_prj = graph_time_us(lambda: td.ma_deform_attn(*a, mode='project'), 100, 3)
                pick = td.choose_mode(a[0], a[1], a[5])
                t_auto = t_fus if pick == 'fused' else t_prj
                print(f'| {name} | {B} | {Q} | {t_ref:.1f} | {t_fus:.1f} | {t_prj:.1f} | {t_auto:.1f} ({pick}) | '
                      f'{t_ref / t_auto:.1f}x | {diff:.1e} |', flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=1000)
    ap.add_argument('--warmup', type=int, default=50)
    ap.add_argument('--workload', default='rtdetr640-fp16-b1-q300', choices=sorted(WORKLOADS))
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--cpu-seconds', type=float, default=10.0)
    ap.add_argument('--modes-only', action='store_true', help='time the modes, skip per-kernel legs')
    ap.add_argument('--fit-auto', metavar='OUT.json', default=None,
                    help='time fused and project over the auto grid, fit the per-dtype cost model of '
                         'marearts_tinydeform_amd.FUSED_LIMIT and report how far auto is from the faster mode')
    ap.add_argument('--holdout', metavar='OUT.json', default=None,
                    help='time fused and project over shapes the selector was not fitted on and report how far '
                         'auto is from the faster mode in each')
    ap.add_argument('--table', action='store_true',
                    help="the reference's sweep (its bench/bench.py): PyTorch path, fused, project and auto per dtype, "
                         'batch and query count, as a markdown table on stdout')
    ap.add_argument('--queries', type=int, nargs='+', default=[50, 100, 300], help='--table: query counts')
    ap.add_argument('--batch', type=int, nargs='+', default=[1, 4], help='--table: batch sizes')
    ap.add_argument('--dtype', nargs='+', default=['float32', 'float16'], help='--table: dtypes')
    ap.add_argument('--levels', default='80x80,40x40,20x20', help='--table: level sizes HxW')
    ap.add_argument('--channels', type=int, default=256, help='--table: C')
    ap.add_argument('--heads', type=int, default=8, help='--table: H')
    ap.add_argument('--points', type=int, default=4, help='--table: P')
    ap.add_argument('--ceiling', action='store_true',
                    help='the gather ceiling (td_probe_gather) for row widths 64..1024 bytes and buffers from 2 MB '
                         'to 512 MB, as a markdown table')
    ap.add_argument('--atomic-ceiling', action='store_true',
                    help='the float-atomic probe (td_probe_atomic): adds of 64-, 128- and 256-byte chunks, random or '
                         'in sequence, over value-gradient-sized buffers, as a markdown table')
    ap.add_argument('--trace-run', action='store_true',
                    help='for rocprofv3 --kernel-trace: --steps operator calls and --steps empty kernels, each in '
                         'a graph timed like the headline')
    ap.add_argument('--train-run', action='store_true',
                    help='for rocprofv3 --kernel-trace: --steps eager training steps of the operator (forward and '
                         'backward), then the same step graph-timed')
    ap.add_argument('--phases', action='store_true',
                    help='the fused kernel\'s phase timeline from the measurement build libtinydeform_phases.so')
    ap.add_argument('--pmc-run', action='store_true',
                    help='for rocprofv3 --pmc: one plain copy of COPY_BYTES (the counter calibration), then '
                         '--steps eager calls of the fused kernel, the value projection and the sampling kernel')
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU: this operator has no multi-GPU path to time (every (batch, query, head) '
              'row is independent; sharding is data parallel with no exchange). Run with --gpus 1.', file=sys.stderr)
        sys.exit(2)
    if _native.lib is None:
        raise SystemExit(f'HIP extension missing: {_native.load_error}')
    assert torch.cuda.is_available(), 'no HIP device'
    if args.fit_auto:
        fit_auto(args.fit_auto)
        return
    if args.holdout:
        holdout(args.holdout)
        return
    if args.table:
        table(args)
        return
    if args.ceiling:
        ceiling_table()
        return
    if args.atomic_ceiling:
        atomic_table()
        return

    spec = WORKLOADS[args.workload]
    B, Q, H, D, C, levels, P, dtype, bias, loc_dist = spec
    cpu_args = workload(B, Q, H, D, C, levels, P, dtype, bias=bias, loc_dist=loc_dist)
    dev = [None if t is None else t.cuda() for t in cpu_args]
    N, L = dev[0].shape[1], len(levels)
    s = dev[0].element_size()
    alg = algorithmic(B, Q, H, D, C, N, L, P, s)
    torch.backends.cuda.matmul.allow_tf32 = False
    log(f'{torch.cuda.get_device_name()} ({torch.cuda.get_device_properties(0).gcnArchName}), torch '
        f'{torch.__version__}, workload {args.workload}: B={B} Q={Q} N={N} C={C} H={H} D={D} L={L} P={P}')

    if args.pmc_run:
        pmc_run(dev, H, args.steps)
        return
    if args.trace_run:
        trace_run(dev, args.steps, args.warmup)
        return
    if args.train_run:
        train_run(cpu_args, args.steps, args.warmup)
        return
    if args.phases:
        phases_run(dev, args.steps, args.warmup)
        return

    pick = td.choose_mode(dev[0], dev[1], dev[5])
    times = {}
    with torch.inference_mode():
        for mode in ('fused', 'project'):
            times[mode] = graph_time_us(lambda m=mode: td.ma_deform_attn(*dev, mode=m), args.steps, args.warmup)
            log(f'  {mode:8s} {times[mode]:9.2f} µs/call')
        times['auto'] = graph_time_us(lambda: td.ma_deform_attn(*dev), args.steps, args.warmup)
        log(f'  auto     {times["auto"]:9.2f} µs/call (picks {pick})')
        kern = {}
        if not args.modes_only:
            # the two halves td_project_forward runs (head-major value when a head row is 64 bytes or less)
            proj, smp = project_halves(dev, H, D, dtype)
            value = proj()
            kern['value_proj'] = graph_time_us(proj, args.steps, args.warmup)
            kern['sample'] = graph_time_us(lambda: smp(value), args.steps, args.warmup)
            kern['fused'] = times['fused']
            log(f'  kernels: value_proj {kern["value_proj"]:.2f} µs, sample {kern["sample"]:.2f} µs')
            # the standard PyTorch path (F.linear + per-level grid_sample) on the same device, same graph timing;
            # it reads the level shapes on the host, so they stay in host memory (no sync inside the graph)
            ref_args = dev[:3] + [cpu_args[3], cpu_args[4]] + dev[5:]
            kern['pytorch_reference'] = graph_time_us(lambda: td.ma_deform_attn_reference(*ref_args),
                                                      min(args.steps, 200), min(args.warmup, 10))
            log(f'  PyTorch reference path on the GPU: {kern["pytorch_reference"]:.2f} µs/call')
            lay = layer_times(B, Q, H, D, C, levels, P, dtype, args.steps, args.warmup)
            log('  decoder layer (prologue + value_proj + MSDeformAttn + output_proj): ' +
                ', '.join(f'{k[6:]} {v:.2f}' for k, v in lay.items()) + ' µs/call')
            kern.update(lay)
            with torch.inference_mode(False), torch.enable_grad():
                tr = train_times(cpu_args, min(args.steps, 200), args.warmup)
            log(f'  training step (forward + backward): {tr["train_step"]:.2f} µs, PyTorch reference path '
                f'{tr["pytorch_train_step"]:.2f} µs')
            kern.update(tr)

    # Roofline of the dominant kernel. The gather kernels read rows that mostly sit in L2, so their bound is the rate
    # at which the CUs receive such rows from L2 ("l2-gather"), measured here, on this device, by td_probe_gather with
    # the kernel's row width over an L2-resident buffer (the gathered tensor, or one XCD's 4 MB of it when larger: the
    # kernels deal each XCD a contiguous share of the work, whose rows it keeps in its own L2, so the probe's random
    # rows over a whole large tensor would understate what the kernels reach). The HBM figures (counter-measured bytes
    # over the same time, and the algorithmic bytes against 8 TB/s) stand beside it.
    ceiling = None
    if pick == 'fused':
        t = times['fused']
        ceiling = gather_ceiling(C * s, min(B * N * C * s, td.L2_BYTES))
        roof = {'kernel': 'fused_vec_kernel', 'bound': 'l2-gather', 'achieved': alg['fused_bytes'] / (t * 1e-6) / 1e9,
                'peak': ceiling['gbps'], 'unit': 'GB/s'}
    else:
        t_gemm, t_smp = kern.get('value_proj', times['project']), kern.get('sample', 0.0)
        gk = gemm_kernel(B * N, C, H * D, s)
        if t_gemm >= t_smp:
            t = t_gemm
            flops = alg['gemm_flops']
            if dtype in (torch.float16, torch.bfloat16) and flops / alg['gemm_bytes'] > MFMA_PEAK_16 / HBM_PEAK:
                roof = {'kernel': gk, 'bound': 'mfma', 'achieved': flops / (t_gemm * 1e-6) / 1e12,
                        'peak': 2500.0, 'unit': 'TFLOP/s'}
            else:
                roof = {'kernel': gk, 'bound': 'hbm',
                        'achieved': alg['gemm_bytes'] / (t_gemm * 1e-6) / 1e9, 'peak': 8000.0, 'unit': 'GB/s'}
        else:
            t = t_smp
            # with the head-major value the two corners (x0, x0 + 1) of a row are one 2 D-wide run
            ceiling = gather_ceiling((2 if head_major(dtype, D) else 1) * D * s, min(B * N * H * D * s, td.L2_BYTES))
            roof = {'kernel': 'sample_kernel', 'bound': 'l2-gather',
                    'achieved': alg['sample_bytes'] / (t_smp * 1e-6) / 1e9, 'peak': ceiling['gbps'], 'unit': 'GB/s'}
    roof['achieved'] = round(roof['achieved'], 1)
    roof['frac'] = round(roof['achieved'] / roof['peak'], 4)
    roof['traffic'] = measured_traffic(args.workload, roof['kernel'])
    if ceiling is not None:
        roof['ceiling_probe'] = ceiling
        roof['hbm'] = {'achieved': None if roof['traffic'] is None else round(roof['traffic'] / (t * 1e-6) / 1e9, 1),
                       'peak': 8000.0, 'unit': 'GB/s', 'what': 'counter-measured HBM bytes per launch / time'}
        if roof['hbm']['achieved'] is not None:
            roof['hbm']['frac'] = round(roof['hbm']['achieved'] / 8000.0, 4)
        roof['algorithmic_vs_hbm_peak'] = round(roof['achieved'] / 8000.0, 4)

    path_bytes = alg['fused_bytes'] if pick == 'fused' else alg['gemm_bytes'] + alg['sample_bytes']
    # HBM rate from the counters: the bytes the path's kernels moved to and from the memory fabric per launch
    # (committed rocprofv3 --pmc summary of this workload) over the measured time per call
    if pick == 'fused':
        traffic = measured_traffic(args.workload, roof['kernel'])
    else:
        parts = [measured_traffic(args.workload, k) for k in (gemm_kernel(B * N, C, H * D, s), 'sample_kernel')]
        traffic = None if None in parts else sum(parts)
    result = {
        'metric': ('µs per layer call (value_proj+MSDeformAttn) RT-DETR-640 fp16 B=1 Q=300; HBM GB/s'
                   if args.workload == 'rtdetr640-fp16-b1-q300'
                   else f'µs per layer call (value_proj+MSDeformAttn) {args.workload}; HBM GB/s'),
        'value': round(times['auto'], 2),
        'unit': 'µs',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(times['auto'] / 1e3, 5),
        'higher_is_better': False,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': DTYPE_NAMES[dtype],
        'data': f'synthetic (seeded CPU generator; locations {loc_dist})',
        'config': {'workload': args.workload, 'B': B, 'Q': Q, 'N': N, 'C': C, 'H': H, 'D': D, 'L': L, 'P': P,
                   'mode': 'auto'},
        'modes_us': {k: round(v, 2) for k, v in times.items()},
        'timing': f'best of 7 replays of a {args.steps}-call graph; each replay also carries 10-17 µs of fixed '
                  f'cost (graph launch and the two timing events), up to {17.0 / args.steps:.2f} µs per call here',
        'auto_pick': pick,
        'kernels_us': {k: round(v, 2) for k, v in kern.items()},
        'queries_per_s': round(B * Q / (times['auto'] * 1e-6)),
        'effective_gbps': round(path_bytes / (times['auto'] * 1e-6) / 1e9, 1),
        'hbm_gbps': None if traffic is None else round(traffic / (times['auto'] * 1e-6) / 1e9, 1),
        'roofline': roof,
    }
    if not args.no_cpu:
        log('CPU baseline ...')
        result['cpu_baseline'] = cpu_baseline(spec, args.cpu_seconds)
        log(f'  cpu {result["cpu_baseline"]["value"]} µs/call on {result["cpu_baseline"]["cores"]} threads')
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
