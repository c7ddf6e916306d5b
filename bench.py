"""Benchmark of the BDM routed-memory hot path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

Workload ("C2"): BSDM layer geometry d_model=1024, H=8,
J=256 banks (16x16 product key), S=8 rows per bank, B=8 read and 8 write
banks, v=128 per head, batch 8, T=4096 -> 32,768 tokens.  Weights are the
seeded random init of ``BankedDeltaMemory``, x ~ N(0,1) (synthetic data).
Controllers and router scores are computed once before the timed region; a
timed step is one prefill pass of the hot path over the batch:

    router (write and read roles) and dispatch in one call -> recurrence + ordered read
    combine, final bank state written (BF16 cache), FP32 recurrence math on a
    state rounded to BF16 every 16 packed events (the reference module
    forward's policy at this geometry)

``value`` is tokens/s of that step with every input already in HBM.  Extra
fields report the full-layer prefill (controller GEMMs and output interface
included), the C3 decode step (batch 64 against a resident BF16 state of
[64, 256, 8, 8, 128]) and an HBM copy probe.

roofline: the dominant launch is ``bdm_forward`` (recurrence + ordered
combine).  Its algorithmic bytes per token are the bytes it must move once:
q,k,b (3*H*S*2), g (H*S*4), v,w (2*V*2), route weights ww,rw ((KW+KR)*2),
read indices (KR*8), packed order ((KW+KR)*8), y (V*2) and the final state
(J*H*S*v*2 per sequence, spread over its T tokens), plus the shared initial
state once per launch.  ``achieved`` divides them by the launch's average
duration, measured with events on the stream the kernels run on.

cpu_baseline: the CPU oracle's port of the reference ``backend='reference'``
forward (per-event loop + index_add_, oracle/bdm_oracle.py) at C1 (BASELINE
batch 1, T 512, d_model 512, H4, v64, J256, FP32), 1 warmup + 5
timed runs, median, on the host's cores (at most 16, one GPU's share); the
HIP module forward at C1 is timed in the same run (``c1_forward``).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
# The reference module forward at the C2 geometry (H = 8) runs bank_training
# per head with training_state_dtype='bfloat16' (heads.py:40-46), which rounds
# the FP32 state to BF16 every 16 packed events (role_bank_kernel.py:153-165);
# the FP32-state prefill policy exists in the reference for H = 1 only.
ROUND_INTERVAL = 16
# GPU clocks ramp up over the first tens of milliseconds of load: on a device
# that was idle, 20 timed C2 steps after 3 warmup steps read ~0.47 ms per step
# where 50 read ~0.435 ms (the same build and box).  Before its warmup steps
# the hot path runs for this much wall time (counted from the end of a first
# batch of 8 steps, which takes the process's one-time costs: on a fresh
# process the first steps are host-bound), so that the timed steps measure the
# steady state; the line reports it as device_warmup.
DEVICE_WARMUP_S = 0.15
TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'forward_c2_traffic.json')


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--batch', type=int, default=8)
    ap.add_argument('--time', type=int, default=4096)
    ap.add_argument('--decode-steps', type=int, default=256)
    ap.add_argument('--no-cpu-baseline', dest='cpu_baseline', action='store_false',
                    help='skip the CPU baseline (the reference CPU path at C1, ~10 s)')
    ap.add_argument('--no-extras', action='store_true', help='skip the full-layer and decode measurements')
    ap.add_argument('--only', choices=('c2-forward', 'c3', 'c3-kernel', 'c4', 'c4-module', 'c5', 'prefill', 'lm',
                                       'lm-prefill', 'lm-train'),
                    help='run one named workload alone (C3 decode, C4 skewed forward, C5 training, C2 full-layer '
                         'prefill, whole-model prefill and decode) and print its figures as one JSON line; used to '
                         'profile a workload on its own')
    ap.add_argument('--c3-routes', choices=('init', 'independent'), default='independent',
                    help='--only c3-kernel: the route case of the kernel-only decode leg (for profilers)')
    ap.add_argument('--lm-context', type=int, default=8192,
                    help='prompt length T (= memory rows N) of the whole-model L16/D2048 measurement')
    ap.add_argument('--lm-gemm-tuning', choices=('on', 'off'), default='on',
                    help='whole-model inference: pick GEMM solutions with PyTorch TunableOp (on) or take the '
                         "library's heuristic choice (off, e.g. under a profiler)")
    return ap.parse_args()


def c2_config():
    from bdm_amd import BSDMConfig
    return BSDMConfig(dim=1024, bank_count=256, bank_size=8, selected_banks=8, value_width=1024, num_heads=8)


def make_inputs(layer, batch, time_, device, seed=0):
    import torch
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, time_, layer.hidden_size, generator=gen).to(torch.bfloat16).to(device)
    with torch.no_grad():
        q, k, v, g, b, w = layer._controllers(x)
        read_scores, write_scores = layer._route_projections(x)
        initial = layer._state_heads(layer.materialize_initial_state()).contiguous()
    return x, (q, k, v, g, b, w), (read_scores, write_scores), initial


def forward_algorithmic_bytes(cfg, batch, time_, initial_bytes):
    """Bytes one bdm_forward launch must move once (module docstring)."""
    h, s, j, kk = cfg.num_heads, cfg.bank_size, cfg.bank_count, cfg.selected_banks
    v_total = cfg.value_width
    per_token = (3 * h * s * 2 + h * s * 4 + 2 * v_total * 2 + 2 * kk * 2 + kk * 8 + 2 * kk * 8 + v_total * 2)
    final = batch * j * h * s * (v_total // h) * 2
    return per_token * batch * time_ + final + initial_bytes


def hot_path_algorithmic_bytes(cfg, batch, time_):
    """Hot path from router scores and controllers to y, final state written:
    2*(J1+J2)*2 + 3*H*S*2 + H*S*4 + 2*V*2 + V*2 per token + J*H*S*v*2 per
    sequence (7,936 B/token at C2)."""
    from bdm_amd.config import near_square_factors
    j1, j2 = near_square_factors(cfg.bank_count)
    h, s, v_total = cfg.num_heads, cfg.bank_size, cfg.value_width
    per_token = 2 * (j1 + j2) * 2 + 3 * h * s * 2 + h * s * 4 + 2 * v_total * 2 + v_total * 2
    return per_token * batch * time_ + batch * cfg.bank_count * h * s * (v_total // h) * 2


VALU_FP32_TFLOPS = 78.6   # MI355X FP32 vector peak without packed-FP32 instructions (disabled in this build)
MFMA_FP32_TFLOPS = 157.3  # MI355X FP32 matrix peak
MFMA_BF16_TFLOPS = 2500.0  # MI355X BF16 matrix peak, dense


def recurrence_flop(cfg, batch, time_):
    """Algorithmic FLOPs of the sequential recurrence: 5*S*v per write and
    2*S*v per read, per head (458,752 per token at C2)."""
    s, v, h, k = cfg.bank_size, cfg.head_value_width, cfg.num_heads, cfg.selected_banks
    return batch * time_ * h * k * (5 * s * v + 2 * s * v)


def recurrence_roofline(cfg, batch, time_, ms):
    """The recurrence kernels, timed with events bdm_forward records around
    them: algorithmic FLOPs against the compute peaks.  The default kernel runs
    on the vector ALUs (no MFMA: BDM_FORWARD_KERNEL=mfma selects the
    matrix-core variant)."""
    flop = recurrence_flop(cfg, batch, time_)
    tflops = flop / (ms * 1e-3) / 1e12
    kernel = os.environ.get('BDM_FORWARD_KERNEL', 'vector')
    return {'kernel': 'chunk_forward_kernel (MFMA)' if kernel == 'mfma' else 'lazy_forward_kernel (vector ALU)',
            'ms': round(ms, 4), 'flop': flop, 'achieved_tflops': round(tflops, 2),
            'bound': 'mfma' if kernel == 'mfma' else 'valu',
            'valu_fp32_peak_tflops': VALU_FP32_TFLOPS, 'frac_valu_fp32': round(tflops / VALU_FP32_TFLOPS, 4),
            'mfma_fp32_peak_tflops': MFMA_FP32_TFLOPS, 'frac_mfma_fp32': round(tflops / MFMA_FP32_TFLOPS, 4),
            'mfma_utilisation': None if kernel == 'mfma' else 0.0,
            'fma_floor': fma_floor(cfg, batch, time_, ms),
            'note': 'FLOPs of the sequential form (5Sv per write, 2Sv per read, per head); the vector kernel '
                    'issues 2 FMAs per state element per write, 1 per read (lazy decay)'}


# MI355X: 256 CUs, 64 non-packed FP32 FMA lanes per CU per clock; 2.4 GHz is
# the clock of the 78.6 TFLOP/s figure, and PROFILED_CLOCK_GHZ the shader
# clock the C2 recurrence ran at under rocprofv3 (GRBM_GUI_ACTIVE cycles of
# one XCD over the kernel's duration: 403 K in 182 us, profiles/bdm_forward_c2.md)
CU_COUNT, FMA_PER_CU_CLOCK, RATED_CLOCK_GHZ, PROFILED_CLOCK_GHZ = 256, 64, 2.4, 2.2


def fma_floor(cfg, batch, time_, ms):
    """The lazy recurrence's state-update FMAs alone (2*S*v per write and head,
    S*v per read and head), issued at the full non-packed FP32 rate: the time
    no vector-ALU form of this recurrence can beat, at the rated and at the
    profiled clock, and the kernel's fraction of it."""
    s, v, h, k = cfg.bank_size, cfg.head_value_width, cfg.num_heads, cfg.selected_banks
    fmas = batch * time_ * h * k * (2 * s * v + s * v)
    floor = {}
    for name, ghz in (('rated', RATED_CLOCK_GHZ), ('profiled', PROFILED_CLOCK_GHZ)):
        us = fmas / (CU_COUNT * FMA_PER_CU_CLOCK * ghz * 1e9) * 1e6
        floor[f'{name}_clock_ghz'] = ghz
        floor[f'{name}_floor_us'] = round(us, 1)
        floor[f'frac_of_{name}_floor'] = round(us / (ms * 1e3), 4)
    floor['state_update_fmas'] = fmas
    return floor


def combine_exposed(cfg, batch, time_, ms):
    """The read combine's time after the recurrence (bdm_forward's phase
    events 1 -> 2).  With the combine beside the recurrence (the default) that
    is the last head-group round's combine and the join; with
    BDM_COMBINE_OVERLAP=0 the whole combine."""
    overlapped = (os.environ.get('BDM_COMBINE_OVERLAP', '1') != '0'
                  and os.environ.get('BDM_FORWARD_KERNEL', 'vector') != 'mfma')
    if not overlapped:
        return dict(combine_roofline(cfg, batch, time_, ms), exposed_ms=round(ms, 4), overlapped=False)
    return {'kernel': 'ordered_combine_kernel', 'exposed_ms': round(ms, 4), 'overlapped': overlapped,
            'note': ("the last round's combine (its heads' columns); the earlier rounds' combines run beside the "
                     'recurrence and are inside the recurrence phase' if overlapped else
                     'the whole combine after the recurrence')}


def combine_roofline(cfg, batch, time_, ms):
    """The ordered read combine: KR rows of V BF16 values in, V out, per token."""
    nbytes = batch * time_ * (cfg.selected_banks + 1) * cfg.value_width * 2
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {'kernel': 'ordered_combine_kernel', 'ms': round(ms, 4), 'bytes': nbytes, 'achieved_GBps': round(gbps, 1),
            'peak_GBps': HBM_PEAK_GBPS, 'frac': round(gbps / HBM_PEAK_GBPS, 4)}


def timed(fn, steps, warmup):
    """Run fn warmup times, then time exactly `steps` calls between two
    device synchronisations.  Returns (seconds per step, last result)."""
    import torch
    out = None
    for _ in range(warmup):
        out = fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps, out


def copy_probe(device):
    """Achieved HBM bandwidth of a plain streaming kernel (read + write bytes):
    torch.neg over 512 MiB of BF16 into another 512 MiB.  It is also the
    known-size kernel that calibrates the FETCH_SIZE/WRITE_SIZE counters."""
    import torch
    n = 1 << 28  # 256 Mi bf16 = 512 MiB each way
    src = torch.empty(n, device=device, dtype=torch.bfloat16).normal_()
    dst = torch.empty_like(src)
    sec, _ = timed(lambda: torch.neg(src, out=dst), 10, 2)
    del src, dst
    return 2 * n * 2 / sec / 1e9


def decode_routes(layer, xs, routes, seed):
    """Per-step inputs of the kernel-only decode legs: the layer's controllers
    of each step's token and its routes.  routes='init': the layer's own
    routers, which at random init give every token the same read and write
    banks (the router residuals are zero, routing.py:37-68), so every read is
    served from a bank the same token just wrote; 'independent': write and
    read banks from independent N(0, 1) factor scores per step, so a token
    touches up to 24 banks (BASELINE's byte count assumes 24)."""
    import torch
    from bdm_amd import ops
    cfg = layer.config
    gen = torch.Generator().manual_seed(seed)
    j1, j2 = cfg.route_factors
    pre = []
    with torch.no_grad():
        for i in range(xs.shape[0]):
            q, k, v, g, b, w = layer._controllers(xs[i])
            if routes == 'init':
                rr, wr = layer._route_projections(xs[i])
                ww, wi = layer._route(wr, cfg.selected_banks)
                rw, ri = layer._route(rr, cfg.selected_banks)
            else:
                scores = torch.randn(2, xs.shape[1], 1, j1 + j2, generator=gen).to(xs.dtype).to(xs.device)
                ww, wi = ops.router_select(scores[0], bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
                rw, ri = ops.router_select(scores[1], bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
            pre.append(tuple(t[:, 0].contiguous() for t in (q, k, v, g, b, w, wi, ww, ri, rw)))
    return pre


def decode_moved_bytes(cfg, pre):
    """Bank-state bytes one decode step must move, averaged over the steps:
    each write bank read and written, each read bank that the same token does
    not also write read once (a read of a written bank takes the written
    value, which the kernel keeps on chip)."""
    bank_bytes = cfg.num_heads * cfg.bank_size * cfg.head_value_width * 2
    total = 0
    for step in pre:
        wi, ri = step[6].cpu(), step[8].cpu()
        extra = sum(len(set(ri[b].tolist()) - set(wi[b].tolist())) for b in range(wi.shape[0]))
        total += (2 * wi.numel() + extra) * bank_bytes
    return total / len(pre)


def decode_kernel_leg(layer, state, pre):
    """All steps' bdm_decode launches captured in one HIP graph and replayed:
    the kernel's time per step without host launch overhead."""
    import torch
    from bdm_amd import ops
    cfg = layer.config
    device = state.device
    scale = cfg.bank_size ** -0.5
    launch = lambda i: ops.decode_step(*pre[i], state, bank_count=cfg.bank_count, scale=scale,  # noqa: E731
                                       routed_decay=True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        for i in range(min(8, len(pre))):  # warmup
            launch(i)
        torch.cuda.synchronize()
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for i in range(len(pre)):
                    launch(i)
        torch.cuda.current_stream(device).wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(device)
        start.record(stream)
        graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        eager_sec, _ = timed(lambda: [launch(i) for i in range(len(pre))], 1, 0)
    del graph
    return start.elapsed_time(stop) * 1e3 / len(pre), eager_sec * 1e6 / len(pre)


def decode_bench(layer, device, steps, seed=1, legs=('init', 'independent'), full_step=True):
    """C3: batch 64, one token per sequence, resident BF16 state ~ N(0, 0.02).
    Kernel-only legs for both route cases (decode_routes), each reported on
    the bytes it moves (decode_moved_bytes); the full layer step (controllers,
    routes, decode, output interface) eagerly and from one HIP graph."""
    import torch
    cfg = layer.config
    batch = 64
    gen = torch.Generator().manual_seed(seed)
    state = (torch.randn(batch, cfg.bank_count, cfg.num_heads, cfg.bank_size, cfg.head_value_width,
                         generator=gen) * 0.02).to(torch.bfloat16).to(device)
    xs = torch.randn(steps, batch, 1, cfg.dim, generator=gen).to(torch.bfloat16).to(device)
    bank_bytes = cfg.num_heads * cfg.bank_size * cfg.head_value_width * 2
    # BASELINE's count: every step reads and writes KW banks and reads KR banks
    baseline_bytes = batch * (2 * cfg.selected_banks + cfg.selected_banks) * bank_bytes
    out = {'batch': batch, 'steps': steps, 'baseline_state_bytes_per_step': baseline_bytes}
    for routes in legs:
        pre = decode_routes(layer, xs, routes, seed + 17)
        kernel_us, eager_us = decode_kernel_leg(layer, state, pre)
        moved = decode_moved_bytes(cfg, pre)
        gbps = moved / (kernel_us * 1e-6) / 1e9
        out[f'{routes}_routes'] = {
            'kernel_us_per_step': round(kernel_us, 3), 'eager_launch_us_per_step': round(eager_us, 2),
            'moved_state_bytes_per_step': round(moved), 'moved_state_GBps': round(gbps, 1),
            'moved_state_frac_of_hbm_peak': round(gbps / HBM_PEAK_GBPS, 4)}
        del pre
    if full_step:
        with torch.no_grad():
            sec, _ = timed(lambda: [layer.step(xs[i], state) for i in range(steps)], 1, 1)
            full_graph_us, graph_check = full_step_graph(layer, xs, state, steps)
        out.update({'full_step_us_eager': round(sec * 1e6 / steps, 2), 'full_step_us_graph': full_graph_us,
                    'full_step_graph_check': graph_check,
                    'full_step_routes': 'the layer\'s own routers at random init (read banks = write banks)'})
    # the kernel leg whose bytes match BASELINE's 24-bank count most closely
    lead = out.get('independent_routes') or out.get('init_routes')
    out['kernel_us_per_step'] = lead['kernel_us_per_step']
    out['state_frac_of_hbm_peak'] = lead['moved_state_frac_of_hbm_peak']
    return out


def full_layer_prefill(layer, device, batch, time_, steps):
    """C2 geometry through the whole layer: controllers, route projections,
    routers, dispatch, recurrence, combine and the output interface (LN x gate,
    o_proj), from x ~ N(0, 1)."""
    import torch
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(batch, time_, layer.hidden_size, generator=gen).to(torch.bfloat16).to(device)
    with torch.no_grad():
        sec, _ = timed(lambda: layer.prefill(x), steps, 1)
    return {'tokens_per_s': round(batch * time_ / sec, 1), 'ms_per_step': round(sec * 1e3, 3)}


def full_step_graph(layer, xs, state, steps):
    """The full decode step (controllers, both routes, decode kernel, output
    projection) replayed per token from a HIP graph (bdm_amd.GraphDecoder: one
    input copy and one replay per token).  Before it is timed, the replays of
    all steps from a copy of the state are checked against the same steps run
    eagerly: every output and the final state must be identical.  Returns
    (us per step or None, check result)."""
    import torch
    from bdm_amd import GraphDecoder
    device = state.device
    try:
        with torch.no_grad():
            eager_state = state.clone()
            graph_state = state.clone()
            decoder = GraphDecoder(layer, graph_state)
            for i in range(steps):
                want, _ = layer.step(xs[i], eager_state)
                if not torch.equal(decoder.step(xs[i]), want):
                    return None, f'graph replay differs from the eager step {i}'
            if not torch.equal(graph_state, eager_state):
                return None, 'graph replays leave a different state'
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream(device)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(steps):
                decoder.step(xs[i])
            b.record(stream)
            torch.cuda.synchronize()
            return round(a.elapsed_time(b) * 1e3 / steps, 2), 'replays equal the eager steps'
    except RuntimeError as exc:  # a step that cannot be captured is reported, not hidden
        return None, f'capture failed: {str(exc)[:120]}'


# Published H200 whole-model figures for L16/D2048/FFN5632, batch 1, N = T
# (data/inference-performance.json:2497,2656,2868; data/decode-performance.json:851)
H200_PREFILL_SECONDS = {8192: 0.0504, 65536: 0.3757, 1048576: 6.709}
H200_DECODE_MS = {8192: 2.523}


def lm_graph_decode(model, tokens, caches, pos, count):
    """Whole-model decode replayed from one HIP graph
    (bdm_amd.LanguageModelGraphDecoder).  The replays of the first 4 tokens
    are checked against eager steps on a copy of the caches (logits and caches
    identical), then `count` more replays are timed.  Returns (ms per token or
    None, check result)."""
    import torch
    from bdm_amd import LanguageModelGraphDecoder
    try:
        eager = [c.clone() for c in caches]
        decoder = LanguageModelGraphDecoder(model, caches)
        for i in range(4):
            want, eager = model.step(tokens[:, pos + i:pos + i + 1], eager)
            if not torch.equal(decoder.step(tokens[:, pos + i:pos + i + 1]), want):
                return None, f'graph replay differs from the eager step {i}'
        if not all(torch.equal(a, b) for a, b in zip(decoder.caches, eager)):
            return None, 'graph replays leave different caches'
        del eager
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(count):
            decoder.step(tokens[:, pos + 4 + i:pos + 5 + i])
        torch.cuda.synchronize()
        return round((time.perf_counter() - t0) * 1e3 / count, 3), 'replays equal the eager steps'
    except RuntimeError as exc:  # a step that cannot be captured is reported, not hidden
        return None, f'capture failed: {str(exc)[:120]}'


def whole_model(device, context, timed_runs=3, decode_tokens=16, tune=True, decode=True):
    """The reference's whole-model inference case (perf_inference_case.py:15-56,
    80-160): BDMLanguageModel L16/D2048/FFN5632, vocab 50,257, one head of width
    2,048, N = T memory rows (J = T/8 banks of 8), K = 8, BF16 weights, batch
    1.  Prefill = embedding, every block's prefill from a fresh cache (the
    caches are created inside, as the reference's run does) and the head on
    the last position; decode = one eager step per token through all blocks
    and the full-vocabulary head.  Random-init weights, token ids uniform.
    ``tune``: GEMM selection by TunableOp in the warmup run (the library's
    heuristic otherwise); ``decode``: also time the eager and graph decode."""
    import torch
    from bdm_amd import BSDMConfig
    from bdm_amd.lm import BDMLanguageModel, LanguageModelConfig
    memory = BSDMConfig(dim=2048, bank_count=context // 8, bank_size=8, selected_banks=8, value_width=2048,
                        num_heads=1)
    config = LanguageModelConfig(memory=memory, vocab_size=50257, layers=16, seed=0)
    with torch.device(device):
        model = BDMLanguageModel(config)
    model = model.to(torch.bfloat16).eval()
    # GEMM selection by measurement (PyTorch TunableOp over the hipBLASLt and
    # rocBLAS solutions): each shape is tuned on its first call, in the warmup
    tunable = torch.cuda.tunable
    tunable.enable(tune)
    tunable.tuning_enable(tune)
    tunable.set_max_tuning_duration(30)
    tunable.set_filename(os.path.join(tempfile.gettempdir(), f'bdm_tunableop_{os.getpid()}_%d.csv'))
    gen = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, config.vocab_size, (1, context + 128), generator=gen).to(device)
    prompt = tokens[:, :context]
    samples = []
    with torch.inference_mode():
        for i in range(timed_runs + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            logits, caches = model.prefill(prompt)
            torch.cuda.synchronize()
            if i:  # the first run warms up (and tunes) the GEMMs and kernel caches
                samples.append(time.perf_counter() - t0)
            elif decode:
                for j in range(2):  # tune the decode shapes too, then only look up
                    model.step(tokens[:, context + 100 + j:context + 101 + j], [c.clone() for c in caches])
            tunable.tuning_enable(False)
        if not bool(torch.isfinite(logits).all()):
            raise RuntimeError('whole-model prefill produced non-finite logits')
        prefill_s = statistics.mean(samples)
        out = {'context': context, 'layers': 16, 'd_model': 2048, 'ffn': model.layers[0].feed_forward.hidden_dim,
               'bank_count': memory.bank_count, 'prefill_seconds': round(prefill_s, 5),
               'prefill_tokens_per_s': round(context / prefill_s, 1),
               'cache_bytes': sum(c.numel() * c.element_size() for c in caches)}
        if context in H200_PREFILL_SECONDS:
            out['h200_prefill_seconds'] = H200_PREFILL_SECONDS[context]
            out['prefill_speedup_vs_h200'] = round(H200_PREFILL_SECONDS[context] / prefill_s, 3)
        out['gemm_selection'] = ('PyTorch TunableOp (hipBLASLt and rocBLAS solutions, tuned in the warmup run)'
                                 if tune else 'library heuristic')
        if not decode:
            tunable.enable(False)
            del model, caches
            torch.cuda.empty_cache()
            return out
        for i in range(4):
            logits, caches = model.step(tokens[:, context + i:context + i + 1], caches)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(decode_tokens):
            pos = context + 4 + i
            logits, caches = model.step(tokens[:, pos:pos + 1], caches)
        torch.cuda.synchronize()
        decode_ms = (time.perf_counter() - t0) * 1e3 / decode_tokens
        graph_ms, graph_check = lm_graph_decode(model, tokens, caches, context + 4 + decode_tokens, decode_tokens)
    out.update({'decode_ms_per_token_eager': round(decode_ms, 3), 'decode_ms_per_token_graph': graph_ms,
                'decode_graph_check': graph_check})
    if context in H200_DECODE_MS:
        out['h200_decode_ms_per_token'] = H200_DECODE_MS[context]
        if graph_ms:
            out['decode_speedup_vs_h200'] = round(H200_DECODE_MS[context] / graph_ms, 3)
    tunable.enable(False)
    del model, caches
    torch.cuda.empty_cache()
    return out


H200_TRAIN_MS = {8192: 342.8}  # data/training-performance.json:1640-1643


def whole_model_training(device, context, timed_steps=3, warmup=2):
    """One full optimizer update of the reference's training case
    (reproduction/experiments/profile_final.py:30-80 with optim.py:7-50):
    BDMLanguageModel L16/D2048/FFN5632, vocab 50,257, batch 1, N = T, BF16
    weights with FP32 master copies; forward to the cross-entropy loss,
    backward, gradient-norm clipping at 1.0, AdamW on the FP32 masters
    (weight decay 0.01 except the no-decay parameters), masters copied back
    to the BF16 weights.  The clip scaling, the update and the copy back run
    as one pass (``MasterAdamW``, bit-identical to the reference's four).
    Random-init weights and token ids."""
    import torch
    from bdm_amd import BSDMConfig
    from bdm_amd.lm import BDMLanguageModel, LanguageModelConfig
    from bdm_amd.optim import MasterAdamW
    memory = BSDMConfig(dim=2048, bank_count=context // 8, bank_size=8, selected_banks=8, value_width=2048,
                        num_heads=1)
    config = LanguageModelConfig(memory=memory, vocab_size=50257, layers=16, seed=0)
    with torch.device(device):
        model = BDMLanguageModel(config)
    model = model.to(torch.bfloat16).train()
    params = list(model.parameters())
    optimizer = MasterAdamW(params, lr=0.0, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01, max_norm=1.0)
    gen = torch.Generator().manual_seed(7)
    tokens = torch.randint(0, config.vocab_size, (1, context + 1), generator=gen).to(device)
    x, y = tokens[:, :-1], tokens[:, 1:]

    def step():
        for p in params:
            p.grad = None
        loss = model(x, y)
        loss.backward()
        norm = optimizer.step()  # raises if a parameter received no gradient
        return loss.detach(), norm

    for i in range(warmup):
        loss, norm = step()
        torch.cuda.synchronize()
        progress('training warmup step', i + 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(timed_steps):
        loss, norm = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / timed_steps
    if not (math.isfinite(float(loss)) and math.isfinite(float(norm))):
        raise RuntimeError('whole-model training produced a non-finite loss or gradient norm')
    out = {'context': context, 'ms_per_step': round(ms, 2), 'tokens_per_s': round(context / ms * 1e3, 1),
           'loss': round(float(loss), 4), 'grad_norm': round(float(norm), 4),
           'peak_allocated_GiB': round(torch.cuda.max_memory_allocated() / 2 ** 30, 2)}
    if context in H200_TRAIN_MS:
        out['h200_ms_per_step'] = H200_TRAIN_MS[context]
        out['speedup_vs_h200'] = round(H200_TRAIN_MS[context] / ms, 3)
    del model, optimizer, params
    torch.cuda.empty_cache()
    return out


def c4_forward(device, steps=10, policy='prefill'):
    """C4: batch 4, T8192, J2048 (32x64), Zipf s=1.1 bias on the factor scores,
    hot-path prefill forward (router x2, dispatch, recurrence + combine, final
    state).  policy 'prefill': FP32 state, never rounded inside the
    recurrence (the reference's H = 1 prefill policy, inference.py:114-130),
    which lets long segments run as pieces composed by a scan; 'module': the
    module forward's BF16 training-state policy at H = 8 (heads.py:40-46,
    state rounded every 16 events, role_bank_kernel.py:153-165), under which a
    segment is not an affine map of its start state and runs as one serial
    chain, so the step is bound by the longest segment.  Reports tokens/s and
    the segment-length skew; under 'module' also the step with the opt-in
    stage path (BDM_STAGE_PATH=1: segments longer than 512 events as
    per-stage affine maps and a scan along the stages)."""
    import torch
    from bdm_amd import BSDMConfig, BankedDeltaMemory, ops
    from bdm_amd.config import near_square_factors
    cfg = BSDMConfig(dim=1024, bank_count=2048, bank_size=8, selected_banks=8, value_width=1024, num_heads=8)
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=0).to(device=device, dtype=torch.bfloat16)
    x, (q, k, v, g, b, w), (rr, wr), initial = make_inputs(layer, 4, 8192, device, seed=4)
    j1, j2 = near_square_factors(cfg.bank_count)
    gen = torch.Generator().manual_seed(11)
    bias = torch.cat([-1.1 * torch.log1p(torch.randperm(j1, generator=gen).float()),
                      -1.1 * torch.log1p(torch.randperm(j2, generator=gen).float())]).to(device)
    rr = (rr.float() + bias).to(rr.dtype)
    wr = (wr.float() + bias).to(wr.dtype)
    final = torch.empty(4, cfg.bank_count, cfg.num_heads, cfg.bank_size, cfg.head_value_width, device=device,
                        dtype=torch.bfloat16)
    interval = ROUND_INTERVAL if policy == 'module' else 0

    def step():
        (ww, wi), (rw, ri), meta = ops.route_dispatch(wr, rr, bank_count=cfg.bank_count, selected_banks=8)
        ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, initial, meta, bank_count=cfg.bank_count,
                           scale=cfg.bank_size ** -0.5, routed_decay=True, round_interval=interval,
                           final_state=final)
        return meta

    with torch.no_grad():
        sec, meta = timed(step, steps, 1)
    lengths = (meta.cu_seqlens[1:] - meta.cu_seqlens[:-1]).float()
    hot_bytes = hot_path_algorithmic_bytes(cfg, 4, 8192)
    described = {'prefill': 'FP32 state (prefill), long segments cut into pieces',
                 'module': 'BF16 state rounded every 16 events (module forward at H = 8), each segment serial'}
    result = {'tokens_per_s': round(4 * 8192 / sec, 1), 'ms_per_step': round(sec * 1e3, 3), 'steps': steps,
              'policy': described[policy],
              'hot_path_bytes_per_token': hot_bytes // (4 * 8192),
              'hot_path_roofline_frac': round(hot_bytes / sec / 1e9 / HBM_PEAK_GBPS, 4),
              'max_segment_events': int(lengths.max()), 'mean_segment_events': round(float(lengths.mean()), 1)}
    if policy == 'module':
        previous = os.environ.get('BDM_STAGE_PATH')
        os.environ['BDM_STAGE_PATH'] = '1'
        try:
            with torch.no_grad():
                sec_stage, _ = timed(step, steps, 1)
        finally:
            if previous is None:
                del os.environ['BDM_STAGE_PATH']
            else:
                os.environ['BDM_STAGE_PATH'] = previous
        result['stage_path'] = {'ms_per_step': round(sec_stage * 1e3, 3),
                                'tokens_per_s': round(4 * 8192 / sec_stage, 1),
                                'switch': 'BDM_STAGE_PATH=1'}
    return result


def c5_training(device, steps=10):
    """C5: batch 4, T2048, H8, BF16 training state: routed operator forward +
    backward (bank_training with all controller, route and state gradients)."""
    import torch
    from bdm_amd import BankedDeltaMemory, bank_training
    cfg = c2_config()
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=0).to(device=device, dtype=torch.bfloat16)
    x, ctrl, (rr, wr), initial = make_inputs(layer, 4, 2048, device, seed=5)
    gen = torch.Generator().manual_seed(12)
    dy = torch.randn(4, 2048, cfg.value_width, generator=gen).to(torch.bfloat16).to(device)
    with torch.no_grad():
        ww, wi = layer._route(wr, cfg.selected_banks)
        rw, ri = layer._route(rr, cfg.selected_banks)
    leaves = [t.detach().clone().requires_grad_(True) for t in (*ctrl, ww, rw, initial)]

    def step():
        for t in leaves:
            t.grad = None
        y = bank_training(*leaves[:6], wi, leaves[6], ri, leaves[7], leaves[8], cfg.bank_count,
                          cfg.bank_size ** -0.5, state_dtype=torch.bfloat16)
        y.backward(dy)

    sec, _ = timed(step, steps, 1)
    tokens = 4 * 2048
    hbm = training_algorithmic_bytes(cfg, 4, 2048)
    flop = training_flop(cfg, 4, 2048)
    return {'tokens_per_s': round(tokens / sec, 1), 'ms_per_step': round(sec * 1e3, 3), 'steps': steps,
            'hot_path_bytes_per_token': hbm // tokens,
            'hot_path_roofline_frac': round(hbm / sec / 1e9 / HBM_PEAK_GBPS, 4),
            'flop_per_token': flop // tokens, 'achieved_tflops': round(flop / sec / 1e12, 2),
            'frac_valu_fp32': round(flop / sec / 1e12 / VALU_FP32_TFLOPS, 4),
            'roofline_note': ('bytes: the forward hot path without the final state, the BF16 snapshot at every '
                              '16th event written and read back, the controllers read again, dy read and every '
                              'controller and route gradient written; FLOPs: the sequential forward (5Sv per '
                              'write, 2Sv per read) plus the replay (5Sv per write) and the adjoint (11Sv per '
                              'write, 4Sv per read), per head')}


def training_algorithmic_bytes(cfg, batch, time_):
    """C5 forward + backward bytes (the roofline_note of c5_training)."""
    h, s, v_total, kk = cfg.num_heads, cfg.bank_size, cfg.value_width, cfg.selected_banks
    controllers = 3 * h * s * 2 + h * s * 4 + 2 * v_total * 2
    forward = hot_path_algorithmic_bytes(cfg, batch, time_) - batch * cfg.bank_count * h * s * (v_total // h) * 2
    tokens = batch * time_
    # one snapshot of S x v BF16 per head every 16 events; 2K events per token and head
    snapshots = tokens * h * (2 * kk) // 16 * s * (v_total // h) * 2
    backward = tokens * (controllers + v_total * 2 + controllers + 2 * kk * 2)
    return forward + 2 * snapshots + backward


def training_flop(cfg, batch, time_):
    s, v, h, k = cfg.bank_size, cfg.head_value_width, cfg.num_heads, cfg.selected_banks
    return batch * time_ * h * k * ((5 + 5 + 11) * s * v + (2 + 4) * s * v)


def c2_forward_only(layer, device, batch, time_, launches):
    """``launches`` bdm_forward launches of the C2 hot path (routes and dispatch
    built once), for profilers; BDM_FORWARD_KERNEL picks the recurrence."""
    import torch
    from bdm_amd import ops
    _, (q, k, v, g, b, w), (read_scores, write_scores), initial = make_inputs(layer, batch, time_, device)
    cfg = layer.config
    final = torch.empty(batch, cfg.bank_count, cfg.num_heads, cfg.bank_size, cfg.head_value_width,
                        device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        (ww, wi), (rw, ri), meta = ops.route_dispatch(write_scores, read_scores, bank_count=cfg.bank_count,
                                                       selected_banks=cfg.selected_banks)
        t0 = time.perf_counter()
        for _ in range(launches):
            ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, initial, meta, bank_count=cfg.bank_count,
                               scale=cfg.bank_size ** -0.5, routed_decay=True, round_interval=ROUND_INTERVAL,
                               final_state=final)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / launches * 1e3
        # one copy of known size, the reference for calibrating FETCH_SIZE and
        # WRITE_SIZE counters: 512 MiB read and 512 MiB written by torch.neg
        src = torch.empty(256 * 1024 * 1024, device=device, dtype=torch.bfloat16).fill_(1.0)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
    return {'launches': launches, 'ms_per_launch': round(ms, 4),
            'recurrence': os.environ.get('BDM_FORWARD_KERNEL', 'vector'), 'copy_probe_bytes': 2 * src.numel() * 2}


def graph_step(step, final, steps, tokens):
    """The same hot-path step captured in one HIP graph (torch.cuda.graph) and
    replayed: the kernels' launch gaps without the host.  Replays, with eager
    steps between them, must equal the eager step's y and final state."""
    import torch
    with torch.no_grad():
        y_eager = step().clone()
        torch.cuda.synchronize()
        f_eager = final.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_graph = step()
        equal = True
        for _ in range(3):
            final.zero_()
            graph.replay()
            torch.cuda.synchronize()
            equal = equal and torch.equal(y_graph, y_eager) and torch.equal(final, f_eager)
            step()
            torch.cuda.synchronize()
        # replays for DEVICE_WARMUP_S first, as before the eager timed steps
        w0 = time.perf_counter()
        while time.perf_counter() - w0 < DEVICE_WARMUP_S:
            for _ in range(8):
                graph.replay()
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        sec = (time.perf_counter() - t0) / steps
    return {'ms_per_step': round(sec * 1e3, 4), 'tokens_per_s': round(tokens / sec, 1),
            'replays_equal_eager': bool(equal)}


def c1_config():
    """BASELINE configs[0] (the reference's CPU-runnable case): d_model 512, H4 of
    v = 64, J256 = 16x16, S8, K8, FP32 weights, FP32 training state."""
    from bdm_amd import BSDMConfig
    return BSDMConfig(dim=512, bank_count=256, bank_size=8, selected_banks=8, value_width=256, num_heads=4,
                      training_state_dtype='float32')


def c1_input():
    import torch
    return torch.randn(1, 512, 512, generator=torch.Generator().manual_seed(512))


def c1_gpu(device, steps=20):
    """The HIP module forward at C1 (FP32): controllers, routing, dispatch,
    recurrence, combine and output interface; tokens/s of one forward."""
    import torch
    from bdm_amd import BankedDeltaMemory
    layer = BankedDeltaMemory(c1_config(), layer_id=0, seed=0).to(device)
    x = c1_input().to(device)
    with torch.no_grad():
        sec, _ = timed(lambda: layer(x), steps, 3)
    # FP32 controllers and state: the hot-path bytes of hot_path_algorithmic_bytes at 4 bytes per element
    cfg = c1_config()
    hot = 2 * hot_path_algorithmic_bytes(cfg, 1, 512)
    return {'tokens_per_s': round(512 / sec, 1), 'ms_per_forward': round(sec * 1e3, 4),
            'hot_path_roofline_frac': round(hot / sec / 1e9 / HBM_PEAK_GBPS, 6),
            'roofline_note': 'host-bound: ~15 launches of microseconds for 512 tokens',
            'config': 'C1: batch 1, T 512, d_model 512, H4, v64, J256 (16x16), S8, K8, FP32, FP32 state'}


def cpu_threads():
    """Host threads for the CPU baseline: the cores this process may run on,
    at most 16 (one GPU's share of the box, whatever os.cpu_count() reports)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return max(1, min(usable, 16)), usable


def cpu_baseline():
    """The reference's CPU path timed at C1: the backend='reference' forward
    (oracle/bdm_oracle.py OracleBankedDeltaMemory.forward, the per-event loop
    of reference_packed_gdn2 and index_add_), under no_grad, 1 warmup and 5
    timed runs, the median; tokens/s = 512 / median."""
    import torch
    from oracle import bdm_oracle as O
    threads, usable = cpu_threads()
    torch.set_num_threads(threads)
    oracle = O.OracleBankedDeltaMemory(c1_config(), layer_id=0, seed=0)
    x = c1_input()

    def run():
        with torch.no_grad():
            return oracle(x, combine='index_add', lockstep=False)

    run()  # warmup
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    model = ''
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    return {'value': round(512 / med, 2), 'unit': 'tokens/s', 'cores': threads, 'kind': 'port',
            'sample': (f'C1 whole: batch 1 x T=512, d_model 512, H4 v64 J256 (16x16) S8 K8, FP32 weights and '
                       f'state; OracleBankedDeltaMemory.forward (per-event loop + index_add_), 1 warmup + 5 runs, '
                       f'median {med:.3f} s; {threads} threads ({usable} usable cores, os.cpu_count() = '
                       f'{os.cpu_count()}); host CPU: {model}')}


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def progress(*what):
    print('bench:', *what, file=sys.stderr, flush=True)


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: this build has no multi-GPU path '
              '(every GPU box here has one GPU); run with --gpus 1', file=sys.stderr)
        sys.exit(2)
    import torch
    from bdm_amd import BankedDeltaMemory, ops

    if not torch.cuda.is_available():
        print('bench.py needs a ROCm GPU', file=sys.stderr)
        sys.exit(2)
    device = torch.device('cuda', 0)
    cfg = c2_config()
    batch, time_ = args.batch, args.time
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=0).to(device=device, dtype=torch.bfloat16)
    if args.only:
        run = {'c2-forward': lambda: c2_forward_only(layer, device, batch, time_, args.steps),
               'c3': lambda: decode_bench(layer, device, args.decode_steps),
               'c3-kernel': lambda: decode_bench(layer, device, args.decode_steps, legs=(args.c3_routes,),
                                                 full_step=False),
               'c4': lambda: c4_forward(device), 'c4-module': lambda: c4_forward(device, steps=3, policy='module'),
               'c5': lambda: c5_training(device),
               'prefill': lambda: full_layer_prefill(layer, device, batch, time_, max(3, args.steps // 4)),
               'lm': lambda: whole_model(device, args.lm_context, tune=args.lm_gemm_tuning == 'on'),
               'lm-prefill': lambda: whole_model(device, args.lm_context, tune=args.lm_gemm_tuning == 'on',
                                                 decode=False),
               'lm-train': lambda: whole_model_training(device, args.lm_context)}[args.only]
        progress('workload', args.only)
        print(json.dumps({'workload': args.only, 'result': run()}), flush=True)
        return
    x, (q, k, v, g, b, w), (read_scores, write_scores), initial = make_inputs(layer, batch, time_, device)
    final = torch.empty(batch, cfg.bank_count, cfg.num_heads, cfg.bank_size, cfg.head_value_width,
                        device=device, dtype=torch.bfloat16)
    j, kk, scale = cfg.bank_count, cfg.selected_banks, cfg.bank_size ** -0.5
    stream = torch.cuda.current_stream(device)
    # Timing events are recorded in a profiling pass after the timed steps: a
    # timestamp event drains the stream before the next kernel starts, and five
    # of them per step cost ~20 us of overlap between kernels.
    prof_steps = min(args.steps, 10)
    ev_front = [torch.cuda.Event(enable_timing=True) for _ in range(prof_steps)]
    ev_start = [torch.cuda.Event(enable_timing=True) for _ in range(prof_steps)]
    ev_stop = [torch.cuda.Event(enable_timing=True) for _ in range(prof_steps)]
    # recorded by bdm_forward itself: before the recurrence, before the combine, after it
    ev_phase = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(prof_steps)]

    def step(rec=None):
        if rec is not None:
            ev_front[rec].record(stream)
        (ww, wi), (rw, ri), meta = ops.route_dispatch(write_scores, read_scores, bank_count=j, selected_banks=kk)
        if rec is not None:
            ev_start[rec].record(stream)
        y = ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, initial, meta, bank_count=j, scale=scale,
                               routed_decay=True, round_interval=ROUND_INTERVAL, final_state=final,
                               phase_events=ev_phase[rec] if rec is not None else None)
        if rec is not None:
            ev_stop[rec].record(stream)
        return y

    progress('hot path', batch, time_)
    with torch.no_grad():
        for _ in range(8):
            step()
        torch.cuda.synchronize()
        warm_steps, w0 = 8, time.perf_counter()
        while time.perf_counter() - w0 < DEVICE_WARMUP_S:
            for _ in range(8):
                step()
            torch.cuda.synchronize()
            warm_steps += 8
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        progress('hot path profiling pass', prof_steps)
        for i in range(prof_steps):
            step(i)
        torch.cuda.synchronize()
    sec = elapsed / args.steps
    tokens = batch * time_
    fwd_ms = statistics.mean(a.elapsed_time(bb) for a, bb in zip(ev_start, ev_stop))
    front_ms = statistics.mean(a.elapsed_time(bb) for a, bb in zip(ev_front, ev_start))
    rec_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in ev_phase)
    comb_ms = statistics.mean(e[1].elapsed_time(e[2]) for e in ev_phase)
    fwd_bytes = forward_algorithmic_bytes(cfg, batch, time_, initial.numel() * initial.element_size())
    achieved = fwd_bytes / (fwd_ms * 1e-3) / 1e9
    hot_bytes = hot_path_algorithmic_bytes(cfg, batch, time_)
    traffic = load_traffic()

    result = {
        'metric': 'BDM-layer prefill tokens/sec (routed-memory hot path, N=2048,S=8,B=8)',
        'value': round(tokens / sec, 1), 'unit': 'tokens/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(sec * 1e3, 4), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'bf16 controllers and state storage (state rounded every 16 events), fp32 recurrence math',
        'data': 'synthetic: x ~ N(0,1), seeded random-init BSDM layer weights',
        'config': {'workload': 'C2 prefill hot path: router x2 + dispatch + recurrence + ordered combine '
                               '+ final BF16 state', 'state_rounding_interval': ROUND_INTERVAL, 'batch': batch, 'seq_len': time_, 'd_model': cfg.dim,
                   'heads': cfg.num_heads, 'bank_count': j, 'bank_size': cfg.bank_size,
                   'selected_banks': kk, 'head_value_width': cfg.head_value_width},
        'roofline': {'bound': 'hbm', 'kernel': ('bdm_forward (segment_order_kernel, lazy_forward_kernel in head-group '
                                                'rounds, ordered_combine_kernel per round beside the next)'),
                     'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
                     'frac': round(achieved / HBM_PEAK_GBPS, 4),
                     'traffic': traffic.get('bytes_per_launch') if traffic else None,
                     'traffic_source': ('FETCH_SIZE x2 + WRITE_SIZE x1 per launch from rocprofv3 --pmc runs of '
                                        'bench.py --only c2-forward, calibrated on a 512 MiB copy in the same '
                                        'process (profiles/forward_c2_traffic.json)') if traffic else None,
                     'launch_ms': round(fwd_ms, 4), 'algorithmic_bytes': fwd_bytes},
        'hot_path_roofline_frac': round(hot_bytes / sec / 1e9 / HBM_PEAK_GBPS, 4),
        'recurrence': recurrence_roofline(cfg, batch, time_, rec_ms),
        'combine': combine_exposed(cfg, batch, time_, comb_ms),
        'front_end_ms': round(front_ms, 4),
        'timing': ('ms_per_step: wall clock over the timed steps, no events inside; launch_ms, recurrence, '
                   f'combine and front_end_ms: events of {prof_steps} further steps'),
        'device_warmup': {'seconds': DEVICE_WARMUP_S, 'steps': warm_steps,
                          'note': 'hot-path steps run before the warmup steps while the GPU clocks ramp up'},
    }
    progress('hot path from one HIP graph')
    result['hip_graph'] = graph_step(step, final, args.steps, tokens)
    if not args.no_extras:
        progress('full layer prefill')
        result['full_layer_prefill_tokens_per_s'] = full_layer_prefill(layer, device, batch, time_,
                                                                       max(3, args.steps // 4))['tokens_per_s']
        progress('decode C3')
        result['decode_c3'] = decode_bench(layer, device, args.decode_steps)
        progress('skewed forward C4')
        result['forward_c4'] = c4_forward(device)
        progress('skewed forward C4, module policy')
        result['forward_c4_module_policy'] = c4_forward(device, steps=3, policy='module')
        progress('training C5')
        result['training_c5'] = c5_training(device)
        progress('whole model L16/D2048', args.lm_context)
        result['whole_model'] = whole_model(device, args.lm_context, tune=args.lm_gemm_tuning == 'on')
        progress('whole model training step', args.lm_context)
        result['whole_model_training'] = whole_model_training(device, args.lm_context)
    progress('copy probe')
    result['hbm_copy_GBps'] = round(copy_probe(device), 1)
    progress('C1 forward on the GPU')
    result['c1_forward'] = c1_gpu(device)
    if args.cpu_baseline:
        progress('cpu baseline at C1')
        result['cpu_baseline'] = cpu_baseline()
        result['c1_forward']['gpu_over_cpu'] = round(result['c1_forward']['tokens_per_s']
                                                     / result['cpu_baseline']['value'], 1)
    else:
        result['cpu_baseline'] = None
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
