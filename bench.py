"""Benchmark of the ASRN layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--config cfg2] [--no-cpu-baseline] [--no-decode]

A step is one forward + backward of one ASRN layer (asrn.ASRNLayer, group-A protections) over one batch of
synthetic tokens: BASELINE.json configs[1] = cfg2, B 8, N 4096, d 256, V 256, fp32, 30% copied spans. Inputs and
weights are resident in HBM before the timed region. The step is captured once into a HIP graph and the timed steps
are its replays (the same kernels, launched without the host's per-op overhead); --eager times Python-launched steps
instead. The per-kernel device events (roofline, hip_aggregate, kernels) come from an eager pass of the same number of
steps, since events recorded while capturing are not replayed. Prints one JSON line with the driver's keys plus:
  roofline      the dominant HIP kernel: algorithmic bytes per launch / its mean launch time (device events recorded
                on the stream it runs on), against MI355X's 8 TB/s
  hip_aggregate all HIP kernels: 25,552 B/token (cfg2) x tokens / (8 TB/s x their summed time per step)
  layer         whole-layer tokens/s and its HBM fraction at 41,552 B/token (the HIP kernels' bytes plus the GEMMs'
                operands and results, 16,000 B/token at cfg2)
  decode        the O(1) generation step of one layer (BASELINE.json configs[4] at one layer): per-token latency
                against the context, 1K to 64K, and its slope
  cpu_baseline  the CPU oracle (oracle/layer.py, PyTorch on the host cores) on the same workload
"""
import argparse
import copy
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = 'ASRN layer fwd+bwd tokens/sec at N=4096 (1 GPU); % HBM roofline; decode tok/s'
HBM_PEAK = 8.0e12

# algorithmic bytes per token at cfg2 (fp32, T 8, P 112, cf 16, d 256): every tensor the kernel must touch, read
# once and written once. The entry point timed below and its per-token figure.
def algorithmic_bytes(d, P, cf, T, a=4):
    reads_fwd = P * a + 2 * cf * a + d * a + 8 + 8 + 4 + 2 * T * 4       # phi, Qc, Kc, V, x, Bt, log_alfa, order+ids
    fwd = reads_fwd + d * a + 4 * 4                                     # + salida, 4 signals
    bwd = reads_fwd + d * a + (P * a + 2 * cf * a + d * a + 8 + 4)      # + dsalida; dphi, dQc, dKc, dV, dBt, dlog_alfa
    return {'asrn_candidates_fwd': fwd, 'asrn_candidates_bwd': bwd}


def gate_bytes(d, n, a=4):
    """The fused gate (asrn_gate_fwd/bwd): h, A (W_o salida, a bytes), signals, seen flags, Hawkes, streak, logit in;
    h' out; the backward also reads dh' and writes dh, dA, dHawkes, dstreak."""
    small = 16 + 8 * n + 4 + 4
    fwd = 4 * d + a * d + small + 4 * d
    bwd = 4 * d + 4 * d + a * d + small + 4 * d + a * d + 4 * n + 4
    return fwd, bwd


def context_bytes(d):
    """The fused LayerNorm + clock projection (asrn_context_fwd/bwd), fp32: h in, hh, (mean, rstd, u) and beta (fp64),
    log_alfa out; the backward reads h, dhh, the gate's dh, the stats, dbeta, dlog_alfa and writes dh."""
    return 4 * d + 4 * d + 16 + 8 + 4, 4 * d + 4 * d + 4 * d + 16 + 8 + 4 + 4 * d


def hidden_bytes(m=64, mc=64):
    """The hash MLPs' hidden layer (asrn_hidden_fwd/bwd, the path under autocast), fp32: the forward reads the three
    first-layer blocks and writes g; the backward reads them and dg and writes their gradients."""
    return 4 * (m + 2 * mc) + 4 * (m + mc), 4 * (m + 2 * mc) + 4 * (m + mc) + 4 * (m + 2 * mc)


def hash_bytes(P, m=64, mc=64):
    """The fused hash MLPs (asrn_hash_fwd/bwd, the fp32 path): the forward reads the three first-layer blocks and
    writes phi; the backward reads them and dphi and writes the blocks' gradients (g, dg and the second layer's
    GEMM operands stay on chip; the parameter gradients are per-workgroup partials, not per token)."""
    return 4 * (m + 2 * mc) + 4 * P, 4 * (m + 2 * mc) + 4 * P + 4 * (m + 2 * mc)


def hip_bytes_per_token(d, P, cf, T, n=4, a=4, m=64, mc=64, K=4, fused=True):
    """All HIP kernels of one fwd+bwd, each distinct tensor read once and written once: hash + bucket sort (phi in, ids
    and order out), clock 16 + 16, n-gram sort 28, Hawkes/streak scans 60 + 100, candidates, gate, context producer,
    the hash MLPs (fused: hash_bytes; else the hidden layer and its bias column sums), and the column sums of the
    candidates' per-token partials (the weight gradients' slab sums scale with the weights, not the tokens, and are
    left out).
    cfg2 fp32 (fused): 512 + 32 + 28 + 160 + 7,044 + 8,324 + 6,200 + 3,200 + 52 = 25,552."""
    cand = algorithmic_bytes(d, P, cf, T, a)
    colsums = 4 * (T + K + 1) + (0 if fused else 4 * (m + mc) + 4 * P)
    mlp = sum(hash_bytes(P, m, mc)) if fused else sum(hidden_bytes(m, mc))
    return (P * a + 8 * T + 32 + 28 + 160 + sum(cand.values()) + sum(gate_bytes(d, n, a))
            + sum(context_bytes(d)) + mlp + colsums)


def gemm_bytes_per_token(d, P, cf, a=4, m=64, mc=64, fused=True):
    """Operands and results of the layer's GEMMs per token, each read or written once (activations in a bytes;
    weights are per step, not per token): forward E -> [hp|za|zb], hh -> [Qc|Kc], sum -> W_o W_v sum and, unfused,
    g -> phi; backward the input gradients (the E one accumulating into the candidates' dE) and the weight gradients
    (both operands read). cfg2 fp32 (fused): 4,992 + 11,008 = 16,000."""
    h, q = m + 2 * mc, 2 * cf
    fwd = (d + h) + (d + q) + (d + d) + (0 if fused else (m + mc) + P)
    bwd = (d + d) + 2 * d + (q + d) + (q + d) + (h + 2 * d) + (h + d) + (0 if fused else 2 * (P + m + mc))
    return a * (fwd + bwd)


TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'cfg2_traffic.json')


def measured_traffic(kernel):
    """HBM bytes per launch of an entry point from the committed counter passes (FETCH_SIZE and WRITE_SIZE, scaled
    by a copy of known size), or None when they were not taken for this build."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)['bytes_per_launch'].get(kernel)
    except (OSError, ValueError, KeyError):
        return None


def cpu_baseline(layer_cpu, x, E, h, gy, reps=2):
    """The CPU oracle's layer forward + backward on the same inputs (oracle/layer.py, PyTorch on all host cores)."""
    import torch
    from oracle import layer as O
    torch.set_num_threads(os.cpu_count() or 1)
    p = {k: (v.clone().requires_grad_() if v.is_floating_point() and k not in ('c_vistos', 'r_firma') else v.clone())
         for k, v in layer_cpu.state_dict().items()}
    sh = O.shape_from_params(p, E.shape[-1], n_bits=layer_cpu.n_bits, C=layer_cpu.chunk)
    times = []
    for i in range(reps + 1):
        Ec, hc = E.clone().requires_grad_(), h.clone().requires_grad_()
        t0 = time.perf_counter()
        y = O.layer_forward(p, Ec, hc, x, sh)
        (y * gy).sum().backward()
        dt = time.perf_counter() - t0
        if i:
            times.append(dt)
    t = statistics.median(times)
    tokens = x.numel()
    return {'value': round(tokens / t, 1), 'unit': 'tokens/s', 'cores': torch.get_num_threads(), 'kind': 'port',
            'sample': f'full workload ({x.shape[0]}x{x.shape[1]} tokens), fp32, median of {reps} after 1 warm-up; '
                      f'cpu_count={os.cpu_count()}',
            'seconds_per_step': round(t, 3)}


DECODE = dict(B=16, d=768, V=50304, contexts=(1024, 4096, 16384, 32768, 65536), frac=0.2, span=(16, 256),
              zipf=1.1)


def decode_bench(dev, steps, warmup, seed=0, contexts=None):
    """BASELINE.json configs[4], one layer: the O(1) generation step of one ASRN layer at d = 768, B = 16, after a
    prefill of each context length. Per-token latency (wall clock over `steps` back-to-back steps, synchronized at
    both ends) against the context, and the least-squares slope with its 95% interval (O(1): it includes 0). The
    step is the writer's HIP graph replay (EscritorCapa(grafo=True)); its first step runs op by op, and there the two
    HIP kernels are timed with events (a replay makes no library call to time); the second captures the graph."""
    import torch

    import asrn_amd
    from asrn_amd import _lib, synth

    cfg = DECODE
    B, d, V = cfg['B'], cfg['d'], cfg['V']
    contexts = contexts or cfg['contexts']
    torch.manual_seed(seed)
    layer = synth.move_params(asrn_amd.ASRNLayer(d), seed=seed).to(dev)
    g = torch.Generator(device=dev).manual_seed(seed + 7)
    emb = torch.randn(V, d, generator=g, device=dev)
    rows = []
    kern = {}
    for ctx in contexts:
        x = synth.tokens(B, ctx + max(warmup, 2) + steps, V, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'],
                         seed=seed + ctx).to(dev)
        E = emb[x]
        h = torch.randn(B, x.shape[1], d, generator=g, device=dev)
        # every position a key (the rings update); the step replayed from a HIP graph
        esc = asrn_amd.EscritorCapa(layer, memoria_de_lo_ajeno=False, grafo=True)
        esc.inicio(E[:, :ctx], h[:, :ctx], x[:, :ctx], capacidad=ctx + max(warmup, 2) + steps + 1)
        timed = _lib.time_calls(['asrn_decode_attend', 'asrn_repetition_step'])
        esc.paso(E[:, ctx], h[:, ctx], x[:, ctx])                        # op by op: its kernels timed
        timed = _lib.stop_timing()
        for t in range(ctx + 1, ctx + max(warmup, 2)):                    # the first of these captures the graph
            esc.paso(E[:, t], h[:, t], x[:, t])
        w = max(warmup, 2)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(ctx + w, ctx + w + steps):
            esc.paso(E[:, t], h[:, t], x[:, t])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for n, evs in timed.items():
            kern.setdefault(n, []).extend(s.elapsed_time(e) for s, e in evs)
        ms = 1e3 * (t1 - t0) / steps
        rows.append({'context': ctx, 'ms_per_step': round(ms, 4), 'tokens_per_s': round(B * 1e3 / ms, 1),
                     'kernel_us': {n: round(1e3 * sum(s.elapsed_time(e) for s, e in evs) / len(evs), 2)
                                   for n, evs in timed.items() if evs}})
        del esc, E, h, x
        torch.cuda.empty_cache()
    xs = [r['context'] for r in rows]
    ys = [r['ms_per_step'] * 1e6 for r in rows]        # ns
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    sxx = sum((a - mx) ** 2 for a in xs)
    slope = sum((a - mx) * (b - my) for a, b in zip(xs, ys)) / sxx if sxx else 0.0
    res = [b - (my + slope * (a - mx)) for a, b in zip(xs, ys)]
    se = (sum(r * r for r in res) / max(n - 2, 1) / sxx) ** 0.5 if sxx else 0.0
    t975 = {1: 12.71, 2: 4.30, 3: 3.18, 4: 2.78, 5: 2.57}.get(n - 2, 2.0)
    return {'workload': f'configs[4], one layer: O(1) generation step of one ASRN layer, d={d}, B={B}, V={V}, '
                        f'Zipf 1.1 with 20% copied spans, prefill of each context then {warmup} + {steps} steps',
            'launch': 'hip graph replay of the step', 'per_context': rows, 'tokens_per_s': rows[-1]['tokens_per_s'],
            'slope_ns_per_context_token': round(slope, 4),
            'slope_ci95': [round(slope - t975 * se, 4), round(slope + t975 * se, 4)],
            'kernels': {k: {'launches': len(v), 'mean_us': round(1e3 * sum(v) / len(v), 3)} for k, v in kern.items()
                        if v}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    # 200 replays (about 0.17 s) measure the steady state: 20 read about 3% slower, the clocks still settling
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--config', default='cfg2')
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-decode', action='store_true')
    ap.add_argument('--decode-steps', type=int, default=256)
    ap.add_argument('--decode-only', action='store_true',
                    help='only the generation-step leg (configs[4], one layer); prints its JSON object')
    ap.add_argument('--eager', action='store_true', help='time Python-launched steps instead of HIP graph replays')
    ap.add_argument('--default-gemms', action='store_true',
                    help="leave the GEMMs on the libraries' default picks instead of the shipped MI355X picks")
    ap.add_argument('--copy-calibration', type=int, default=0, metavar='BYTES',
                    help='only run a plain device-to-device copy of BYTES, 3 times: the reference point that scales '
                         'the FETCH_SIZE / WRITE_SIZE counters of a profiler run into bytes')
    args = ap.parse_args()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(f'bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): the ASRN hot path '
              'shards over the batch with no exchange between GPUs.', file=sys.stderr)
        sys.exit(2)

    import torch

    import asrn_amd
    from asrn_amd import _lib, synth

    if args.copy_calibration:
        src = torch.ones(args.copy_calibration // 4, dtype=torch.float32, device='cuda:0')
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_calibration_bytes': src.numel() * 4, 'launches': 3}), flush=True)
        return

    asrn_amd.load()
    gemm_picks = 'library defaults'
    if not args.default_gemms:
        from asrn_amd import tuning
        if tuning.use_tuned_gemms():
            gemm_picks = 'TunableOp picks, asrn_amd/data/gemm_picks_mi355x.csv'
    if args.decode_only:
        print(json.dumps({'decode': decode_bench(torch.device('cuda:0'), args.decode_steps, 20, seed=args.seed),
                          'gemm_picks': gemm_picks}), flush=True)
        return
    cfg = synth.CONFIGS[args.config]
    B, N, d, V = cfg['B'], cfg['N'], cfg['d'], cfg['V']
    dev = torch.device('cuda:0')
    torch.manual_seed(args.seed)
    layer_cpu = synth.move_params(asrn_amd.ASRNLayer(d), seed=args.seed)
    layer = copy.deepcopy(layer_cpu).to(dev)
    x, E, h = synth.layer_inputs(B, N, d, V, seed=args.seed, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'])
    gy = torch.randn(B, N, d, generator=torch.Generator().manual_seed(args.seed + 1))
    xd, Ed, hd, gyd = x.to(dev), E.to(dev).requires_grad_(), h.to(dev).requires_grad_(), gy.to(dev)

    bf16 = args.config == 'cfg3'           # configs[2]: bf16 activations, fp32 scan state (autocast)
    dtype = 'bf16' if bf16 else 'fp32'

    def fwd_bwd():
        with torch.autocast('cuda', dtype=torch.bfloat16, enabled=bf16):
            y = layer(Ed, hd, xd)
        y.backward(gyd.to(y.dtype))                     # the gradient of sum(y * gy)

    def step():
        layer.zero_grad(set_to_none=True)
        Ed.grad = None
        hd.grad = None
        fwd_bwd()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # eager pass with HIP-event timing of every library entry point (on the stream each one launches on)
    names = [n for n in _lib.SIGNATURES if n not in ('asrn_hip_last_error', 'asrn_hip_abi_version')
             and not n.endswith('_workspace')]
    timed = _lib.time_calls(names)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    timed = _lib.stop_timing()
    eager_wall = (t1 - t0) / args.steps

    graph = None
    if not args.eager:
        # capture one step; the gradients are written into the graph's buffers on every replay
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        layer.zero_grad(set_to_none=True)
        Ed.grad = None
        hd.grad = None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fwd_bwd()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()

    per_call = {}
    for n, evs in timed.items():
        if evs:
            ms = [s.elapsed_time(e) for s, e in evs]
            per_call[n] = {'launches': len(ms), 'mean_us': 1e3 * sum(ms) / len(ms), 'total_ms': sum(ms)}
    wall = (t1 - t0) / args.steps
    tokens = B * N
    value = tokens * args.steps / (t1 - t0)

    P, cf, T = layer.n_tablas * layer.n_bits, layer.confirmar, layer.n_tablas
    algo = algorithmic_bytes(d, P, cf, T, a=2 if bf16 else 4)
    dom = max(algo, key=lambda n: per_call.get(n, {}).get('total_ms', 0.0))
    dom_us = per_call[dom]['mean_us']
    achieved = algo[dom] * tokens / (dom_us * 1e-6)
    hip_ms_per_step = sum(v['total_ms'] for v in per_call.values()) / args.steps
    fused = not bf16                    # the fused hash kernels run in fp32 outside autocast
    hip_b = hip_bytes_per_token(d, P, cf, T, layer.vistos, a=2 if bf16 else 4, K=layer.sufijo, fused=fused)
    layer_b = hip_b + gemm_bytes_per_token(d, P, cf, a=2 if bf16 else 4, fused=fused)

    out = {
        'metric': METRIC, 'value': round(value, 1), 'unit': 'tokens/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(wall * 1e3, 4), 'higher_is_better': True, 'scaling': 'weak',
        'vs_baseline': None, 'dtype': dtype, 'data': f'synthetic (seeded tokens, {int(cfg["frac"] * 100)}% copied '
        'spans; random-init layer moved off its neutral values)',
        'config': {'workload': f'{args.config}: one ASRN layer fwd+bwd, B={B}, N={N}, d={d}, V={V}, T=8 tables x 14 '
                               f'bits, C=32, {dtype}', 'global_batch': B, 'seq_len': N, 'parallelism': 'none (1 GPU)',
                   'launch': 'eager' if graph is None else 'hip graph replay', 'gemms': gemm_picks},
        'eager_ms_per_step': round(eager_wall * 1e3, 4),
        'roofline': {'bound': 'hbm', 'kernel': dom, 'achieved': round(achieved / 1e9, 1), 'peak': HBM_PEAK / 1e9,
                     'unit': 'GB/s', 'frac': round(achieved / HBM_PEAK, 4), 'traffic': measured_traffic(dom) if args.config == 'cfg2' else None,
                     'bytes_per_token': algo[dom], 'mean_launch_us': round(dom_us, 2)},
        'hip_aggregate': {'bytes_per_token': hip_b, 'hip_ms_per_step': round(hip_ms_per_step, 4),
                          'frac': round(hip_b * tokens / (HBM_PEAK * hip_ms_per_step * 1e-3), 4)},
        'layer': {'tokens_per_s': round(value, 1),
                  'bytes_per_token': layer_b, 'hbm_frac': round(layer_b * tokens / (HBM_PEAK * wall), 4)},
        'kernels': {n: {k: round(v, 3) if isinstance(v, float) else v for k, v in s.items()}
                    for n, s in sorted(per_call.items(), key=lambda kv: -kv[1]['total_ms'])},
    }
    if not args.no_decode:
        out['decode'] = decode_bench(dev, args.decode_steps, 20, seed=args.seed)
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline(layer_cpu, x, E, h, gy)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
