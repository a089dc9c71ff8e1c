"""Benchmark of the ASRN layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--config cfg2|cfg3] [--no-cpu-baseline] [--no-decode]
                    [--decode-steps 1024] [--decode-only] [--no-model] [--model-only]
                    [--model-steps 20]

A step is one forward + backward of one ASRN layer (asrn.ASRNLayer, group-A protections) over one batch of
synthetic tokens: BASELINE.json configs[1] = cfg2, B 8, N 4096, d 256, V 256, fp32, 30% copied spans (--config cfg3:
configs[2], B 4, N 65,536, d 512, V 32,000, Zipf tokens, bf16 autocast; run it with --no-decode). Inputs and
weights are resident in HBM before the timed region. The step is captured once into a HIP graph and the timed steps
are its replays (the same kernels, launched without the host's per-op overhead); --eager times Python-launched steps
instead. The per-kernel device events (roofline, hip_aggregate, kernels) come from an eager pass of the same number of
steps, since events recorded while capturing are not replayed. Prints one JSON line with the driver's keys plus:
  roofline      the dominant HIP kernel: algorithmic bytes per launch / its mean launch time (device events recorded
                on the stream it runs on), against MI355X's 8 TB/s
  survey_headline  SURVEY.md section 8(d)'s headline: the compulsory bytes of the HIP kernels K1-K5 (7,776 B/token at
                cfg2) over their summed kernel time per fwd+bwd (the committed rocprofv3 kernel trace, and the eager
                pass's device events beside it), against 8 TB/s; its target is 0.5
  hip_aggregate all HIP kernels: 24,240 B/token (cfg2) x tokens / (8 TB/s x their summed time per step), the time
                from the committed rocprofv3 kernel trace (profiles/cfg2_kernel_times.json) where there is one
  layer         whole-layer tokens/s and its HBM fraction at SURVEY.md 8(d)'s compulsory 25,876 B/token (cfg2; 24,436
                at cfg3), and beside it at the implementation's own count (the HIP kernels' bytes plus the GEMMs'
                operands and results, 39,088 B/token at cfg2)
  decode        configs[4]'s greedy generation with the whole d = 768 model (B 16): per-token latency over 1,024
                steps against the context, 1K to 64K, and its slope
  modelo        the whole model's training step as PasoGrafado replays it: configs[3] (V 50,304, d 768, 12 local
                blocks, 6 ASRN layers, B 8, N 2,048, bf16 autocast, AdamW) and configs[0] (the quick-start model,
                fp32, 8 x 256 tokens)
  cpu_baseline  the CPU oracle (oracle/layer.py, PyTorch fp32 on the host cores) on the same workload (a bounded
                sample of it for cfg3)
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


def context_bytes(d, cf=16, proj=True):
    """The fused LayerNorm + clock projection (asrn_context_fwd/bwd), fp32: h in, hh, (mean, rstd, u) and beta (fp64),
    log_alfa out; the backward reads h, the Qc/Kc gradient (proj: the 2 cf values of dy, from which it forms dhh;
    else the GEMM's dhh), the gate's dh, the stats, dbeta, dlog_alfa and writes dh."""
    dq = 4 * 2 * cf if proj else 4 * d
    return 4 * d + 4 * d + 16 + 8 + 4, 4 * d + dq + 4 * d + 16 + 8 + 4 + 4 * d


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
    """All HIP kernels of one fwd+bwd, each distinct tensor read once and written once: sign hash + bucket sort (fused:
    the hash kernel writes the ids, the sort reads them and writes the order; else the sort reads phi and writes ids
    and order), clock 16 + 16, n-gram sort 28, Hawkes/streak scans 60 + 100, candidates, gate, context producer, the
    hash MLPs (fused: hash_bytes; else the hidden layer and its bias column sums), and the column sums of the
    candidates' per-token partials (the weight gradients' slab sums scale with the weights, not the tokens, and are
    left out).
    cfg2 fp32 (fused): 96 + 32 + 28 + 160 + 7,044 + 8,324 + 5,304 + 3,200 + 52 = 24,240."""
    cand = algorithmic_bytes(d, P, cf, T, a)
    colsums = 4 * (T + K + 1) + (0 if fused else 4 * (m + mc) + 4 * P)
    mlp = sum(hash_bytes(P, m, mc)) if fused else sum(hidden_bytes(m, mc))
    return ((4 * T if fused else P * a) + 8 * T + 32 + 28 + 160 + sum(cand.values()) + sum(gate_bytes(d, n, a))
            + sum(context_bytes(d, cf, proj=fused)) + mlp + colsums)


def gemm_bytes_per_token(d, P, cf, a=4, m=64, mc=64, fused=True):
    """Operands and results of the layer's GEMMs per token, each read or written once (activations in a bytes;
    weights are per step, not per token): forward E -> [hp|za|zb], hh -> [Qc|Kc], sum -> W_o W_v sum and, unfused,
    g -> phi; backward the input gradients (the E one accumulating into the candidates' dE; fused, the [Qc|Kc] one is
    formed inside the context backward instead) and the weight gradients (both operands read).
    cfg2 fp32 (fused): 4,992 + 9,856 = 14,848."""
    h, q = m + 2 * mc, 2 * cf
    fwd = (d + h) + (d + q) + (d + d) + (0 if fused else (m + mc) + P)
    bwd = (d + d) + 2 * d + (0 if fused else (q + d)) + (q + d) + (h + 2 * d) + (h + d) + (0 if fused else 2 * (P + m + mc))
    return a * (fwd + bwd)


# SURVEY.md section 8(d)'s compulsory bytes per token (each distinct tensor read once and written once per pass) at its
# two layer configurations: the HIP kernels K1-K5 (hash + bucket sort, clock, n-gram sort, Hawkes/streak scans,
# candidates; forward + backward) and the whole layer (adding the GEMM-boundary tensors)
SURVEY_BYTES = {'cfg2': {'hip': 3340 + 4436, 'layer': 10680 + 15196},
                'cfg3': {'hip': 2828 + 3860, 'layer': 24436}}
# the library entry points whose kernels are K1-K5 (the clock scan runs forward and backward)
K1_K5 = {'K1 hash + bucket sort': ['asrn_bucket_sort'], 'K2 clock': ['asrn_clock_scan'],
         'K3 n-gram sort': ['asrn_ngram_sort'],
         'K4 Hawkes/streak scans': ['asrn_hawkes_fwd', 'asrn_hawkes_bwd', 'asrn_streak_fwd', 'asrn_streak_bwd',
                                    'asrn_repetition_fwd', 'asrn_repetition_bwd'],
         'K5 candidates': ['asrn_candidates_fwd', 'asrn_candidates_bwd']}


def survey_headline(config, tokens, per_call, steps, prof):
    """SURVEY section 8(d)'s headline: K1-K5's compulsory bytes over their summed kernel time per fwd+bwd, against
    8 TB/s. From the committed rocprofv3 kernel trace of this configuration (profiles/<config>_kernel_times.json,
    'k1_k5_us_per_step') when there is one, and from the device events around each entry point in the eager pass
    (these also hold the host's launch gaps of a host-bound step, so they read high)."""
    b = SURVEY_BYTES.get(config)
    if b is None:
        return None
    groups = {}
    for g, names in K1_K5.items():
        groups[g] = round(1e3 * sum(per_call[n]['total_ms'] for n in names if n in per_call) / steps, 2)
    ev_us = sum(groups.values())
    out = {'bytes_per_token': b['hip'], 'target_frac': 0.5,
           'events_us_per_step': round(ev_us, 1), 'events_us_by_kernel': groups,
           'frac_events': round(b['hip'] * tokens / (HBM_PEAK * ev_us * 1e-6), 4) if ev_us else None}
    if prof and prof.get('k1_k5_us_per_step'):
        us = prof['k1_k5_us_per_step']
        out.update({'rocprof_us_per_step': us, 'rocprof_us_by_kernel': prof.get('k1_k5_us_by_kernel'),
                    'frac': round(b['hip'] * tokens / (HBM_PEAK * us * 1e-6), 4),
                    'source': 'rocprofv3 kernel trace, profiles/%s_kernel_times.json' % config})
    return out


TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'cfg2_traffic.json')


def measured_traffic(kernel):
    """HBM bytes per launch of an entry point from the committed counter passes (FETCH_SIZE and WRITE_SIZE, scaled
    by a copy of known size), or None when they were not taken for this build."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)['bytes_per_launch'].get(kernel)
    except (OSError, ValueError, KeyError):
        return None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or '' where it cannot be read."""
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return ''


def cpu_baseline(layer_cpu, x, E, h, gy, reps=3, max_tokens=32768):
    """The CPU oracle's layer forward + backward (oracle/layer.py, PyTorch fp32 on all host cores), median of `reps`
    after 1 warm-up, on the same inputs; workloads over `max_tokens` tokens are timed on a bounded sample (the first
    rows, cut to at most max_tokens tokens in all) so that the run stays within about half a minute."""
    import torch
    from oracle import layer as O
    torch.set_num_threads(os.cpu_count() or 1)
    B, N = x.shape
    full = B * N <= max_tokens
    if not full:
        rows = max(1, max_tokens // N)
        n = min(N, max_tokens // rows)
        x, E, h, gy = x[:rows, :n], E[:rows, :n], h[:rows, :n], gy[:rows, :n]
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
    what = (f'full workload ({x.shape[0]}x{x.shape[1]} tokens)' if full else
            f'bounded sample: the first {x.shape[0]}x{x.shape[1]} tokens of the {B}x{N} workload')
    return {'value': round(tokens / t, 1), 'unit': 'tokens/s', 'cores': torch.get_num_threads(), 'kind': 'port',
            'sample': f'{what}, fp32, median of {reps} after 1 warm-up; cpu_count={os.cpu_count()}',
            'cpu_model': cpu_model(), 'seconds_per_step': round(t, 3)}


def kernel_times(config):
    """The committed rocprofv3 kernel-trace summary of this configuration (profiles/<config>_kernel_times.json:
    'hip_us_per_step', 'k1_k5_us_per_step', ...), or None when there is none."""
    try:
        with open(os.path.join(ROOT, 'profiles', f'{config}_kernel_times.json')) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def profiled_hip_us(config):
    """The HIP kernels' summed time per step from the committed rocprofv3 kernel trace of this configuration, or None
    when there is none."""
    return (kernel_times(config) or {}).get('hip_us_per_step')


DECODE = dict(B=16, V=50304, d=768, n_capas=12, contexts=(1024, 4096, 16384, 32768, 65536), frac=0.2,
              span=(16, 256), zipf=1.1)


def decode_bench(dev, steps, warmup, seed=0, contexts=None):
    """greedy generation (top_k=1, memoria_de_lo_ajeno=False, so every new position enters
    the rings; the quote correction on, the reference's default) with the whole d = 768 model of configs[3] (12 local
    blocks, 6 ASRN layers, tied head; random-init weights from the seed, fp32), B = 16, after a prefill of each context
    length, 1K to 64K. A step is escribir's loop step: the token choice (asrn_sample) and the model's O(1) step, one HIP
    graph replay. Per-token latency is wall clock over `steps` back-to-back steps (synchronized at both ends); the
    least-squares slope against the context, with its 95% interval, is the O(1) check. The first step runs op by op,
    and there each HIP entry point is timed with device events (a replay makes no library call to time)."""
    import torch

    import asrn_amd
    from asrn_amd import _lib, synth
    from asrn_amd.generacion import EscritorModelo, _Bucle

    cfg = DECODE
    B, V = cfg['B'], cfg['V']
    contexts = contexts or cfg['contexts']
    m = asrn_amd.crear_modelo(V, d=cfg['d'], n_capas=cfg['n_capas'], largo_cada=2, semilla=seed).to(dev).eval()
    rows, kern = [], {}
    w = max(warmup, 2)
    nombres = ['asrn_sample', 'asrn_decode_produce', 'asrn_repetition_step', 'asrn_decode_attend', 'asrn_gate_step',
               'asrn_block_step']
    with torch.no_grad():
        for ctx in contexts:
            x = synth.tokens(B, ctx, V, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'], seed=seed + ctx).to(dev)
            n = w + steps + 1
            esc = EscritorModelo(m, memoria_de_lo_ajeno=False)
            lg = esc.inicio(x, capacidad=ctx + n)
            esc.reservar(ctx + n)
            bucle = _Bucle(esc, x, n, 1.0, 1, seed, 1.0, 64, 0, None, 1.0, False, True, True)
            bucle.lg.copy_(lg)
            del lg
            timed = _lib.time_calls(nombres)
            bucle.paso(0)                                          # op by op: its kernels timed
            timed = _lib.stop_timing()
            for k in range(1, w):                                  # the first of these captures the step
                bucle.paso(k)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for k in range(w, w + steps):
                bucle.paso(k)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for name, evs in timed.items():
                kern.setdefault(name, []).extend(s.elapsed_time(e) for s, e in evs)
            ms = 1e3 * (t1 - t0) / steps
            rows.append({'context': ctx, 'ms_per_step': round(ms, 4), 'tokens_per_s': round(B * 1e3 / ms, 1),
                         'kernel_us_first_step': {name: round(1e3 * sum(s.elapsed_time(e) for s, e in evs), 2)
                                                  for name, evs in timed.items() if evs}})
            del bucle, esc, x
            torch.cuda.empty_cache()
    xs = [r['context'] for r in rows]
    ys = [r['ms_per_step'] * 1e6 for r in rows]        # ns
    k = len(xs)
    mx, my = sum(xs) / k, sum(ys) / k
    sxx = sum((a - mx) ** 2 for a in xs)
    slope = sum((a - mx) * (b - my) for a, b in zip(xs, ys)) / sxx if sxx else 0.0
    res = [b - (my + slope * (a - mx)) for a, b in zip(xs, ys)]
    se = (sum(r * r for r in res) / max(k - 2, 1) / sxx) ** 0.5 if sxx else 0.0
    t975 = {1: 12.71, 2: 4.30, 3: 3.18, 4: 2.78, 5: 2.57}.get(k - 2, 2.0)
    return {'workload': f"configs[4]: greedy generation with the whole configs[3] model (V={V}, d={cfg['d']}, "
                        f"{cfg['n_capas']} local blocks, {len(m.largos)} ASRN layers, random-init fp32), B={B}, Zipf 1.1 "
                        f'tokens with 20% copied spans, prefill of each context then {w} + {steps} steps, every '
                        'position a key, quote correction on',
            'parameters': m.num_parametros(), 'launch': 'hip graph replay of the whole loop step (choice + model)',
            'per_context': rows, 'tokens_per_s': rows[-1]['tokens_per_s'],
            'slope_ns_per_context_token': round(slope, 4),
            'slope_ci95': [round(slope - t975 * se, 4), round(slope + t975 * se, 4)],
            'kernels_op_by_op_step': {name: {'launches': len(v), 'mean_us': round(1e3 * sum(v) / len(v), 3)}
                                      for name, v in kern.items() if v}}


# BASELINE.json configs[3] (the d = 768 LM training step) and configs[0] (the quick-start model's step)
MODELOS = {
    'cfg4': dict(kw=dict(V=50304, d=768, n_capas=12, largo_cada=2), B=8, N=2048, precision='bf16', frac=0.15,
                 span=(8, 128), zipf=1.1),
    'cfg1': dict(kw=dict(V=256, d=64, n_capas=4), B=8, N=256, precision='fp32', frac=0.3, span=(8, 64), zipf=None),
}


def modelo_bench(dev, nombre, steps, warmup, seed=0, eager_steps=5):
    """One whole training step of ModeloASRN (forward, fp32 cross-entropy, backward, clipping at 1.0, fused AdamW)
    as PasoGrafado replays it: the step captured once into a HIP graph, new batches copied into its inputs each
    step. Weights random-init from the seed (create_model(..., semilla=seed)), synthetic tokens of the config's
    distribution, all resident in HBM. Also the same step launched op by op (eager_steps of them), for the host
    overhead the graph removes."""
    import torch

    import asrn_amd
    from asrn_amd import synth

    cfg = MODELOS[nombre]
    B, N = cfg['B'], cfg['N']
    m = asrn_amd.crear_modelo(**cfg['kw'], semilla=seed).to(dev).train()
    opt = asrn_amd.crear_optimizador(m, lr=1e-3, capturable=True)
    nb = 4
    w = synth.tokens(B * nb, N + 1, cfg['kw']['V'], frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'],
                     seed=seed + 11).to(dev)
    lotes = [(w[B * i:B * i + B, :-1].contiguous(), w[B * i:B * i + B, 1:].contiguous()) for i in range(nb)]

    def correr(paso, n, desde):
        ultimo = None
        for i in range(n):
            x, y = lotes[(desde + i) % nb]
            ultimo = paso(x, y, lr=1e-3)
        return ultimo

    eager = asrn_amd.PasoGrafado(m, opt, B, N, precision=cfg['precision'], grabar=False)
    correr(eager, 2, 0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    correr(eager, eager_steps, 0)
    torch.cuda.synchronize()
    eager_ms = 1e3 * (time.perf_counter() - t0) / eager_steps
    del eager
    grafo = asrn_amd.PasoGrafado(m, opt, B, N, precision=cfg['precision'], calentar=2)
    correr(grafo, max(warmup, 3), 0)                              # 2 side-stream steps, then capture and replays
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    perdida, norma, salto = correr(grafo, steps, 0)
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / steps
    return {'workload': f"configs[{'3' if nombre == 'cfg4' else '0'}]: ModeloASRN training step, "
                        f"V={cfg['kw']['V']}, d={cfg['kw']['d']}, {cfg['kw']['n_capas']} local blocks, "
                        f"{len(m.largos)} ASRN layers, B={B}, N={N}, {cfg['precision']} autocast, fp32 weights, "
                        'AdamW (fused, capturable), clip 1.0; synthetic tokens, random-init weights',
            'parameters': m.num_parametros(), 'tokens_per_s': round(B * N * 1e3 / ms, 1), 'ms_per_step': round(ms, 3),
            'steps': steps, 'launch': 'PasoGrafado: hip graph replay of the whole step',
            'eager_ms_per_step': round(eager_ms, 3), 'last_loss': round(float(perdida), 5),
            'skipped_last': float(salto)}


def hip_aggregate(hip_b, tokens, eager_ms, prof_us):
    """All HIP kernels' algorithmic bytes over their summed time per step: from the committed rocprofv3 kernel trace
    when there is one (the eager pass's event times include the host's launch gaps of a host-bound step), else from
    those events."""
    if prof_us:
        return {'bytes_per_token': hip_b, 'hip_us_per_step': prof_us, 'source': 'rocprofv3 kernel trace, '
                'profiles/cfg2_kernel_times.json', 'frac': round(hip_b * tokens / (HBM_PEAK * prof_us * 1e-6), 4)}
    return {'bytes_per_token': hip_b, 'hip_us_per_step': round(eager_ms * 1e3, 1),
            'source': 'device events around each library call in the eager pass (include launch gaps)',
            'frac': round(hip_b * tokens / (HBM_PEAK * eager_ms * 1e-3), 4)}


# kernel names (rocprofv3) of the K1-K5 groups and of the entry points whose traffic is reported
K1_K5_KERNELS = {'K1 hash + bucket sort': ('k_bucket_',), 'K2 clock': ('ClockOp',),
                 'K3 n-gram sort': ('k_ngram_', 'k_merge_pass'),
                 'K4 Hawkes/streak scans': ('Hawkes', 'Streak', 'k_hawkes_'), 'K5 candidates': ('k_cand_',)}
ENTRY_KERNELS = {'asrn_candidates_fwd': ('k_cand_fwd',), 'asrn_candidates_bwd': ('k_cand_bwd_q', 'k_cand_bwd_k'),
                 'asrn_bucket_sort': ('k_bucket_',), 'asrn_ngram_sort': ('k_ngram_', 'k_merge_pass')}


def _csv_rows(path):
    import csv
    import glob
    files = glob.glob(os.path.join(path, '**', '*.csv'), recursive=True) if os.path.isdir(path) else [path]
    return files, csv


def summarize_trace(path, steps, command):
    """A rocprofv3 --kernel-trace --stats run (its directory) of `steps` traced steps -> the per-step summary that
    profiles/<config>_kernel_times.json holds: all kernels, the HIP library's, and K1-K5 by group and kernel."""
    files, csv = _csv_rows(path)
    stats = [f for f in files if f.endswith('kernel_stats.csv')]
    if not stats:
        raise SystemExit(f'no kernel_stats.csv under {path}')
    rows = list(csv.DictReader(open(stats[0])))
    per = {r['Name']: float(r['TotalDurationNs']) / 1e3 / steps for r in rows}
    calls = {r['Name']: int(r['Calls']) / steps for r in rows}
    groups, by_kernel = {}, {}
    for g, keys in K1_K5_KERNELS.items():
        ks = {n: us for n, us in per.items() if 'asrn::' in n and any(k in n for k in keys)}
        groups[g] = round(sum(ks.values()), 2)
        for n, us in ks.items():
            by_kernel[n.split('(')[0]] = {'us_per_step': round(us, 2), 'launches_per_step': calls[n]}
    return {'hip_us_per_step': round(sum(us for n, us in per.items() if 'asrn::' in n), 1),
            'all_kernels_us_per_step': round(sum(per.values()), 1),
            'k1_k5_us_per_step': round(sum(groups.values()), 1), 'k1_k5_us_by_kernel': groups,
            'k1_k5_kernels': by_kernel, 'traced_steps': steps, 'source': command}


def summarize_traffic(fetch, write, cal_fetch, cal_write, cal_bytes, command):
    """rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE runs of the eager bench, and the same passes over a plain copy
    of cal_bytes (bench.py --copy-calibration) -> HBM bytes per launch of the entry points in ENTRY_KERNELS."""
    def per_kernel(path, counter):
        files, csv = _csv_rows(path)
        vals = {}
        for f in files:
            if f.endswith('counter_collection.csv'):
                for r in csv.DictReader(open(f)):
                    if r['Counter_Name'] == counter:
                        vals.setdefault(r['Kernel_Name'], []).append(float(r['Counter_Value']))
        return {k: sum(v) / len(v) for k, v in vals.items()}
    def copy_kib(path, counter):
        v = per_kernel(path, counter)
        return max(v.values()) if v else None
    f_scale = cal_bytes / 1024 / copy_kib(cal_fetch, 'FETCH_SIZE')
    w_scale = cal_bytes / 1024 / copy_kib(cal_write, 'WRITE_SIZE')
    fk, wk = per_kernel(fetch, 'FETCH_SIZE'), per_kernel(write, 'WRITE_SIZE')
    out = {}
    for e, keys in ENTRY_KERNELS.items():
        names = [n for n in fk if 'asrn::' in n and any(k in n for k in keys)]
        if names:
            out[e] = int(1024 * sum(f_scale * fk[n] + w_scale * wk.get(n, 0.0) for n in names))
    return {'calibration': {'FETCH_SIZE_KiB_scale': f_scale, 'WRITE_SIZE_KiB_scale': w_scale,
                            'copy_bytes': cal_bytes},
            'bytes_per_launch': out, 'source': command}


def summarize_kernels(trace, steps, fetch, write, sq1, sq2, cal_fetch, cal_write, cal_bytes, algo_mb=None, top=30):
    """A markdown table of the HIP kernels of one traced configuration: launches and mean time (kernel trace), VGPRs,
    LDS and workgroup size (dispatch records), HBM bytes per launch (FETCH_SIZE / WRITE_SIZE calibrated by a copy),
    L2 hit rate, LDS bank-conflict cycles per LDS instruction, VALU and LDS instructions per wave and the SIMDs'
    VALU-busy fraction: SQ_ACTIVE_INST_VALU (quad-cycles, summed over the chip) over CU_NUM x the kernel's cycles
    (GRBM_GUI_ACTIVE, which the profiler sums over the 8 XCDs)."""
    import csv
    def counters(path):
        files, _ = _csv_rows(path)
        acc = {}
        for f in files:
            if f.endswith('counter_collection.csv'):
                for r in csv.DictReader(open(f)):
                    d = acc.setdefault(r['Kernel_Name'], {'meta': r})
                    d.setdefault(r['Counter_Name'], []).append(float(r['Counter_Value']))
        return {k: {c: (sum(v) / len(v) if c != 'meta' else v) for c, v in d.items()} for k, d in acc.items()}
    files, _ = _csv_rows(trace)
    stats = list(csv.DictReader(open([f for f in files if f.endswith('kernel_stats.csv')][0])))
    disp = {}
    for r in csv.DictReader(open([f for f in files if f.endswith('kernel_trace.csv')][0])):
        disp.setdefault(r['Kernel_Name'], r)
    cf, cw = counters(cal_fetch), counters(cal_write)
    f_scale = cal_bytes / 1024 / max(v.get('FETCH_SIZE', 0) for v in cf.values())
    w_scale = cal_bytes / 1024 / max(v.get('WRITE_SIZE', 0) for v in cw.values())
    F, W, S1, S2 = counters(fetch), counters(write), counters(sq1), counters(sq2)
    rows = []
    for r in stats:
        n = r['Name']
        if 'asrn::' not in n:
            continue
        us = float(r['AverageNs']) / 1e3
        d = disp.get(n, {})
        mb = (f_scale * F.get(n, {}).get('FETCH_SIZE', 0.0) + w_scale * W.get(n, {}).get('WRITE_SIZE', 0.0)) * 1024 / 1e6
        s1, s2 = S1.get(n, {}), S2.get(n, {})
        waves = s1.get('SQ_WAVES') or float('nan')
        hit = s2.get('TCC_HIT_sum', 0.0)
        miss = s2.get('TCC_MISS_sum', 0.0)
        lds = s2.get('SQ_ACTIVE_INST_LDS') or float('nan')
        grbm = s1.get('GRBM_GUI_ACTIVE') or float('nan')
        rows.append((int(r['Calls']) / steps * us, n.split('(')[0][:60], int(r['Calls']) / steps, us,
                     d.get('LDS_Block_Size', ''), d.get('Workgroup_Size_X', ''), mb,
                     mb / 1e3 / (us * 1e-6) if us else 0.0, hit / (hit + miss) if hit + miss else float('nan'),
                     s2.get('SQ_LDS_BANK_CONFLICT', 0.0) / lds, s1.get('SQ_INSTS_VALU', float('nan')) / waves,
                     s1.get('SQ_INSTS_LDS', float('nan')) / waves,
                     s1.get('SQ_ACTIVE_INST_VALU', float('nan')) / (256 * grbm / 8)))
    rows.sort(key=lambda x: -x[0])
    out = ['| kernel | launches/step | us | LDS B | WG | HBM MB/launch | GB/s | L2 hit | LDS conflict/inst | '
           'VALU inst/wave | LDS inst/wave | SIMD VALU busy |', '|' + '---|' * 12]
    for x in rows[:top]:
        out.append(f'| `{x[1]}` | {x[2]:.1f} | {x[3]:.1f} | {x[4]} | {x[5]} | {x[6]:.1f} | {x[7]:.0f} | '
                   f'{x[8]:.2f} | {x[9]:.2f} | {x[10]:.0f} | {x[11]:.0f} | {x[12]:.2f} |')
    out.append('')
    out.append(f'Copy calibration: FETCH_SIZE x {f_scale:.3f} KiB, WRITE_SIZE x {w_scale:.3f} KiB '
               f'(a {cal_bytes}-byte device copy).')
    return '\n'.join(out)


def _short(name):
    """A kernel's name without its namespace noise and argument list."""
    return name.replace('(anonymous namespace)::', '').split('(')[0].replace('void ', '')


def summarize_decode(trace, fetch, write, cal_fetch, cal_write, cal_bytes, steps=64):
    """The decode leg's per-step kernels: from a rocprofv3 --kernel-trace of bench.py --decode-only, the last `steps`
    intervals from one k_sample launch to the next (graph replays): each kernel's (and grid's) launches per step and
    mean time; from --pmc FETCH_SIZE and WRITE_SIZE runs of the same command (optional), the HBM bytes per dispatch of
    that kernel and grid (calibrated by a copy, as summarize_traffic does), and the rate they make over the traced mean
    time. A markdown table."""
    import csv
    import collections
    files, _ = _csv_rows(trace)
    rows = list(csv.DictReader(open([f for f in files if f.endswith('kernel_trace.csv')][0])))
    rows.sort(key=lambda r: int(r['Start_Timestamp']))
    ks = [i for i, r in enumerate(rows) if 'k_sample' in r['Kernel_Name']]
    spans = [(ks[j], ks[j + 1]) for j in range(len(ks) - 1)][-steps:]
    dur, cnt, tot, kern = collections.defaultdict(list), collections.Counter(), [], []

    def grid(r):
        return int(r['Grid_Size_X']) * int(r.get('Grid_Size_Y') or 1) * int(r.get('Grid_Size_Z') or 1)

    for a, b in spans:
        tot.append((int(rows[b]['Start_Timestamp']) - int(rows[a]['Start_Timestamp'])) / 1e3)
        kern.append(sum(int(r['End_Timestamp']) - int(r['Start_Timestamp']) for r in rows[a:b]) / 1e3)
        for r in rows[a:b]:
            key = (_short(r['Kernel_Name']), grid(r))
            dur[key].append((int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3)
            cnt[key] += 1

    def per_dispatch(path, counter):
        if not path:
            return {}
        fs, _ = _csv_rows(path)
        vals = collections.defaultdict(list)
        for f in fs:
            if f.endswith('counter_collection.csv'):
                for r in csv.DictReader(open(f)):
                    if r['Counter_Name'] == counter:
                        vals[(_short(r['Kernel_Name']), int(r.get('Grid_Size') or 0))].append(float(r['Counter_Value']))
        return {k: sum(v) / len(v) for k, v in vals.items()}

    scale = {}
    if cal_fetch and cal_write:
        cf, cw = per_dispatch(cal_fetch, 'FETCH_SIZE'), per_dispatch(cal_write, 'WRITE_SIZE')
        scale = {'f': cal_bytes / 1024 / max(cf.values()), 'w': cal_bytes / 1024 / max(cw.values())}
    F, W = per_dispatch(fetch, 'FETCH_SIZE'), per_dispatch(write, 'WRITE_SIZE')
    n_steps = len(spans)
    out = [f'{n_steps} steps: {sum(kern) / n_steps:.1f} us of kernel time and {sum(tot) / n_steps:.1f} us from one token '
           f'choice to the next per step, {sum(cnt.values()) / n_steps:.0f} kernels per step.', '',
           '| kernel | grid (threads) | launches/step | us/step | mean us | HBM KB/dispatch | GB/s |',
           '|---|---|---|---|---|---|---|']
    for key in sorted(dur, key=lambda k: -sum(dur[k])):
        n, g = key
        mean = sum(dur[key]) / len(dur[key])
        kb = rate = ''
        if scale and key in F:
            b = 1024 * (scale['f'] * F[key] + scale['w'] * W.get(key, 0.0))
            kb, rate = f'{b / 1e3:.0f}', f'{b / 1e3 / mean:.0f}'
        out.append(f'| `{n[:60]}` | {g} | {cnt[key] / n_steps:.1f} | {sum(dur[key]) / n_steps:.1f} | {mean:.2f} | '
                   f'{kb} | {rate} |')
    return '\n'.join(out)


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
    ap.add_argument('--decode-steps', type=int, default=1024)
    ap.add_argument('--decode-contexts', default=None, help='comma-separated prefill lengths (default 1K,4K,16K,32K,64K)')
    ap.add_argument('--decode-only', action='store_true',
                    help='only the generation leg (configs[4], the whole model); prints its JSON object')
    ap.add_argument('--eager', action='store_true', help='time Python-launched steps instead of HIP graph replays')
    ap.add_argument('--no-model', action='store_true', help='skip the whole-model training-step legs')
    ap.add_argument('--model-only', action='store_true',
                    help='only the whole-model training-step legs (configs[3] and configs[0]); prints their JSON')
    ap.add_argument('--model-steps', type=int, default=20)
    ap.add_argument('--default-gemms', action='store_true',
                    help="leave the GEMMs on the libraries' default picks instead of the shipped MI355X picks")
    ap.add_argument('--copy-calibration', type=int, default=0, metavar='BYTES',
                    help='only run a plain device-to-device copy of BYTES, 3 times: the reference point that scales '
                         'the FETCH_SIZE / WRITE_SIZE counters of a profiler run into bytes')
    ap.add_argument('--summarize-trace', metavar='DIR', default=None,
                    help='only summarize a rocprofv3 kernel-trace directory of --trace-steps steps into the JSON of '
                         'profiles/<config>_kernel_times.json (printed); needs no GPU')
    ap.add_argument('--trace-steps', type=int, default=13)
    ap.add_argument('--summarize-decode', nargs=6, default=None,
                    metavar=('TRACE', 'FETCH', 'WRITE', 'CAL_FETCH', 'CAL_WRITE', 'CAL_BYTES'),
                    help="only summarize the decode leg's kernel trace and its FETCH_SIZE / WRITE_SIZE runs ('-' for "
                         'none) into a markdown table of the per-step kernels')
    ap.add_argument('--summarize-traffic', nargs=5, metavar=('FETCH', 'WRITE', 'CAL_FETCH', 'CAL_WRITE', 'CAL_BYTES'),
                    default=None, help='only turn FETCH_SIZE / WRITE_SIZE counter runs and their copy calibration '
                                       'into the JSON of profiles/cfg2_traffic.json (printed); needs no GPU')
    ap.add_argument('--summarize-kernels', nargs=9, default=None,
                    metavar=('TRACE', 'FETCH', 'WRITE', 'SQ1', 'SQ2', 'CAL_FETCH', 'CAL_WRITE', 'CAL_BYTES', 'STEPS'),
                    help='only print the markdown kernel table of a traced configuration (profiles/*_kernels.md) '
                         'from its trace and counter runs; needs no GPU')
    ap.add_argument('--command', default='', help='the profiler command recorded with a summary')
    args = ap.parse_args()
    if args.summarize_decode:
        t, f, w, cf, cw, nb = args.summarize_decode
        print(summarize_decode(t, f if f != '-' else None, w if w != '-' else None, cf if cf != '-' else None,
                               cw if cw != '-' else None, int(nb)))
        return
    if args.summarize_trace:
        print(json.dumps(summarize_trace(args.summarize_trace, args.trace_steps, args.command), indent=1))
        return
    if args.summarize_kernels:
        t, f, w, q1, q2, cf, cw, nb, st = args.summarize_kernels
        print(summarize_kernels(t, int(st), f, w, q1, q2, cf, cw, int(nb)))
        return
    if args.summarize_traffic:
        f, w, cf, cw, nb = args.summarize_traffic
        print(json.dumps(summarize_traffic(f, w, cf, cw, int(nb), args.command), indent=1))
        return
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

    asrn_amd.cargar_biblioteca()
    gemm_picks = 'library defaults'
    if not args.default_gemms:
        from asrn_amd import tuning
        if tuning.use_tuned_gemms():
            gemm_picks = 'TunableOp picks, asrn_amd/data/gemm_picks_mi355x.csv'
    if args.model_only:
        print(json.dumps({'modelo': {n: modelo_bench(torch.device('cuda:0'), n, args.model_steps, 5, seed=args.seed)
                                     for n in MODELOS}, 'gemm_picks': gemm_picks}), flush=True)
        return
    contexts = [int(c) for c in args.decode_contexts.split(',')] if args.decode_contexts else None
    if args.decode_only:
        print(json.dumps({'decode': decode_bench(torch.device('cuda:0'), args.decode_steps, 20, seed=args.seed,
                                                  contexts=contexts),
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
    impl_b = hip_b + gemm_bytes_per_token(d, P, cf, a=2 if bf16 else 4, fused=fused)
    layer_b = SURVEY_BYTES.get(args.config, {}).get('layer', impl_b)

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
        'survey_headline': survey_headline(args.config, tokens, per_call, args.steps, kernel_times(args.config)),
        'hip_aggregate': hip_aggregate(hip_b, tokens, hip_ms_per_step, profiled_hip_us(args.config)),
        'layer': {'tokens_per_s': round(value, 1),
                  'bytes_per_token': layer_b, 'hbm_frac': round(layer_b * tokens / (HBM_PEAK * wall), 4),
                  'bytes_source': "SURVEY.md 8(d)'s compulsory whole-layer bytes",
                  'implementation_bytes_per_token': impl_b,
                  'implementation_hbm_frac': round(impl_b * tokens / (HBM_PEAK * wall), 4)},
        'kernels': {n: {k: round(v, 3) if isinstance(v, float) else v for k, v in s.items()}
                    for n, s in sorted(per_call.items(), key=lambda kv: -kv[1]['total_ms'])},
    }
    if not args.no_decode:
        out['decode'] = decode_bench(dev, args.decode_steps, 20, seed=args.seed, contexts=contexts)
    if not args.no_model:
        out['modelo'] = {n: modelo_bench(dev, n, args.model_steps, 5, seed=args.seed) for n in MODELOS}
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline(layer_cpu, x, E, h, gy)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
