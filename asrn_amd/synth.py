"""Seeded synthetic token streams and layer inputs for the benchmark configurations.

Tokens are uniform (or Zipf) ids with a fraction of positions overwritten by copies of earlier spans, so buckets
fill, suffixes match and n-grams repeat. Layer inputs follow the reference's single-layer benchmark
(benchmarks/banco_gpu.py:102-110, 293-296): E = randn(V, d)[x], h = randn(B, N, d), and the layer's parameters are
moved off their neutral values (p += 0.5 randn for the clock/Hawkes/gate parameters, 0.05 randn otherwise, then
gamma = |gamma|).
"""
import torch

# the parameters that start neutral in the reference (asrn/nucleo.py:2093)
NUEVOS = ('w_reloj', 'b_reloj', 'gamma', 'log_kappa', 'log_kappa_racha', 'u_hawkes', 'd_racha')

CONFIGS = {
    'cfg1': dict(B=8, N=256, d=64, V=256, frac=0.30, span=(8, 64), zipf=None),
    'cfg2': dict(B=8, N=4096, d=256, V=256, frac=0.30, span=(8, 64), zipf=None),
    'cfg3': dict(B=4, N=65536, d=512, V=32000, frac=0.20, span=(16, 256), zipf=1.1),
}


def tokens(B, N, V, frac=0.3, span=(8, 64), zipf=None, seed=0):
    """(B, N) int64 token ids: uniform over V (or Zipf with exponent `zipf`), then, per row, copies of earlier spans
    (length uniform in `span`, destination p uniform in [1, N - l], source uniform in [0, p - l]) until `frac` of the
    positions are covered."""
    g = torch.Generator().manual_seed(seed)
    if zipf:
        p = (torch.arange(V, dtype=torch.float64) + 1) ** -zipf
        x = torch.multinomial(p, B * N, replacement=True, generator=g).view(B, N)
    else:
        x = torch.randint(0, V, (B, N), generator=g)
    lo, hi = span
    for b in range(B):
        covered = torch.zeros(N, dtype=torch.bool)
        target = int(frac * N)
        tries = 0
        while int(covered.sum()) < target and tries < 100 * N:
            tries += 1
            ln = int(torch.randint(lo, hi + 1, (1,), generator=g))
            if N - ln < 1:
                continue
            dst = int(torch.randint(1, N - ln + 1, (1,), generator=g))
            if dst < ln:
                continue
            src = int(torch.randint(0, dst - ln + 1, (1,), generator=g))
            x[b, dst:dst + ln] = x[b, src:src + ln].clone()
            covered[dst:dst + ln] = True
    return x


def move_params(layer, seed=0):
    """Moves the layer's parameters off their neutral values, deterministically."""
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            p.add_((torch.randn(p.shape, generator=g) * (0.5 if n in NUEVOS else 0.05)).to(p.device, p.dtype))
        layer.gamma.abs_()
    return layer


def layer_inputs(B, N, d, V, seed=0, **tok):
    """x (B, N), E (B, N, d), h (B, N, d) on the CPU, seeded."""
    x = tokens(B, N, V, seed=seed, **tok)
    g = torch.Generator().manual_seed(seed + 100)
    E = torch.randn(V, d, generator=g)[x]
    h = torch.randn(B, N, d, generator=g)
    return x, E, h
