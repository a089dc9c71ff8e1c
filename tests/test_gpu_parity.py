"""HIP kernels against the oracle and the reference's golden fixtures, on the GPU, through the C ABI.

Bit-exact: bucket ids, sorted orders, candidate lists, suffix-match lengths, n-gram keys, their order, the repeated
and seen flags, integer streaks. Within the north-star tolerance (1e-3 relative at fp32): outputs and gradients of
the candidate attention, the Hawkes and streak scans, the clock, and the whole layer. Each test prints the case it
runs before touching the device."""
import os
import math

import numpy as np
import pytest
import torch

import asrn_amd
from asrn_amd import ops, synth
from asrn_amd.capa import CapaASRNEstable
from asrn_amd.lineal import lineal
from oracle import layer as O
from tests import fixtures

pytestmark = pytest.mark.gpu
DEV = 'cuda'
TOL = 1e-3           # fp32 relative tolerance of the north star, on max |error| / max |reference|
CASES = fixtures.names(False)    # the fp32 fixtures (the bf16 ones: tests/test_gpu_fullsize.py)


def say(*a):
    print('[case]', *a, flush=True)


def rel_err(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    if a.numel() == 0:
        return 0.0
    return (a - b).abs().max().item() / (b.abs().max().item() + 1e-12)


def assert_close(a, b, what, tol=TOL):
    e = rel_err(a, b)
    assert e <= tol, f'{what}: relative error {e:.3g} > {tol}'


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    asrn_amd.cargar_biblioteca()


# ---------------------------------------------------------------------------------------------------------------------
# a1 + a2: bucket ids and the stable sort
# ---------------------------------------------------------------------------------------------------------------------

def check_bucket_sort(phi, T, nb):
    C = 32
    ids, order, ids_s, rank, win = ops.bucket_sort(phi.to(DEV), T, nb, C)
    ref_ids, ref_order = O.bucket_rows(phi.cpu(), T, nb)
    assert torch.equal(ids.cpu().long(), ref_ids.long())
    assert torch.equal(order.cpu().long(), ref_order)
    assert torch.equal(ids_s.cpu().long(), torch.gather(ref_ids.long(), 1, ref_order))
    B, L = phi.shape[0], phi.shape[1]
    inv = torch.empty_like(ref_order).scatter_(1, ref_order, torch.arange(L).expand(B * T, L))
    assert torch.equal(rank.cpu().long().permute(0, 2, 1).reshape(B * T, L), inv)
    # the recent-mates index: bucket mates before and after each position, clamped to C
    ids_np = ref_ids.numpy()
    before = np.zeros((B * T, L), dtype=np.int64)
    total = np.zeros((B * T, L), dtype=np.int64)
    for r in range(B * T):
        _, inv_r, counts = np.unique(ids_np[r], return_inverse=True, return_counts=True)
        seen = np.zeros(len(counts), dtype=np.int64)
        for t, g in enumerate(inv_r):
            before[r, t] = seen[g]
            seen[g] += 1
        total[r] = counts[inv_r]
    after = total - 1 - before
    want = torch.from_numpy(np.minimum(before, C) | (np.minimum(after, C) << 8))
    assert torch.equal(win.cpu().long().permute(0, 2, 1).reshape(B * T, L), want)
    return ids, order, ids_s, rank, win


@pytest.mark.parametrize('name', CASES)
def test_bucket_sort_golden(name):
    say('bucket_sort golden', name)
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    ids, order, ids_s, rank, win = ops.bucket_sort(g['phi'].to(DEV), sh.T, sh.nb, sh.C)
    assert torch.equal(ids.cpu().long(), g['ids'].long())
    assert torch.equal(order.cpu().long(), g['orden'])


@pytest.mark.parametrize('B,L,T,nb,mode', [(8, 4096, 8, 14, 'randn'), (2, 5000, 8, 14, 'few'), (1, 1, 8, 14, 'randn'),
                                           (3, 1023, 5, 3, 'randn'), (1, 2049, 8, 14, 'same'),
                                           (1, 65536, 8, 14, 'few'), (1, 4097, 8, 14, 'randn'),
                                           (4, 4096, 8, 14, 'few'), (5, 3, 3, 2, 'randn'), (3, 8200, 2, 1, 'randn')])
def test_bucket_sort_vs_numpy(B, L, T, nb, mode):
    say('bucket_sort', B, L, T, nb, mode)
    g = torch.Generator().manual_seed(L)
    P = T * nb
    if mode == 'randn':
        phi = torch.randn(B, L, P, generator=g)
    elif mode == 'few':                           # few distinct rows: long runs of ties in every bucket
        phi = torch.randn(7, P, generator=g)[torch.randint(0, 7, (B, L), generator=g)]
    else:                                         # one bucket for everything, with exact zeros (strict > 0)
        phi = torch.zeros(B, L, P)
    check_bucket_sort(phi, T, nb)


# ---------------------------------------------------------------------------------------------------------------------
# a3 + a4: candidate lists and suffix lengths
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('B,L,T,nb,C,K,V', [(2, 300, 8, 3, 16, 4, 5), (1, 200, 4, 2, 4, 4, 3), (2, 700, 8, 14, 32, 4, 6),
                                            (1, 130, 3, 2, 64, 6, 4), (1, 50, 2, 1, 1, 1, 2)])
def test_candidate_lists_bruteforce(B, L, T, nb, C, K, V):
    say('candidate_lists', B, L, T, nb, C, K, V)
    g = torch.Generator().manual_seed(B * 1000 + L)
    x = torch.randint(0, V, (B, L), generator=g)
    phi = torch.randn(V, T * nb, generator=g)[x]
    sig = x.float()
    ids, order, ids_s, rank, _ = check_bucket_sort(phi, T, nb)
    _, order, ids_s, rank, win = ops.bucket_sort(phi.to(DEV), T, nb, C)
    pos, ell = ops.candidate_lists(sig.to(DEV), order, win, rank, C, K)
    pos, ell = pos.cpu().long(), ell.cpu().long()
    lists = O.candidate_lists_bruteforce(ids.cpu(), C)
    want = torch.full((B, L, T, C), -1, dtype=torch.long)
    for b in range(B):
        for tau in range(T):
            for t, lst in enumerate(lists[b * T + tau]):
                if lst:
                    want[b, t, tau, C - len(lst):] = torch.tensor(lst)
    assert torch.equal(pos, want)
    Pf = O.previous(sig, K)                                                   # (B, L, K)
    valid = want >= 0
    kk = want.clamp(min=0)
    Pk = Pf.reshape(B * L, K)[(torch.arange(B).view(B, 1, 1, 1) * L + kk)]   # (B, L, T, C, K)
    Pq = Pf[:, :, None, None, :].expand_as(Pk)
    ref_ell = O.suffix_len(Pq, Pk)
    assert torch.equal(ell[valid], ref_ell[valid])
    assert bool((ell[~valid] == -1).all())


# ---------------------------------------------------------------------------------------------------------------------
# a10: n-gram keys and their sort
# ---------------------------------------------------------------------------------------------------------------------

def check_ngram(sig, coef, n):
    keys, order, rep, rank_k, vistos = ops.ngram_sort(sig.to(DEV), coef.to(DEV), n)
    rk = O.ngram_keys(sig, coef, n)
    k = keys.cpu()
    assert torch.equal(torch.isnan(k), torch.isnan(rk))
    assert torch.equal(k.nan_to_num(-5.0).view(torch.int64), rk.nan_to_num(-5.0).view(torch.int64))
    ro, rr = O.ngram_sort(rk)
    assert torch.equal(order.cpu().long(), ro)
    assert torch.equal(rep.cpu().bool(), rr)
    B, L = sig.shape
    inv = torch.empty_like(ro).scatter_(-1, ro, torch.arange(L).expand_as(ro))
    assert torch.equal(rank_k.cpu().long(), inv)
    rv = torch.zeros_like(rr).scatter(-1, ro, rr).transpose(1, 2).float()
    assert torch.equal(vistos.cpu(), rv)
    return keys, order, rep, rank_k, vistos


@pytest.mark.parametrize('name', CASES)
def test_ngram_golden(name):
    say('ngram golden', name)
    g, p, m = fixtures.load(name)
    keys, order, rep, rank_k, vistos = ops.ngram_sort(g['sig'].to(DEV), p['c_vistos'].to(DEV), 4)
    k = keys.cpu()
    assert torch.equal(torch.isnan(k), torch.isnan(g['claves']))
    assert torch.equal(k.nan_to_num(-5.0), g['claves'].nan_to_num(-5.0))
    assert torch.equal(order.cpu().long(), g['orden_k'])
    assert torch.equal(rep.cpu().bool(), g['repetido'].bool())
    assert torch.equal(vistos.cpu(), g['rep.vistos'])


@pytest.mark.parametrize('B,L,V,zipf', [(8, 4096, 256, None), (2, 10000, 6, None), (1, 1, 5, None), (3, 3, 5, None),
                                        (1, 65536, 32000, 1.1), (2, 333, 50304, 1.1), (1, 4097, 3, None),
                                        (3, 4095, 2, None), (2, 12289, 40, 1.1)])
def test_ngram_vs_oracle(B, L, V, zipf):
    say('ngram', B, L, V, zipf)
    x = synth.tokens(B, L, V, frac=0.3, span=(2, 8), zipf=zipf, seed=L)
    coef = torch.rand(4, generator=torch.Generator().manual_seed(12345), dtype=torch.float64) + 0.5
    check_ngram(x.float(), coef, 4)


# ---------------------------------------------------------------------------------------------------------------------
# a9, a11, a12: scans
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('N', [1, 2, 3, 7, 64, 1000, 1025, 4096, 4097, 10000, 70000])
def test_affine_scan_vs_sequential(N):
    say('scan', N)
    g = torch.Generator().manual_seed(N)
    a = torch.rand(3, 5, N, generator=g)
    b = torch.randn(3, 5, N, generator=g)
    a[..., ::7] = 0
    w = torch.randn(3, 5, N, generator=g)
    ar, br = a.clone().requires_grad_(), b.clone().requires_grad_()
    (O.scan(ar, br) * w).sum().backward()
    ad, bd = a.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    S = ops.escaneo(ad, bd)
    (S * w.to(DEV)).sum().backward()
    assert_close(S, O.scan(a, b), 'S', 1e-5)
    assert_close(ad.grad, ar.grad, 'dL/da', 1e-5)
    assert_close(bd.grad, br.grad, 'dL/db', 1e-5)


@pytest.mark.parametrize('B,L', [(8, 4096), (4, 65536), (3, 1), (2, 5000)])
def test_clock_scan(B, L):
    say('clock', B, L)
    beta = torch.rand(B, L, generator=torch.Generator().manual_seed(L), dtype=torch.float64) * 2
    bd = beta.to(DEV).requires_grad_()
    Bt = ops.ClockScan.apply(bd)
    assert_close(Bt, beta.cumsum(1), 'Bt', 1e-12)
    g = torch.randn(B, L, dtype=torch.float64)
    Bt.backward(g.to(DEV))
    assert_close(bd.grad, g.flip(1).cumsum(1).flip(1), 'dbeta', 1e-12)


@pytest.mark.parametrize('B,L', [(8, 4096), (4, 65536), (2, 5000)])
def test_clock_scan_fp32_core_layer(B, L):
    """The core layer's fp32 clock (reloj32): bit for bit the reference's fp32 cumsum on the CPU, which accumulates in
    double and rounds each sum (torch.rand's fp32 values are multiples of 2^-24 here, so every fp64 partial sum is
    exact and the order of the additions cannot matter); a sequential fp32 sum differs. The gradient is the suffix
    sum."""
    say('clock fp32', B, L)
    beta = torch.rand(B, L, generator=torch.Generator().manual_seed(L)) * 2
    bd = beta.double().to(DEV).requires_grad_()
    Bt = ops.ClockScan.apply(bd, True)
    ref = beta.cumsum(1)
    assert torch.equal(Bt.cpu().float(), ref)
    assert torch.equal(Bt.cpu(), ref.double())
    g = torch.randn(B, L, dtype=torch.float64)
    Bt.backward(g.to(DEV))
    assert_close(bd.grad, g.flip(1).cumsum(1).flip(1), 'dbeta', 1e-12)


def repetition(Bt, la, kappa, beta, kappa_r, order, rep, rank_k, vistos, joint):
    """hawkes and racha through the two autograd functions, or (joint) through ops.Repeticion, whose two scans share
    their launches."""
    if joint:
        return ops.Repeticion.apply(Bt, la, kappa, beta, kappa_r, order, rep, rank_k, vistos)
    return ops.Hawkes.apply(Bt, la, kappa, order, rep, rank_k), ops.Streak.apply(beta, kappa_r, vistos)


def run_repetition_stage(g, p, sh, kappa_min=None, joint=False):
    """HIP hawkes/streak on the fixture's stage inputs, with gradients (the rates floored at kappa_min when the
    fixture's protections have one, as the layer's _kappas does)."""
    beta = g['beta'].to(DEV).requires_grad_()
    Bt = g['Bt'].to(DEV).requires_grad_()
    la = g['log_alfa'].to(DEV).requires_grad_()
    lk = p['log_kappa'].to(DEV).requires_grad_()
    lkr = p['log_kappa_racha'].to(DEV).requires_grad_()
    _, order, rep, rank_k, vistos = ops.ngram_sort(g['sig'].to(DEV), p['c_vistos'].to(DEV), sh.n)
    kappa, kappa_r = lk.exp(), lkr.exp()
    if kappa_min is not None:
        kappa, kappa_r = kappa.clamp(min=kappa_min), kappa_r.clamp(min=kappa_min)
    hawkes, racha = repetition(Bt, la, kappa, beta, kappa_r, order, rep, rank_k, vistos, joint)
    ((hawkes * g['rep.gh'].to(DEV)).sum() + (racha * g['rep.gr'].to(DEV)).sum()).backward()
    return vistos, hawkes, racha, beta.grad, Bt.grad, la.grad, lk.grad, lkr.grad


@pytest.mark.parametrize('joint', [False, True], ids=['apart', 'joint'])
@pytest.mark.parametrize('name', CASES)
def test_repetition_golden(name, joint):
    say('repetition golden', name, joint)
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    vistos, hawkes, racha, gb, gB, gla, glk, glkr = run_repetition_stage(g, p, sh, fixtures.prot(m).kappa_min, joint)
    assert torch.equal(vistos.cpu(), g['rep.vistos'])
    assert_close(hawkes, g['rep.hawkes'], 'hawkes')
    if m['extra'].get('kappa_r_zero'):
        assert torch.equal(racha.cpu(), g['rep.racha'])          # integer run lengths, bit-exact
    else:
        assert_close(racha, g['rep.racha'], 'racha')
    assert_close(gb, g['rep.g_beta'], 'grad beta')
    assert_close(gB, g['rep.g_Bt'], 'grad Bt')
    assert_close(gla, g['rep.g_log_alfa'], 'grad log_alfa')
    assert_close(glk, g['rep.g_log_kappa'], 'grad log_kappa')
    assert_close(glkr, g['rep.g_log_kappa_racha'], 'grad log_kappa_racha')


@pytest.mark.parametrize('joint', [False, True], ids=['apart', 'joint'])
@pytest.mark.parametrize('B,L,n,V', [(2, 1025, 4, 3), (3, 4096, 4, 4), (2, 5000, 4, 5), (1, 70000, 3, 8)])
def test_repetition_vs_oracle_long_rows(B, L, n, V, joint):
    """Hawkes and streak scans over rows that span many chunks (the carry between chunks and the chunk-summed d kappa)
    against the oracle's sequential scans, outputs and every gradient."""
    say('repetition long rows', B, L, n, V, joint)
    g = torch.Generator().manual_seed(L)
    x = torch.randint(0, V, (B, L), generator=g)
    sig = O.firmas(x)
    beta = (torch.rand(B, L, generator=g, dtype=torch.float64) * 0.2).requires_grad_()
    Bt = (torch.rand(B, L, generator=g, dtype=torch.float64) * 0.2).cumsum(1).requires_grad_()
    la = (torch.randn(B, L, generator=g) * 0.3).requires_grad_()
    lk = (torch.randn(n, generator=g) * 0.5 - 1.0).requires_grad_()
    lkr = torch.tensor([-2.0]).requires_grad_()
    c = torch.rand(n, generator=g, dtype=torch.float64) + 0.5                  # the c_vistos buffer's law
    gh = torch.randn(B, L, n, generator=g)
    gr = torch.randn(B, L, generator=g)
    p = {'log_kappa': lk, 'log_kappa_racha': lkr, 'c_vistos': c}
    ref = O.repetition(p, sig, beta, Bt, la, O.Shape(d=32, n=n), O.Prot())
    ((ref['hawkes'] * gh).sum() + (ref['racha'] * gr).sum()).backward()
    leaves = [t.detach().to(DEV).requires_grad_() for t in (beta, Bt, la, lk, lkr)]
    _, order, rep, rank_k, vistos = ops.ngram_sort(sig.to(DEV), c.to(DEV), n)
    hawkes, racha = repetition(leaves[1], leaves[2], leaves[3].exp(), leaves[0], leaves[4].exp(), order, rep, rank_k,
                               vistos, joint)
    ((hawkes * gh.to(DEV)).sum() + (racha * gr.to(DEV)).sum()).backward()
    assert torch.equal(vistos.cpu(), ref['vistos'])
    assert_close(hawkes, ref['hawkes'], 'hawkes')
    assert_close(racha, ref['racha'], 'racha')
    for name, mine, want in zip(('beta', 'Bt', 'log_alfa', 'log_kappa', 'log_kappa_racha'), leaves,
                                (beta, Bt, la, lk, lkr)):
        assert_close(mine.grad, want.grad, 'grad ' + name)


# ---------------------------------------------------------------------------------------------------------------------
# a3 - a8: candidate attention forward and backward
# ---------------------------------------------------------------------------------------------------------------------

def run_candidates(stage, sig, w_suf, gamma, sh, gs, prot=None, fugas=None):
    """HIP candidate stage on CPU-provided stage tensors; returns outputs and grads on the CPU. prot: the core layer's
    clock term without reloj_64; fugas: a list that receives the leak count without mascara_exacta."""
    leaves = {k: stage[k].to(DEV).requires_grad_() for k in ('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa')}
    w = w_suf.to(DEV).requires_grad_()
    gam = gamma.to(DEV).requires_grad_()
    _, order, _, rank, win = ops.bucket_sort(leaves['phi'].detach(), sh.T, sh.nb, sh.C)
    shape = dict(T=sh.T, Tc=sh.Tc, C=sh.C, K=sh.K)
    if prot is not None and not prot.reloj_64:
        shape['reloj32'] = True
    if prot is not None and not prot.mascara_exacta:
        shape['fuga'] = torch.zeros(1, dtype=torch.int32, device=DEV)
    salida, sen = ops.Candidates.apply(leaves['phi'], leaves['V'], leaves['Qc'], leaves['Kc'], leaves['Bt'],
                                       leaves['log_alfa'], w, gam, sig.to(DEV), order, win, rank, shape)
    (salida * gs.to(DEV)).sum().backward()
    grads = {k: t.grad.cpu() for k, t in leaves.items()}
    grads['w_sufijo'], grads['gamma'] = w.grad.cpu(), gam.grad.cpu()
    if fugas is not None and 'fuga' in shape:
        fugas.append(int(shape['fuga'].item()))
    return salida.detach().cpu(), sen.cpu(), grads


def oracle_candidates(stage, sig, w_suf, gamma, sh, gs, prot=None):
    leaves = {k: stage[k].clone().requires_grad_() for k in ('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa')}
    w, gam = w_suf.clone().requires_grad_(), gamma.clone().requires_grad_()
    salida, sen = O.candidates(leaves['phi'], leaves['V'], leaves['Qc'], leaves['Kc'], leaves['Bt'],
                               leaves['log_alfa'], sig, w, gam, sh, prot)
    acc = O.gate_signals(salida, sen, sh.T, sh.Tc)
    (salida * gs).sum().backward()
    grads = {k: t.grad for k, t in leaves.items()}
    grads['w_sufijo'], grads['gamma'] = w.grad, gam.grad
    return acc, grads


def check_signals(sen, acc):
    assert torch.equal(sen[..., 0:1], acc['peso_total'])
    assert torch.equal(sen[..., 3:4], acc['peso_ctx'])
    assert_close(sen[..., 1:2], acc['mejor'], 'mejor')
    assert_close(sen[..., 2:3], acc['pico'], 'pico')


@pytest.mark.parametrize('name', CASES)
def test_candidates_golden(name):
    """Every fp32 fixture, the core layer's (v89 numerics: the fp32 clock term, the -1e9 fill) included. On the core
    layer's gamma = 1e9 fixture the reference's fill leaks weight to invalid keys: there the kernels count the leaking
    (query, table) pairs, equal the oracle's core mode with the exact mask everywhere, and equal the reference at every
    query none of whose tables leaks. On the moved-clock core fixture the reference's d gamma is a difference of two
    sums of ds B over clocks of ~4e5, which rounds away ~3e-3 of it; the kernels form d gamma from the clock
    differences, so it is held to 1e-2 there."""
    import dataclasses
    say('candidates golden', name)
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    prot = fixtures.prot(m)
    stage = {k: fixtures.stage_input(g, k) for k in ('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa')}
    fugas = []
    salida, sen, grads = run_candidates(stage, g['sig'], p['w_sufijo'], p['gamma'], sh, g['acc.gs'], prot, fugas)
    if fixtures.nucleo(m) and 'gamma_fill' in m['extra']:
        print('  leaking (query, table) pairs counted:', fugas, flush=True)
        assert fugas[0] > 0
        exacta = dataclasses.replace(prot, mascara_exacta=True)
        acc, rg = oracle_candidates(stage, g['sig'], p['w_sufijo'], p['gamma'], sh, g['acc.gs'], exacta)
        assert_close(salida, acc['salida'], 'salida vs the exact mask')
        check_signals(sen, acc)
        for k in rg:
            assert_close(grads[k], rg[k], 'grad ' + k)
        same = ((acc['salida'] - g['acc.salida']).abs().amax(-1) == 0)           # queries where nothing leaks
        assert same.any() and not same.all()
        assert_close(salida[same], g['acc.salida'][same], 'salida where the reference does not leak')
        return
    if fugas:
        assert fugas[0] == 0
    assert_close(salida, g['acc.salida'], 'salida')
    check_signals(sen, {k: g['acc.' + k] for k in ('peso_total', 'mejor', 'pico', 'peso_ctx')})
    for k in ('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa', 'w_sufijo', 'gamma'):
        tol = 1e-2 if k == 'gamma' and 'reloj_extra' in m['extra'] else TOL
        assert_close(grads[k], g['acc.g_' + k], 'grad ' + k, tol)


def random_stage(B, L, d, V, nb=14, T=8, cf=16, K=4, seed=0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    x = synth.tokens(B, L, V, frac=0.3, span=(8, 64), seed=seed)
    P = T * nb
    emb = torch.randn(V, P, generator=g)
    word = emb[x][..., :P // 2]
    ctx = torch.randn(V, V, P - P // 2, generator=g) if V <= 64 else None
    prev = torch.cat([x[:, :1], x[:, :-1]], 1)
    ctxv = ctx[x, prev] if ctx is not None else (emb[x][..., P // 2:] + 0.7 * emb[prev][..., P // 2:])
    phi = torch.cat([word, ctxv], -1).contiguous()
    stage = dict(phi=phi, V=torch.randn(B, L, d, generator=g), Qc=torch.randn(B, L, cf, generator=g),
                 Kc=torch.randn(B, L, cf, generator=g),
                 Bt=(torch.rand(B, L, generator=g, dtype=torch.float64) * 1.5).cumsum(1) + shift,
                 log_alfa=torch.randn(B, L, generator=g) * 0.3)
    w_suf = torch.randn(K + 1, generator=g) * 0.5
    gamma = torch.rand(T, generator=g) * 2
    gs = torch.randn(B, L, d, generator=g)
    return x.float(), stage, w_suf, gamma, gs


@pytest.mark.parametrize('B,L,d,V,C,nb,T,shift', [(2, 1500, 256, 6, 32, 14, 8, 0.0), (2, 777, 96, 40, 16, 4, 8, 0.0),
                                                  (1, 600, 64, 5, 64, 6, 4, 1e6), (2, 300, 1024, 8, 8, 3, 8, 0.0),
                                                  (1, 2, 32, 3, 32, 14, 8, 0.0), (2, 900, 768, 7, 32, 14, 8, 0.0),
                                                  (1, 500, 512, 9, 32, 14, 8, 0.0)])
def test_candidates_vs_oracle(B, L, d, V, C, nb, T, shift):
    say('candidates', B, L, d, V, C, nb, T, shift)
    sig, stage, w_suf, gamma, gs = random_stage(B, L, d, V, nb=nb, T=T, seed=L, shift=shift)
    sh = O.Shape(d=d, nb=nb, C=C, T=T, Tc=T // 2)
    salida, sen, grads = run_candidates(stage, sig, w_suf, gamma, sh, gs)
    acc, rg = oracle_candidates(stage, sig, w_suf, gamma, sh, gs)
    assert_close(salida, acc['salida'], 'salida')
    check_signals(sen, acc)
    for k in rg:
        assert_close(grads[k], rg[k], 'grad ' + k)


def test_candidates_cfg2_full_size():
    """BASELINE cfg2 (B 8, N 4096, d 256, fp32) on the synthetic generator, candidate stage vs the oracle."""
    say('candidates cfg2 full size')
    sig, stage, w_suf, gamma, gs = random_stage(8, 4096, 256, 256, seed=0)
    sh = O.Shape(d=256)
    salida, sen, grads = run_candidates(stage, sig, w_suf, gamma, sh, gs)
    acc, rg = oracle_candidates(stage, sig, w_suf, gamma, sh, gs)
    assert_close(salida, acc['salida'], 'salida')
    check_signals(sen, acc)
    for k in rg:
        assert_close(grads[k], rg[k], 'grad ' + k)


@pytest.mark.parametrize('B,L,d', [(3, 1504, 256), (2, 808, 96), (1, 64, 64)])
def test_candidates_rowwise_xcd_mapping_bit_identical(B, L, d):
    """The row-wise XCD mapping (all XCDs on one batch row at a time, which the kernels take by themselves when the
    rows outgrow the last-level cache, as at cfg3) forced on and off with ASRN_ROWWISE: the same bits, forward and
    backward, since every wave computes its own token whatever order the waves take them in."""
    say('candidates row-wise mapping', B, L, d)
    sig, stage, w_suf, gamma, gs = random_stage(B, L, d, 40, seed=L + d)
    sh = O.Shape(d=d)
    runs = []
    try:
        for flag in ('1', '0'):
            os.environ['ASRN_ROWWISE'] = flag
            runs.append(run_candidates(stage, sig, w_suf, gamma, sh, gs))
    finally:
        os.environ.pop('ASRN_ROWWISE', None)
    (s1, e1, g1), (s0, e0, g0) = runs
    assert torch.equal(s1, s0) and torch.equal(e1, e0)
    for k in g0:
        assert torch.equal(g1[k], g0[k]), k


@pytest.mark.parametrize('B,L,d,T,nb,C', [(2, 900, 96, 4, 6, 16), (2, 1500, 64, 8, 3, 32), (1, 1, 64, 8, 14, 32),
                                         (3, 700, 256, 8, 2, 8)])
def test_candidates_lists_match_regather(B, L, d, T, nb, C):
    """The backward's query pass reading the forward's candidate lists gives the same outputs and gradients, bit for
    bit, as gathering and deduplicating again (few bits per table: many queries have more than 64 candidates); both
    match the oracle."""
    say('candidate lists', B, L, d, T, nb, C)
    P, cf = T * nb + (-(T * nb)) % 4, 16
    g = torch.Generator().manual_seed(L + nb)
    phi = torch.randn(B, L, P, generator=g)
    phi[..., T * nb:] = 0                              # the float4 padding columns
    phi = phi.to(DEV)
    V = torch.randn(B, L, d, generator=g).to(DEV)
    Qc, Kc = torch.randn(B, L, cf, generator=g).to(DEV), torch.randn(B, L, cf, generator=g).to(DEV)
    Bt = (torch.rand(B, L, generator=g, dtype=torch.float64) * 0.1).cumsum(1).to(DEV)
    la = (torch.randn(B, L, generator=g) * 0.3).to(DEV)
    sig = torch.randint(0, 7, (B, L), generator=g).float().to(DEV)
    w, gam = torch.randn(5, generator=g).to(DEV), torch.rand(T, generator=g).to(DEV)
    _, order, _, rank, win = ops.bucket_sort(phi[..., :T * nb].contiguous(), T, nb, C)
    gs = torch.randn(B, L, d, generator=g).to(DEV)
    outs = []
    for listas in (True, False):
        leaves = [t.detach().clone().requires_grad_() for t in (phi, V, Qc, Kc, Bt, la, w, gam)]
        shape = dict(T=T, Tc=T // 2, C=C, K=4, listas=listas)
        sal, sen = ops.Candidates.apply(*leaves[:6], leaves[6], leaves[7], sig, order, win, rank, shape)
        (sal * gs).sum().backward()
        outs.append([sal.detach(), sen] + [t.grad for t in leaves])
    for i, (a, b) in enumerate(zip(outs[0], outs[1])):
        assert torch.equal(a, b), f'output {i} differs'
    sh = O.Shape(d=d, T=T, nb=nb, C=C, Tc=T // 2, cf=cf, K=4)
    stage = {k: v.detach().cpu() for k, v in zip(('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa'), (phi, V, Qc, Kc, Bt, la))}
    stage['phi'] = stage['phi'][..., :T * nb]
    acc, rg = oracle_candidates(stage, sig.cpu(), w.cpu(), gam.cpu(), sh, gs.cpu())
    assert_close(outs[1][0], acc['salida'], 'salida vs oracle')
    check_signals(outs[1][1].cpu(), acc)
    for i, k in enumerate(('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa', 'w_sufijo', 'gamma')):
        got = outs[1][2 + i]
        assert_close(got[..., :T * nb] if k == 'phi' else got, rg[k], 'grad ' + k + ' vs oracle')


def test_candidates_v_shift_in_place():
    """v_shift = 1 with v a column block of a wider fp32 tensor (read in place through its row stride) against
    v_shift = 0 with the reference's shifted, contiguous V[t] = v[t+1]: the same outputs bit for bit, and dv = dV
    moved one row down with row 0 zero."""
    say('candidates v_shift')
    B, L, d, P, cf, T, nb, C = 2, 900, 96, 56, 16, 4, 6, 16
    g = torch.Generator().manual_seed(21)
    wide = torch.randn(B, L, 40 + d + 12, generator=g).to(DEV)
    v = wide[..., 40:40 + d]
    V = torch.cat([v[:, 1:], torch.zeros_like(v[:, :1])], 1).contiguous()
    phi = torch.randn(B, L, P, generator=g).to(DEV)
    Qc, Kc = torch.randn(B, L, cf, generator=g).to(DEV), torch.randn(B, L, cf, generator=g).to(DEV)
    Bt = (torch.rand(B, L, generator=g, dtype=torch.float64) * 0.1).cumsum(1).to(DEV)
    la = (torch.randn(B, L, generator=g) * 0.3).to(DEV)
    sig = torch.randint(0, 7, (B, L), generator=g).float().to(DEV)
    w, gam = torch.randn(5, generator=g).to(DEV), torch.rand(T, generator=g).to(DEV)
    _, order, _, rank, win = ops.bucket_sort(phi, T, nb, C)
    gs = torch.randn(B, L, d, generator=g).to(DEV)
    outs = []
    for vv, shift in ((V, 0), (v, 1)):
        leaf = vv.detach().clone() if shift == 0 else wide.detach().clone().requires_grad_()
        vin = leaf.requires_grad_() if shift == 0 else leaf[..., 40:40 + d]
        shape = dict(T=T, Tc=2, C=C, K=4, v_shift=shift)
        sal, sen = ops.Candidates.apply(phi, vin, Qc, Kc, Bt, la, w, gam, sig, order, win, rank, shape)
        (sal * gs).sum().backward()
        outs.append((sal.detach(), sen, leaf.grad if shift == 0 else leaf.grad[..., 40:40 + d]))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    dV, dv = outs[0][2], outs[1][2]
    assert torch.equal(dv[:, 1:], dV[:, :-1]) and torch.equal(dv[:, 0], torch.zeros_like(dv[:, 0]))
    assert torch.equal(dV[:, -1], torch.zeros_like(dV[:, -1]))


# ---------------------------------------------------------------------------------------------------------------------
# a0: the hash producer (one GEMM, the fused hidden layer) and the column sums of the parameter gradients
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('rows,cols,ld,off,bf16', [(32768, 13, 13, 0, False), (32768, 112, 448, 192, False),
                                                   (16, 114688, 114688, 0, False), (4096, 7, 9, 1, False),
                                                   (1, 5, 5, 0, False), (0, 6, 6, 0, False), (5000, 64, 64, 0, True),
                                                   (20000, 448, 448, 0, True), (300, 1024, 1030, 2, True)])
def test_column_sums_exact(rows, cols, ld, off, bf16):
    """asrn_column_sums on small integers, whose fp32 sums are exact in any order: every column must equal the integer
    sum bit for bit (one slab or two passes, float4 or scalar loads, strided and offset rows, bf16 input)."""
    say('column sums', rows, cols, ld, off, bf16)
    from asrn_amd.lineal import _hip_sums
    g = torch.Generator().manual_seed(rows + cols)
    flat = torch.randint(-8, 9, (rows * ld + off + 8,), generator=g)
    ref = flat[off:off + rows * ld].view(rows, ld)[:, :cols].sum(0) if rows else torch.zeros(cols, dtype=torch.int64)
    x = flat.to(torch.bfloat16 if bf16 else torch.float32).to(DEV)
    xv = x.as_strided((rows, cols), (ld, 1), off)
    out = _hip_sums(xv, rows, cols, ld)
    assert torch.equal(out.cpu().double(), ref.double())


@pytest.mark.parametrize('d,kw', [(256, {}), (32, dict(n_tablas=5, tablas_contexto=2, n_bits=3, confirmar=6))])
def test_weight_assembly_is_exact(d, kw):
    """The one-launch assembly of the fused GEMMs' weights (asrn_copy_blocks) equals torch.cat / block_diag of the
    parameters bit for bit, and its backward hands each parameter exactly its block of the gradients."""
    say('weight assembly', d, kw)
    from asrn_amd.capa import _Pesos
    layer = synth.move_params(CapaASRNEstable(d, **kw), seed=7).to(DEV)
    pal, ctx = layer.afin_palabra, layer.afin_contexto
    mc = ctx[0].out_features
    ref = [torch.cat([pal[0].weight, ctx[0].weight.view(mc, 2, d).transpose(0, 1).reshape(2 * mc, d)]),
           torch.cat([layer.cq.weight, layer.ck.weight]), torch.block_diag(pal[2].weight, ctx[2].weight),
           torch.cat([pal[2].bias, ctx[2].bias])]
    params = [pal[0].weight, ctx[0].weight, layer.cq.weight, layer.ck.weight, pal[2].weight, ctx[2].weight,
              pal[2].bias, ctx[2].bias]
    g = torch.Generator().manual_seed(d)
    gs = [torch.randn(r.shape, generator=g).to(DEV) for r in ref]
    for k in (8, 4):             # with the second layers' blocks, and without (the fused hash kernels' path)
        got = _Pesos.apply(*params[:k])
        assert len(got) == k // 2
        want = torch.autograd.grad(sum((r * x).sum() for r, x in zip(ref[:k // 2], gs)), params[:k])
        have = torch.autograd.grad(sum((r * x).sum() for r, x in zip(got, gs)), params[:k])
        for r, x in zip(ref, got):
            assert torch.equal(r, x)
        for a, b in zip(want, have):
            assert torch.equal(a, b)


@pytest.mark.parametrize('M,N,K,autocast', [(256, 256, 256, False), (33, 70, 129, False), (1, 17, 5, False),
                                            (512, 96, 768, False), (768, 768, 768, False), (768, 768, 768, True)])
def test_small_matmul_vs_fp64(M, N, K, autocast):
    """ops.SmallMatmul (the layer's W_o W_v; asrn_small_gemm up to 256^3 multiply-adds, the library's fp32 GEMM beyond):
    the product and both gradients against fp64 on the CPU, including sizes that leave partial 16 x 16 tiles, and
    fp32 also when called under bf16 autocast."""
    say('small matmul', M, N, K, autocast)
    g = torch.Generator().manual_seed(M * N + K)
    A, B, gC = torch.randn(M, K, generator=g), torch.randn(K, N, generator=g), torch.randn(M, N, generator=g)
    Ar, Br = A.double().requires_grad_(), B.double().requires_grad_()
    (Ar @ Br * gC.double()).sum().backward()
    Ad, Bd = A.to(DEV).requires_grad_(), B.to(DEV).requires_grad_()
    with torch.autocast(device_type='cuda', dtype=torch.bfloat16, enabled=autocast):
        C = ops.SmallMatmul.apply(Ad, Bd)
        (C * gC.to(DEV)).sum().backward()
    assert C.dtype == torch.float32
    assert_close(C, Ar @ Br, 'C', 1e-5)
    assert_close(Ad.grad, Ar.grad, 'dA', 1e-5)
    assert_close(Bd.grad, Br.grad, 'dB', 1e-5)


@pytest.mark.parametrize('B,L,d,kw,rows_grad', [(2, 777, 96, {}, True), (2, 777, 96, {}, False), (3, 1, 64, {}, True),
                                                (1, 2048, 256, {}, True), (8, 4096, 256, {}, True),
                                                (3, 3000, 256, {}, True), (2, 300, 32, dict(n_tablas=5, tablas_contexto=2,
                                                                                          n_bits=3), True),
                                                (2, 300, 32, dict(afin_oculto=16), True),
                                                (2, 300, 32, dict(afin_oculto=160), True)])
def test_hash_producer_vs_oracle(B, L, d, kw, rows_grad):
    """phi from the fused hash producer (one GEMM, then asrn_hash_fwd/bwd: the hidden layer and both second layers
    on the matrix cores, every parameter gradient summed in order) against the oracle's word and context MLPs on the
    materialized key [E_t; E_{t-1}] (fp64 on the CPU): phi, the gradient of E and of every MLP parameter. Odd output
    widths (9 and 6) and 8 hidden units take the same kernels; 80 hidden units take the unfused path (the first
    layers' GEMM, asrn_hidden_fwd/bwd, a block-diagonal GEMM). rows_grad: the E rows the producer hands on (the
    candidate kernels' values) also receive a gradient, which the producer's input-gradient GEMM accumulates into.
    (8, 4096, 256) is cfg2's shape: asrn_hash_bwd's persistent workgroups (at most 128) each run 4 of the 512 tiles
    and carry dW2 and the bias partials across them; (3, 3000, 256) adds a ragged last round (141 tiles, the last
    one partial)."""
    say('hash producer', B, L, d, kw, rows_grad)
    layer = synth.move_params(CapaASRNEstable(d, **kw), seed=B + d)
    p = {k: v.detach().clone() for k, v in layer.state_dict().items()}
    g = torch.Generator().manual_seed(L)
    E = torch.randn(B, L, d, generator=g)
    gphi = torch.randn(B, L, layer.n_tablas * layer.n_bits, generator=g)
    gr = torch.randn(B, L, d, generator=g)
    names = [k for k in p if k.startswith(('afin_palabra', 'afin_contexto'))]
    leaves = {k: (v.double().requires_grad_() if k in names else v) for k, v in p.items()}
    Ec = E.double().requires_grad_()
    phi_r, _ = O.phi_and_values(leaves, Ec)
    ((phi_r * gphi.double()).sum() + ((Ec * gr.double()).sum() if rows_grad else 0)).backward()
    layer = layer.to(DEV)
    Ed = E.to(DEV).requires_grad_()
    phi, filas = layer._phi_y_valores(Ed)
    assert filas.data_ptr() == Ed.data_ptr()          # the values are E's own rows, read in place
    ((phi * gphi.to(DEV)).sum() + ((filas * gr.to(DEV)).sum() if rows_grad else 0)).backward()
    assert_close(phi, phi_r, 'phi')
    assert_close(Ed.grad, Ec.grad, 'grad E')
    named = dict(layer.named_parameters())
    for k in names:
        assert_close(named[k].grad, leaves[k].grad, 'grad ' + k)


@pytest.mark.parametrize('B,L,T,nb,m,mc', [(2, 1500, 8, 14, 64, 64), (3, 700, 5, 14, 32, 32), (1, 65, 3, 6, 8, 8),
                                           (1, 5000, 8, 14, 64, 64)])
def test_hash_producer_bucket_ids(B, L, T, nb, m, mc):
    """The bucket ids the fused hash kernel writes with phi equal the sign hash the bucket sort takes of that phi,
    bit for bit, and the sort fed those ids gives the same order, ranks and windows: tables inside either MLP's
    columns, a table across the word/context boundary (T 5, nb 14: columns 28-41 around 35), a few tokens (the small
    GEMM), and rows that take the sort's one-launch (700), chunked (1,500) and merge (5,000) paths."""
    say('hash producer bucket ids', B, L, T, nb, m, mc)
    d, C = 64, 32
    P = T * nb
    Pw, Pc = P // 2, P - P // 2
    g = torch.Generator().manual_seed(L + T)
    r = lambda *s: torch.randn(*s, generator=g).to(DEV)
    E = r(B, L, d)
    args = (r(m + 2 * mc, d) * 0.2, r(m) * 0.1, r(mc) * 0.1, r(Pw, m) * 0.3, r(Pw) * 0.1, r(Pc, mc) * 0.3,
            r(Pc) * 0.1)
    with torch.no_grad():
        phi, _, ids = ops.HashProducer.apply(E, *args, m, mc, T, nb)
        ref = ops.bucket_sort(phi, T, nb, C)
        got = ops.bucket_sort(phi, T, nb, C, ids=ids.clone())
    assert torch.equal(ids, ref[0])
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    pos = (phi > 0).float().mean().item()
    assert 0.2 < pos < 0.8                                   # both signs occur


# ---------------------------------------------------------------------------------------------------------------------
# a0: the context producer
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('case', ['plain', 'clamped', 'bf16', 'wide', 'wide20', 'many'])
def test_context_vs_oracle(case):
    """LayerNorm + Qc/Kc + the fp32 clock projection with softplus / logsigmoid and the group-A clamps (the fused
    asrn_context_fwd/bwd and the Qc/Kc GEMM, whose input gradient the fp32 backward forms in the kernel) against the
    oracle's context: outputs and the gradients of h and every parameter. 'clamped' drives some tokens past beta_max
    and below log_alfa_min; 'bf16' runs under bf16 autocast (the Qc/Kc GEMM in bf16 with its own backward, the clock
    in fp32), within the bf16 tolerance; 'wide' takes d = 384 (two float4 columns a lane) and 16 + 16 outputs, 'wide20'
    20 + 20 outputs (more than the kernel forms: the projection's own backward); 'many' takes 30,035 tokens, 939
    per-workgroup partial rows of the parameter gradients (a full and a ragged batch of the fixed-order sum)."""
    say('context', case)
    B, L, d, cf = {'wide': (3, 301, 384, 16), 'wide20': (3, 301, 384, 20), 'many': (5, 6007, 96, 16)}.get(case, (2, 777, 96, 16))
    g = torch.Generator().manual_seed(11)
    sh = O.Shape(d=d, cf=cf)
    prot = O.Prot()
    p = {'ln_ctx.weight': 1 + 0.1 * torch.randn(d, generator=g), 'ln_ctx.bias': 0.1 * torch.randn(d, generator=g),
         'cq.weight': 0.1 * torch.randn(cf, d, generator=g), 'ck.weight': 0.1 * torch.randn(cf, d, generator=g),
         'w_reloj': 0.3 * torch.randn(2, d, generator=g), 'b_reloj': torch.tensor([0.5, -0.2])}
    h = torch.randn(B, L, d, generator=g) * 2 + 0.5
    if case == 'clamped':                 # large |u|: softplus past 1e4 and logsigmoid below -30 on some tokens
        p['w_reloj'] = p['w_reloj'] * 4000
    gQ, gK = torch.randn(B, L, cf, generator=g), torch.randn(B, L, cf, generator=g)
    gb, gl = torch.randn(B, L, generator=g, dtype=torch.float64), torch.randn(B, L, generator=g)
    hr = h.clone().requires_grad_()
    pr = {k: v.clone().requires_grad_() for k, v in p.items()}
    Qr, Kr, br, lr = O.context(pr, hr, sh, prot)
    ((Qr * gQ).sum() + (Kr * gK).sum() + (br * gb).sum() + (lr * gl).sum()).backward()
    if case == 'clamped':
        assert (br == prot.beta_max).any() and (lr == prot.log_alfa_min).any()
    layer = CapaASRNEstable(d, confirmar=cf).to(DEV)
    with torch.no_grad():
        for k, v in p.items():
            dict(layer.named_parameters())[k].copy_(v)
    hd = h.to(DEV).requires_grad_()
    with torch.autocast('cuda', dtype=torch.bfloat16, enabled=case == 'bf16'):
        Q, K, be, la = layer._contexto(hd)
    assert be.dtype == torch.float64 and la.dtype == torch.float32
    ((Q.float() * gQ.to(DEV)).sum() + (K.float() * gK.to(DEV)).sum() + (be * gb.to(DEV)).sum()
     + (la * gl.to(DEV)).sum()).backward()
    tol = 2e-2 if case == 'bf16' else TOL
    assert_close(Q, Qr, 'Qc', tol)
    assert_close(K, Kr, 'Kc', tol)
    assert_close(be, br, 'beta', TOL)                  # the clock stays fp32 under autocast
    assert_close(la, lr, 'log_alfa', TOL)
    assert_close(hd.grad, hr.grad, 'grad h', tol)
    named = dict(layer.named_parameters())
    for k in p:
        assert_close(named[k].grad, pr[k].grad, 'grad ' + k, tol)


# ---------------------------------------------------------------------------------------------------------------------
# a13: the gate
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('tope,bf16', [(None, False), (10.0, False), (None, True)])
def test_gate_vs_oracle(tope, bf16):
    """The fused gate (asrn_gate_fwd/bwd, with W_o on hipBLASLt) against the oracle's combine: rows without any
    candidate (peso_total 0, mejor -1e9), mejor beyond the clip, streaks past the last response node, and the optional
    tanh cap; output and the gradients of h, salida, hawkes, racha and every gate parameter. bf16: W_o under bf16
    autocast, within the bf16 tolerance."""
    say('gate', tope, bf16)
    B, L, d, n, T, Tc = 2, 333, 64, 4, 8, 4
    sh = O.Shape(d=d, T=T, Tc=Tc, n=n)
    prot = O.Prot(tope_puerta=tope)
    g = torch.Generator().manual_seed(7 + int(bf16) + (0 if tope is None else 1))
    p = {'g.weight': torch.randn(1, d, generator=g) * 0.1, 'g.bias': torch.randn(1, generator=g),
         'g_conf.weight': torch.randn(1, 4, generator=g) * 0.5, 'g_conf.bias': torch.randn(1, generator=g),
         'w_vistos': torch.randn(n, generator=g), 'u_hawkes': torch.randn(n, generator=g),
         'd_racha': torch.randn(sh.nodos, generator=g) * 0.3, 'o.weight': torch.randn(d, d, generator=g) * 0.1}
    pt = torch.randint(0, T + 1, (B, L, 1), generator=g).float()
    mejor = torch.randn(B, L, 1, generator=g) * 3
    mejor[:, ::17] = 2e4                                                   # beyond the clip at 1e4
    mejor = torch.where(pt > 0, mejor, torch.full_like(mejor, -1e9))
    pico = torch.rand(B, L, 1, generator=g) * pt
    ctx = torch.minimum(pt, torch.randint(0, Tc + 1, (B, L, 1), generator=g).float())
    top = math.log1p(sh.racha_max) * 1.3
    leaves = {'h': torch.randn(B, L, d, generator=g), 'salida': torch.randn(B, L, d, generator=g) * 2,
              'hawkes': torch.rand(B, L, n, generator=g) * 5,
              'racha': torch.expm1(torch.rand(B, L, generator=g) * top)}
    vistos = (torch.rand(B, L, n, generator=g) < 0.5).float()
    gy = torch.randn(B, L, d, generator=g)
    ref = {k: v.clone().requires_grad_() for k, v in leaves.items()}
    pr = {k: v.clone().requires_grad_() for k, v in p.items()}
    acc = {'salida': ref['salida'], 'peso_total': pt, 'mejor': mejor, 'pico': pico, 'peso_ctx': ctx,
           'vistos': vistos, 'hawkes': ref['hawkes'], 'racha': ref['racha']}
    yo = O.combine(pr, acc, ref['h'], sh, prot)
    (yo * gy).sum().backward()
    mine = {k: v.to(DEV).requires_grad_() for k, v in leaves.items()}
    pm = {k: v.to(DEV).requires_grad_() for k, v in p.items()}
    sen = torch.cat([pt, mejor, pico, ctx], -1).to(DEV)
    meta = (T, Tc, sh.racha_paso, float(prot.mejor_max), 0.0 if tope is None else tope)
    with torch.autocast('cuda', dtype=torch.bfloat16, enabled=bf16):
        A = lineal(mine['salida'], pm['o.weight'])
    y = ops.Gate.apply(mine['h'], A, sen, vistos.to(DEV), mine['hawkes'], mine['racha'], pm['g.weight'],
                       pm['g.bias'], pm['g_conf.weight'], pm['g_conf.bias'], pm['w_vistos'], pm['u_hawkes'],
                       pm['d_racha'], meta)
    (y * gy.to(DEV)).sum().backward()
    tol = 2e-2 if bf16 else TOL
    assert y.dtype == torch.float32
    assert_close(y, yo, 'out', tol)
    for k in leaves:
        assert_close(mine[k].grad, ref[k].grad, 'grad ' + k, tol)
    for k in p:
        assert_close(pm[k].grad, pr[k].grad, 'grad ' + k, tol)


@pytest.mark.parametrize('B,d,tope', [(16, 768, None), (40, 256, 10.0), (3, 96, None), (5, 1024, None), (16, 512, 3.0)])
def test_gate_step_vs_oracle(B, d, tope):
    """The generation step's W_o product and gate in one kernel (asrn_gate_step: 16 x 16 tiles of W_o salida on the
    matrix cores, the logit recomputed by every column tile) against the oracle's combine in fp64, the edge rows as in
    test_gate_vs_oracle; 40 tokens take three row tiles, 96 and 1024 the narrowest and widest depths."""
    say('gate step', B, d, tope)
    n, T, Tc = 4, 8, 4
    sh = O.Shape(d=d, T=T, Tc=Tc, n=n)
    prot = O.Prot(tope_puerta=tope)
    g = torch.Generator().manual_seed(B + d)
    p = {'g.weight': torch.randn(1, d, generator=g) * 0.1, 'g.bias': torch.randn(1, generator=g),
         'g_conf.weight': torch.randn(1, 4, generator=g) * 0.5, 'g_conf.bias': torch.randn(1, generator=g),
         'w_vistos': torch.randn(n, generator=g), 'u_hawkes': torch.randn(n, generator=g),
         'd_racha': torch.randn(sh.nodos, generator=g) * 0.3, 'o.weight': torch.randn(d, d, generator=g) * 0.1}
    pt = torch.randint(0, T + 1, (B, 1, 1), generator=g).float()
    mejor = torch.randn(B, 1, 1, generator=g) * 3
    mejor[::7] = 2e4
    mejor = torch.where(pt > 0, mejor, torch.full_like(mejor, -1e9))
    pico = torch.rand(B, 1, 1, generator=g) * pt
    ctx = torch.minimum(pt, torch.randint(0, Tc + 1, (B, 1, 1), generator=g).float())
    top = math.log1p(sh.racha_max) * 1.3
    h = torch.randn(B, 1, d, generator=g)
    salida = torch.randn(B, 1, d, generator=g) * 2
    hawkes = torch.rand(B, 1, n, generator=g) * 5
    racha = torch.expm1(torch.rand(B, 1, generator=g) * top)
    vistos = (torch.rand(B, 1, n, generator=g) < 0.5).float()
    acc = {'salida': salida.double(), 'peso_total': pt.double(), 'mejor': mejor.double(), 'pico': pico.double(),
           'peso_ctx': ctx.double(), 'vistos': vistos.double(), 'hawkes': hawkes.double(), 'racha': racha.double()}
    yo = O.combine({k: v.double() for k, v in p.items()}, acc, h.double(), sh, prot)[:, 0]
    sen = torch.cat([pt, mejor, pico, ctx], -1)[:, 0].to(DEV)
    meta = (T, Tc, sh.racha_paso, float(prot.mejor_max), 0.0 if tope is None else tope)
    with torch.no_grad():
        y = ops.gate_step(h[:, 0].to(DEV), salida[:, 0].to(DEV), p['o.weight'].to(DEV), sen, vistos[:, 0].to(DEV),
                          hawkes[:, 0].to(DEV), racha[:, 0].to(DEV), *[p[k].to(DEV) for k in (
                              'g.weight', 'g.bias', 'g_conf.weight', 'g_conf.bias', 'w_vistos', 'u_hawkes', 'd_racha')],
                          meta)
    assert_close(y, yo, 'out')

# ---------------------------------------------------------------------------------------------------------------------
# the whole layer
# ---------------------------------------------------------------------------------------------------------------------

def layer_from_fixture(p, m):
    layer = CapaASRNEstable(m['d'], protecciones=fixtures.protecciones(m), **m['kw'])
    layer.load_state_dict(p)
    return layer.to(DEV)


def run_layer(layer, E, h, x, gy):
    layer.zero_grad()
    Ed, hd = E.to(DEV).requires_grad_(), h.to(DEV).requires_grad_()
    y = layer(Ed, hd, None if x is None else x.to(DEV))
    (y * gy.to(DEV)).sum().backward()
    grads = {'E': Ed.grad.cpu(), 'h': hd.grad.cpu()}
    grads.update({n: q.grad.cpu() for n, q in layer.named_parameters() if q.grad is not None})
    return y.detach().cpu(), grads


@pytest.mark.parametrize('name', CASES)
def test_layer_golden(name):
    """The whole layer against every fp32 fixture; the core layer's (asrn_amd.CapaASRN, v89 numerics) against the
    reference's core-layer fixtures, and on the gamma = 1e9 one, where the reference's -1e9 fill leaks, the leak is
    counted and the output equals the oracle's core mode with the exact mask."""
    import dataclasses
    say('layer golden', name)
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    layer = layer_from_fixture(p, m)
    with torch.no_grad():
        phi, _ = layer._phi_y_valores(g['E'].to(DEV))
    ids, _ = O.bucket_rows(phi.cpu(), sh.T, sh.nb)
    flips = (ids != g['ids']).sum().item()
    if flips:
        pytest.skip(f'{flips} bucket ids differ between the GPU GEMM and the CPU one (sign of phi near 0)')
    y, grads = run_layer(layer, g['E'], g['h'], g['x'], g['gy'])
    if fixtures.nucleo(m):
        print('  core layer: leaking (query, table) pairs', layer.fugas(), flush=True)
        if 'gamma_fill' in m['extra']:
            assert layer.fugas() > 0
            pp = {k: (v.clone().requires_grad_() if v.is_floating_point() and k not in ('c_vistos', 'r_firma', 'pot')
                      else v) for k, v in p.items()}
            E, h = g['E'].clone().requires_grad_(), g['h'].clone().requires_grad_()
            yo = O.layer_forward(pp, E, h, g['x'], sh, dataclasses.replace(fixtures.prot(m), mascara_exacta=True))
            (yo * g['gy']).sum().backward()
            assert_close(y, yo, 'y vs the exact mask')
            assert_close(grads['E'], E.grad, 'grad E')
            assert_close(grads['h'], h.grad, 'grad h')
            return
        assert layer.fugas() == 0
    assert_close(y, g['y'], 'y')
    assert_close(grads['E'], g['gE'], 'grad E')
    assert_close(grads['h'], g['gh'], 'grad h')
    for n in grads:
        if ('g.' + n) in g:
            assert_close(grads[n], g['g.' + n], 'grad ' + n)


def test_layer_deterministic_and_causal():
    say('layer determinism + causality')
    torch.manual_seed(0)
    layer = synth.move_params(CapaASRNEstable(64)).to(DEV)
    x, E, h = synth.layer_inputs(2, 700, 64, 40, seed=3)
    gy = torch.randn(2, 700, 64)
    y1, g1 = run_layer(layer, E, h, x, gy)
    y2, g2 = run_layer(layer, E, h, x, gy)
    assert torch.equal(y1, y2)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
    cut = 400
    x2, E2, h2 = x.clone(), E.clone(), h.clone()
    x2[:, cut:] = torch.randint(0, 40, (2, 700 - cut))
    E2[:, cut:] = torch.randn(2, 700 - cut, 64)
    h2[:, cut:] = torch.randn(2, 700 - cut, 64)
    with torch.no_grad():
        ya = layer(E.to(DEV), h.to(DEV), x.to(DEV))[:, :cut]
        yb = layer(E2.to(DEV), h2.to(DEV), x2.to(DEV))[:, :cut]
    assert (ya - yb).abs().max().item() <= 1e-6 * ya.abs().max().item()


def test_layer_exact_mask_no_leak_with_huge_gamma():
    """gamma = 1e9: every valid score sinks below -1e9; the exact mask still gives no weight to invalid keys, so
    the future never changes the past (asrn/estable.py:20-24, tests te:283-310)."""
    say('layer gamma huge')
    torch.manual_seed(0)
    layer = CapaASRNEstable(32, chunk=16, n_bits=3).to(DEV)
    with torch.no_grad():
        layer.gamma.fill_(1e9)
    L, cut = 96, 60
    g = torch.Generator().manual_seed(0)
    E, h, x = torch.randn(1, L, 32, generator=g), torch.randn(1, L, 32, generator=g), torch.randint(0, 7, (1, L), generator=g)
    E2, h2, x2 = E.clone(), h.clone(), x.clone()
    E2[:, cut:], h2[:, cut:] = torch.randn(1, L - cut, 32), torch.randn(1, L - cut, 32)
    x2[:, cut:] = torch.randint(0, 7, (1, L - cut))
    with torch.no_grad():
        ya = layer(E.to(DEV), h.to(DEV), x.to(DEV))[:, :cut]
        yb = layer(E2.to(DEV), h2.to(DEV), x2.to(DEV))[:, :cut]
    assert torch.isfinite(ya).all()
    assert (ya - yb).abs().max().item() <= 1e-6 * ya.abs().max().item()


def test_layer_odd_feature_widths_vs_oracle():
    """P = 15 and cf = 6 (not multiples of 4): the host pads the feature rows with zero columns for the float4 reads;
    outputs and every gradient must still match the oracle."""
    say('layer odd widths P=15 cf=6')
    torch.manual_seed(2)
    kw = dict(n_tablas=5, tablas_contexto=2, n_bits=3, confirmar=6, chunk=8)
    layer = synth.move_params(CapaASRNEstable(32, **kw), 2)
    p = {k: v.detach().clone() for k, v in layer.state_dict().items()}
    sh = O.shape_from_params(p, 32, n_bits=3, C=8)
    x, E, h = synth.layer_inputs(2, 300, 32, 7, seed=4)
    gy = torch.randn(2, 300, 32, generator=torch.Generator().manual_seed(5))
    layer = layer.to(DEV)
    with torch.no_grad():
        phi, _ = layer._phi_y_valores(E.to(DEV))
    ids, _ = O.bucket_rows(phi.cpu(), sh.T, sh.nb)
    ref_phi, _ = O.phi_and_values(p, E)
    ref_ids, _ = O.bucket_rows(ref_phi, sh.T, sh.nb)
    if not torch.equal(ids, ref_ids):
        pytest.skip('a bucket id differs between the GPU GEMM and the CPU one (sign of phi near 0)')
    y, grads = run_layer(layer, E, h, x, gy)
    leaves = {k: (v.clone().requires_grad_() if v.is_floating_point() and k not in ('c_vistos', 'r_firma') else v)
              for k, v in p.items()}
    Ec, hc = E.clone().requires_grad_(), h.clone().requires_grad_()
    yo = O.layer_forward(leaves, Ec, hc, x, sh)
    (yo * gy).sum().backward()
    assert_close(y, yo, 'y')
    assert_close(grads['E'], Ec.grad, 'grad E')
    assert_close(grads['h'], hc.grad, 'grad h')
    for n, g in grads.items():
        if n in leaves and leaves[n].grad is not None:
            assert_close(g, leaves[n].grad, 'grad ' + n)


def test_layer_signatures_from_E_vs_oracle():
    """No token ids: the signatures are E r_firma (asrn/nucleo.py:161-164), computed on the layer's second stream.
    Outputs and every gradient match the oracle, and E's gradient is accumulated without a stream-mismatch warning
    (the signatures take no gradient, so the second stream holds no edge to E)."""
    say('layer signatures from E')
    torch.manual_seed(6)
    kw = dict(n_tablas=5, tablas_contexto=2, n_bits=4, confirmar=8, chunk=8)
    layer = synth.move_params(CapaASRNEstable(32, **kw), 6)
    p = {k: v.detach().clone() for k, v in layer.state_dict().items()}
    sh = O.shape_from_params(p, 32, n_bits=4, C=8)
    _, E, h = synth.layer_inputs(2, 400, 32, 9, seed=7)
    gy = torch.randn(2, 400, 32, generator=torch.Generator().manual_seed(8))
    layer = layer.to(DEV)
    with torch.no_grad():
        phi, _ = layer._phi_y_valores(E.to(DEV))
    ids, _ = O.bucket_rows(phi.cpu(), sh.T, sh.nb)
    ref_ids, _ = O.bucket_rows(O.phi_and_values(p, E)[0], sh.T, sh.nb)
    if not torch.equal(ids, ref_ids):
        pytest.skip('a bucket id differs between the GPU GEMM and the CPU one (sign of phi near 0)')
    import warnings
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter('always')
        y, grads = run_layer(layer, E, h, None, gy)
    assert not [w for w in caught if 'AccumulateGrad' in str(w.message)]
    leaves = {k: (v.clone().requires_grad_() if v.is_floating_point() and k not in ('c_vistos', 'r_firma') else v)
              for k, v in p.items()}
    Ec, hc = E.clone().requires_grad_(), h.clone().requires_grad_()
    yo = O.layer_forward(leaves, Ec, hc, None, sh)
    (yo * gy).sum().backward()
    assert_close(y, yo, 'y')
    assert_close(grads['E'], Ec.grad, 'grad E')
    assert_close(grads['h'], hc.grad, 'grad h')
    for n, g in grads.items():
        if n in leaves and leaves[n].grad is not None:
            assert_close(g, leaves[n].grad, 'grad ' + n)


def test_shared_ngram_sort_across_layers_is_bit_identical():
    """One n-gram sort for a stack of 6 layers (asrn_amd.ngramas, handed to every layer's forward) gives the same
    outputs and gradients, bit for bit, as each layer sorting the same tokens itself; a sort made for other tokens
    is refused."""
    say('shared n-gram sort, 6 layers')
    d, B, L = 64, 2, 700
    torch.manual_seed(5)
    capas = [synth.move_params(CapaASRNEstable(d), 10 + j).to(DEV) for j in range(6)]
    x, E, h = synth.layer_inputs(B, L, d, 40, seed=9)
    gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(2)).to(DEV)
    xd = x.to(DEV)
    outs = []
    for shared in (False, True):
        for c in capas:
            c.zero_grad()
        Ed, hd = E.to(DEV).requires_grad_(), h.to(DEV).requires_grad_()
        ng = asrn_amd.ngramas(xd, capas[0]) if shared else None
        y = hd
        for c in capas:
            y = c(Ed, y, xd, ngramas=ng)
        (y * gy).sum().backward()
        outs.append([y.detach(), Ed.grad, hd.grad] + [p.grad.clone() for c in capas for p in c.parameters()
                                                       if p.grad is not None])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    other = xd.clone()
    with pytest.raises(ValueError, match='other token ids'):
        capas[0](E.to(DEV), h.to(DEV), xd, ngramas=asrn_amd.ngramas(other, capas[0]))
