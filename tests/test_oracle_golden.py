"""Pins the CPU oracle against golden fixtures written from the reference (tests/golden/make_golden.py).

Stage-wise: each stage of the oracle runs on the reference's own upstream tensors, so integer outputs (bucket ids,
sorted orders, n-gram keys, their order, repeated flags, seen flags) must be bit-exact and floating-point ones must
agree to rounding. Whole layer: forward and every gradient."""
import pytest
import torch

from oracle import layer as O
from tests import fixtures

CASES = fixtures.names()


def close(a, b, rel, what):
    a, b = a.double(), b.double()
    scale = b.abs().max().item() + 1e-6
    err = (a - b).abs().max().item() if a.numel() else 0.0
    assert err <= rel * scale, f'{what}: max err {err:.3g} vs scale {scale:.3g}'


@pytest.mark.parametrize('name', CASES)
def test_bucket_ids_and_order_bit_exact(name):
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    ids, order = O.bucket_rows(g['phi'], sh.T, sh.nb)
    assert torch.equal(ids, g['ids'])
    assert torch.equal(order, g['orden'])


@pytest.mark.parametrize('name', CASES)
def test_producers(name):
    """phi, V, Qc, Kc, beta and log_alfa; a bf16 fixture runs the oracle under CPU autocast, where Qc/Kc come from
    the 16-bit LayerNorm output and the clock projection stays fp32 (estable:176-180): every output keeps the
    reference's dtype."""
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    with fixtures.cpu_autocast(m):
        phi, V = O.phi_and_values(p, g['E'])
        Qc, Kc, beta, la = O.context(p, g['h'], sh, fixtures.prot(m))
    close(phi, g['phi'], 1e-6, 'phi')
    close(V, g['V'], 1e-6, 'V')
    for a, k in ((phi, 'phi'), (V, 'V'), (Qc, 'Qc'), (Kc, 'Kc'), (beta, 'beta'), (la, 'log_alfa')):
        assert a.dtype == g[k].dtype, (k, a.dtype, g[k].dtype)
    for a, k in ((Qc, 'Qc'), (Kc, 'Kc'), (beta, 'beta'), (la, 'log_alfa')):
        close(a, g[k], 1e-6, k)
    assert beta.dtype == (torch.float32 if fixtures.nucleo(m) else torch.float64)


@pytest.mark.parametrize('name', CASES)
def test_candidate_stage_forward_and_gradients(name):
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    leaves = {k: fixtures.stage_input(g, k).clone().requires_grad_() for k in ('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa')}
    w = p['w_sufijo'].clone().requires_grad_()
    gam = p['gamma'].clone().requires_grad_()
    with fixtures.cpu_autocast(m):
        salida, sen = O.candidates(leaves['phi'], leaves['V'], leaves['Qc'], leaves['Kc'], leaves['Bt'],
                                   leaves['log_alfa'], g['sig'], w, gam, sh, fixtures.prot(m))
        acc = O.gate_signals(salida, sen, sh.T, sh.Tc)
    assert salida.dtype == g['acc.salida'].dtype
    for k in ('salida', 'pico'):
        close(acc[k], g['acc.' + k], 1e-5, k)
    for k in ('peso_total', 'peso_ctx'):
        assert torch.equal(acc[k], g['acc.' + k]), k
    close(acc['mejor'], g['acc.mejor'], 1e-5, 'mejor')
    (salida.float() * g['acc.gs']).sum().backward()
    for k, t in leaves.items():
        close(t.grad, g['acc.g_' + k], 1e-4, 'grad ' + k)
    close(w.grad, g['acc.g_w_sufijo'], 1e-4, 'grad w_sufijo')
    close(gam.grad, g['acc.g_gamma'], 1e-4, 'grad gamma')


@pytest.mark.parametrize('name', CASES)
def test_ngram_keys_order_and_flags_bit_exact(name):
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    keys = O.ngram_keys(g['sig'], p['c_vistos'], sh.n)
    ref = g['claves']
    assert torch.equal(torch.isnan(keys), torch.isnan(ref))
    assert torch.equal(torch.nan_to_num(keys, nan=-7.0), torch.nan_to_num(ref, nan=-7.0))
    order, rep = O.ngram_sort(keys)
    assert torch.equal(order, g['orden_k'])
    assert torch.equal(rep, g['repetido'].bool())


@pytest.mark.parametrize('name', CASES)
def test_repetition_stage_forward_and_gradients(name):
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    rl = {k: g[k].clone().requires_grad_() for k in ('beta', 'Bt', 'log_alfa')}
    pp = dict(p)
    pp['log_kappa'] = p['log_kappa'].clone().requires_grad_()
    pp['log_kappa_racha'] = p['log_kappa_racha'].clone().requires_grad_()
    r = O.repetition(pp, g['sig'], rl['beta'], rl['Bt'], rl['log_alfa'], sh, fixtures.prot(m))
    assert torch.equal(r['vistos'], g['rep.vistos'])
    if 'corrimiento' not in m['extra']:                          # with huge clock steps exp(-kappa dB) underflows
        assert torch.equal(r['hawkes'] > 0, g['rep.vistos'] > 0)
    close(r['hawkes'], g['rep.hawkes'], 1e-5, 'hawkes')
    if m['extra'].get('kappa_r_zero'):
        assert torch.equal(r['racha'], g['rep.racha'])            # integer run lengths: bit-exact
    else:
        close(r['racha'], g['rep.racha'], 1e-5, 'racha')
    ((r['hawkes'] * g['rep.gh']).sum() + (r['racha'] * g['rep.gr']).sum()).backward()
    for k, t in rl.items():
        close(t.grad, g['rep.g_' + k], 1e-4, 'grad ' + k)
    close(pp['log_kappa'].grad, g['rep.g_log_kappa'], 1e-4, 'grad log_kappa')
    close(pp['log_kappa_racha'].grad, g['rep.g_log_kappa_racha'], 1e-4, 'grad log_kappa_racha')


@pytest.mark.parametrize('name', CASES)
def test_whole_layer_forward_and_gradients(name):
    g, p, m = fixtures.load(name)
    sh = fixtures.shape_of(p, m)
    pp = {k: (v.clone().requires_grad_() if v.is_floating_point() and not k.startswith(('pot', 'c_vistos', 'r_firma'))
              else v) for k, v in p.items()}
    E, h = g['E'].clone().requires_grad_(), g['h'].clone().requires_grad_()
    with fixtures.cpu_autocast(m):
        y = O.layer_forward(pp, E, h, g['x'], sh, fixtures.prot(m))
    assert y.dtype == torch.float32
    close(y, g['y'], 1e-5, 'y')
    (y * g['gy']).sum().backward()
    close(E.grad, g['gE'], 1e-4, 'grad E')
    close(h.grad, g['gh'], 1e-4, 'grad h')
    for k, t in pp.items():
        if ('g.' + k) in g:
            assert t.grad is not None, k
            close(t.grad, g['g.' + k], 1e-4, 'grad ' + k)


def test_core_layer_mistakes_fail_the_fixtures():
    """Planted mistakes in the oracle's core-layer mode fail the reference's core fixtures: the protected layer's clock
    difference instead of v89's (log alfa_k + rate B_k) - rate B_q (the offset-clock fixture: salida and every gradient
    off by ~1e-4, d gamma by ~3e-3), and the exact mask instead of v89's -1e9 fill (the gamma = 1e9 fixture, where the
    fill leaks weight to invalid keys: salida off by ~0.4)."""
    import dataclasses

    def stage_error(name, prot):
        g, p, m = fixtures.load(name)
        sh = fixtures.shape_of(p, m)
        leaves = {k: fixtures.stage_input(g, k).clone().requires_grad_()
                  for k in ('phi', 'V', 'Qc', 'Kc', 'Bt', 'log_alfa')}
        gam = p['gamma'].clone().requires_grad_()
        salida, _ = O.candidates(leaves['phi'], leaves['V'], leaves['Qc'], leaves['Kc'], leaves['Bt'],
                                 leaves['log_alfa'], g['sig'], p['w_sufijo'], gam, sh, prot)
        (salida * g['acc.gs']).sum().backward()
        e_s = ((salida - g['acc.salida']).abs().max() / g['acc.salida'].abs().max()).item()
        e_g = ((gam.grad - g['acc.g_gamma']).abs().max() / g['acc.g_gamma'].abs().max()).item()
        return e_s, e_g

    core = O.Prot.ninguna()
    assert stage_error('n_nucleo_reloj_desplazado', core) == (0.0, 0.0)
    e_s, e_g = stage_error('n_nucleo_reloj_desplazado', dataclasses.replace(core, reloj_64=True))
    assert e_s > 3e-5 and e_g > 1e-3, (e_s, e_g)
    assert stage_error('m_nucleo_gamma_huge', core)[0] == 0.0
    assert stage_error('m_nucleo_gamma_huge', dataclasses.replace(core, mascara_exacta=True))[0] > 0.1
