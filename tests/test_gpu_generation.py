"""The O(1) generation step on the GPU, through the C ABI, against the oracle (oracle/generation.py) and against the
whole-text layer.

Bit-exact: ring contents slot by slot and counts (after the prompt and after every insert), the step's bucket ids,
the Hawkes memory's seen flags. Within 1e-3 relative (fp32): the step's candidate attention output and gate
signals, Hawkes intensities, streak, and the layer output written step by step. Each test prints its case first."""
import numpy as np
import pytest
import torch

import asrn_amd
from asrn_amd import ops, synth
from asrn_amd.capa import CapaASRNEstable
from asrn_amd.escritura import EscritorCapa
from oracle import generation as G
from oracle import layer as O

pytestmark = pytest.mark.gpu
DEV = 'cuda'
TOL = 1e-3


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


def token_phi(B, L, V, T, nb, seed):
    """phi whose word half depends on the token and context half on (token, previous token): buckets repeat."""
    g = torch.Generator().manual_seed(seed)
    x = synth.tokens(B, L, V, frac=0.3, span=(4, 16), seed=seed)
    P = T * nb
    emb = torch.randn(V, P, generator=g)
    prev = torch.cat([x[:, :1], x[:, :-1]], 1)
    phi = torch.cat([emb[x][..., :P // 2], emb[x][..., P // 2:] + 0.7 * emb[prev][..., P // 2:]], -1).contiguous()
    return x, phi, g


def gpu_rings_as_oracle(rings, counts, B, T):
    nc, C = rings.shape[1], rings.shape[2]
    return rings.cpu().numpy().reshape(B, T, nc, C), counts.cpu().numpy().reshape(B, T, nc).astype(np.int64)


# ---------------------------------------------------------------------------------------------------------------------
# rings
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('B,n,T,nb,C,V', [(2, 300, 8, 14, 32, 6), (3, 200, 4, 2, 4, 5), (2, 0, 8, 3, 4, 5),
                                          (1, 1, 8, 3, 4, 5), (16, 4096, 8, 14, 32, 40), (2, 5000, 8, 4, 64, 3)])
def test_ring_build_vs_oracle(B, n, T, nb, C, V):
    say('ring build', B, n, T, nb, C)
    x, phi, _ = token_phi(B, max(n, 1), V, T, nb, seed=n)
    phi = phi[:, :n]
    rings, counts = ops.ring_build(phi.to(DEV), T, nb, C)
    ids = O.bucket_ids(phi, T, nb).numpy() if n else np.zeros((B, 0, T), dtype=np.int32)
    ring_ref, count_ref = G.ring_from(ids, n, C, 2 ** nb)
    got_ring, got_count = gpu_rings_as_oracle(rings, counts, B, T)
    assert np.array_equal(got_count, count_ref)
    assert np.array_equal(got_ring, ring_ref)


# ---------------------------------------------------------------------------------------------------------------------
# the step's candidate attention, with inserts
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('B,t0,steps,d,C,nb,T,V,split', [
    (2, 300, 24, 64, 32, 14, 8, 6, True), (3, 100, 40, 96, 4, 2, 4, 5, True), (2, 1, 30, 256, 16, 4, 8, 4, True),
    (1, 500, 8, 1024, 8, 3, 8, 7, True), (16, 2000, 4, 768, 32, 14, 8, 50, True), (2, 200, 6, 64, 8, 14, 16, 6, True),
    (16, 2000, 4, 768, 32, 14, 8, 50, False), (3, 60, 30, 520, 4, 2, 4, 5, True)])
def test_decode_attend_vs_oracle(B, t0, steps, d, C, nb, T, V, split):
    """The step's attention against the oracle, step after step, and the rings after each insert. split: with the
    per-row count buffer, so that d > 256 runs each row's value columns on several workgroups (the last of a row to
    finish its ring reads inserting); the buffer is back to zero after every launch."""
    say('decode attend', B, t0, steps, d, C, nb, T, split)
    L = t0 + steps
    cf, K, Tc = 16, 4, T // 2
    x, phi, g = token_phi(B, L, V, T, nb, seed=t0 + d)
    cache = dict(phi=phi, V=torch.randn(B, L, d, generator=g), Qc=torch.randn(B, L, cf, generator=g),
                 Kc=torch.randn(B, L, cf, generator=g), sig=x.float(),
                 Bt=(torch.rand(B, L, generator=g, dtype=torch.float64) * 1.5).cumsum(1),
                 log_alfa=torch.randn(B, L, generator=g) * 0.3)
    w_suf = torch.randn(K + 1, generator=g) * 0.5
    gamma = torch.rand(T, generator=g) * 2
    sh = O.Shape(d=d, T=T, nb=nb, C=C, Tc=Tc, cf=cf, K=K)
    ids = O.bucket_ids(phi, T, nb).numpy()
    ring, count = G.ring_from(ids, t0, C, 2 ** nb)
    dcache = {k: v.to(DEV).contiguous() for k, v in cache.items()}
    rings = torch.from_numpy(ring.reshape(B * T, 2 ** nb, C)).to(DEV)
    counts = torch.from_numpy(count.reshape(B * T, 2 ** nb).astype(np.int32)).to(DEV)
    shape = dict(T=T, Tc=Tc, C=C, K=K, nb=nb)
    hechos = torch.zeros(B, dtype=torch.int32, device=DEV) if split else None
    for t in range(t0, L):
        sal, sen, got_ids = ops.decode_attend(dcache, t, rings, counts, w_suf.to(DEV), gamma.to(DEV), shape,
                                              insert=True, hechos=hechos)
        assert hechos is None or not hechos.any(), t
        ref_sal, ref_sen = G.attend(G.ring_positions(ring, ids[:, t]), t, cache['phi'], cache['V'], cache['Qc'],
                                    cache['Kc'], cache['sig'], cache['Bt'], cache['log_alfa'], w_suf, gamma, sh)
        assert np.array_equal(got_ids.cpu().numpy(), ids[:, t]), t
        assert_close(sal, ref_sal, f'salida t={t}')
        assert torch.equal(sen[:, 0].cpu(), ref_sen[:, 0]), t                  # tables with candidates
        assert torch.equal(sen[:, 3].cpu(), ref_sen[:, 3]), t
        assert_close(sen[:, 1], ref_sen[:, 1], f'mejor t={t}')
        assert_close(sen[:, 2], ref_sen[:, 2], f'pico t={t}')
        G.ring_insert(ring, count, ids[:, t], t)
        got_ring, got_count = gpu_rings_as_oracle(rings, counts, B, T)
        assert np.array_equal(got_count, count) and np.array_equal(got_ring, ring), f'rings after insert t={t}'


def test_decode_attend_without_insert_leaves_rings():
    say('decode attend, no insert')
    B, L, T, nb, C, d = 2, 80, 8, 3, 4, 64
    x, phi, g = token_phi(B, L, 5, T, nb, seed=11)
    cache = dict(phi=phi, V=torch.randn(B, L, d, generator=g), Qc=torch.randn(B, L, 16, generator=g),
                 Kc=torch.randn(B, L, 16, generator=g), sig=x.float(),
                 Bt=torch.rand(B, L, generator=g, dtype=torch.float64).cumsum(1), log_alfa=torch.zeros(B, L))
    dcache = {k: v.to(DEV).contiguous() for k, v in cache.items()}
    rings, counts = ops.ring_build(phi[:, :40].to(DEV), T, nb, C)
    r0, c0 = rings.clone(), counts.clone()
    for t in range(40, 60):
        ops.decode_attend(dcache, t, rings, counts, torch.zeros(5, device=DEV), torch.ones(T, device=DEV),
                          dict(T=T, Tc=4, C=C, K=4, nb=nb), insert=False)
    assert torch.equal(rings, r0) and torch.equal(counts, c0)


# ---------------------------------------------------------------------------------------------------------------------
# Hawkes memory and streak
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('B,L0,steps,V,n', [(3, 50, 150, 5, 4), (2, 1, 60, 3, 4), (4, 700, 40, 30, 4), (2, 20, 30, 4, 6)])
def test_hawkes_table_vs_oracle(B, L0, steps, V, n):
    say('hawkes table', B, L0, steps, V, n)
    L = L0 + steps
    g = torch.Generator().manual_seed(L0)
    x = synth.tokens(B, L, V, frac=0.3, span=(3, 10), seed=L0)
    sig = x.float()
    beta = torch.rand(B, L, generator=g, dtype=torch.float64) * 2
    Bt = beta.cumsum(1)
    la = torch.randn(B, L, generator=g) * 0.5
    coef = torch.rand(n, generator=torch.Generator().manual_seed(12345), dtype=torch.float64) + 0.5
    kappa = torch.rand(n, generator=g) * 0.3 + 0.01
    kappa_r = torch.rand(1, generator=g) * 0.1 + 0.01
    keys, order, rep, rank_k, vistos = ops.ngram_sort(sig[:, :L0].to(DEV), coef.to(DEV), n)
    hk = ops.Hawkes.apply(Bt[:, :L0].to(DEV), la[:, :L0].to(DEV), kappa.to(DEV), order, rep, rank_k)
    tab = ops.HawkesTable.load(keys, order, rep, hk, Bt[:, :L0].to(DEV), la[:, :L0].to(DEV))
    mem = G.HawkesMemory(B, n)
    mem.load(keys.cpu(), hk.cpu(), Bt[:, :L0], la[:, :L0])
    cache = dict(sig=sig.to(DEV).contiguous(), Bt=torch.zeros(B, L, dtype=torch.float64, device=DEV),
                 log_alfa=la.to(DEV).contiguous())
    cache['Bt'][:, :L0] = Bt[:, :L0].to(DEV)
    racha = torch.rand(B, generator=g).to(DEV)
    racha_ref = racha.cpu().clone()
    all_keys = O.ngram_keys(sig, coef, n)
    cap0 = tab.cap
    for t in range(L0, L):
        v, h = tab.step(cache, t, beta[:, t].to(DEV), coef.to(DEV), kappa.to(DEV), kappa_r.to(DEV), racha)
        Bq = cache['Bt'][:, t].cpu()
        assert torch.equal(Bq, Bt[:, t - 1] + beta[:, t]), t
        v_ref, h_ref = mem.step(all_keys[:, t], Bq, la[:, t], kappa)
        racha_ref = G.streak_step(v_ref, beta[:, t], racha_ref, kappa_r)
        assert torch.equal(v.cpu(), v_ref), t
        assert_close(h, h_ref, f'hawkes t={t}', 1e-5)
        assert_close(racha, racha_ref, f'racha t={t}', 1e-5)
    assert tab.cap > cap0 or 2 * L <= cap0                 # the tables grew when they had to


def table_contents(tab):
    """Each group's (key, Bu, A) ordered by key code, empty slots zeroed: the prompt's load and a growth place
    colliding keys by concurrent compare-and-swap, so two tables with the same contents may differ slot by slot."""
    keys, idx = torch.sort(tab.keys, dim=1)
    held = keys != -1                                      # Bu and A are only defined where a key is stored
    return (keys, torch.where(held, tab.Bu.gather(1, idx), torch.zeros((), dtype=tab.Bu.dtype, device=DEV)),
            torch.where(held, tab.A.gather(1, idx), torch.zeros((), dtype=tab.A.dtype, device=DEV)))


@pytest.mark.parametrize('B,t0,steps,d,C,nb,T,V,n,reloj32,dev_pos', [
    (2, 300, 24, 64, 32, 14, 8, 6, 4, False, False), (3, 40, 30, 96, 4, 2, 4, 5, 4, True, True),
    (16, 500, 6, 768, 32, 14, 8, 50, 4, False, True), (2, 1, 20, 64, 8, 3, 8, 4, 6, True, False)])
def test_decode_attend_repeat_equals_two_calls(B, t0, steps, d, C, nb, T, V, n, reloj32, dev_pos):
    """asrn_decode_attend_repeat (the repetition step in the attention's launch) against asrn_repetition_step then
    asrn_decode_attend on a copy of the same state, bit for bit, step after step: the attention's outputs and ids, the
    step's vistos and hawkes, the clock cache, the streak, the rings and counts and the Hawkes tables (which also
    grow on the way in the t0 = 1 case)."""
    say('decode attend + repetition = two calls', B, t0, steps, d, C, nb, T, n, reloj32, dev_pos)
    L = t0 + steps
    cf, K, Tc = 16, 4, T // 2
    x, phi, g = token_phi(B, L, V, T, nb, seed=t0 + d + n)
    beta = torch.rand(B, L, generator=g, dtype=torch.float64) * 1.5
    Bt = beta.cumsum(1)
    if reloj32:                                            # the core layer's clock holds fp32 values
        Bt = Bt.float().double()
    la = torch.randn(B, L, generator=g) * 0.3
    coef = torch.rand(n, generator=g, dtype=torch.float64) + 0.5
    kappa = (torch.rand(n, generator=g) * 0.3 + 0.01).to(DEV)
    kappa_r = (torch.rand(1, generator=g) * 0.1 + 0.01).to(DEV)
    w_suf = (torch.randn(K + 1, generator=g) * 0.5).to(DEV)
    gamma = (torch.rand(T, generator=g) * 2).to(DEV)
    cache = dict(phi=phi, V=torch.randn(B, L, d, generator=g), Qc=torch.randn(B, L, cf, generator=g),
                 Kc=torch.randn(B, L, cf, generator=g), sig=x.float(), Bt=torch.zeros(B, L, dtype=torch.float64),
                 log_alfa=la)
    cache['Bt'][:, :t0] = Bt[:, :t0]
    sig_d = x.float().to(DEV)
    keys, order, rep, rank_k, _ = ops.ngram_sort(sig_d[:, :t0], coef.to(DEV), n)
    hk = ops.Hawkes.apply(Bt[:, :t0].to(DEV), la[:, :t0].to(DEV), kappa, order, rep, rank_k)
    states = []
    for _ in range(2):
        tab = ops.HawkesTable.load(keys, order, rep, hk, Bt[:, :t0].to(DEV), la[:, :t0].to(DEV))
        rings, counts = ops.ring_build(phi[:, :t0].to(DEV), T, nb, C)
        states.append(dict(cache={k: v.to(DEV).contiguous() for k, v in cache.items()}, tab=tab, rings=rings,
                           counts=counts, racha=torch.rand(B, generator=torch.Generator().manual_seed(3)).to(DEV)))
    sep, fus = states
    shape = dict(T=T, Tc=Tc, C=C, K=K, nb=nb)
    hechos = [torch.zeros(B, dtype=torch.int32, device=DEV) for _ in range(2)]   # d > 256: the column split
    for t in range(t0, L):
        pos = torch.full((1,), t, dtype=torch.int64, device=DEV) if dev_pos else t
        t_max = L - 1 if dev_pos else None
        bt = beta[:, t].to(DEV)
        v1, h1 = sep['tab'].step(sep['cache'], pos, bt, coef.to(DEV), kappa, kappa_r, sep['racha'], t_max=t_max,
                                 reloj32=reloj32)
        s1, g1, i1 = ops.decode_attend(sep['cache'], pos, sep['rings'], sep['counts'], w_suf, gamma, shape,
                                       insert=True, t_max=t_max, hechos=hechos[0])
        s2, g2, i2, v2, h2 = ops.decode_attend_repeat(fus['cache'], pos, fus['rings'], fus['counts'], w_suf, gamma,
                                                      shape, True, fus['tab'], bt, coef.to(DEV), kappa, kappa_r,
                                                      fus['racha'], t_max=t_max, reloj32=reloj32, hechos=hechos[1])
        for a_, b_, what in ((s1, s2, 'salida'), (g1, g2, 'signals'), (i1, i2, 'ids'), (v1, v2, 'vistos'),
                             (h1, h2, 'hawkes'), (sep['racha'], fus['racha'], 'racha'),
                             (sep['cache']['Bt'], fus['cache']['Bt'], 'Bt'), (sep['rings'], fus['rings'], 'rings'),
                             (sep['counts'], fus['counts'], 'counts')):
            assert torch.equal(a_, b_), f'{what} t={t}'
        assert sep['tab'].cap == fus['tab'].cap
        for a_, b_, what in zip(table_contents(sep['tab']), table_contents(fus['tab']), ('keys', 'Bu', 'A')):
            assert torch.equal(a_, b_), f'table {what} t={t}'
    assert fus['tab'].cap >= 2 * L


# ---------------------------------------------------------------------------------------------------------------------
# the layer written step by step
# ---------------------------------------------------------------------------------------------------------------------

def write(layer, E, h, x, L0, ajeno, capacidad):
    esc = EscritorCapa(layer, memoria_de_lo_ajeno=ajeno)
    Ed, hd, xd = E.to(DEV), h.to(DEV), x.to(DEV)
    y0 = esc.inicio(Ed[:, :L0], hd[:, :L0], xd[:, :L0], capacidad=capacidad)
    ys = [esc.paso(Ed[:, t], hd[:, t], xd[:, t]) for t in range(L0, E.shape[1])]
    return y0, torch.stack(ys, 1), esc


def ids_agree(layer, E, sh, ref=None):
    """The step's phi (the producer over two rows) and the whole text's give the same bucket ids (and `ref`)."""
    with torch.no_grad():
        whole, _ = layer._phi_y_valores(E.to(DEV))
        Ed = E.to(DEV)
        step = torch.stack([layer._phi_y_valores(Ed[:, max(0, t - 1):t + 1])[0][:, -1] for t in range(E.shape[1])],
                           1)
    a, b = O.bucket_ids(whole.cpu(), sh.T, sh.nb), O.bucket_ids(step.cpu(), sh.T, sh.nb)
    return torch.equal(a, b) and (ref is None or torch.equal(a, ref))


SMALL = dict(chunk=4, n_bits=2, n_tablas=4, tablas_contexto=2)


@pytest.mark.parametrize('clase', ['estable', 'nucleo'])
@pytest.mark.parametrize('B,L0,n,kw', [(2, 40, 50, SMALL), (1, 2, 30, SMALL), (3, 1, 20, SMALL), (2, 300, 60, {}),
                                       (2, 64, 40, dict(chunk=16, n_bits=4))])
def test_writer_equals_whole_text(B, L0, n, kw, clase):
    """The writer's steps equal the whole-text layer position by position: the protected layer, and the core layer
    (CapaASRN, v89 numerics), whose step advances its fp32 clock in fp32 and takes the clock difference (nucleo:937,
    1826) where the whole text forms (log alfa_k + rate B_k) - rate B_q from the rounded cumsum; no leak counted."""
    say('writer = whole text', B, L0, n, kw, clase)
    d = 64
    torch.manual_seed(0)
    capa = asrn_amd.CapaASRN(d, **kw) if clase == 'nucleo' else CapaASRNEstable(d, **kw)
    layer = synth.move_params(capa, 0).to(DEV)
    x, E, h = synth.layer_inputs(B, L0 + n, d, 12, seed=L0, frac=0.4, span=(3, 8))
    sh = O.shape_from_params({k: v.cpu() for k, v in layer.state_dict().items()}, d, n_bits=layer.n_bits,
                             C=layer.chunk)
    if not ids_agree(layer, E, sh):
        pytest.skip('a bucket id differs between the step GEMM and the whole-text GEMM (sign of phi near 0)')
    y0, ys, esc = write(layer, E, h, x, L0, ajeno=False, capacidad=L0 + 3)
    with torch.no_grad():
        y = layer(E.to(DEV), h.to(DEV), x.to(DEV))
    assert_close(y0, y[:, :L0], 'prompt')
    assert_close(ys, y[:, L0:], 'steps')
    assert esc.cap >= L0 + n
    if clase == 'nucleo':
        assert layer.fugas() == 0 and int(esc.fugas_t.item()) == 0


# the generation step's fallback branch (not asrn_decode_produce): widths past the fused producer's limits
FALLBACK = [dict(confirmar=80), dict(afin_oculto=256)]


@pytest.mark.parametrize('ajeno', [True, False])
@pytest.mark.parametrize('B,L0,n,kw', [(2, 40, 30, SMALL), (1, 2, 12, SMALL), (2, 100, 20, {}),
                                       (2, 60, 16, FALLBACK[0]), (2, 60, 16, FALLBACK[1])])
def test_writer_vs_oracle(B, L0, n, kw, ajeno):
    say('writer vs oracle', B, L0, n, kw, ajeno)
    d = 32
    torch.manual_seed(1)
    layer = synth.move_params(CapaASRNEstable(d, **kw), 1).to(DEV)
    assert ops.decode_produce_ok(layer, torch.zeros(B, d, device=DEV)) == (kw not in FALLBACK)
    p = {k: v.detach().cpu() for k, v in layer.state_dict().items()}
    sh = O.shape_from_params(p, d, n_bits=layer.n_bits, C=layer.chunk)
    x, E, h = synth.layer_inputs(B, L0 + n, d, 10, seed=5, frac=0.4, span=(3, 8))
    phi_cpu = torch.stack([O.phi_and_values(p, E[:, max(0, t - 1):t + 1])[0][:, -1] for t in range(L0 + n)], 1)
    if not ids_agree(layer, E, sh, O.bucket_ids(phi_cpu, sh.T, sh.nb)):
        pytest.skip('a bucket id differs between the GPU GEMMs and the CPU one (sign of phi near 0)')
    _, ys, _ = write(layer, E, h, x, L0, ajeno=ajeno, capacidad=0)
    ref, _ = G.decode_layer(p, E, h, x, L0, sh, ajeno=ajeno)
    assert_close(ys, ref, f'steps ajeno={ajeno}')


@pytest.mark.parametrize('ajeno', [True, False])
@pytest.mark.parametrize('B,L0,n,cap,kw,bf16', [(2, 40, 30, 45, SMALL, False), (3, 300, 24, 0, {}, False),
                                                (1, 2, 20, 4, SMALL, False), (2, 60, 20, 70, FALLBACK[0], False),
                                                (2, 60, 20, 0, FALLBACK[1], False), (2, 60, 20, 70, {}, True)])
def test_writer_graph_equals_eager(B, L0, n, cap, kw, bf16, ajeno):
    """The step captured in a HIP graph and replayed (its position copied before each replay, with its inputs, from
    a device table of positions into the buffer the kernels read; a capacity doubling captures again) writes the
    same outputs, caches, rings, counts and streak as the step launched op by op, bit for bit, step after step. The
    FALLBACK widths and bf16 autocast take the step's PyTorch-producer branch, whose cache rows are written with
    index_copy_ at the device-held position."""
    say('writer graph = eager', B, L0, n, cap, kw, bf16, ajeno)
    d = 32
    torch.manual_seed(2)
    layer = synth.move_params(CapaASRNEstable(d, **kw), 2).to(DEV)
    x, E, h = synth.layer_inputs(B, L0 + n, d, 9, seed=7, frac=0.4, span=(3, 8))
    Ed, hd, xd = E.to(DEV), h.to(DEV), x.to(DEV)
    with torch.autocast('cuda', dtype=torch.bfloat16, enabled=bf16):
        ok = ops.decode_produce_ok(layer, Ed[:, 0])
    assert ok == (kw not in FALLBACK and not bf16)
    outs = []
    for grafo in (False, True):
        esc = EscritorCapa(layer, memoria_de_lo_ajeno=ajeno, grafo=grafo)
        with torch.autocast('cuda', dtype=torch.bfloat16, enabled=bf16):
            esc.inicio(Ed[:, :L0], hd[:, :L0], xd[:, :L0], capacidad=cap)
            ys = [esc.paso(Ed[:, t], hd[:, t], xd[:, t]) for t in range(L0, L0 + n)]
        torch.cuda.synchronize()
        outs.append((torch.stack(ys, 1), esc))
    (ye, ee), (yg, eg) = outs
    assert eg._g is not None and eg.t == ee.t == L0 + n and eg.cap == ee.cap
    assert torch.equal(yg, ye)
    for k in ee.cache:
        assert torch.equal(eg.cache[k][:, :L0 + n], ee.cache[k][:, :L0 + n]), k
    assert torch.equal(eg.anillos, ee.anillos) and torch.equal(eg.cuentas, ee.cuentas)
    assert torch.equal(eg.racha, ee.racha)


@pytest.mark.parametrize('B,d,kw', [(16, 768, {}), (3, 64, SMALL), (2, 32, dict(confirmar=8, n_tablas=5, n_bits=4))])
def test_decode_produce_matches_the_ops(B, d, kw):
    """asrn_decode_produce (the step's V, phi, Qc, Kc, log_alfa, id rows and beta in two kernels) against the same rows
    from the layer's own ops (the hash producer, the context producer, W_v), within 1e-5 relative: the same products
    summed in another order. Also through a device-held position, and from strided views of the text (the wrapper's
    contiguous copies held until the launch: freed early, the next copy reused their memory)."""
    say('decode produce = ops', B, d, kw)
    torch.manual_seed(4)
    layer = synth.move_params(CapaASRNEstable(d, **kw), 4).to(DEV)
    x, E, h = synth.layer_inputs(B, 40, d, 9, seed=3)
    Ed, hd, xd = E.to(DEV), h.to(DEV), x.to(DEV)
    esc = EscritorCapa(layer, memoria_de_lo_ajeno=False)
    esc.inicio(Ed[:, :30], hd[:, :30], xd[:, :30], capacidad=40)
    t = 30
    e_t, e_prev, h_t = Ed[:, t].contiguous(), Ed[:, t - 1].contiguous(), hd[:, t].contiguous()
    assert ops.decode_produce_ok(layer, e_t)
    with torch.no_grad():
        v = layer.v(e_t)
        phi = layer._phi_y_valores(torch.stack([e_prev, e_t], 1))[0][:, -1]
        Qc, Kc, beta, la = layer._contexto(h_t.unsqueeze(1))
    strided = (Ed[:, t], Ed[:, t - 1], hd[:, t])             # views: the wrapper's converted copies must live on
    for pos, ins in ((t, (e_t, e_prev, h_t)), (torch.full((1,), t, dtype=torch.int64, device=DEV), strided),
                     (t, strided)):
        cache = {k: v_.clone() for k, v_ in esc.cache.items()}
        got_beta = ops.decode_produce(layer, cache, *ins, xd[:, t], pos, t_max=t)
        assert_close(cache['V'][:, t - 1], v, 'V', 1e-5)
        assert_close(cache['phi'][:, t], phi, 'phi', 1e-5)
        assert_close(cache['Qc'][:, t], Qc[:, 0], 'Qc', 1e-5)
        assert_close(cache['Kc'][:, t], Kc[:, 0], 'Kc', 1e-5)
        assert_close(cache['log_alfa'][:, t], la[:, 0], 'log_alfa', 1e-5)
        assert_close(got_beta, beta[:, 0], 'beta', 1e-5)
        assert torch.equal(cache['sig'][:, t], xd[:, t].float())
        for k in cache:                                    # nothing else written
            rows = [t - 1, t] if k == 'V' else [t]
            keep = [i for i in range(cache[k].shape[1]) if i not in rows]
            assert torch.equal(cache[k][:, keep], esc.cache[k][:, keep]), k


@pytest.mark.parametrize('B,d,kw,L', [(16, 768, {}, 3), (3, 64, SMALL, 2), (2, 32, dict(confirmar=8, n_tablas=5, n_bits=4), 1)])
def test_decode_produce_split_equals_whole(B, d, kw, L):
    """asrn_decode_produce_e for L layers at once, then asrn_decode_produce_h for each layer, write what
    asrn_decode_produce writes layer by layer, bit for bit: every cache (V at t - 1; phi, Qc, Kc, log_alfa, sig at t;
    nothing else) and beta, through a device-held position as the captured model step passes it."""
    say('decode produce split', B, d, kw, L)
    capas, caches, hs = [], [], []
    x, E, h = synth.layer_inputs(B, 40, d, 9, seed=3)
    Ed, xd = E.to(DEV), x.to(DEV)
    for l in range(L):
        torch.manual_seed(10 + l)
        layer = synth.move_params(CapaASRNEstable(d, **kw), 10 + l).to(DEV)
        esc = EscritorCapa(layer, memoria_de_lo_ajeno=False)
        hl = (h + 0.3 * l).to(DEV)
        esc.inicio(Ed[:, :30], hl[:, :30], xd[:, :30], capacidad=40)
        capas.append(layer)
        caches.append(esc.cache)
        hs.append(hl[:, 30].contiguous())
    t = 30
    e_t, e_prev = Ed[:, t].contiguous(), Ed[:, t - 1].contiguous()
    pos = torch.full((1,), t, dtype=torch.int64, device=DEV)
    whole = [{k: v.clone() for k, v in c.items()} for c in caches]
    split = [{k: v.clone() for k, v in c.items()} for c in caches]
    assert ops.decode_produce_e_ok(capas, split, e_t)
    betas_w = [ops.decode_produce(capas[l], whole[l], e_t, e_prev, hs[l], xd[:, t], pos, t_max=t) for l in range(L)]
    ops.decode_produce_e(capas, split, e_t, e_prev, xd[:, t], pos, t_max=t)
    betas_s = [ops.decode_produce_h(capas[l], split[l], hs[l], pos, t_max=t) for l in range(L)]
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(betas_w[l], betas_s[l]), l
        for k in whole[l]:
            assert torch.equal(whole[l][k], split[l][k]), (l, k)
        assert not torch.equal(whole[l]['phi'], caches[l]['phi'])     # the step wrote something


@pytest.mark.parametrize('B,d,kw,k,ff', [(16, 768, {}, 4, 1536), (3, 64, SMALL, 1, 40),
                                         (2, 32, dict(confirmar=8, n_tablas=5, n_bits=4), 3, 4096)])
def test_decode_produce_h_finishes_pending_block(B, d, kw, k, ff):
    """A local block step left pending (asrn_block_step_ex, finish = 0) then finished by the layer's producer
    (asrn_decode_produce_h_ex) against the finished block step then asrn_decode_produce_h on its output, bit for bit:
    the block's output and ring, every cache and beta. The feed-forward widths give 6, 1 and 16 depth splits of the
    second product (the 8-, 4- and 16-load instances); k = 1 has no ring."""
    say('decode produce h pending', B, d, kw, k, ff)
    x, E, h = synth.layer_inputs(B, 40, d, 9, seed=4)
    torch.manual_seed(20)
    layer = synth.move_params(CapaASRNEstable(d, **kw), 20).to(DEV)
    esc = EscritorCapa(layer, memoria_de_lo_ajeno=False)
    esc.inicio(E.to(DEV)[:, :30], h.to(DEV)[:, :30], x.to(DEV)[:, :30], capacidad=40)
    t = 30
    pos = torch.full((1,), t, dtype=torch.int64, device=DEV)
    with torch.no_grad():
        blq = asrn_amd.BloqueLocal(d, k, ff).to(DEV)
        for p in blq.parameters():
            p.add_(torch.randn_like(p) * 0.1)
        hin = torch.randn(B, d, device=DEV)
        anillo = torch.randn(B, d, k - 1, device=DEV) if k > 1 else None
        anillo2 = anillo.clone() if k > 1 else None
        espacio = ops.espacio_bloque(B, d, ff, DEV)
        whole = {kk: v.clone() for kk, v in esc.cache.items()}
        fused = {kk: v.clone() for kk, v in esc.cache.items()}
        out = ops.paso_bloque(blq, hin, anillo, pos, espacio)
        beta_w = ops.decode_produce_h(layer, whole, out, pos, t_max=t)
        pend = ops.paso_bloque(blq, hin, anillo2, pos, espacio, terminar=False)
        assert isinstance(pend, ops.BloquePendiente)
        beta_f = ops.decode_produce_h(layer, fused, None, pos, t_max=t, previo=pend)
        torch.cuda.synchronize()
    assert torch.equal(out, pend.out)
    assert k == 1 or torch.equal(anillo, anillo2)
    assert torch.equal(beta_w, beta_f)
    for kk in whole:
        assert torch.equal(whole[kk], fused[kk]), kk
    assert not torch.equal(whole['Qc'], esc.cache['Qc'])              # the step wrote something
