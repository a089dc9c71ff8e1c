"""The HIP layer at the benchmark configurations' full sizes and under bf16 autocast, against the oracle.

- cfg2 (B 8, N 4096, d 256, fp32): the whole layer and every gradient against the oracle with the reference's own
  full-size GPU-vs-CPU criterion (tests/verificar_gpu.py:221-229): at least 99% of positions within 1e-3 (a bucket id
  is the sign of a GEMM output, and the GPU and CPU GEMMs may round one near 0 differently) and the gradients'
  relative norm below 1e-3. The bucket-id flips between the HIP phi and the oracle's are counted and printed.
- bf16: the reference's acceptance rule for a 16-bit kernel (tests/test_nucleo.py:462-468): per output and gradient,
  |hip_bf16 - fp32| / n <= 1.5 |reference_bf16 - fp32| / n + 1e-2 with n = max|fp32| + 1e-3, against the bf16
  fixture the reference wrote and against the oracle's own bf16 branch (pinned by that fixture) on a larger input.
- cfg3 (B 4, N 65,536, d 512, V 32,000, Zipf, bf16): the layer forward and backward is finite, bit-identical run to
  run and causal; the candidate stage at that shape is checked query by query against the oracle's per-query
  restatement on 2,048 sampled queries, forward and backward (the upstream gradient is nonzero only at those
  queries, so every gradient, key side included, comes from them alone).
- configs[4]'s decode (B 16, d 768, a 32,768-token prompt): rings bit-exact after the prompt and after every insert,
  and each of 64 steps' candidate attention, Hawkes intensities and streak against the oracle.
Each test prints its case first."""
import copy
import math

import numpy as np
import pytest
import torch

import asrn_amd
from asrn_amd import ops, synth
from asrn_amd.capa import CapaASRNEstable
from asrn_amd.escritura import EscritorCapa
from oracle import generation as G
from oracle import layer as O
from tests import fixtures

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def say(*a):
    print('[case]', *a, flush=True)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    asrn_amd.cargar_biblioteca()


def leaves_of(layer_cpu):
    return {k: (v.detach().clone().requires_grad_() if v.is_floating_point() and k not in ('c_vistos', 'r_firma')
                else v.detach().clone()) for k, v in layer_cpu.state_dict().items()}


def run_hip(layer, E, h, x, gy, bf16=False):
    layer.zero_grad()
    Ed, hd = E.to(DEV).requires_grad_(), h.to(DEV).requires_grad_()
    with torch.autocast('cuda', dtype=torch.bfloat16, enabled=bf16):
        y = layer(Ed, hd, None if x is None else x.to(DEV))
    (y.float() * gy.to(DEV)).sum().backward()
    grads = {'E': Ed.grad.cpu(), 'h': hd.grad.cpu()}
    grads.update({n: q.grad.cpu() for n, q in layer.named_parameters() if q.grad is not None})
    return y.detach().float().cpu(), grads


def run_oracle(p, E, h, x, gy, sh, prot=O.Prot(), bf16=False):
    p = {k: (v.detach().clone().requires_grad_() if v.requires_grad else v) for k, v in p.items()}
    Ec, hc = E.clone().requires_grad_(), h.clone().requires_grad_()
    with torch.autocast('cpu', dtype=torch.bfloat16, enabled=bf16):
        y = O.layer_forward(p, Ec, hc, x, sh, prot)
    (y.float() * gy).sum().backward()
    grads = {'E': Ec.grad, 'h': hc.grad}
    grads.update({k: v.grad for k, v in p.items() if getattr(v, 'grad', None) is not None})
    return y.detach().float(), grads


# ---------------------------------------------------------------------------------------------------------------------
# cfg2 at full size
# ---------------------------------------------------------------------------------------------------------------------

def test_layer_cfg2_full_size_vs_oracle():
    cfg = synth.CONFIGS['cfg2']
    B, N, d, V = cfg['B'], cfg['N'], cfg['d'], cfg['V']
    say('layer cfg2 full size vs oracle', B, N, d, V)
    torch.manual_seed(0)
    layer_cpu = synth.move_params(CapaASRNEstable(d), seed=0)
    x, E, h = synth.layer_inputs(B, N, d, V, seed=0, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'])
    gy = torch.randn(B, N, d, generator=torch.Generator().manual_seed(1))
    p = leaves_of(layer_cpu)
    sh = O.shape_from_params(p, d)
    layer = copy.deepcopy(layer_cpu).to(DEV)
    with torch.no_grad():
        phi_hip, _ = layer._phi_y_valores(E.to(DEV))
        phi_ref, _ = O.phi_and_values({k: v.detach() for k, v in p.items()}, E)
    flips = (O.bucket_ids(phi_hip.cpu(), sh.T, sh.nb) != O.bucket_ids(phi_ref, sh.T, sh.nb)).sum().item()
    y, gg = run_hip(layer, E, h, x, gy)
    yo, go = run_oracle(p, E, h, x, gy, sh)
    dif = (y - yo).abs().amax(-1)
    same = (dif < 1e-3).float().mean().item()
    names = [k for k in go if k not in ('E', 'h')]
    gc = torch.cat([go[k].flatten() for k in names])
    gh = torch.cat([gg[k].flatten() for k in names])
    rel = ((gh - gc).norm() / gc.norm()).item()
    rel_E = ((gg['E'] - go['E']).norm() / go['E'].norm()).item()
    rel_h = ((gg['h'] - go['h']).norm() / go['h'].norm()).item()
    print(f'cfg2: bucket-id flips {flips} of {B * N * sh.T}; positions within 1e-3: {100 * same:.3f}% '
          f'(max dif {dif.max():.2e}); parameter gradients rel. norm {rel:.2e}; dE {rel_E:.2e}; dh {rel_h:.2e}',
          flush=True)
    assert same >= 0.99
    assert rel < 1e-3 and rel_E < 1e-3 and rel_h < 1e-3


# ---------------------------------------------------------------------------------------------------------------------
# bf16 under autocast: the reference's rule
# ---------------------------------------------------------------------------------------------------------------------

def bf16_rule(hip, ref16, truth, what):
    """tests/test_nucleo.py:462-468: the 16-bit result is no farther from fp32 than the reference's 16-bit one."""
    n = truth.abs().max().item() + 1e-3
    e_hip = (hip.double() - truth.double()).abs().max().item() / n
    e_ref = (ref16.double() - truth.double()).abs().max().item() / n
    print(f'  {what}: hip {e_hip:.3e}  reference bf16 {e_ref:.3e}  bound {1.5 * e_ref + 1e-2:.3e}', flush=True)
    assert e_hip <= 1.5 * e_ref + 1e-2, f'{what}: {e_hip:.3e} > 1.5 * {e_ref:.3e} + 1e-2'


@pytest.mark.parametrize('name', fixtures.names('bf16'))
def test_layer_bf16_golden_rule(name):
    say('layer bf16 vs the reference bf16 fixture', name)
    g, p, m = fixtures.load(name)
    layer = CapaASRNEstable(m['d'], protecciones=fixtures.protecciones(m), **m['kw'])
    layer.load_state_dict(p)
    layer = layer.to(DEV)
    y, grads = run_hip(layer, g['E'], g['h'], g['x'], g['gy'], bf16=True)
    assert torch.isfinite(y).all()
    bf16_rule(y, g['y'], g['y32'], 'y')
    bf16_rule(grads['E'], g['gE'], g['gE32'], 'grad E')
    bf16_rule(grads['h'], g['gh'], g['gh32'], 'grad h')
    for k, v in grads.items():
        if ('g32.' + k) in g:
            bf16_rule(v, g['g.' + k], g['g32.' + k], 'grad ' + k)


@pytest.mark.parametrize('B,L,d,V', [(2, 2048, 64, 300), (2, 1500, 256, 1000)])
def test_layer_bf16_vs_oracle_rule(B, L, d, V):
    """A larger bf16 case with Zipf tokens and long copies: the oracle's fp32 layer is the truth and its bf16 branch
    (the reference's autocast code path, pinned by the bf16 fixture) the 16-bit reference."""
    say('layer bf16 vs oracle', B, L, d, V)
    torch.manual_seed(3)
    layer_cpu = synth.move_params(CapaASRNEstable(d), 3)
    x, E, h = synth.layer_inputs(B, L, d, V, seed=8, frac=0.2, span=(16, 64), zipf=1.1)
    gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(9))
    p = leaves_of(layer_cpu)
    sh = O.shape_from_params(p, d)
    y, gg = run_hip(copy.deepcopy(layer_cpu).to(DEV), E, h, x, gy, bf16=True)
    y32, g32 = run_oracle(p, E, h, x, gy, sh)
    y16, g16 = run_oracle(p, E, h, x, gy, sh, bf16=True)
    assert torch.isfinite(y).all()
    bf16_rule(y, y16, y32, 'y')
    for k in g32:
        bf16_rule(gg[k], g16[k], g32[k], 'grad ' + k)


# ---------------------------------------------------------------------------------------------------------------------
# cfg3 at full size
# ---------------------------------------------------------------------------------------------------------------------

def test_layer_cfg3_full_size_deterministic_causal():
    cfg = synth.CONFIGS['cfg3']
    B, N, d, V = cfg['B'], cfg['N'], cfg['d'], cfg['V']
    say('layer cfg3 full size, bf16: finite, deterministic, causal', B, N, d, V)
    torch.manual_seed(0)
    layer = synth.move_params(CapaASRNEstable(d), seed=0).to(DEV)
    x, E, h = synth.layer_inputs(B, N, d, V, seed=0, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'])
    gy = torch.randn(B, N, d, generator=torch.Generator().manual_seed(1))
    y1, g1 = run_hip(layer, E, h, x, gy, bf16=True)
    print('  first pass done', flush=True)
    assert torch.isfinite(y1).all()
    for k, v in g1.items():
        assert torch.isfinite(v).all(), k
    y2, g2 = run_hip(layer, E, h, x, gy, bf16=True)
    assert torch.equal(y1, y2)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
    cut = 40000
    x2, E2, h2 = x.clone(), E.clone(), h.clone()
    gen = torch.Generator().manual_seed(5)
    x2[:, cut:] = torch.randint(0, V, (B, N - cut), generator=gen)
    E2[:, cut:] = torch.randn(B, N - cut, d, generator=gen)
    h2[:, cut:] = torch.randn(B, N - cut, d, generator=gen)
    with torch.no_grad(), torch.autocast('cuda', dtype=torch.bfloat16):
        ya = layer(E.to(DEV), h.to(DEV), x.to(DEV))[:, :cut].float()
        yb = layer(E2.to(DEV), h2.to(DEV), x2.to(DEV))[:, :cut].float()
    assert (ya - yb).abs().max().item() <= 1e-6 * ya.abs().max().item()


def test_candidates_cfg3_shape_sampled_vs_oracle():
    cfg = synth.CONFIGS['cfg3']
    B, N, d, V = cfg['B'], cfg['N'], cfg['d'], cfg['V']
    T, nb, C, cf, K = 8, 14, 32, 16, 4
    say('candidates at cfg3 shape, 2048 sampled queries vs oracle', B, N, d)
    sh = O.Shape(d=d, T=T, nb=nb, C=C, Tc=4, cf=cf, K=K)
    gen = torch.Generator().manual_seed(0)
    x = synth.tokens(B, N, V, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'], seed=0)
    # phi from the tokens (the word half from the token, the context half from it and the one before), so buckets
    # fill as the layer's do
    emb = torch.randn(V, sh.P, generator=gen)
    prev = torch.cat([x[:, :1], x[:, :-1]], 1)
    half = sh.P // 2
    phi = torch.cat([emb[x][..., :half], emb[x][..., half:] + 0.7 * emb[prev][..., half:]], -1).contiguous()
    st = dict(phi=phi, V=torch.randn(B, N, d, generator=gen), Qc=torch.randn(B, N, cf, generator=gen),
              Kc=torch.randn(B, N, cf, generator=gen),
              Bt=(torch.rand(B, N, generator=gen, dtype=torch.float64) * 2).cumsum(1),
              log_alfa=torch.randn(B, N, generator=gen) * 0.3)
    w_suf = torch.randn(K + 1, generator=gen) * 0.5
    gamma = torch.rand(T, generator=gen) * 2
    sig = x.float()
    q = torch.stack([torch.randint(0, B, (2048,), generator=gen), torch.randint(0, N, (2048,), generator=gen)], 1)
    q = torch.unique(q, dim=0)
    gs = torch.zeros(B, N, d)
    gq = torch.randn(len(q), d, generator=gen)
    gs[q[:, 0], q[:, 1]] = gq

    lv = {k: v.to(DEV).requires_grad_() for k, v in st.items()}
    w, gam = w_suf.to(DEV).requires_grad_(), gamma.to(DEV).requires_grad_()
    ids_rows, order, _, rank, win = ops.bucket_sort(lv['phi'].detach(), T, nb, C)
    sal, sen = ops.Candidates.apply(lv['phi'], lv['V'], lv['Qc'], lv['Kc'], lv['Bt'], lv['log_alfa'], w, gam,
                                    sig.to(DEV), order, win, rank, dict(T=T, Tc=4, C=C, K=K))
    (sal * gs.to(DEV)).sum().backward()
    ids = ids_rows.view(B, T, N).transpose(1, 2).cpu()
    assert torch.equal(ids, O.bucket_ids(phi, T, nb))                           # the GPU's ids are the sign hash
    print('  GPU stage done', flush=True)

    ol = {k: v.clone().requires_grad_() for k, v in st.items()}
    wo, go_ = w_suf.clone().requires_grad_(), gamma.clone().requires_grad_()
    ref, ref_sen = O.candidates_at(ol['phi'], ol['V'], ol['Qc'], ol['Kc'], ol['Bt'], ol['log_alfa'], sig, wo, go_,
                                   sh, ids.numpy(), q)
    (ref * gq).sum().backward()

    def close(a, b, what, tol=1e-3):
        a, b = a.detach().double().cpu(), b.detach().double()
        e = (a - b).abs().max().item() / (b.abs().max().item() + 1e-12)
        assert e <= tol, f'{what}: relative error {e:.3g}'

    close(sal.detach()[q[:, 0], q[:, 1]], ref, 'salida')
    got = sen.cpu()[q[:, 0], q[:, 1]]
    hay = ref_sen[..., 0]
    assert torch.equal(got[:, 0], hay.sum(1))
    assert torch.equal(got[:, 3], hay[:, T - 4:].sum(1))
    mejor = torch.where(hay > 0, ref_sen[..., 1], torch.full_like(hay, O.PROHIBIDO)).amax(1)
    close(got[:, 1], mejor, 'mejor')
    close(got[:, 2], (ref_sen[..., 2] * hay).sum(1), 'pico')
    ncand = int(hay.sum().item())
    print(f'  {len(q)} queries, {ncand} (query, table) pairs with candidates', flush=True)
    for k in st:
        close(lv[k].grad, ol[k].grad, 'grad ' + k)
    close(w.grad, wo.grad, 'grad w_sufijo')
    close(gam.grad, go_.grad, 'grad gamma')


# ---------------------------------------------------------------------------------------------------------------------
# configs[4]'s decode at scale
# ---------------------------------------------------------------------------------------------------------------------

def test_decode_cfg5_scale_vs_oracle():
    B, d, V, L0, steps = 16, 768, 50304, 32768, 64
    say('decode at configs[4] scale vs oracle', B, d, L0, steps)
    torch.manual_seed(0)
    layer = synth.move_params(CapaASRNEstable(d), seed=0).to(DEV)
    T, nb, C, n = layer.n_tablas, layer.n_bits, layer.chunk, layer.vistos
    sh = O.Shape(d=d, T=T, nb=nb, C=C)
    x = synth.tokens(B, L0 + steps, V, frac=0.2, span=(16, 256), zipf=1.1, seed=0)
    g = torch.Generator(device=DEV).manual_seed(7)
    emb = torch.randn(V, d, generator=g, device=DEV)
    xd = x.to(DEV)
    E = emb[xd]
    h = torch.randn(B, L0 + steps, d, generator=g, device=DEV)
    esc = EscritorCapa(layer, memoria_de_lo_ajeno=False)
    esc.inicio(E[:, :L0], h[:, :L0], xd[:, :L0], capacidad=L0 + steps + 1)
    torch.cuda.synchronize()
    print('  prompt done', flush=True)
    mirror = {k: v[:, :L0 + steps].cpu() for k, v in esc.cache.items()}
    ids = O.bucket_ids(mirror['phi'][:, :L0], T, nb).numpy()
    ring, count = G.ring_from(ids, L0, C, 2 ** nb)
    got_ring = esc.anillos.cpu().numpy().reshape(B, T, 2 ** nb, C)
    got_count = esc.cuentas.cpu().numpy().reshape(B, T, 2 ** nb).astype(np.int64)
    assert np.array_equal(got_count, count) and np.array_equal(got_ring, ring), 'rings after the prompt'
    print('  rings after the prompt bit-exact', flush=True)
    # the oracle's Hawkes memory from the prompt (its intensities by the oracle's scan over the same clock)
    Bt0 = mirror['Bt'][:, :L0]
    beta0 = torch.cat([Bt0[:, :1], Bt0[:, 1:] - Bt0[:, :-1]], 1)
    p = {k: v.detach().cpu() for k, v in layer.state_dict().items()}
    rep = O.repetition(p, mirror['sig'][:, :L0], beta0, Bt0, mirror['log_alfa'][:, :L0], sh, O.Prot())
    mem = G.HawkesMemory(B, n)
    keys_all = O.ngram_keys(x.float(), p['c_vistos'], n)
    mem.load(keys_all[:, :L0], rep['hawkes'], Bt0, mirror['log_alfa'][:, :L0])
    racha_ref = esc.racha.cpu().clone()
    with torch.no_grad():
        kappa, kappa_r = (t.detach() for t in layer._kappas())
    shape = dict(T=T, Tc=layer.tablas_contexto, C=C, K=layer.sufijo, nb=nb)
    e_prev = E[:, L0 - 1].contiguous()
    for t in range(L0, L0 + steps):
        e_t, h_t = E[:, t].contiguous(), h[:, t].contiguous()
        with torch.no_grad():
            beta_t = ops.decode_produce(layer, esc.cache, e_t, e_prev, h_t, xd[:, t], t)
            v, hk = esc.hawkes.step(esc.cache, t, beta_t, layer.c_vistos, kappa, kappa_r, esc.racha)
            sal, sen, got_ids = ops.decode_attend(esc.cache, t, esc.anillos, esc.cuentas, layer.w_sufijo, layer.gamma,
                                                  shape, insert=True)
        e_prev = e_t
        for k in mirror:
            mirror[k][:, t] = esc.cache[k][:, t].cpu()
        mirror['V'][:, t - 1] = esc.cache['V'][:, t - 1].cpu()
        ids_t = O.bucket_ids(mirror['phi'][:, t:t + 1], T, nb)[:, 0].numpy()
        assert np.array_equal(got_ids.cpu().numpy(), ids_t), t
        ref_sal, ref_sen = G.attend(G.ring_positions(ring, ids_t), t, mirror['phi'], mirror['V'], mirror['Qc'],
                                    mirror['Kc'], mirror['sig'], mirror['Bt'], mirror['log_alfa'],
                                    p['w_sufijo'], p['gamma'], sh)
        e = (sal.cpu().double() - ref_sal.double()).abs().max() / ref_sal.abs().max()
        assert e <= 1e-3, (t, e.item())
        assert torch.equal(sen[:, 0].cpu(), ref_sen[:, 0]) and torch.equal(sen[:, 3].cpu(), ref_sen[:, 3]), t
        Bq = mirror['Bt'][:, t]
        assert torch.equal(Bq, mirror['Bt'][:, t - 1] + beta_t.cpu().double()), t
        v_ref, h_ref = mem.step(keys_all[:, t], Bq, mirror['log_alfa'][:, t], kappa.cpu())
        racha_ref = G.streak_step(v_ref, beta_t.cpu().double(), racha_ref, kappa_r.cpu())
        assert torch.equal(v.cpu(), v_ref), t
        assert (hk.cpu() - h_ref).abs().max() <= 1e-4 * max(1.0, h_ref.abs().max().item()), t
        assert (esc.racha.cpu() - racha_ref).abs().max() <= 1e-4 * max(1.0, racha_ref.abs().max().item()), t
        G.ring_insert(ring, count, ids_t, t)
        rows = esc.anillos.view(B, T, 2 ** nb, C)[torch.arange(B)[:, None], torch.arange(T)[None, :],
                                                  torch.from_numpy(ids_t).long()].cpu().numpy()
        assert np.array_equal(rows, ring[np.arange(B)[:, None], np.arange(T)[None, :], ids_t]), t
    got_ring = esc.anillos.cpu().numpy().reshape(B, T, 2 ** nb, C)
    got_count = esc.cuentas.cpu().numpy().reshape(B, T, 2 ** nb).astype(np.int64)
    assert np.array_equal(got_count, count) and np.array_equal(got_ring, ring), 'rings after the steps'
