"""The HIP layer at the widths and precisions the benchmark configurations run, against the oracle, one gradient at a
time.

- fp32 whole layer at d = 512, 768 and 1024 (the candidate kernels' forms with 2, 3 and 4 column chunks of 256, the
  gate's and the context kernels' wider forms): the output and every parameter's gradient, each against the oracle on
  its own (relative norm below 1e-3, the reference's GPU-vs-CPU criterion of tests/verificar_gpu.py:221-229 applied
  per tensor), and dE, dh.
- cfg2 (B 8, N 4096, d 256) with the same per-parameter check.
- bf16 under autocast at d = 512 and 768: the reference's acceptance rule for a 16-bit kernel
  (tests/test_nucleo.py:462-468) per output and gradient, every parameter included, against the oracle's bf16 branch
  (pinned by the reference's bf16 fixture) with the oracle's fp32 layer as the truth.
- the candidate stage at cfg3's shape (B 4, N 65,536, d 512) fed bf16 phi, Qc, Kc and value rows (the kernels' form
  that cfg3 runs: every row read as bf16 and widened exactly), checked query by query against the oracle's per-query
  restatement given the same values in fp32.
- widths past 1,024 (the candidate kernels' value phases over column slabs of 1,024; the context producer and the
  gate as PyTorch ops on the GPU): fp32 layers at d = 1,536 and 2,048 against the oracle per parameter, the bf16 rule
  at d = 2,048, the generation step at d = 2,048 against the whole text, and the named size '1b' (d 2,048)
  forward and backward.

A bucket id is the sign of a hash output, so a value within rounding of 0 can land in the other bucket on the GPU and
on the CPU. The bucket-id flips between the HIP phi and the oracle's are counted and printed; when there are any, the
oracle takes the HIP phi's values through a straight-through term (its own phi still carries the gradient), so both
sides sort the same buckets and every gradient can be held to 1e-3 (phi itself is checked against the oracle in
tests/test_gpu_parity.py). Each test prints its case first."""
import copy

import pytest
import torch

import asrn_amd
from asrn_amd import ops, synth
from asrn_amd.capa import CapaASRNEstable
from oracle import layer as O

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
        y = layer(Ed, hd, x.to(DEV))
    (y.float() * gy.to(DEV)).sum().backward()
    grads = {'E': Ed.grad.cpu(), 'h': hd.grad.cpu()}
    grads.update({n: q.grad.cpu() for n, q in layer.named_parameters() if q.grad is not None})
    return y.detach().float().cpu(), grads


def oracle_forward(p, E, h, x, sh, prot=O.Prot(), phi_values=None):
    """oracle.layer.layer_forward with, optionally, phi's values replaced by `phi_values` through a straight-through
    term (the gradient still flows through the oracle's own phi)."""
    sig = O.firmas(x)
    Qc, Kc, beta, log_alfa = O.context(p, h, sh, prot)
    Bt = beta.cumsum(1)
    phi, V = O.phi_and_values(p, E)
    if phi_values is not None:
        phi = phi + (phi_values.to(phi.dtype) - phi).detach()
    salida, sen = O.candidates(phi, V, Qc, Kc, Bt, log_alfa, sig, p['w_sufijo'], p['gamma'], sh)
    acc = O.gate_signals(salida, sen, sh.T, sh.Tc)
    acc.update(O.repetition(p, sig, beta, Bt, log_alfa, sh, prot))
    return O.combine(p, acc, h, sh, prot)


def run_oracle(p, E, h, x, gy, sh, bf16=False, phi_values=None):
    p = {k: (v.detach().clone().requires_grad_() if v.requires_grad else v) for k, v in p.items()}
    Ec, hc = E.clone().requires_grad_(), h.clone().requires_grad_()
    with torch.autocast('cpu', dtype=torch.bfloat16, enabled=bf16):
        y = oracle_forward(p, Ec, hc, x, sh, phi_values=phi_values)
    (y.float() * gy).sum().backward()
    grads = {'E': Ec.grad, 'h': hc.grad}
    grads.update({k: v.grad for k, v in p.items() if getattr(v, 'grad', None) is not None})
    return y.detach().float(), grads


def flips_and_phi(layer, p, E, sh):
    """The HIP phi (fp32, as the layer computes it) and its bucket-id differences from the oracle's phi."""
    with torch.no_grad():
        phi_hip, _ = layer._phi_y_valores(E.to(DEV))
        phi_ref, _ = O.phi_and_values({k: v.detach() for k, v in p.items()}, E)
    phi_hip = phi_hip.float().cpu()
    flips = (O.bucket_ids(phi_hip, sh.T, sh.nb) != O.bucket_ids(phi_ref, sh.T, sh.nb)).sum().item()
    return flips, phi_hip


def check_per_parameter(gg, go, tol=1e-3):
    """Every gradient's relative norm against the oracle's, each on its own; a tensor whose reference gradient is
    exactly 0 must come out (near) 0 too. Returns the worst (error, name)."""
    total = torch.cat([go[k].flatten() for k in go]).norm().item()
    worst = (0.0, '')
    for k, ref in go.items():
        got = gg[k]
        assert got.shape == ref.shape, k
        scale = ref.norm().item()
        err = (got.double() - ref.double()).norm().item()
        print(f'  grad {k:24s} rel {err / max(scale, 1e-30):.2e}  (norm {scale:.3e})', flush=True)
        if scale == 0.0:
            assert got.abs().max().item() <= 1e-7 * max(total, 1.0), k
            continue
        worst = max(worst, (err / scale, k))
        assert err <= tol * scale, f'grad {k}: relative norm {err / scale:.2e} > {tol}'
    return worst


def whole_layer_fp32(B, L, d, V, seed, zipf=None, frac=0.3, span=(8, 64)):
    torch.manual_seed(seed)
    layer_cpu = synth.move_params(CapaASRNEstable(d), seed=seed)
    x, E, h = synth.layer_inputs(B, L, d, V, seed=seed, frac=frac, span=span, zipf=zipf)
    gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(seed + 1))
    p = leaves_of(layer_cpu)
    sh = O.shape_from_params(p, d)
    layer = copy.deepcopy(layer_cpu).to(DEV)
    flips, phi_hip = flips_and_phi(layer, p, E, sh)
    y, gg = run_hip(layer, E, h, x, gy)
    yo, go = run_oracle(p, E, h, x, gy, sh, phi_values=phi_hip if flips else None)
    dif = (y - yo).abs().amax(-1)
    rel_y = ((y - yo).norm() / yo.norm()).item()
    print(f'  bucket-id flips {flips} of {B * L * sh.T} (oracle on the HIP phi: {bool(flips)}); '
          f'y max dif {dif.max():.2e}, rel. norm {rel_y:.2e}; positions within 1e-3: '
          f'{100 * (dif < 1e-3).float().mean():.3f}%', flush=True)
    assert rel_y < 1e-3 and (dif < 1e-3).float().mean().item() >= 0.999
    worst = check_per_parameter(gg, go)
    print('  worst gradient', worst, flush=True)


@pytest.mark.parametrize('B,L,d,V', [(2, 1024, 512, 1000), (1, 1536, 768, 2000), (1, 1024, 1024, 500)])
def test_layer_fp32_wide_vs_oracle(B, L, d, V):
    say('layer fp32 wide vs oracle, per parameter', B, L, d, V)
    whole_layer_fp32(B, L, d, V, seed=d, zipf=1.1, frac=0.2, span=(16, 128))


def test_layer_cfg2_per_parameter_vs_oracle():
    cfg = synth.CONFIGS['cfg2']
    say('layer cfg2 full size vs oracle, per parameter', cfg['B'], cfg['N'], cfg['d'], cfg['V'])
    whole_layer_fp32(cfg['B'], cfg['N'], cfg['d'], cfg['V'], seed=0, zipf=cfg['zipf'], frac=cfg['frac'],
                     span=cfg['span'])


def bf16_rule(hip, ref16, truth, what):
    """tests/test_nucleo.py:462-468: the 16-bit result is no farther from fp32 than the reference's 16-bit one."""
    n = truth.abs().max().item() + 1e-3
    e_hip = (hip.double() - truth.double()).abs().max().item() / n
    e_ref = (ref16.double() - truth.double()).abs().max().item() / n
    print(f'  {what:24s}: hip {e_hip:.3e}  reference bf16 {e_ref:.3e}  bound {1.5 * e_ref + 1e-2:.3e}', flush=True)
    assert e_hip <= 1.5 * e_ref + 1e-2, f'{what}: {e_hip:.3e} > 1.5 * {e_ref:.3e} + 1e-2'


@pytest.mark.parametrize('B,L,d,V', [(2, 1024, 512, 32000), (1, 1536, 768, 50304)])
def test_layer_bf16_wide_vs_oracle_rule(B, L, d, V):
    """cfg3's width (d = 512) and the configs[3] model's (d = 768) under bf16 autocast: the candidate kernels read bf16
    feature and value rows there (with 2 and 3 column chunks), the gate and the context kernels run their wider forms.
    The oracle's fp32 layer is the truth, its bf16 branch the 16-bit reference."""
    say('layer bf16 wide vs oracle rule', B, L, d, V)
    torch.manual_seed(d)
    layer_cpu = synth.move_params(CapaASRNEstable(d), d)
    x, E, h = synth.layer_inputs(B, L, d, V, seed=d + 5, frac=0.2, span=(16, 128), zipf=1.1)
    gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(d + 6))
    p = leaves_of(layer_cpu)
    sh = O.shape_from_params(p, d)
    y, gg = run_hip(copy.deepcopy(layer_cpu).to(DEV), E, h, x, gy, bf16=True)
    y32, g32 = run_oracle(p, E, h, x, gy, sh)
    y16, g16 = run_oracle(p, E, h, x, gy, sh, bf16=True)
    assert torch.isfinite(y).all()
    bf16_rule(y, y16, y32, 'y')
    for k in g32:
        bf16_rule(gg[k], g16[k], g32[k], 'grad ' + k)


def test_candidates_cfg3_shape_bf16_rows_sampled_vs_oracle():
    """The candidate stage at cfg3's shape with every row in bf16 (phi, Qc, Kc and V: the kernels' rows_bf16 = 2 form,
    the one cfg3's layer runs), against the oracle given the same values widened to fp32, on 2,048 sampled queries:
    salida (bf16, one rounding of the fp32 sum), the gate signals and every gradient, key side included (the upstream
    gradient, bf16, is nonzero only at those queries). Tolerance 2e-2 relative to each tensor's largest value (the bf16
    bound of the task); salida and dV are stored in bf16."""
    cfg = synth.CONFIGS['cfg3']
    B, N, d, V = cfg['B'], cfg['N'], cfg['d'], cfg['V']
    T, nb, C, cf, K = 8, 14, 32, 16, 4
    say('candidates at cfg3 shape, bf16 rows, 2048 sampled queries vs oracle', B, N, d)
    sh = O.Shape(d=d, T=T, nb=nb, C=C, Tc=4, cf=cf, K=K)
    gen = torch.Generator().manual_seed(1)
    x = synth.tokens(B, N, V, frac=cfg['frac'], span=cfg['span'], zipf=cfg['zipf'], seed=1)
    emb = torch.randn(V, sh.P, generator=gen)
    prev = torch.cat([x[:, :1], x[:, :-1]], 1)
    half = sh.P // 2
    phi = torch.cat([emb[x][..., :half], emb[x][..., half:] + 0.7 * emb[prev][..., half:]], -1)
    bf = torch.bfloat16
    st16 = dict(phi=phi.to(bf), V=torch.randn(B, N, d, generator=gen).to(bf),
                Qc=torch.randn(B, N, cf, generator=gen).to(bf), Kc=torch.randn(B, N, cf, generator=gen).to(bf))
    st32 = dict(Bt=(torch.rand(B, N, generator=gen, dtype=torch.float64) * 2).cumsum(1),
                log_alfa=torch.randn(B, N, generator=gen) * 0.3)
    w_suf = torch.randn(K + 1, generator=gen) * 0.5
    gamma = torch.rand(T, generator=gen) * 2
    sig = x.float()
    q = torch.stack([torch.randint(0, B, (2048,), generator=gen), torch.randint(0, N, (2048,), generator=gen)], 1)
    q = torch.unique(q, dim=0)
    gq = torch.randn(len(q), d, generator=gen).to(bf)
    gs = torch.zeros(B, N, d, dtype=bf)
    gs[q[:, 0], q[:, 1]] = gq

    lv = {k: v.to(DEV).requires_grad_() for k, v in list(st16.items()) + list(st32.items())}
    w, gam = w_suf.to(DEV).requires_grad_(), gamma.to(DEV).requires_grad_()
    ids_rows, order, _, rank, win = ops.bucket_sort(lv['phi'].detach().float(), T, nb, C)
    sal, sen = ops.Candidates.apply(lv['phi'], lv['V'], lv['Qc'], lv['Kc'], lv['Bt'], lv['log_alfa'], w, gam,
                                    sig.to(DEV), order, win, rank, dict(T=T, Tc=4, C=C, K=K))
    assert sal.dtype == bf
    (sal * gs.to(DEV)).float().sum().backward()
    ids = ids_rows.view(B, T, N).transpose(1, 2).cpu()
    print('  GPU stage done', flush=True)

    ol = {k: v.float().clone().requires_grad_() for k, v in st16.items()}
    ol.update({k: v.clone().requires_grad_() for k, v in st32.items()})
    wo, go_ = w_suf.clone().requires_grad_(), gamma.clone().requires_grad_()
    ref, ref_sen = O.candidates_at(ol['phi'], ol['V'], ol['Qc'], ol['Kc'], ol['Bt'], ol['log_alfa'], sig, wo, go_,
                                   sh, ids.numpy(), q)
    (ref * gq.float()).sum().backward()

    def close(a, b, what, tol=2e-2):
        a, b = a.detach().double().cpu(), b.detach().double()
        e = (a - b).abs().max().item() / (b.abs().max().item() + 1e-12)
        print(f'  {what:16s} rel {e:.2e}', flush=True)
        assert e <= tol, f'{what}: relative error {e:.3g}'

    close(sal.detach()[q[:, 0], q[:, 1]], ref, 'salida')
    got = sen.cpu()[q[:, 0], q[:, 1]]
    hay = ref_sen[..., 0]
    assert torch.equal(got[:, 0], hay.sum(1))
    assert torch.equal(got[:, 3], hay[:, T - 4:].sum(1))
    mejor = torch.where(hay > 0, ref_sen[..., 1], torch.full_like(hay, O.PROHIBIDO)).amax(1)
    close(got[:, 1], mejor, 'mejor', 1e-3)
    close(got[:, 2], (ref_sen[..., 2] * hay).sum(1), 'pico', 1e-3)
    print(f'  {len(q)} queries, {int(hay.sum().item())} (query, table) pairs with candidates', flush=True)
    for k in lv:
        close(lv[k].grad, ol[k].grad, 'grad ' + k)
    close(w.grad, wo.grad, 'grad w_sufijo')
    close(gam.grad, go_.grad, 'grad gamma')


# ---------------------------------------------------------------------------------------------------------------------
# widths past 1,024: the candidate kernels' value phases over column slabs of 1,024; the context producer and the gate
# as PyTorch ops on the GPU
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('B,L,d,V', [(1, 600, 1536, 300), (1, 512, 2048, 500)])
def test_layer_fp32_past_1024_vs_oracle(B, L, d, V):
    """d = 1,536 (one full slab and a half one) and 2,048 (two slabs): the output and every gradient against the
    oracle, each on its own."""
    say('layer fp32 past 1024 vs oracle, per parameter', B, L, d, V)
    whole_layer_fp32(B, L, d, V, seed=d, zipf=1.1, frac=0.2, span=(16, 64))


def test_layer_bf16_2048_vs_oracle_rule():
    B, L, d, V = 1, 512, 2048, 1000
    say('layer bf16 d 2048 vs oracle rule', B, L, d, V)
    torch.manual_seed(d)
    layer_cpu = synth.move_params(CapaASRNEstable(d), d)
    x, E, h = synth.layer_inputs(B, L, d, V, seed=d + 5, frac=0.2, span=(16, 64), zipf=1.1)
    gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(d + 6))
    p = leaves_of(layer_cpu)
    sh = O.shape_from_params(p, d)
    y, gg = run_hip(copy.deepcopy(layer_cpu).to(DEV), E, h, x, gy, bf16=True)
    y32, g32 = run_oracle(p, E, h, x, gy, sh)
    y16, g16 = run_oracle(p, E, h, x, gy, sh, bf16=True)
    bf16_rule(y, y16, y32, 'y')
    for k in g32:
        bf16_rule(gg[k], g16[k], g32[k], 'grad ' + k)


def test_writer_d2048_equals_whole_text():
    """The generation step at d = 2,048 (the writer's PyTorch producers, the decode attention over two slabs, the
    gate as PyTorch ops) equals the whole-text layer position by position."""
    from asrn_amd.escritura import EscritorCapa
    B, L0, n, d = 2, 200, 40, 2048
    say('writer d 2048 = whole text', B, L0, n, d)
    torch.manual_seed(0)
    layer = synth.move_params(CapaASRNEstable(d), 0).to(DEV)
    x, E, h = synth.layer_inputs(B, L0 + n, d, 12, seed=4, frac=0.4, span=(3, 8))
    Ed, hd, xd = E.to(DEV), h.to(DEV), x.to(DEV)
    esc = EscritorCapa(layer, memoria_de_lo_ajeno=False)
    with torch.no_grad():
        y0 = esc.inicio(Ed[:, :L0], hd[:, :L0], xd[:, :L0], capacidad=L0 + n)
        ys = torch.stack([esc.paso(Ed[:, t], hd[:, t], xd[:, t]) for t in range(L0, L0 + n)], 1)
        y = layer(Ed, hd, xd)
        whole, _ = layer._phi_y_valores(Ed)
        step = torch.stack([layer._phi_y_valores(Ed[:, max(0, t - 1):t + 1])[0][:, -1] for t in range(L0 + n)], 1)
    if not torch.equal(O.bucket_ids(whole.cpu(), 8, 14), O.bucket_ids(step.cpu(), 8, 14)):
        pytest.skip('a bucket id differs between the step GEMM and the whole-text GEMM (sign of phi near 0)')
    e0 = ((y0 - y[:, :L0]).abs().max() / y.abs().max()).item()
    e1 = ((ys - y[:, L0:]).abs().max() / y.abs().max()).item()
    print(f'  prompt {e0:.2e}, steps {e1:.2e}', flush=True)
    assert e0 <= 1e-3 and e1 <= 1e-3


def test_tallas_1b_forward_backward():
    """The named size '1b' (d 2,048, 27 local blocks, 13 ASRN layers, V 32,768; 1.0 B parameters in fp32) runs a
    forward and backward on one GPU: finite loss and gradients, and the loss equals a second forward's bit for bit."""
    say("TALLAS['1b'] forward + backward", 1, 256)
    m = asrn_amd.crear_desde_config('1b', semilla=0).to(DEV).train()
    assert m.largos[0].v.weight.shape[0] == 2048
    x = synth.tokens(1, 257, 32768, frac=0.2, span=(8, 32), zipf=1.1, seed=0).to(DEV)
    perdida = m.perdida(x[:, :-1], x[:, 1:])
    perdida.backward()
    torch.cuda.synchronize()
    print(f'  {m.num_parametros() / 1e9:.3f} B parameters, loss {float(perdida):.5f}', flush=True)
    assert torch.isfinite(perdida)
    for nombre, q in m.named_parameters():
        assert q.grad is not None and torch.isfinite(q.grad).all(), nombre
    with torch.no_grad():
        assert float(m.perdida(x[:, :-1], x[:, 1:])) == float(perdida)
