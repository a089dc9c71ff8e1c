"""The whole model on the GPU (HIP ASRN layers inside the reference's model) against the reference's own training step.

- configs[0] (create_model(V=256, d=64, n_capas=4, semilla=0), one fp32 step on 8 x 256 tokens) and a mezcla='memoria'
  model: the loss, the gradient norm and every parameter's gradient against what the reference computed on the CPU
  (tests/golden/make_golden_modelo.py), with the reference's GPU-vs-CPU criterion for gradients
  (tests/verificar_gpu.py:221-229): relative norm below 1e-3, plus an absolute floor of 1e-7 times the whole
  gradient's norm for tensors whose gradient is rounding noise at the start (the clock bias's is ~1e-12 there).
- checkpointing ('asrn', 'todo') recomputes the same numbers as no checkpointing.
- PasoGrafado: the step captured once and replayed equals the eager step, replay after replay, with new batches and a
  new learning rate each time (graph nodes that misbehave on replays after the first show up here).
- entrenar() runs, writes a training state that cargar() reads, and resumes a training state the reference wrote.
Each test prints its case first."""
import copy
import json
import os
import tempfile

import pytest
import torch
from safetensors import safe_open

import asrn_amd
from asrn_amd import archivo, synth

pytestmark = pytest.mark.gpu
DEV = 'cuda'
AQUI = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'modelo')
REDUCIDA = dict(n_tablas=2, tablas_contexto=1, n_bits=6, afin_oculto=16, confirmar=4, vistos=2, nodos_racha=4)


def say(*a):
    print('[case]', *a, flush=True)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    asrn_amd.cargar_biblioteca()


def _fixture(nombre):
    with safe_open(os.path.join(AQUI, nombre + '.safetensors'), framework='pt') as f:
        return {k: f.get_tensor(k) for k in f.keys()}, json.loads(f.metadata()['kw'])


def _grads(m, x, y, checkpoint='no'):
    m.checkpoint = checkpoint
    m.zero_grad(set_to_none=True)
    perdida = m.perdida(x.to(DEV), y.to(DEV))
    perdida.backward()
    norma = torch.nn.utils.clip_grad_norm_(m.parameters(), float('inf'))
    return float(perdida.detach()), float(norma), {n: p.grad.detach().cpu() for n, p in m.named_parameters()}


@pytest.mark.parametrize('dtype,V,rows,reduction', [(torch.bfloat16, 50304, 300, 'mean'),
                                                     (torch.float32, 50304, 300, 'mean'),
                                                     (torch.bfloat16, 1001, 257, 'sum'),
                                                     (torch.float32, 6, 5, 'mean'),
                                                     (torch.bfloat16, 7, 33, 'mean')])
def test_cross_entropy_matches_torch(dtype, V, rows, reduction):
    """asrn_cross_entropy_fwd/bwd (the model's loss) against F.cross_entropy(logits.float(), y, ignore_index) as the
    reference computes it: the loss to 2e-6 relative and the gradient (in the logits' dtype, after PyTorch's cast back)
    to one bf16 rounding step or 1e-6 in fp32; ignored targets; odd V (a padded row stride); a row of +-inf and huge
    logits; a NaN row makes the loss NaN."""
    say('cross_entropy', dtype, V, rows, reduction)
    g = torch.Generator().manual_seed(V + rows)
    x = (torch.randn(rows, V, generator=g) * 4).to(dtype).to(DEV)
    x[1, :3] = float('-inf')
    x[2, 0] = 1e4 if dtype == torch.float32 else 3e38
    y = torch.randint(0, V, (rows,), generator=g).to(DEV)
    y[::7] = -100
    y[1] = 4 if V > 4 else V - 1
    a = x.clone().requires_grad_()
    b = x.clone().requires_grad_()
    la = asrn_amd.ops.cross_entropy(a, y, ignore_index=-100, reduction=reduction)
    lb = torch.nn.functional.cross_entropy(b.float(), y, ignore_index=-100, reduction=reduction)
    assert abs(float(la) - float(lb)) <= 2e-6 * abs(float(lb)), (float(la), float(lb))
    la.backward()
    lb.backward()
    assert a.grad.dtype == dtype
    d = (a.grad.float() - b.grad.float()).abs()
    if dtype == torch.bfloat16:
        assert bool((d <= b.grad.float().abs() * 2 ** -7 + 1e-12).all()), float(d.max())
    else:
        assert float(d.max()) <= 1e-6 * float(b.grad.abs().max()), float(d.max())
    xn = x.clone()
    xn[3, 3] = float('nan')                         # row 3 counts (row 0 is ignored, as in PyTorch)
    assert torch.isnan(asrn_amd.ops.cross_entropy(xn, y)).item()


@pytest.mark.parametrize('dtype,B,L,d,k', [(torch.bfloat16, 3, 517, 96, 4), (torch.float32, 2, 300, 64, 4),
                                            (torch.bfloat16, 2, 40, 10, 3), (torch.float32, 1, 5, 8, 7),
                                            (torch.bfloat16, 2, 2048, 768, 4), (torch.bfloat16, 3, 8, 12, 4)])
def test_conv_window_matches_unfold(dtype, B, L, d, k):
    """asrn_conv_window_fwd/bwd (the 'conv' block's convolution columns) against pad + unfold + reshape and the cast to
    the GEMM's dtype: the columns bit-identical, the z gradient to fp32 rounding (the fold sums k terms in another
    order); k = 4 takes the vectorized kernels (4 tokens a thread when L is a multiple of 4: 300, 2048, 8), 3 and 7
    the general ones, and rows shorter than k are covered."""
    say('conv window', dtype, B, L, d, k)
    g = torch.Generator().manual_seed(L + k)
    z = torch.randn(B, L, d, generator=g).to(DEV)
    gc = torch.randn(B, L, d * k, generator=g).to(DEV).to(dtype)
    a = z.clone().requires_grad_()
    b = z.clone().requires_grad_()
    ca = asrn_amd.ops.ventana_causal(a, k, dtype)
    cb = torch.nn.functional.pad(b, (0, 0, k - 1, 0)).unfold(1, k, 1).reshape(B, L, -1).to(dtype)
    assert ca.dtype == dtype and torch.equal(ca, cb)
    (ca.float() * gc.float()).sum().backward()
    (cb.float() * gc.float()).sum().backward()
    assert torch.allclose(a.grad, b.grad, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize('dtype,rows,d,res', [(torch.float32, 1000, 768, True), (torch.bfloat16, 4099, 768, True),
                                              (torch.bfloat16, 33, 64, False), (torch.float32, 7, 1024, True),
                                              (torch.float32, 70, 12, False)])
def test_layer_norm_matches_torch(dtype, rows, d, res):
    """asrn_layer_norm_fwd/bwd (ops.NormaResidual) against torch.nn.LayerNorm in fp32 followed by the cast to the
    product's dtype: the output within one bf16 rounding (fp32: 2e-6), the gradients of x (with the residual path's
    gradient added in the kernel) and of gamma and beta to fp32 rounding; rows that leave partial workgroups (1000,
    4099, 33, 7, 70) and widths of 1 to 4 float4 columns a lane."""
    say('layer norm', dtype, rows, d, res)
    g = torch.Generator().manual_seed(rows + d)
    x = (torch.randn(rows, d, generator=g) * 3 + 1).to(DEV)
    ln = torch.nn.LayerNorm(d).to(DEV)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.2 * torch.randn(d, generator=g))
        ln.bias.copy_(0.2 * torch.randn(d, generator=g))
    gy = torch.randn(rows, d, generator=g).to(DEV).to(dtype)
    gr = torch.randn(rows, d, generator=g).to(DEV)
    a = x.clone().requires_grad_()
    b = x.clone().requires_grad_()
    ya, ra = asrn_amd.ops.norma_residual(ln, a, dtype)
    assert ya.dtype == dtype
    ((ya.float() * gy.float()).sum() + ((ra * gr).sum() if res else 0)).backward()
    wa, ba = ln.weight.grad.clone(), ln.bias.grad.clone()
    ln.weight.grad = ln.bias.grad = None
    yb = ln(b)
    ((yb.to(dtype).float() * gy.float()).sum() + ((b * gr).sum() if res else 0)).backward()
    if dtype == torch.bfloat16:     # one rounding apart at most: the fp32 values differ in the last bits
        assert torch.allclose(ya.float(), yb.to(dtype).float(), rtol=8e-3, atol=1e-2)
    else:
        assert torch.allclose(ya, yb, rtol=2e-6, atol=2e-6)
    assert torch.allclose(a.grad, b.grad, rtol=1e-4, atol=1e-4)
    assert torch.allclose(wa, ln.weight.grad, rtol=1e-4, atol=1e-3)
    assert torch.allclose(ba, ln.bias.grad, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize('nombre', ['paso_cfg0', 'paso_memoria'])
def test_training_step_matches_reference(nombre):
    t, kw = _fixture(nombre)
    say(nombre, kw, tuple(t['x'].shape))
    m = asrn_amd.crear_modelo(**kw).to(DEV).train()
    perdida, norma, g = _grads(m, t['x'], t['y'])
    ref_p, ref_n = float(t['perdida']), float(t['norma'])
    print(f'loss {perdida:.8f} vs {ref_p:.8f}; norm {norma:.6f} vs {ref_n:.6f}', flush=True)
    assert abs(perdida - ref_p) <= 1e-5 * abs(ref_p)
    assert abs(norma - ref_n) <= 1e-4 * ref_n
    peor = (0.0, '')
    for n, gr in g.items():
        ref = t['g.' + n]
        escala = ref.norm().item()
        err = (gr - ref).norm().item()
        if escala == 0:
            assert gr.abs().max().item() <= 1e-7, n
            continue
        peor = max(peor, (err / escala, n))
        assert err <= 1e-3 * escala + 1e-7 * ref_n, f'{n}: relative gradient error {err / escala:.2e}'
    print('worst relative gradient error', peor, flush=True)


@pytest.mark.parametrize('modo', ['asrn', 'todo'])
def test_checkpointing_recomputes_the_same(modo):
    say('checkpoint', modo)
    t, kw = _fixture('paso_cfg0')
    m = asrn_amd.crear_modelo(**kw).to(DEV).train()
    p0, n0, g0 = _grads(m, t['x'], t['y'])
    p1, n1, g1 = _grads(m, t['x'], t['y'], modo)
    assert p0 == p1
    for n in g0:
        assert torch.allclose(g0[n], g1[n], rtol=1e-6, atol=1e-9), n


def _sincronizar(dst_m, dst_o, src_m, src_o):
    """Copies weights and AdamW state in place (the graph keeps pointing at dst's tensors)."""
    with torch.no_grad():
        for a, b in zip(dst_m.parameters(), src_m.parameters()):
            a.copy_(b)
        for a, b in zip(dst_m.parameters(), src_m.parameters()):
            for k, v in src_o.state[b].items():
                dst_o.state[a][k].copy_(v)


def _peor_grad(m1, m2):
    peor = (0.0, '')
    for (n, a), (_, b) in zip(m1.named_parameters(), m2.named_parameters()):
        escala = a.grad.norm().item()
        if escala > 0:
            peor = max(peor, ((a.grad - b.grad).norm().item() / escala, n))
    return peor


@pytest.mark.parametrize('precision', ['fp32', 'bf16'])
def test_graphed_step_equals_eager_step(precision):
    """From the same weights and AdamW state, the replayed step computes the eager step's loss, norm and gradients:
    fp32 to 1e-6, bf16 to 1e-3 relative (the bf16 GEMMs may take other library kernels under capture). Both models
    are brought back to the same state after every step, so a difference cannot accumulate."""
    say('PasoGrafado', precision)
    torch.manual_seed(0)
    kw = dict(V=256, d=64, n_capas=4, semilla=0)
    m1 = asrn_amd.crear_modelo(**kw).to(DEV).train()
    m2 = copy.deepcopy(m1)
    o1 = asrn_amd.crear_optimizador(m1, lr=1e-3, capturable=True)
    o2 = asrn_amd.crear_optimizador(m2, lr=1e-3, capturable=True)
    ansioso = asrn_amd.PasoGrafado(m1, o1, 4, 128, precision=precision, grabar=False)
    grafo = asrn_amd.PasoGrafado(m2, o2, 4, 128, precision=precision, calentar=2)
    tol = 1e-6 if precision == 'fp32' else 1e-3
    w = synth.tokens(4 * 7, 129, 256, seed=3)
    for i in range(7):
        x, y = w[4 * i:4 * i + 4, :-1].to(DEV), w[4 * i:4 * i + 4, 1:].to(DEV)
        lr = asrn_amd.tasa_aprendizaje(i, 1e-3, 7, 2, 1e-4)
        a = [float(v) for v in ansioso(x, y, lr=lr)]
        b = [float(v) for v in grafo(x, y, lr=lr)]
        torch.cuda.synchronize()
        peor = _peor_grad(m1, m2)
        print(i, 'eager', a, 'graph', b, 'worst gradient difference', peor, flush=True)
        assert a[2] == b[2] == 0.0
        assert abs(a[0] - b[0]) <= tol * abs(a[0]) and abs(a[1] - b[1]) <= tol * abs(a[1])
        assert peor[0] <= tol, peor
        _sincronizar(m2, o2, m1, o1)
        # eager work between replays (the graph must not depend on leftovers of it)
        torch.randn(1 << 20, device=DEV).sum().item()
    assert grafo.grafo is not None


@pytest.mark.parametrize('precision', ['fp32', 'bf16'])
def test_graph_replays_from_one_state_are_bit_identical(precision):
    """Two replays from the same weights, AdamW state and batch give the same bits: nothing a replay leaves behind
    (a buffer not cleared, a counter not reset) reaches the next one."""
    say('PasoGrafado replay determinism', precision)
    m = asrn_amd.crear_modelo(V=256, d=64, n_capas=4, semilla=0).to(DEV).train()
    opt = asrn_amd.crear_optimizador(m, lr=1e-3, capturable=True)
    paso = asrn_amd.PasoGrafado(m, opt, 4, 128, precision=precision, calentar=2)
    w = synth.tokens(8, 129, 256, seed=4).to(DEV)
    lotes = [(w[:4, :-1], w[:4, 1:]), (w[4:, :-1], w[4:, 1:])]
    for x, y in lotes * 2:
        paso(x, y, lr=1e-3)                             # 2 eager steps, the capture, replays
    pesos = [p.detach().clone() for p in m.parameters()]
    estado = [{k: v.clone() for k, v in opt.state[p].items()} for p in m.parameters()]
    resultados = []
    for _ in range(2):
        with torch.no_grad():
            for p, q, st in zip(m.parameters(), pesos, estado):
                p.copy_(q)
                for k, v in st.items():
                    opt.state[p][k].copy_(v)
        perdida, norma, _ = paso(*lotes[0], lr=1e-3)
        perdida2, _, _ = paso(*lotes[1], lr=1e-3)
        torch.cuda.synchronize()
        resultados.append((float(perdida), float(norma), float(perdida2),
                           [p.grad.detach().clone() for p in m.parameters()],
                           [p.detach().clone() for p in m.parameters()]))
        torch.randn(1 << 20, device=DEV).sum().item()
    (a0, a1, a2, ga, pa), (b0, b1, b2, gb, pb) = resultados
    print('replays', (a0, a1, a2), (b0, b1, b2), flush=True)
    assert (a0, a1, a2) == (b0, b1, b2)
    assert all(torch.equal(u, v) for u, v in zip(ga, gb))
    assert all(torch.equal(u, v) for u, v in zip(pa, pb))


def test_graphed_step_skips_a_non_finite_step():
    say('PasoGrafado skip')
    m = asrn_amd.crear_modelo(V=64, d=32, n_capas=2, semilla=1, **REDUCIDA).to(DEV).train()
    opt = asrn_amd.crear_optimizador(m, lr=1e-3, capturable=True)
    paso = asrn_amd.PasoGrafado(m, opt, 2, 64, precision='fp32', calentar=1)
    w = synth.tokens(2, 65, 64, seed=1).to(DEV)
    paso(w[:, :-1], w[:, 1:])
    paso(w[:, :-1], w[:, 1:])                     # captured here
    antes = {n: p.detach().clone() for n, p in m.named_parameters()}
    with torch.no_grad():
        m.ln_f.weight[0] = float('nan')
    perdida, norma, salto = paso(w[:, :-1], w[:, 1:])
    torch.cuda.synchronize()
    assert float(salto) == 1.0
    for n, p in m.named_parameters():
        if n != 'ln_f.weight':
            assert torch.equal(p, antes[n]), n


def test_entrenar_writes_and_resumes():
    say('entrenar tiny model')
    r = archivo.leer(os.path.join(AQUI, 'ckpt_entrenar.pt'))
    datos = synth.tokens(1, 4000, r['config']['V'], seed=3)[0]
    lineas = []
    with tempfile.TemporaryDirectory() as tmp:
        ruta = os.path.join(tmp, 'e.pt')
        m = archivo.modelo_de_config(dict(r['config'])).to(DEV)
        hist = asrn_amd.entrenar(m, datos, validacion=datos[:1000], largo=32, lote=2, pasos=4, lr=1e-3,
                                 precision='bf16', guardar_en=ruta, registrar_cada=1, evaluar_cada=2, lotes_eval=2,
                                 registro=lineas.append, semilla=5)
        assert [h['paso'] for h in hist if 'perdida' in h] == [1, 2, 3, 4]
        assert all(torch.isfinite(torch.tensor(h['perdida'])) for h in hist if 'perdida' in h)
        assert os.path.exists(os.path.join(tmp, 'e.mejor.pt'))
        m2 = asrn_amd.cargar(ruta)
        for (n, a), (_, b) in zip(m.state_dict().items(), m2.state_dict().items()):
            assert torch.equal(a.cpu(), b.cpu()), n
        ev = asrn_amd.evaluar(m2, datos[:1000], largo=32, lote=2, max_lotes=2)
        assert ev['piezas'] == 2 * 2 * 32 and ev['perdida'] > 0
        # resume the reference's own training state (written after 2 fp32 steps) for 2 more
        m3 = archivo.modelo_de_config(dict(r['config'])).to(DEV)
        hist = asrn_amd.entrenar(m3, datos, largo=32, lote=2, pasos=4, lr=1e-3, precision='fp32',
                                 reanudar=os.path.join(AQUI, 'ckpt_entrenar.pt'), registrar_cada=1,
                                 registro=lineas.append, semilla=5)
        assert [h['paso'] for h in hist if 'perdida' in h] == [1, 2, 3, 4]
        assert any('resuming from step 2' in s for s in lineas)


def test_configs3_model_step_bf16():
    """the whole d = 768 LM (V 50,304, 12 local blocks, an ASRN layer after every second one: 6 layers, tied
    head), B 8 x N 2,048, bf16 autocast over fp32 weights, fused AdamW, clipping at 1.0. From the same weights and
    AdamW state, PasoGrafado's replayed step computes its eager step's loss, gradient norm and every parameter's
    gradient to 1e-3 relative (both brought back to the same state after each step); two replays from one state are
    bit-identical; every loss is finite; and the loss falls over 5 steps on one batch."""
    kw = dict(V=50304, d=768, n_capas=12, largo_cada=2, semilla=0)
    B, N = 8, 2048
    say('configs[3] model step, bf16', kw, B, N)
    m1 = asrn_amd.crear_modelo(**kw).to(DEV).train()
    assert len(m1.largos) == 6
    m2 = copy.deepcopy(m1)
    o1 = asrn_amd.crear_optimizador(m1, lr=1e-3, capturable=True)
    o2 = asrn_amd.crear_optimizador(m2, lr=1e-3, capturable=True)
    ansioso = asrn_amd.PasoGrafado(m1, o1, B, N, precision='bf16', grabar=False)
    grafo = asrn_amd.PasoGrafado(m2, o2, B, N, precision='bf16', calentar=2)
    w = synth.tokens(4 * B, N + 1, kw['V'], frac=0.15, span=(8, 128), zipf=1.1, seed=21).to(DEV)
    lotes = [(w[B * i:B * i + B, :-1].contiguous(), w[B * i:B * i + B, 1:].contiguous()) for i in range(4)]
    for i, (x, y) in enumerate(lotes):             # 2 side-stream steps, the capture, a replay
        a = [float(v) for v in ansioso(x, y, lr=1e-3)]
        b = [float(v) for v in grafo(x, y, lr=1e-3)]
        torch.cuda.synchronize()
        peor = _peor_grad(m1, m2)
        print(i, 'eager', a, 'graph', b, 'worst gradient difference', peor, flush=True)
        assert all(torch.isfinite(torch.tensor(a[:2]))) and a[2] == b[2] == 0.0
        assert abs(a[0] - b[0]) <= 1e-3 * abs(a[0]) and abs(a[1] - b[1]) <= 1e-3 * abs(a[1])
        assert peor[0] <= 1e-3, peor
        _sincronizar(m2, o2, m1, o1)
        torch.randn(1 << 20, device=DEV).sum().item()
    assert grafo.grafo is not None
    del ansioso, o1, m1
    torch.cuda.empty_cache()
    # two replays from one state
    pesos = [p.detach().clone() for p in m2.parameters()]
    estado = [{k: v.clone() for k, v in o2.state[p].items()} for p in m2.parameters()]
    res = []
    for _ in range(2):
        with torch.no_grad():
            for p, q, st in zip(m2.parameters(), pesos, estado):
                p.copy_(q)
                for k, v in st.items():
                    o2.state[p][k].copy_(v)
        perdida, norma, _ = grafo(*lotes[0], lr=1e-3)
        torch.cuda.synchronize()
        res.append((float(perdida), float(norma), [p.detach().clone() for p in m2.parameters()]))
    assert res[0][:2] == res[1][:2]
    assert all(torch.equal(u, v) for u, v in zip(res[0][2], res[1][2]))
    del res, pesos, estado
    # the loss falls on one batch
    perdidas = [float(grafo(*lotes[1], lr=1e-3)[0]) for _ in range(5)]
    print('losses on one batch', perdidas, flush=True)
    assert all(torch.isfinite(torch.tensor(perdidas)))
    assert perdidas[-1] < perdidas[0]
