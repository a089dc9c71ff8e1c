"""Generation with the whole model on the GPU: the device sampler against the oracle's restatement of the reference's
per-token choice, the model's O(1) step against the reference's writer (tests/golden/make_golden_modelo.py), and
escribir against the reference's own tests of it (tests/test_nucleo.py:86-140, 632-639, 1237-1257).

- ops.muestrear (asrn_sample): the final probability row equals oracle.muestreo's (penalty, bans with their fallback,
  quote mask, temperature, top-k, top-p, the quote-mass correction) within fp32 rounding, with the same support, both
  where the n-gram contexts' successor lists answer and where a context overflows them and every token is probed,
  with the row in registers (V up to 16,384) and read from memory (larger V);
  the token lies in that support and is written into the text; the n-gram sets take the new n-grams (checked by a
  second step against the oracle on the longer text); draws follow the distribution (chi-square) and repeat for a
  seed.
- EscritorModelo: teacher-forced logits equal the reference's O(1) writer's, with and without memoria_de_lo_ajeno, to
  the reference's tolerance (1e-4); with every position a key they equal the whole-text model.
- escribir: the logits of every step equal the whole-text model on the written text (tests/test_nucleo.py:105-115);
  greedy tokens equal the reference's greedy run; the graphed loop equals the eagerly launched one; conservar_cita
  changes nothing at temperature 1; edge cases and errors as the reference's.
Each test prints its case first."""
import json
import os

import pytest
import torch
from safetensors import safe_open

import asrn_amd
from asrn_amd import ops
from oracle import muestreo as M

pytestmark = pytest.mark.gpu
DEV = 'cuda'
AQUI = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'modelo')
TOL = 1e-4


def say(*a):
    print('[case]', *a, flush=True)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    asrn_amd.cargar_biblioteca()


def _mover(m, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for n, p in m.named_parameters():
            nuevo = n.rsplit('.', 1)[-1] in asrn_amd.archivo.NUEVOS_V87
            p.add_(torch.randn(p.shape, generator=g) * (0.5 if nuevo else 0.05))
        for c in m.largos:
            c.gamma.abs_()
    return m


def _fixture():
    with safe_open(os.path.join(AQUI, 'escritura.safetensors'), framework='pt') as f:
        t = {k: f.get_tensor(k) for k in f.keys()}
        meta = f.metadata()
    kw = json.loads(meta['kw'])
    torch.manual_seed(0)
    m = _mover(asrn_amd.crear_modelo(**kw), 7).to(DEV).eval()
    return t, m, int(meta['L0']), int(meta['n'])


# ---------------------------------------------------------------------------------------------------------------------
# the sampler kernel
# ---------------------------------------------------------------------------------------------------------------------

def _texto(B, L, V, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(0, V, (B, L), generator=g)
    x[:, L // 2:L // 2 + L // 4] = x[:, :L // 4].clone()
    return x


class _Estado:
    def __init__(self, B, V, total):
        self.piezas = torch.zeros(B, dtype=torch.int64, device=DEV)
        self.terminado = torch.zeros(B, dtype=torch.uint8, device=DEV)
        self.paso_fin = torch.full((B,), -1, dtype=torch.int32, device=DEV)
        self.trabajo = torch.empty((B, V), dtype=torch.float32, device=DEV)
        self.bits = torch.empty((B, (V + 31) // 32), dtype=torch.int32, device=DEV)
        self.prob = torch.empty((B, V), dtype=torch.float32, device=DEV)


SAMPLER_CASES = [
    dict(V=300, T=0.8, k=40, p=1.0, pena=1.0, ventana=64, nb=0, nq=0),
    dict(V=300, T=1.0, k=0, p=0.9, pena=1.0, ventana=64, nb=0, nq=0),
    dict(V=300, T=0.7, k=0, p=1.0, pena=1.3, ventana=16, nb=0, nq=0),
    dict(V=300, T=0.9, k=50, p=0.95, pena=1.0, ventana=64, nb=2, nq=0),
    dict(V=40, T=0.6, k=0, p=1.0, pena=1.0, ventana=64, nb=0, nq=4),
    dict(V=40, T=0.5, k=10, p=0.8, pena=1.2, ventana=8, nb=3, nq=4),
    dict(V=2, T=1.0, k=0, p=1.0, pena=1.0, ventana=64, nb=1, nq=0),
    dict(V=50304, T=0.8, k=40, p=0.9, pena=1.1, ventana=64, nb=3, nq=4),
    dict(V=1000, T=1.0, k=1, p=1.0, pena=1.0, ventana=64, nb=0, nq=4),
    dict(V=1000, T=0.8, k=0, p=0.0, pena=1.0, ventana=64, nb=0, nq=0),
    dict(V=10000, T=0.9, k=100, p=0.95, pena=1.2, ventana=32, nb=2, nq=3),
    dict(V=70000, T=0.9, k=100, p=0.95, pena=1.2, ventana=32, nb=2, nq=3),
    # the whole-row branch: V past the register rows with no top-k cut, and more tokens kept at the top-k cut than
    # the LDS candidate list holds (4,096)
    dict(V=50304, T=0.9, k=0, p=0.9, pena=1.1, ventana=64, nb=3, nq=4),
    dict(V=20000, T=1.0, k=5000, p=1.0, pena=1.0, ventana=64, nb=0, nq=0),
    dict(V=30000, T=0.8, k=4500, p=0.7, pena=1.3, ventana=16, nb=2, nq=0),
    # greedy rows past the register sizes: one fused pass over the logits themselves (no penalty, no bans), and over
    # the penalized and banned row
    dict(V=50304, T=1.0, k=1, p=1.0, pena=1.0, ventana=64, nb=0, nq=4),
    dict(V=50304, T=0.7, k=1, p=0.9, pena=1.2, ventana=64, nb=2, nq=3),
    # contexts with more distinct successors than the inline lists hold: the bans and the quote mask probe every token
    dict(V=20, T=0.7, k=0, p=1.0, pena=1.0, ventana=64, nb=1, nq=2),
    dict(V=50, T=1.0, k=5, p=0.9, pena=1.0, ventana=64, nb=1, nq=2),
]


@pytest.mark.parametrize('c', SAMPLER_CASES, ids=lambda c: '-'.join(f'{k}{v}' for k, v in c.items()))
def test_sampler_matches_oracle(c):
    say('sampler', c)
    B, L0, gen = 3, 50, 12
    V = c['V']
    pos = L0 + gen
    x = _texto(B, pos + 2, V, 1 + V)
    if V <= 2:
        x[:, L0:] = torch.arange(x.shape[1] - L0) % 2          # every generated unigram seen: all banned
    texto = x.to(DEV).contiguous()
    g = torch.Generator().manual_seed(V)
    est = _Estado(B, V, pos + 2)
    cita = prohibidas = None
    if c['nq']:
        cita = ops.ConjuntoNgramas(B, c['nq'], V, pos + 2, DEV)
        cita.agregar_texto(texto[:, :pos].contiguous())
    if c['nb']:
        prohibidas = ops.ConjuntoNgramas(B, c['nb'], V, pos + 2, DEV)
        prohibidas.agregar_texto(texto[:, L0:pos].contiguous())
    for paso in range(2):                                      # the second step sees the n-grams the first added
        p_now = pos + paso
        lg = (torch.randn(B, V, generator=g) * 3).to(DEV)
        pdev = torch.tensor([p_now], dtype=torch.int64, device=DEV)
        ops.muestrear(lg, texto, pdev, pos + 1, L0, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits,
                      c['T'], c['k'], c['p'], c['pena'], c['ventana'], 1234 + paso, cita=cita, prohibidas=prohibidas,
                      prob=est.prob)
        torch.cuda.synchronize()
        prob = est.prob.cpu().double()
        texto_cpu = texto.cpu()
        for b in range(B):
            t_b = texto_cpu[b, :p_now].tolist()
            lgr = M.frenar(lg[b].cpu().double(), t_b, L0, c['pena'], c['ventana'], c['nb'])
            q = M.probabilidades(lgr, c['T'], c['k'], c['p'], M.ngramas_siguientes(t_b, c['nq']) if c['nq'] else None)
            assert set(torch.nonzero(prob[b] > 0).view(-1).tolist()) == set(torch.nonzero(q > 0).view(-1).tolist()), b
            assert torch.allclose(prob[b], q, rtol=1e-4, atol=2e-6), (b, (prob[b] - q).abs().max())
            tok = int(est.piezas[b])
            assert q[tok] > 0 and int(texto_cpu[b, p_now]) == tok


@pytest.mark.parametrize('V,nq,nb', [(70000, 4, 2), (50304, 4, 5), (200000, 5, 4)])
def test_sampler_hashed_ngram_keys(V, nq, nb):
    """n-gram sets whose n token ids do not fit 64 bits (n * bits_por_pieza(V) > 64) key them by a 64-bit hash: the
    quote mask and the bans still match the oracle's exact tuple sets, on texts built so that both act (the current
    context repeats a quoted span and closes a banned n-gram of the generated part)."""
    say('sampler hashed keys', V, nq, nb)
    w = ops.bits_por_pieza(V)
    assert nq * w > 64 or nb * w > 64
    B, L0, gen = 2, 40, 30
    pos = L0 + gen
    g = torch.Generator().manual_seed(V + nq)
    x = torch.randint(0, V, (B, pos + 2), generator=g)
    for b in range(B):
        x[b, pos - 8:pos] = x[b, 5:13].clone()                  # the context repeats text 5..12: a quote continues it
        x[b, L0 + 2:L0 + 1 + nb] = x[b, pos - nb + 1:pos].clone()  # the context opens a generated n-gram: a ban
    texto = x.to(DEV).contiguous()
    est = _Estado(B, V, pos + 2)
    cita = ops.ConjuntoNgramas(B, nq, V, pos + 2, DEV)
    cita.agregar_texto(texto[:, :pos].contiguous())
    prohibidas = ops.ConjuntoNgramas(B, nb, V, pos + 2, DEV)
    prohibidas.agregar_texto(texto[:, L0:pos].contiguous())
    lg = (torch.randn(B, V, generator=g) * 3).to(DEV)
    pdev = torch.tensor([pos], dtype=torch.int64, device=DEV)
    ops.muestrear(lg, texto, pdev, pos + 1, L0, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits, 0.9, 0,
                  1.0, 1.0, 64, 77, cita=cita, prohibidas=prohibidas, prob=est.prob)
    torch.cuda.synchronize()
    prob = est.prob.cpu().double()
    texto_cpu = texto.cpu()
    for b in range(B):
        t_b = texto_cpu[b, :pos].tolist()
        lgr = M.frenar(lg[b].cpu().double(), t_b, L0, 1.0, 64, nb)
        sig = M.ngramas_siguientes(t_b, nq)
        assert len(sig) >= 1 and bool(torch.isinf(lgr).any()), 'the text must make both the quote and a ban act'
        q = M.probabilidades(lgr, 0.9, 0, 1.0, sig)
        assert set(torch.nonzero(prob[b] > 0).view(-1).tolist()) == set(torch.nonzero(q > 0).view(-1).tolist()), b
        assert torch.allclose(prob[b], q, rtol=1e-4, atol=2e-6), (b, (prob[b] - q).abs().max())


@pytest.mark.parametrize('caso', ['ties', 'ties_quoted', 'tie_overflow', 'probe'])
def test_sampler_greedy_large_rows(caso):
    """Greedy rows (top_k = 1) of V = 40,000 against the oracle: tied maxima (kept together, so the draw is among
    them), ties of which one continues a quote (the quote-mass correction splits the mass between the two groups),
    six ties held by one thread (more than its four slots: the general count and gather passes), and a quote context
    with more distinct successors than the inline lists hold (the mask probes every token)."""
    say('sampler greedy', caso)
    B, V, L0 = 2, 40000, 30
    pos = 60
    g = torch.Generator().manual_seed(5)
    x = torch.randint(0, V, (B, pos + 2), generator=g)
    nq = 2
    if caso == 'probe':
        for b in range(B):                                      # token 7 followed by 12 distinct tokens, then 7 again
            x[b, 2:26:2] = 7
            x[b, 3:27:2] = torch.arange(100, 112)
            x[b, pos - 1] = 7
    else:
        x[:, pos - 1] = x[:, 10]                                # the context continues the text at 11: a quote
    texto = x.to(DEV).contiguous()
    cita = ops.ConjuntoNgramas(B, nq, V, pos + 2, DEV)
    cita.agregar_texto(texto[:, :pos].contiguous())
    lg = torch.randn(B, V, generator=g) * 3
    top = float(lg.max()) + 1.0
    for b in range(B):
        sig = sorted(M.ngramas_siguientes(x[b, :pos].tolist(), nq))
        if caso == 'ties':
            lg[b, [17, 9000, 39999]] = top
        elif caso == 'ties_quoted':
            lg[b, [sig[0], 123, 31000]] = top
        elif caso == 'tie_overflow':
            lg[b, [300 + 1024 * j for j in range(6)] + [5]] = top
        elif caso == 'probe':
            assert len(sig) > ops.query('asrn_ngram_set_successors')
            lg[b, sig[3]] = top
    lg = lg.to(DEV)
    est = _Estado(B, V, pos + 2)
    pdev = torch.tensor([pos], dtype=torch.int64, device=DEV)
    ops.muestrear(lg, texto, pdev, pos + 1, L0, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits, 1.0, 1,
                  1.0, 1.0, 64, 99, cita=cita, prob=est.prob)
    torch.cuda.synchronize()
    prob = est.prob.cpu().double()
    texto_cpu = texto.cpu()
    for b in range(B):
        t_b = texto_cpu[b, :pos].tolist()
        q = M.probabilidades(lg[b].cpu().double(), 1.0, 1, 1.0, M.ngramas_siguientes(t_b, nq))
        assert set(torch.nonzero(prob[b] > 0).view(-1).tolist()) == set(torch.nonzero(q > 0).view(-1).tolist()), b
        assert torch.allclose(prob[b], q, rtol=1e-4, atol=2e-6), (b, (prob[b] - q).abs().max())
        tok = int(est.piezas[b])
        assert q[tok] > 0 and int(texto_cpu[b, pos]) == tok
        if caso == 'ties_quoted':
            assert 0 < float(q[q > 0].min()) < float(q.max())        # the two groups carry different masses


def _set_contents(s):
    """An n-gram set's contents per row, independent of where colliding keys landed: its keys, and per context its
    successor count and inline successors (as a set: the prompt's build appends them in no fixed order)."""
    slots, ctx, count, succ = (t.cpu() for t in (s.slots, s.ctx, s.count, s.succ))
    out = []
    for r in range(slots.shape[0]):
        keys = sorted(int(k) for k in slots[r] if int(k) != -1)
        ctxs = {}
        for c in torch.nonzero(ctx[r] != -1).view(-1).tolist():
            k = int(count[r, c])
            ctxs[int(ctx[r, c])] = (k, sorted(succ[r, c, :min(k, succ.shape[2])].tolist()))
        out.append((keys, ctxs))
    return out


@pytest.mark.parametrize('caso', ['unique', 'ties', 'nan', 'neg_inf'])
def test_sampler_greedy_prepass(caso):
    """Greedy rows past the register sizes with no penalty, bans, recorded logits or probabilities out go through the
    greedy pre-pass (k_greedy_part, 16 slices a row) and, with one finite maximum, take its token with no pass of
    their own. Over 6 steps each token equals the one the same call makes with probabilities out (the full pass),
    with the maxima placed in every slice, tied maxima (the full pass draws among them), a NaN logit and an all -inf
    row; the quote set, filled by the steps' single-thread inserts, then holds what a set built from the generated
    text holds."""
    say('sampler greedy pre-pass', caso)
    B, V, L0, nq, steps = 4, 50304, 40, 3, 6
    pos0 = 80
    g = torch.Generator().manual_seed(11)
    x = torch.randint(0, 50, (B, pos0 + steps + 1), generator=g)   # a small alphabet: contexts repeat, quotes act
    sets, ests, textos = [], [], []
    for _ in range(2):
        textos.append(x.to(DEV).contiguous())
        s = ops.ConjuntoNgramas(B, nq, V, pos0 + steps + 1, DEV)
        s.agregar_texto(textos[-1][:, :pos0].contiguous())
        sets.append(s)
        ests.append(_Estado(B, V, pos0 + steps + 1))
    per = (V + 15) // 16
    for k in range(steps):
        pos = pos0 + k
        lg = torch.randn(B, V, generator=g) * 3
        for b in range(B):
            if caso == 'unique':                               # the maximum in slice (4 k + b) mod 16, at its ends too
                sl = (4 * k + b) % 16
                lg[b, [sl * per, sl * per + per // 2, min(V - 1, sl * per + per - 1)][b % 3]] = 50.0
            elif caso == 'ties':
                lg[b, [b * 7, V - 1 - k * 13]] = 50.0
            elif caso == 'nan' and b % 2 == 0:
                lg[b, 1000 + k] = float('nan')
            elif caso == 'neg_inf' and b == 1:
                lg[b] = -float('inf')
        lg = lg.to(DEV)
        pdev = torch.tensor([pos], dtype=torch.int64, device=DEV)
        for i in range(2):
            e = ests[i]
            ops.muestrear(lg, textos[i], pdev, pos0 + steps, L0, e.piezas, e.terminado, e.paso_fin, e.trabajo, e.bits,
                          1.0, 1, 1.0, 1.0, 64, 5 + k, cita=sets[i], prob=e.prob if i == 1 else None)
        torch.cuda.synchronize()
        assert torch.equal(ests[0].piezas, ests[1].piezas), (k, ests[0].piezas.tolist(), ests[1].piezas.tolist())
        if caso == 'unique':
            assert torch.equal(ests[0].piezas.cpu(), lg.cpu().argmax(1)), k
    assert torch.equal(textos[0], textos[1])
    whole = ops.ConjuntoNgramas(B, nq, V, pos0 + steps + 1, DEV)
    whole.agregar_texto(textos[0][:, :pos0 + steps].contiguous())
    assert _set_contents(sets[0]) == _set_contents(sets[1]) == _set_contents(whole)


@pytest.mark.parametrize('V,k,p,ntie', [(300, 0, 0.6, 4), (10000, 0, 0.5, 9), (20000, 0, 0.62, 6), (30000, 3000, 0.55, 5),
                                       (3000, 40, 0.8, 7)])
def test_sampler_top_p_ties(V, k, p, ntie):
    """A top-p cut through tied probabilities keeps the tied tokens in token order while the mass before each stays
    below top_p, as the reference's sort-and-cumsum does (a stable sort's order of the ties), not every tie: rows with
    one top token and ntie tied ones after it, on the register rows (V 300, 3,000 and 10,000), the whole-row passes
    (V 20,000, no top-k) and the candidate list (V 30,000, top-k 3,000)."""
    say('sampler top-p ties', V, k, p, ntie)
    B, L0 = 2, 20
    pos = 30
    g = torch.Generator().manual_seed(V + ntie)
    texto = torch.randint(0, V, (B, pos + 2), generator=g).to(DEV).contiguous()
    lg = -8.0 + 0.01 * torch.randn(B, V, generator=g)
    for b in range(B):
        idx = torch.randperm(V, generator=g)[:ntie + 1]
        lg[b, idx[0]] = 2.4                                   # the top token
        lg[b, idx[1:]] = 2.0                                  # the tied group the cut goes through
    lg = lg.to(DEV)
    est = _Estado(B, V, pos + 2)
    pdev = torch.tensor([pos], dtype=torch.int64, device=DEV)
    ops.muestrear(lg, texto, pdev, pos + 1, L0, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits, 1.0, k, p,
                  1.0, 64, 5, prob=est.prob)
    torch.cuda.synchronize()
    prob = est.prob.cpu().double()
    for b in range(B):
        q = M.probabilidades(lg[b].cpu().double(), 1.0, k, p, None)
        tied = torch.nonzero(lg[b].cpu() == 2.0).view(-1)
        assert 0 < int((q[tied] > 0).sum()) < ntie, 'the cut must go through the tied group'
        assert set(torch.nonzero(prob[b] > 0).view(-1).tolist()) == set(torch.nonzero(q > 0).view(-1).tolist()), b
        assert torch.allclose(prob[b], q, rtol=1e-4, atol=2e-6), (b, (prob[b] - q).abs().max())
        tok = int(est.piezas[b])
        assert q[tok] > 0


def test_sampler_distribution_and_seed():
    say('sampler chi-square')
    B, V = 512, 12
    lg0 = torch.linspace(-2, 2, V)
    lg = lg0.expand(B, V).contiguous().to(DEV)
    esperado = torch.softmax(lg0.double() / 0.9, -1)
    texto = torch.zeros((B, 4), dtype=torch.int64, device=DEV)
    est = _Estado(B, V, 4)
    pdev = torch.tensor([1], dtype=torch.int64, device=DEV)
    cuentas = torch.zeros(V, dtype=torch.float64)
    for s in range(20):
        ops.muestrear(lg, texto, pdev, 2, 1, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits, 0.9, 0,
                      1.0, 1.0, 64, s)
        cuentas += torch.bincount(est.piezas.cpu(), minlength=V).double()
    n = cuentas.sum()
    chi2 = float(((cuentas - n * esperado) ** 2 / (n * esperado)).sum())
    print('chi2', chi2, 'draws', int(n), flush=True)
    assert chi2 < 45.0                               # 11 degrees of freedom: p < 1e-5 above 45
    a = est.piezas.clone()
    ops.muestrear(lg, texto, pdev, 2, 1, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits, 0.9, 0, 1.0,
                  1.0, 64, 19)
    assert torch.equal(a, est.piezas)
    ops.muestrear(lg, texto, pdev, 2, 1, est.piezas, est.terminado, est.paso_fin, est.trabajo, est.bits, 0.9, 0, 1.0,
                  1.0, 64, 20)
    assert not torch.equal(a, est.piezas)


# ---------------------------------------------------------------------------------------------------------------------
# the model's step and escribir
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('ajeno', [True, False])
def test_model_writer_matches_reference_writer(ajeno):
    say('EscritorModelo teacher-forced, ajeno', ajeno)
    t, m, L0, n = _fixture()
    x = t['x'].to(DEV)
    esc = asrn_amd.EscritorModelo(m, memoria_de_lo_ajeno=ajeno)
    with torch.no_grad():
        lgs = [esc.inicio(x[:, :L0], capacidad=L0 + 3)] + [esc.paso(x[:, k]) for k in range(L0, L0 + n - 1)]
    got = torch.stack(lgs, 1).cpu()
    ref = t['paso_ajeno' if ajeno else 'paso_todo']
    err = (got - ref).abs().max().item()
    print('max |hip - reference writer|', err, flush=True)
    assert err < TOL
    if not ajeno:
        assert (got - t['entero']).abs().max().item() < TOL


@pytest.mark.parametrize('B,d,k,ff,L', [(16, 768, 4, 1536, 9), (20, 96, 3, 40, 5), (3, 64, 1, 128, 4),
                                          (2, 32, 4, 64, 2), (4, 1100, 12, 300, 14), (3, 2080, 2, 72, 3)])
def test_block_step_equals_whole_text_block(B, d, k, ff, L):
    """asrn_block_step against BloqueLocal.forward at the last position of a short text: the ring built from the
    earlier positions' LayerNorm rows (slot t mod (k - 1)), then the step at position L - 1; 20 rows span two row
    tiles, k = 1 has no ring, L < k starts with zeros; d = 1,100 and 2,080 hold 2 and 3 columns a thread in the row
    kernels, k = 12 has taps past the 8 loaded ahead, and ff1's depth of 1,100 takes two rounds of loads."""
    say('block step', B, d, k, ff, L)
    torch.manual_seed(B + d)
    blq = asrn_amd.BloqueLocal(d, k, ff).to(DEV)
    with torch.no_grad():
        for p in blq.parameters():
            p.add_(torch.randn_like(p) * 0.1)
        h = torch.randn(B, L, d, device=DEV)
        todo = blq(h)[:, -1]
        anillo = None
        if k > 1:
            z = blq.ln1(h[:, :-1])
            ventana = torch.nn.functional.pad(z, (0, 0, k - 1, 0))[:, z.shape[1]:].transpose(1, 2).contiguous()
            anillo = torch.empty_like(ventana)
            anillo[:, :, (L - 1 + torch.arange(k - 1, device=DEV)) % (k - 1)] = ventana
        pos = torch.tensor([L - 1], dtype=torch.int64, device=DEV)
        espacio = ops.espacio_bloque(B, d, ff, DEV)
        anillo0 = anillo.clone() if anillo is not None else None
        out = ops.paso_bloque(blq, h[:, -1], anillo, pos, espacio)
        out2 = ops.paso_bloque(blq, h[:, -1], anillo0, pos, espacio)
        assert torch.equal(out, out2)                           # deterministic, the workspace reused
        err = ((out - todo).abs().max() / todo.abs().max()).item()
        print('max relative difference', err, flush=True)
        assert err < 1e-5
        if k > 1:                                               # the ring took LayerNorm1 of position L - 1
            assert torch.allclose(anillo[:, :, (L - 1) % (k - 1)], blq.ln1(h[:, -1]), atol=1e-5)


@pytest.mark.parametrize('B,d,ks,ffs', [(16, 768, (4, 4, 4), (1536, 1536, 1536)), (20, 96, (4, 1, 3), (40, 200, 64)),
                                         (3, 2080, (2, 12, 1), (72, 300, 48))])
def test_block_step_chained_equals_separate(B, d, ks, ffs):
    """Three blocks in a row with each one's last launch done by the next one's first (asrn_block_step_ex: finish = 0,
    then the pending block taken as the input) against three asrn_block_step calls, bit for bit: every block's output
    and ring. The blocks differ in k (k = 1: no ring) and in the feed-forward width (the pending partials sit where
    the previous call's width put them)."""
    say('block step chained', B, d, ks, ffs)
    torch.manual_seed(B + d)
    blqs = []
    with torch.no_grad():
        for k, ff in zip(ks, ffs):
            blq = asrn_amd.BloqueLocal(d, k, ff).to(DEV)
            for p in blq.parameters():
                p.add_(torch.randn_like(p) * 0.1)
            blqs.append(blq)
        h = torch.randn(B, d, device=DEV)
        anillos = [torch.randn(B, d, k - 1, device=DEV) if k > 1 else None for k in ks]
        anillos2 = [a.clone() if a is not None else None for a in anillos]
        pos = torch.tensor([7], dtype=torch.int64, device=DEV)
        espacio = ops.espacio_bloque(B, d, max(ffs), DEV)
        x, outs = h, []
        for blq, a in zip(blqs, anillos):
            x = ops.paso_bloque(blq, x, a, pos, espacio)
            outs.append(x)
        pend, outs2 = None, []
        for i, (blq, a) in enumerate(zip(blqs, anillos2)):
            r = ops.paso_bloque(blq, h if i == 0 else None, a, pos, espacio, previo=pend, terminar=i == len(blqs) - 1)
            if pend is not None:
                outs2.append(pend.out)
            pend = r if i < len(blqs) - 1 else None
        outs2.append(r)
        torch.cuda.synchronize()
        for i in range(len(blqs)):
            assert torch.equal(outs[i], outs2[i]), i
            assert (anillos[i] is None) or torch.equal(anillos[i], anillos2[i]), i


@pytest.mark.parametrize('B,d,k,ff,avanzar', [(16, 768, 4, 1536, True), (3, 2080, 1, 300, False),
                                               (5, 96, 3, 4096, True)])
def test_block_finish_norm_equals_block_then_layer_norm(B, d, k, ff, avanzar):
    """A block step left pending, then finished with the final LayerNorm in one launch (asrn_block_finish_norm), against
    the finished block step then torch's LayerNorm: the block's output and ring bit for bit, the norm within 2e-6 of
    torch's (a two-pass biased variance against torch's own reduction order). Widths past 1,024 hold several columns
    a thread; the feed-forward widths give 6, 2 and 16 depth splits; k = 1 has no ring. avanzar: the same launch
    advances the position by one (the last workgroup past its use of it), the ring row still at the old one's slot."""
    say('block finish norm', B, d, k, ff, avanzar)
    torch.manual_seed(B + d + k)
    with torch.no_grad():
        blq = asrn_amd.BloqueLocal(d, k, ff).to(DEV)
        for p in blq.parameters():
            p.add_(torch.randn_like(p) * 0.1)
        ln = torch.nn.LayerNorm(d).to(DEV)
        ln.weight.add_(torch.randn_like(ln.weight) * 0.3)
        ln.bias.add_(torch.randn_like(ln.bias) * 0.3)
        h = torch.randn(B, d, device=DEV)
        anillo = torch.randn(B, d, k - 1, device=DEV) if k > 1 else None
        anillo2 = anillo.clone() if k > 1 else None
        pos = torch.tensor([11], dtype=torch.int64, device=DEV)
        espacio = ops.espacio_bloque(B, d, ff, DEV)
        assert ops.norma_pendiente_ok(ln, d, DEV)
        out = ops.paso_bloque(blq, h, anillo, pos, espacio)
        y_ref = ln(out)
        pend = ops.paso_bloque(blq, h, anillo2, pos, espacio, terminar=False)
        cuenta = torch.zeros(1, dtype=torch.int32, device=DEV)
        y = ops.norma_pendiente(ln, pend, avance=(pos, cuenta) if avanzar else None)
        torch.cuda.synchronize()
    assert pos.item() == (12 if avanzar else 11) and cuenta.item() == 0
    assert torch.equal(out, pend.out)
    assert k == 1 or torch.equal(anillo, anillo2)
    err = ((y - y_ref).abs() / (1 + y_ref.abs())).max().item()
    print('max rel |finish_norm - layer_norm|', err, flush=True)
    assert err < 2e-6


@pytest.mark.parametrize('mezcla', ['conv', 'memoria'])
def test_escribir_equals_whole_text(mezcla):
    """tests/test_nucleo.py:105-115: the logits of every step equal the model on the whole written text."""
    say('escribir vs whole text', mezcla)
    torch.manual_seed(1)
    kw = dict(mezcla=mezcla, memoria_max=64) if mezcla == 'memoria' else {}
    m = _mover(asrn_amd.crear_modelo(60, d=32, n_capas=3, largo_cada=1, semilla=1, chunk=8, n_bits=3, **kw), 3)
    m = m.to(DEV).eval()
    x0 = _texto(2, 40, 60, 0).to(DEV)
    for grafo in (True, False):
        sec, pasos = asrn_amd.escribir(m, x0, n_nuevos=60, memoria_de_lo_ajeno=False, top_k=0, grafo=grafo)
        with torch.no_grad():
            entero = m(sec[:, :-1].to(DEV))[:, 40 - 1:].cpu()
        err = (entero - pasos).abs().max().item()
        print('grafo', grafo, 'max |step - whole text|', err, flush=True)
        assert sec.shape == (2, 100) and pasos.shape == (2, 60, 60)
        assert err < TOL


def test_greedy_tokens_match_reference():
    say('greedy vs reference')
    t, m, L0, n = _fixture()
    sec, pasos = asrn_amd.escribir(m, t['x'][:, :L0], n_nuevos=n, top_k=1, semilla=0)
    print(sec[:, L0:].tolist(), flush=True)
    assert torch.equal(sec, t['greedy'])
    assert (pasos - t['greedy_logits']).abs().max().item() < TOL


def test_graph_loop_equals_eager_loop():
    say('escribir graph vs eager, every option on')
    t, m, L0, n = _fixture()
    kw = dict(n_nuevos=48, temperatura=0.8, top_k=20, top_p=0.9, semilla=3, pena_repeticion=1.2, ventana_pena=16,
              no_repetir_ngramas=3, conservar_cita=True)
    a, la = asrn_amd.escribir(m, t['x'][:, :L0], grafo=True, **kw)
    b, lb = asrn_amd.escribir(m, t['x'][:, :L0], grafo=False, **kw)
    assert torch.equal(a, b) and torch.equal(la, lb)
    # no 3-gram of the generated part repeats
    for fila in a[:, L0:].tolist():
        grupos = [tuple(fila[i:i + 3]) for i in range(len(fila) - 2)]
        assert len(grupos) == len(set(grupos))


def test_quote_correction_changes_nothing_at_temperature_one():
    """tests/test_nucleo.py:632-639."""
    say('conservar_cita at T=1')
    t, m, L0, n = _fixture()
    a, _ = asrn_amd.escribir(m, t['x'][:, :L0], n_nuevos=30, temperatura=1.0, top_k=0, semilla=5, conservar_cita=True)
    b, _ = asrn_amd.escribir(m, t['x'][:, :L0], n_nuevos=30, temperatura=1.0, top_k=0, semilla=5, conservar_cita=False)
    assert torch.equal(a, b)


def test_stop_token():
    say('parar_en')
    t, m, L0, n = _fixture()
    x0 = t['x'][:, :L0]
    libre, _ = asrn_amd.escribir(m, x0, n_nuevos=40, temperatura=1.5, top_k=0, semilla=2)
    parar = int(libre[0, L0 + 3])                      # a token the first row writes early
    sec, pasos = asrn_amd.escribir(m, x0, n_nuevos=40, temperatura=1.5, top_k=0, semilla=2, parar_en=parar)
    gen = sec[:, L0:]
    primeros = []
    for fila in gen.tolist():
        i = fila.index(parar) if parar in fila else None
        primeros.append(i)
        if i is not None:
            assert all(v == parar for v in fila[i:])
    assert primeros[0] is not None and primeros[0] <= 3
    if all(i is not None for i in primeros):
        assert gen.shape[1] == max(primeros) + 1 and pasos.shape[1] == gen.shape[1]
    else:
        assert gen.shape[1] == 40


def test_escribir_edge_cases():
    """tests/test_nucleo.py:86-103, 1237-1257."""
    say('escribir edge cases')
    m = asrn_amd.crear_modelo(2, d=16, n_capas=2, semilla=0).to(DEV)
    m.train()
    s, _ = asrn_amd.escribir(m, torch.tensor([[1]]), n_nuevos=12, no_repetir_ngramas=1)
    assert s.shape == (1, 13) and m.training
    s, _ = asrn_amd.escribir(m, torch.tensor([[1, 0]]), n_nuevos=4, top_p=0.0)
    assert s.shape == (1, 6)
    s, lg = asrn_amd.escribir(m, torch.tensor([1, 0, 1]), n_nuevos=0)
    assert s.shape == (1, 3) and lg.shape == (1, 0, 2)
    s, lg = asrn_amd.escribir(m, torch.tensor([[1, 0]]), n_nuevos=3, devolver_logits=False)
    assert s.shape == (1, 5) and lg is None
    with pytest.raises(ValueError, match=r'outside \[0, 2\)'):
        asrn_amd.escribir(m, torch.tensor([[5]]), n_nuevos=2)
    with pytest.raises(AssertionError):
        asrn_amd.escribir(m, torch.zeros(1, 0, dtype=torch.long), n_nuevos=5)
    assert m.training
    m16 = asrn_amd.crear_modelo(30, d=16, n_capas=2, semilla=0).to(DEV).to(torch.bfloat16)
    with pytest.raises(ValueError, match='autocast'):
        asrn_amd.escribir(m16, torch.tensor([[1, 2]]), n_nuevos=2)
