"""Pins oracle/muestreo.py (the per-token choice of the generation loop) with the reference's own tests of those
functions (tests/test_nucleo.py:590-635, 1237-1248) and with direct definitions."""
import random

import torch

from oracle import muestreo as M


def test_ngram_sets_equal_the_direct_search():
    """_Ngramas.siguientes against the search over every window (tests/test_nucleo.py:603-611)."""
    rng = random.Random(0)
    for n in (1, 2, 3, 4):
        for _ in range(40):
            texto = [rng.randrange(5) for _ in range(rng.randrange(0, 60))]
            assert M.ngramas_siguientes(texto, n) == M.ngramas_siguientes_directo(texto, n)
    assert M.ngramas_siguientes([1, 2, 3], 4) == set()


def test_top_p_cases_of_the_reference():
    """top_p 0.5 keeps only the first of [5, 4, 0, -1, -2]; 0.9 the first two; 0 the most probable
    (tests/test_nucleo.py:596-601, 1243-1244)."""
    lg = torch.tensor([5.0, 4.0, 0.0, -1.0, -2.0], dtype=torch.float64)
    soporte = lambda p: set(torch.nonzero(p > 0).view(-1).tolist())
    assert soporte(M.probabilidades(lg, 1.0, 0, 0.5)) == {0}
    assert soporte(M.probabilidades(lg, 1.0, 0, 0.9)) == {0, 1}
    assert soporte(M.probabilidades(torch.tensor([5.0, 4.0, 0.0], dtype=torch.float64), 1.0, 0, 0.0)) == {0}


def test_top_k_keeps_the_k_largest():
    g = torch.Generator().manual_seed(1)
    lg = torch.randn(200, generator=g, dtype=torch.float64)
    for k in (1, 5, 40, 199):
        p = M.probabilidades(lg, 0.7, k, 1.0)
        assert set(torch.nonzero(p > 0).view(-1).tolist()) == set(lg.topk(k).indices.tolist())
        assert abs(float(p.sum()) - 1) < 1e-12


def test_top_p_keeps_the_shortest_prefix_reaching_the_mass():
    g = torch.Generator().manual_seed(2)
    lg = torch.randn(300, generator=g, dtype=torch.float64) * 2
    for tp in (0.1, 0.5, 0.9, 0.99):
        p = M.probabilidades(lg, 1.0, 0, tp)
        full = torch.softmax(lg, -1)
        orden = full.argsort(descending=True)
        cum = full[orden].cumsum(0)
        m = int((cum < tp).sum()) + 1                      # the first prefix whose mass reaches tp
        assert set(torch.nonzero(p > 0).view(-1).tolist()) == set(orden[:m].tolist())


def test_quote_mass_stays_the_temperature_one_mass():
    """_conservar_cita's properties (tests/test_nucleo.py:614-628)."""
    g = torch.Generator().manual_seed(0)
    for _ in range(4):
        lg = torch.randn(50, generator=g, dtype=torch.float64) * 3
        cita = set(torch.nonzero(torch.rand(50, generator=g) < 0.1).view(-1).tolist()) or {3}
        m = torch.zeros(50, dtype=torch.bool)
        m[list(cita)] = True
        p1 = torch.softmax(lg, -1)
        q = torch.softmax(lg / 0.6, -1)
        r = M.probabilidades(lg, 0.6, 0, 1.0, cita)
        assert abs(float(r[m].sum() - p1[m].sum())) < 1e-12
        assert abs(float(r.sum()) - 1) < 1e-12
        assert torch.allclose(r[m] / r[m].sum(), q[m] / q[m].sum(), atol=1e-12)
        assert torch.allclose(r[~m] / r[~m].sum(), q[~m] / q[~m].sum(), atol=1e-12)
    # a part that top-k left empty: nothing changes
    lg = torch.tensor([5.0, 4.0, 0.0, -1.0], dtype=torch.float64)
    assert torch.equal(M.probabilidades(lg, 0.5, 2, 1.0, {2, 3}), M.probabilidades(lg, 0.5, 2, 1.0))
    # temperature 1, no cuts: the quote correction changes nothing (tests/test_nucleo.py:632-639)
    assert torch.allclose(M.probabilidades(lg, 1.0, 0, 1.0, {1, 2}), torch.softmax(lg, -1), atol=1e-15)


def test_penalty_and_bans():
    lg = torch.tensor([2.0, -1.0, 0.5, 3.0], dtype=torch.float64)
    out = M.frenar(lg, [0, 1, 3, 3], 2, 2.0, 2, 0)           # window: the last two tokens, [3, 3]
    assert out.tolist() == [2.0, -1.0, 0.5, 1.5]
    out = M.frenar(lg, [0, 1, 2, 0, 1], 2, 2.0, 64, 0)
    assert out.tolist() == [1.0, -2.0, 0.25, 3.0]
    # bans over the generated part only: generated [0, 1, 0] -> after 0 came 1: 1 is banned
    out = M.frenar(lg, [3, 3, 0, 1, 0], 2, 1.0, 64, 2)
    assert out[1] == -float('inf') and torch.isfinite(out[[0, 2, 3]]).all()
    # every token banned: the plain logits (tests/test_nucleo.py:1239-1241)
    two = torch.tensor([0.3, -0.2], dtype=torch.float64)
    assert torch.equal(M.frenar(two, [1, 0, 1], 1, 1.0, 64, 1), two)
