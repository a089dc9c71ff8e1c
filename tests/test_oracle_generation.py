"""Pins the CPU oracle of the O(1) generation step (oracle/generation.py).

- rings: after a prompt and single inserts, each bucket holds exactly its C most recent positions and its count is
  its number of positions (the reference's own test, tests/test_nucleo.py:143-157), and slot r % C holds the r-th;
- step = whole text: with every earlier position a key, the layer written step by step equals the golden-pinned
  whole-text oracle at every new position (tests/test_nucleo.py:118-140), with buckets that overflow their rings,
  batches of several texts and prompts of 1 and 2 tokens;
- memoria_de_lo_ajeno: the ring path equals a brute-force scan of all earlier positions restricted to k + 1 < L0;
- the Hawkes memory treats -0.0 and +0.0 as one key and skips NaN keys, as the whole-text sort does.
"""
import numpy as np
import pytest
import torch

from asrn_amd import synth
from asrn_amd.capa import CapaASRNEstable
from oracle import generation as G
from oracle import layer as O


def close(a, b, rel, what):
    a, b = a.double(), b.double()
    scale = b.abs().max().item() + 1e-6
    err = (a - b).abs().max().item() if a.numel() else 0.0
    assert err <= rel * scale, f'{what}: max err {err:.3g} vs scale {scale:.3g}'


def small_layer(d=32, seed=0, **kw):
    torch.manual_seed(seed)
    layer = synth.move_params(CapaASRNEstable(d, **kw), seed)
    p = {k: v.detach().clone() for k, v in layer.state_dict().items()}
    sh = O.shape_from_params(p, d, n_bits=kw.get('n_bits', 14), C=kw.get('chunk', 32))
    return p, sh


def test_rings_hold_the_most_recent_positions():
    g = torch.Generator().manual_seed(0)
    B, L, T, nc, C = 2, 70, 3, 5, 4
    ids = torch.randint(0, nc, (B, L, T), generator=g, dtype=torch.int32).numpy()
    ring, count = G.ring_from(ids, 50, C, nc)
    for t in range(50, L):
        G.ring_insert(ring, count, ids[:, t], t)
    for b in range(B):
        for tau in range(T):
            for k in range(nc):
                pos = [p for p in range(L) if ids[b, p, tau] == k]
                assert count[b, tau, k] == len(pos)
                assert sorted(p for p in ring[b, tau, k].tolist() if p >= 0) == pos[-C:], (b, tau, k)
                for r, p in enumerate(pos[-C:], start=max(0, len(pos) - C)):
                    assert ring[b, tau, k, r % C] == p


def test_rings_of_an_empty_prompt_are_empty():
    ids = np.zeros((1, 5, 2), dtype=np.int32)
    ring, count = G.ring_from(ids, 0, 4, 3)
    assert (ring == -1).all() and (count == 0).all()


@pytest.mark.parametrize('B,L0,n', [(2, 40, 50), (1, 2, 30), (3, 1, 20)])
def test_step_by_step_equals_whole_text(B, L0, n):
    d = 32
    p, sh = small_layer(d, chunk=4, n_bits=2, n_tablas=4, tablas_contexto=2)
    x, E, h = synth.layer_inputs(B, L0 + n, d, 12, seed=L0, frac=0.4, span=(3, 8))
    y_steps, _ = G.decode_layer(p, E, h, x, L0, sh, ajeno=False)
    with torch.no_grad():
        y_whole = O.layer_forward(p, E, h, x, sh)
    close(y_steps, y_whole[:, L0:], 1e-5, 'y')


@pytest.mark.parametrize('B,L0,n', [(2, 40, 30), (1, 2, 10)])
def test_rings_equal_bruteforce_with_memoria_de_lo_ajeno(B, L0, n):
    d = 32
    p, sh = small_layer(d, seed=1, chunk=4, n_bits=2, n_tablas=4, tablas_contexto=2)
    x, E, h = synth.layer_inputs(B, L0 + n, d, 12, seed=7, frac=0.4, span=(3, 8))
    for ajeno in (True, False):
        y_ring, s_ring = G.decode_layer(p, E, h, x, L0, sh, ajeno=ajeno)
        y_bf, s_bf = G.decode_layer(p, E, h, x, L0, sh, ajeno=ajeno, rings='bruteforce')
        close(y_ring, y_bf, 1e-6, f'y ajeno={ajeno}')
        for (a, sa, *_), (b, sb, *_) in zip(s_ring, s_bf):
            assert torch.equal(sa[:, 0], sb[:, 0])            # tables with candidates


def test_hawkes_memory_signed_zero_and_nan_keys():
    mem = G.HawkesMemory(1, 2)
    keys = torch.tensor([[[0.0, float('nan')], [1.0, 2.0]]], dtype=torch.float64)
    mem.load(keys, torch.zeros(1, 2, 2), torch.tensor([[1.0, 2.0]], dtype=torch.float64), torch.zeros(1, 2))
    v, hk = mem.step(torch.tensor([[-0.0, float('nan')]], dtype=torch.float64),
                     torch.tensor([3.0], dtype=torch.float64), torch.zeros(1), torch.ones(2))
    assert v.tolist() == [[1.0, 0.0]]
    # lambda = exp(-1 * (3 - 1)) * (0 + exp(0))
    assert abs(hk[0, 0].item() - float(np.exp(-2.0))) < 1e-7 and hk[0, 1].item() == 0.0
