"""CPU-side checks of the product: the C-ABI library loads and exports every symbol include/asrn_hip.h declares, its
argument checks reject bad sizes before any device work, the host layer mirrors the reference's parameters and
construction order, and the product refuses CPU tensors instead of falling back."""
import ctypes
import os
import re

import pytest
import torch

import asrn_amd
from asrn_amd import _lib
from asrn_amd.capa import CapaASRNEstable
from tests import fixtures

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'asrn_hip.h')


def declared():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(asrn_\w+)\s*\(', text)))


@pytest.fixture(scope='module')
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip('libasrn_hip.so not built (run `python -m asrn_amd.build`)')
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared()
    assert len(names) >= 14, names
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f'{n} declared in the header but not bound in _lib.SIGNATURES'
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.asrn_hip_abi_version() == 2


def _err(lib):
    return lib.asrn_hip_last_error().decode()


def test_argument_checks_fail_before_any_device_work(lib):
    N = None
    # n_bits outside [1, 14]
    assert lib.asrn_bucket_sort(N, 2, 16, 8, 15, 120, 32, N, N, N, N, N, N, 0, N) != 0
    assert 'n_bits' in _err(lib)
    # phi row stride shorter than T*nb
    assert lib.asrn_bucket_sort(N, 2, 16, 8, 14, 100, 32, N, N, N, N, N, N, 0, N) != 0
    assert 'stride' in _err(lib)
    # window clamp outside [1, 255]
    assert lib.asrn_bucket_sort(N, 2, 16, 8, 14, 112, 300, N, N, N, N, N, N, 0, N) != 0
    assert 'window' in _err(lib)
    # empty inputs are a no-op
    assert lib.asrn_bucket_sort(N, 0, 16, 8, 14, 112, 32, N, N, N, N, N, N, 0, N) == 0
    # rows of 1025 to 4096 positions need the chunks' workspace: 4 chunks of 1024 int32 per (batch row, table)
    assert lib.asrn_bucket_sort_workspace(2, 1024, 8) == 0 and lib.asrn_bucket_sort_workspace(2, 8192, 8) == 0
    assert lib.asrn_bucket_sort_workspace(2, 3000, 8) == 2 * 8 * 3 * 1024 * 4
    assert lib.asrn_bucket_sort(1, 2, 3000, 8, 14, 112, 32, 1, 1, 1, 1, 1, N, 100, N) != 0
    assert 'workspace' in _err(lib)
    args = [N] * 12 + [2, 16]
    # d not a multiple of 4
    assert lib.asrn_candidates_fwd(*args, 6, 112, 16, 4, 8, 4, 32, 0.1, 0.25, 6, 0, 16, 0, N, N, N, N, 0, N, N) != 0
    assert 'd=6' in _err(lib)
    # chunk above 64
    assert lib.asrn_candidates_fwd(*args, 64, 112, 16, 4, 8, 4, 65, 0.1, 0.25, 64, 0, 16, 0, N, N, N, N, 0, N, N) != 0
    assert 'chunk' in _err(lib)
    # feature width above 256
    assert lib.asrn_candidates_bwd(*args, 64, 250, 16, 4, 8, 4, 32, 0.1, 0.25, 64, 0, 16, 0, *([N] * 11)) != 0
    assert 'P + cf' in _err(lib)
    # feature widths are read as float4 (the host pads them)
    assert lib.asrn_candidates_fwd(*args, 64, 110, 16, 4, 8, 4, 32, 0.1, 0.25, 64, 0, 16, 0, N, N, N, N, 0, N, N) != 0
    assert 'multiples of 4' in _err(lib)
    # V row stride below d
    assert lib.asrn_candidates_fwd(*args, 64, 112, 16, 4, 8, 4, 32, 0.1, 0.25, 60, 1, 16, 0, N, N, N, N, 0, N, N) != 0
    assert 'ldv' in _err(lib)
    # the candidate-list records: 16-byte multiples, sized for T * C entries and uniques
    assert lib.asrn_candidates_record_bytes(8, 32) % 16 == 0 and lib.asrn_candidates_record_bytes(8, 32) >= 11 * 256
    assert lib.asrn_candidates_record_bytes(0, 32) == -1
    # workspace sizes are pure host arithmetic
    assert lib.asrn_ngram_sort_workspace(8, 4096, 4) >= 2 * 8 * 4 * 4096 * 12
    assert lib.asrn_ngram_sort(N, N, 8, 4096, 4, N, N, N, N, N, N, 16, N) != 0
    assert 'workspace' in _err(lib)
    assert lib.asrn_hawkes_bwd_workspace(8, 4096, 4) >= 2 * 8 * 4096 * 4 * 4
    # scans: rows of one chunk need none; longer rows hold 12 bytes per chunk of 256
    assert lib.asrn_scan_workspace(8, 1024) == 0
    assert lib.asrn_scan_workspace(32, 4096) >= 32 * 16 * 12
    assert lib.asrn_scan_workspace(1 << 20, 1 << 20) == -1
    assert lib.asrn_hawkes_bwd_workspace(8, 4096, 4) >= 2 * 8 * 4096 * 4 * 4 + lib.asrn_scan_workspace(32, 4096)
    assert lib.asrn_scan_fwd(N, N, N, 2, 8192, N, 0, N) != 0           # multi-chunk: chunk totals needed
    assert 'workspace' in _err(lib)
    # the scan without a workspace: its static scratch is 4 MiB; larger scans are refused before any device work
    assert lib.asrn_scan_static_scratch_bytes() == 4 << 20
    assert lib.asrn_scan_fwd_static(N, N, N, 4096, 1 << 20, N) != 0
    assert 'static scratch' in _err(lib)
    assert lib.asrn_streak_bwd(*([N] * 5), 2, 2048, 4, N, N, N, 1 << 20, N) != 0
    assert 'workspace' in _err(lib)
    # gate: row width, the small parameters' block, the workspace
    gate = [N, N, 0] + [N] * 11
    assert lib.asrn_gate_fwd(*gate, 10, 6, 4, 16, 8, 4, 0.4, 1e4, 0.0, N, N, N) != 0
    assert 'd=6' in _err(lib)
    assert lib.asrn_gate_fwd(*gate, 10, 256, 16, 40, 8, 4, 0.4, 1e4, 0.0, N, N, N) != 0
    assert 'nodes' in _err(lib)
    assert lib.asrn_gate_bwd(*gate, 10, 256, 4, 16, 8, 4, 0.4, 1e4, 0.0, *([N] * 8), 16, N) != 0
    assert 'workspace' in _err(lib)
    assert lib.asrn_gate_bwd_workspace(32768, 256) >= 320 * 4
    # hidden layer: widths in float4 groups, the row strides
    assert lib.asrn_hidden_fwd(N, 200, N, N, 2, 16, 6, 64, N, N) != 0
    assert 'm=6' in _err(lib)
    assert lib.asrn_hidden_bwd(N, 100, N, N, 2, 16, 64, 64, N, N, 448, N) != 0
    assert 'row stride' in _err(lib)
    # fused hash MLPs: hidden widths, the first layers' row stride, the backward's workspace
    assert lib.asrn_hash_fwd(N, 192, *([N] * 6), 2, 16, 6, 64, 56, 56, N, N, 0, 0, N) != 0
    assert 'm=6' in _err(lib)
    assert lib.asrn_hash_fwd(N, 192, *([N] * 6), 2, 16, 64, 64, 56, 65, N, N, 0, 0, N) != 0
    assert 'Pc=65' in _err(lib)
    assert lib.asrn_hash_fwd(N, 100, *([N] * 6), 2, 16, 64, 64, 56, 56, N, N, 0, 0, N) != 0
    assert 'row stride' in _err(lib)
    assert lib.asrn_hash_bwd_workspace(8, 4096, 64, 64, 56, 56) >= 128 * (56 * 64 * 2 + 56 * 2 + 128) * 4
    assert lib.asrn_hash_bwd(N, 192, N, N, N, N, 8, 4096, 64, 64, 56, 56, N, N, 192, N, N, 0, N) != 0
    assert 'workspace' in _err(lib)
    assert lib.asrn_hash_fwd(N, 192, *([N] * 6), 0, 16, 64, 64, 56, 56, N, N, 0, 0, N) == 0      # no tokens: no launch
    # bucket ids from the hash kernel: T * nb must cover phi's columns exactly
    assert lib.asrn_hash_fwd(N, 192, *([N] * 6), 2, 16, 64, 64, 56, 56, N, 16, 8, 13, N) != 0
    assert 'bucket ids' in _err(lib)
    # column sums: a stride below the width; long columns need the slab workspace, short ones none
    assert lib.asrn_column_sums(N, 0, 16, 13, 12, N, N, 0, N) != 0
    assert 'bad sizes' in _err(lib)
    assert lib.asrn_column_sums_workspace(16, 448 * 256) == 0
    assert lib.asrn_column_sums_workspace(0, 6) == 0 and lib.asrn_column_sums_workspace(1, 0) == 0
    assert lib.asrn_column_sums_workspace(32768, 13) >= 2 * 13 * 4
    assert lib.asrn_column_sums(N, 0, 32768, 13, 13, N, N, 0, N) != 0
    assert 'workspace' in _err(lib)
    # small products: sizes and leading dimensions
    assert lib.asrn_small_gemm(N, 16, 0, N, 16, 0, N, 16, 16, 16, 10000, N) != 0
    assert 'K=10000' in _err(lib)
    assert lib.asrn_small_gemm(N, 8, 0, N, 16, 0, N, 16, 16, 16, 16, N) != 0
    assert 'leading' in _err(lib)
    # generation: ring sizes, the decode position inside the caches, table capacities
    assert lib.asrn_ring_build(N, N, 2, 10, 8, 15, 32, N, N, N) != 0
    assert 'asrn_ring_build' in _err(lib)
    assert lib.asrn_decode_attend(*([N] * 11), 2, 100, 100, N, 64, 14, 16, 4, 8, 4, 32, 0.1, 0.25, 1, N, N, N,
                                  N, N, N) != 0
    assert 'outside the caches' in _err(lib)
    assert lib.asrn_hawkes_table_load(*([N] * 6), 2, 100, 4, 96, N, N, N, N) != 0
    assert 'power of two' in _err(lib)
    assert lib.asrn_repetition_step(*([N] * 7), 2, 1000, 100, N, 4, 128, *([N] * 6), 0, N, N) != 0
    assert 'grow it first' in _err(lib)
    assert lib.asrn_hawkes_table_grow(N, N, N, 8, 256, N, N, N, 128, N) != 0
    assert 'growing' in _err(lib)
    # the chained block step: a pending block needs its parts; the workspace covers the wider of the two widths
    P1 = ctypes.c_void_p(16)                                   # a non-null pointer never dereferenced on these paths
    blk = [P1] * 10
    assert lib.asrn_block_step_ex(N, 0, P1, N, P1, P1, 4, 64, P1, P1, P1, 2, 64, 4, 64, *blk, 1e-5, *([P1] * 5), 1,
                                  P1, 1 << 30, N) != 0
    assert 'pending block' in _err(lib)
    need = lib.asrn_block_step_workspace(2, 64, 512)
    assert lib.asrn_block_step_ex(N, 0, P1, P1, P1, P1, 4, 512, P1, P1, P1, 2, 64, 4, 64, *blk, 1e-5, *([P1] * 5), 1,
                                  P1, need - 4, N) != 0
    assert 'workspace' in _err(lib)
    # the fused attention + repetition step: the attention's checks, then the step's n and table capacity
    att = [2, 100, 50, N, 64, 14, 16, 4, 8, 4, 32, 0.1, 0.25, 1, N, N, N, N]
    assert lib.asrn_decode_attend_repeat(*([N] * 11), 2, 100, 100, *att[3:], *([N] * 4), 4, 128, *([N] * 6), 0, N,
                                         N) != 0
    assert 'outside the caches' in _err(lib)
    assert lib.asrn_decode_attend_repeat(*([N] * 11), *att, *([N] * 4), 0, 128, *([N] * 6), 0, N, N) != 0
    assert 'n=0' in _err(lib)
    assert lib.asrn_decode_attend_repeat(*([N] * 11), *att, *([N] * 4), 4, 64, *([N] * 6), 0, N, N) != 0
    assert 'grow it first' in _err(lib)
    assert lib.asrn_decode_attend_repeat(*([N] * 11), *att, *([N] * 4), 4, 128, *([N] * 6), 0, N, N) != 0
    assert 'null pointer' in _err(lib)
    # the step's producers: width, position, workspace
    prod = [N] * 4
    w = [N] * 9
    assert lib.asrn_decode_produce(*prod, 16, 6, *w, 64, 64, 56, 56, N, N, 1e-5, N, N, 1e4, -30.0, N, N, 16,
                                   *([N] * 6), 100, 50, N, N, N, 0, N) != 0
    assert 'd=6' in _err(lib)
    assert lib.asrn_decode_produce(*prod, 16, 768, *w, 64, 64, 56, 56, N, N, 1e-5, N, N, 1e4, -30.0, N, N, 16,
                                   *([N] * 6), 100, 100, N, N, N, 0, N) != 0
    assert 'outside' in _err(lib)
    assert lib.asrn_decode_produce_workspace(16, 64, 64) == 16 * 192 * 4
    assert lib.asrn_decode_produce(*prod, 16, 768, *w, 64, 64, 56, 56, N, N, 1e-5, N, N, 1e4, -30.0, N, N, 16,
                                   *([N] * 6), 100, 50, N, N, N, 0, N) != 0
    assert 'workspace' in _err(lib)
    # the producer on a pending block: the block's pointers, then its workspace (for the block's feed-forward width)
    hx = [N, 16, 768, P1, P1, 1e-5, P1, P1, 1e4, -30.0, P1, P1, 16, P1, P1, P1, 100, 50, N, P1, N]
    assert lib.asrn_decode_produce_h_ex(N, P1, N, P1, P1, 4, 1536, P1, P1, P1, 1 << 30, *hx[1:]) != 0
    assert 'pending block' in _err(lib)
    need = lib.asrn_block_step_workspace(16, 768, 1536)
    assert lib.asrn_decode_produce_h_ex(N, P1, P1, P1, P1, 4, 1536, P1, P1, P1, need - 4, *hx[1:]) != 0
    assert 'workspace' in _err(lib)
    assert lib.asrn_decode_produce_h_ex(N, N, N, N, N, 0, 0, N, N, N, 0, *hx[1:]) != 0
    assert 'null pointer' in _err(lib)
    # the last block's end with the final norm: sizes, the pending block's pointers, its workspace
    assert lib.asrn_block_finish_norm(P1, P1, P1, P1, 4, 1536, P1, P1, 16, 5000, P1, P1, 1e-5, P1, P1, 1 << 30,
                                      N, N, N) != 0
    assert 'd=5000' in _err(lib)
    assert lib.asrn_block_finish_norm(P1, N, P1, P1, 4, 1536, P1, P1, 16, 768, P1, P1, 1e-5, P1, P1, 1 << 30, N, N,
                                      N) != 0
    assert 'null pointer' in _err(lib)
    assert lib.asrn_block_finish_norm(P1, P1, P1, P1, 4, 1536, P1, P1, 16, 768, P1, P1, 1e-5, P1, P1, need - 4,
                                      N, N, N) != 0
    assert 'workspace' in _err(lib)
    assert lib.asrn_block_finish_norm(P1, P1, P1, P1, 4, 1536, P1, P1, 16, 768, P1, P1, 1e-5, P1, P1, 1 << 30, P1,
                                      N, N) != 0
    assert 'count' in _err(lib)


def test_ops_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match='GPU only'):
        asrn_amd.ops.bucket_sort(torch.zeros(1, 4, 112), 8, 14, 32)
    layer = CapaASRNEstable(16)
    with pytest.raises(RuntimeError, match='GPU only'):
        layer(torch.zeros(1, 4, 16), torch.zeros(1, 4, 16), torch.zeros(1, 4, dtype=torch.long))


@pytest.mark.parametrize('name', fixtures.names())
def test_parameters_and_construction_order_match_the_reference(name):
    """Same names, shapes, registration order and seeded values: building the layer with the fixture's seed and
    moving the parameters exactly as tests/golden/make_golden.py did reproduces the reference's state_dict bit for
    bit (asrn/nucleo.py:585-630)."""
    g, p, m = fixtures.load(name)
    torch.manual_seed(0)
    layer = CapaASRNEstable(m['d'], **m['kw'])
    with torch.no_grad():
        gen = torch.Generator().manual_seed(1)
        for n, par in layer.named_parameters():
            par.add_(torch.randn(par.shape, generator=gen) * (0.5 if n in asrn_amd.synth.NUEVOS else 0.05))
        layer.gamma.abs_()
        if 'corrimiento' in m['extra']:
            layer.b_reloj[0] += m['extra']['corrimiento']
        if 'gamma_fill' in m['extra']:
            layer.gamma.fill_(m['extra']['gamma_fill'])
        if m['extra'].get('kappa_r_zero'):
            layer.log_kappa_racha.fill_(-200.0)
        if m['extra'].get('prot') == 'textos_largos':
            layer.g.weight.mul_(100.0)
            layer.log_kappa[2:] = -12.0
            layer.log_kappa_racha.fill_(-12.0)
    sd = layer.state_dict()
    assert sorted(sd) == sorted(p)              # (safetensors stores keys sorted)
    for k in sd:
        assert sd[k].dtype == p[k].dtype and torch.equal(sd[k], p[k]), k


def test_unsupported_protections_and_shapes_raise_clearly():
    if not torch.cuda.is_available():
        layer = CapaASRNEstable(16, protecciones=asrn_amd.Protecciones.ninguna())
        with pytest.raises(RuntimeError, match='GPU only'):
            layer._revisar(torch.zeros(1, 2, 16))


def test_convertir_swaps_layers_keeping_weights():
    """convertir (the counterpart of asrn/estable.py:424-442) rebuilds each layer with the same hyper-parameters and
    weights; construction only, no device work."""
    class Modelo(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.largos = torch.nn.ModuleList([CapaASRNEstable(16, chunk=8, n_bits=5, racha_max=100, nodos_racha=9),
                                               CapaASRNEstable(16)])
    m = Modelo()
    before = [{k: v.clone() for k, v in c.state_dict().items()} for c in m.largos]
    old = list(m.largos)
    m.eval()
    asrn_amd.convertir(m)
    for c, o, sd in zip(m.largos, old, before):
        assert c is not o and not c.training
        assert (c.chunk, c.n_bits, c.racha_paso) == (o.chunk, o.n_bits, o.racha_paso)
        for k, v in c.state_dict().items():
            assert torch.equal(v, sd[k]), k
