"""The layer's forward + backward captured into a HIP graph (as bench.py times it) replays to the eager results.

Every replay is compared with the eager step, with unrelated eager work and a synchronization between replays, so a
graph node that only works on its first replay (a memset recorded by a library call, a workspace not rewritten) shows
up here. The kernels are deterministic and the graph runs the same launches, so the results must be identical."""
import pytest
import torch

import asrn_amd
from asrn_amd import synth

pytestmark = pytest.mark.gpu
DEV = 'cuda'


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    asrn_amd.cargar_biblioteca()


@pytest.mark.parametrize('B,L,d,bf16', [(2, 1500, 64, False), (2, 2048, 128, True)])
def test_layer_graph_replay_matches_eager(B, L, d, bf16):
    print('[case] graph replay', B, L, d, bf16, flush=True)
    torch.manual_seed(0)
    layer = synth.move_params(asrn_amd.ASRNLayer(d, n_bits=10), seed=3).to(DEV)
    x, E, h = synth.layer_inputs(B, L, d, 40, seed=5)
    gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(6)).to(DEV)
    Ed, hd, xd = E.to(DEV).requires_grad_(), h.to(DEV).requires_grad_(), x.to(DEV)
    params = list(layer.parameters())

    def fwd_bwd():
        with torch.autocast('cuda', dtype=torch.bfloat16, enabled=bf16):
            y = layer(Ed, hd, xd)
        y.backward(gy.to(y.dtype))
        return y

    def clear():
        layer.zero_grad(set_to_none=True)
        Ed.grad = None
        hd.grad = None

    clear()
    y_ref = fwd_bwd().detach().clone()
    ref = [t.grad.clone() for t in [Ed, hd] + params if t.grad is not None]
    assert len(ref) >= 10

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            clear()
            fwd_bwd()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    clear()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static = fwd_bwd()
    for rep in range(3):
        junk = torch.randn(1 << 20, device=DEV)
        (junk * 3).sum().item()                   # eager work (with its own reductions) between replays
        graph.replay()
        torch.cuda.synchronize()
        got = [t.grad for t in [Ed, hd] + params if t.grad is not None]
        assert len(got) == len(ref)
        assert torch.equal(y_static, y_ref), f'replay {rep}: output differs'
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f'replay {rep}: gradient {i} differs (max {(a - b).abs().max().item():.3g})'
