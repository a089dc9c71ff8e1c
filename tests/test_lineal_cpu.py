"""The slab-split weight gradient of asrn_amd.lineal against F.linear's autograd (CPU, fp64): same output, same
input, weight and bias gradients, for token counts that split into 16, 8, 2 or no slabs and for strided inputs."""
import pytest
import torch
import torch.nn.functional as F

from asrn_amd.lineal import lineal, slabs_for


def test_slab_counts():
    assert slabs_for(32768) == 16
    assert slabs_for(8192) == 8
    assert slabs_for(3000) == 2
    assert slabs_for(1000) == 1
    assert slabs_for(4097) == 1


@pytest.mark.parametrize('lead,fin,fout,bias,strided', [((8, 4096), 256, 320, True, False), ((3000,), 64, 56, True, True),
                                                        ((2, 2048), 512, 2, False, False), ((5,), 4, 1, True, False),
                                                        ((4, 1025), 16, 8, True, True)])
def test_lineal_matches_linear(lead, fin, fout, bias, strided):
    g = torch.Generator().manual_seed(fin + fout)
    if strided:                                   # rows of a wider matrix (a split of a fused projection's output)
        x = torch.randn(*lead, fin + 7, generator=g, dtype=torch.float64)[..., 3:3 + fin]
    else:
        x = torch.randn(*lead, fin, generator=g, dtype=torch.float64)
    w = torch.randn(fout, fin, generator=g, dtype=torch.float64)
    b = torch.randn(fout, generator=g, dtype=torch.float64) if bias else None
    gy = torch.randn(*lead, fout, generator=g, dtype=torch.float64)
    leaves = []
    outs = []
    for f in (F.linear, lineal):
        xl, wl = x.clone().requires_grad_(), w.clone().requires_grad_()
        bl = b.clone().requires_grad_() if bias else None
        y = f(xl, wl, bl)
        (y * gy).sum().backward()
        outs.append(y.detach())
        leaves.append((xl, wl, bl))
    torch.testing.assert_close(outs[1], outs[0], rtol=1e-12, atol=1e-12)
    for a, b_ in zip(leaves[0], leaves[1]):
        if a is not None:
            torch.testing.assert_close(b_.grad, a.grad, rtol=1e-10, atol=1e-10)
