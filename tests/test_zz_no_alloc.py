"""asrn_scan_fwd_static (the affine scan with its chunk totals in the library's static device scratch, no workspace
argument and no allocation) against asrn_scan_fwd (the same scan with a caller workspace), through the C ABI: bit for
bit, on two calls in a row, the second on a smaller input; and sizes beyond the scratch are refused with an error."""
import pytest
import torch

import asrn_amd
from asrn_amd import _lib
from asrn_amd._lib import ptr, stream_of

pytestmark = pytest.mark.gpu
DEV = 'cuda'


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    asrn_amd.cargar_biblioteca()


def scan_with_workspace(a, b):
    rows, N = a.shape
    S = torch.empty_like(a)
    need = _lib.query('asrn_scan_workspace', rows, N)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=a.device)
    _lib.call('asrn_scan_fwd', ptr(a), ptr(b), ptr(S), rows, N, ptr(ws), need, stream_of(a.device))
    return S


def scan_static(a, b):
    rows, N = a.shape
    S = torch.full_like(a, float('nan'))
    _lib.call('asrn_scan_fwd_static', ptr(a), ptr(b), ptr(S), rows, N, stream_of(a.device))
    return S


def test_static_scan_equals_workspace_scan_twice():
    print('[case] asrn_scan_fwd_static vs asrn_scan_fwd: (32, 70000) then (5, 30000)', flush=True)
    g = torch.Generator().manual_seed(0)
    for rows, N in ((32, 70000), (5, 30000)):
        a = torch.rand(rows, N, generator=g).to(DEV)
        b = torch.randn(rows, N, generator=g).to(DEV)
        assert _lib.query('asrn_scan_workspace', rows, N) > 0          # multi-chunk scans: the scratch is used
        ref = scan_with_workspace(a, b)
        got = scan_static(a, b)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (rows, N)


def test_static_scan_takes_one_launch_rows_without_scratch():
    """Rows of 1,025 to 4,096 run as one launch (a workgroup a row) and need no chunk totals: the static entry point
    takes them at any row count, also where the workspace bound would exceed its scratch."""
    print('[case] asrn_scan_fwd_static, (32768, 4096): one launch, no scratch', flush=True)
    rows, N = 32768, 4096
    assert _lib.query('asrn_scan_workspace', rows, N) > _lib.query('asrn_scan_static_scratch_bytes')
    g = torch.Generator(device=DEV).manual_seed(1)
    a = torch.rand(rows, N, generator=g, device=DEV)
    b = torch.randn(rows, N, generator=g, device=DEV)
    ref = scan_with_workspace(a, b)
    got = scan_static(a, b)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_static_scan_refuses_sizes_beyond_its_scratch():
    print('[case] asrn_scan_fwd_static refuses an oversized scan', flush=True)
    cap = _lib.query('asrn_scan_static_scratch_bytes')
    rows, N = 4096, 1 << 20
    assert _lib.query('asrn_scan_workspace', rows, N) > cap
    a = torch.empty(0, device=DEV)
    with pytest.raises(_lib.ASRNHipError, match='static scratch'):
        _lib.call('asrn_scan_fwd_static', ptr(a), ptr(a), ptr(a), rows, N, stream_of(a.device))
