"""Dense projections whose weight gradient fits a long token axis on MI355X.

For y = x W^T + b over N tokens, the weight gradient dW = dY^T X reduces over all N (32768 at the layer benchmark's
shape) into a small (out, in) matrix. As one GEMM it has only (out / tile) x (in / tile) output tiles to spread over
256 CUs: hipBLASLt ran this layer's weight gradients on 4 to 70 workgroups, at a few percent of the matrix peak, and
they took a third of the step. Here the token axis is cut into S slabs: one batched GEMM forms the S partial products
(S times the tiles) and they are added in fp32, in slab order. The forward and the input gradient are the usual
GEMMs. Under autocast the operands are cast as autocast casts F.linear's, and the products run in that dtype.

On the GPU, the sums (the slab partials, and the bias gradients' column sums) run in the library's asrn_column_sums
(fp32 accumulation in a fixed order, no memset-cleared semaphores, safe to capture in a HIP graph). fp64 operands,
and CPU tensors (the math checked on the CPU), use torch's sums.
"""
import torch
import torch.nn.functional as F

from . import _lib

MIN_SLAB = 1024            # tokens per slab: below this the batched GEMM's own overhead dominates
MAX_SLAB_WEIGHT = 1 << 20  # weights with this many elements or more keep one GEMM: enough output tiles already, and
                           # S partial copies of them would cost more traffic than they save


def slabs_for(n, weight_elems=0):
    """Slab count for a token axis of n: 16 (or fewer) slabs of at least MIN_SLAB tokens that divide n exactly; 1 for
    weights of MAX_SLAB_WEIGHT elements or more."""
    if weight_elems >= MAX_SLAB_WEIGHT:
        return 1
    for s in (16, 8, 4, 2):
        if n % s == 0 and n // s >= MIN_SLAB:
            return s
    return 1


def _rows(t):
    """(N, k) view of a (..., k) tensor whose last axis is contiguous; copies only when the leading axes do not
    flatten to one stride."""
    k = t.shape[-1]
    if t.stride(-1) != 1:
        t = t.contiguous()
    try:
        return t.view(-1, k)
    except RuntimeError:
        return t.reshape(-1, k)


def _slab(t, s):
    """(s, N / s, k) view of an (N, k) matrix with unit last stride (splitting the row axis never needs a copy)."""
    n, k = t.shape
    return t.view(s, n // s, k)


def _acc_dtype(t):
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def _hip_sums(x, rows, cols, ld):
    """fp32 column sums of the (rows, cols) matrix at x (row stride ld) through asrn_column_sums."""
    out = torch.empty((cols,), dtype=torch.float32, device=x.device)
    wsb = _lib.query('asrn_column_sums_workspace', rows, cols)
    ws = torch.empty((wsb,), dtype=torch.uint8, device=x.device) if wsb > 0 else None
    _lib.call('asrn_column_sums', _lib.ptr(x), int(x.dtype == torch.bfloat16), rows, cols, ld, _lib.ptr(out),
              _lib.ptr(ws), wsb, _lib.stream_of(x.device))
    return out


def _on_hip(t):
    return t.is_cuda and t.dtype in (torch.float32, torch.bfloat16)


def sum_rows(t):
    """t (S, ...) summed over its first axis in fp32 (fp64 for fp64), in order."""
    if _on_hip(t):
        t = t.contiguous()
        n = t[0].numel() if t.shape[0] else 0
        return _hip_sums(t, t.shape[0], n, max(n, 1)).view(t.shape[1:])
    return t.sum(0, dtype=_acc_dtype(t))


def weight_grad(g2, x2):
    """dW = g2^T x2, summed in fp32 (fp64 for fp64 operands): g2 (N, out), x2 (N, in), both with unit last stride."""
    s = slabs_for(g2.shape[0], g2.shape[1] * x2.shape[1])
    if s == 1:
        return g2.t().mm(x2).to(_acc_dtype(g2))
    # left operand: the transposed slab of g2; right operand: x2's slab as stored (never a transposed view)
    return sum_rows(torch.bmm(_slab(g2, s).transpose(1, 2), _slab(x2, s)))


def column_sums(g2):
    """Sum over the rows of g2 (N, k) with unit last stride, in fp32 (fp64 for fp64)."""
    if _on_hip(g2):
        return _hip_sums(g2, g2.shape[0], g2.shape[1], max(g2.stride(0), g2.shape[1], 1))
    return g2.sum(0, dtype=_acc_dtype(g2))


class _Lineal(torch.autograd.Function):

    @staticmethod
    def forward(ctx, x, w, b, dt):
        xc, wc = x.to(dt), w.to(dt)
        bc = b.to(dt) if b is not None else None
        with torch.autocast(device_type=x.device.type, enabled=False):
            y = F.linear(xc, wc, bc)
        ctx.save_for_backward(xc, wc)
        ctx.meta = (x.dtype, w.dtype, None if b is None else b.dtype)
        return y

    @staticmethod
    def backward(ctx, g):
        xc, wc = ctx.saved_tensors
        xdt, wdt, bdt = ctx.meta
        gx = gw = gb = None
        with torch.autocast(device_type=g.device.type, enabled=False):
            g = g.to(wc.dtype)
            g2 = _rows(g)
            if ctx.needs_input_grad[0]:
                gx = g.matmul(wc).to(xdt)
            if ctx.needs_input_grad[1]:
                gw = weight_grad(g2, _rows(xc)).to(wdt)
            if bdt is not None and ctx.needs_input_grad[2]:
                gb = column_sums(g2).to(bdt)
        return gx, gw, gb, None


def lineal(x, w, b=None):
    """F.linear(x, w, b) with the slab-split weight gradient; honours autocast like F.linear."""
    dev = x.device.type
    dt = torch.get_autocast_dtype(dev) if torch.is_autocast_enabled(dev) else x.dtype
    return _Lineal.apply(x, w, b, dt)
