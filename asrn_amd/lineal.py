"""Dense projections whose weight gradient fits a long token axis on MI355X.

For y = x W^T + b over N tokens, the weight gradient dW = dY^T X reduces over all N (32768 at the layer benchmark's
shape) into a small (out, in) matrix. As one GEMM it has only (out / tile) x (in / tile) output tiles to spread over
256 CUs: hipBLASLt ran this layer's weight gradients on 4 to 70 workgroups, at a few percent of the matrix peak, and
they took a third of the step. Here the token axis is cut into S slabs: one batched GEMM forms the S partial products
(S times the tiles) and they are added in fp32, in slab order. The forward and the input gradient are the usual
GEMMs. Under autocast the operands are cast as autocast casts F.linear's, and the products run in that dtype.
"""
import torch
import torch.nn.functional as F

MIN_SLAB = 1024            # tokens per slab: below this the batched GEMM's own overhead dominates


def slabs_for(n):
    """Slab count for a token axis of n: 16 (or fewer) slabs of at least MIN_SLAB tokens that divide n exactly."""
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


def weight_grad(g2, x2):
    """dW = g2^T x2, summed in fp32 (fp64 for fp64 operands): g2 (N, out), x2 (N, in), both with unit last stride."""
    s = slabs_for(g2.shape[0])
    if s == 1:
        return g2.t().mm(x2).to(_acc_dtype(g2))
    # left operand: the transposed slab of g2; right operand: x2's slab as stored (never a transposed view)
    return torch.bmm(_slab(g2, s).transpose(1, 2), _slab(x2, s)).sum(0, dtype=_acc_dtype(g2))


_ONES = {}


def column_sums(g2):
    """Sum over the rows of g2 (N, k), in fp32 (fp64 for fp64): per-slab products with a ones vector on the matrix
    cores, then the slab sum. (A plain sum over N is a multi-workgroup reduction, whose semaphores are cleared with a
    memset before every call.)"""
    s = slabs_for(g2.shape[0])
    if s == 1:
        return g2.sum(0, dtype=_acc_dtype(g2))
    key = (s, g2.shape[0] // s, g2.dtype, g2.device)
    ones = _ONES.get(key)
    if ones is None:
        ones = _ONES[key] = torch.ones((s, 1, key[1]), dtype=g2.dtype, device=g2.device)
    return torch.bmm(ones, _slab(g2, s)).sum(0, dtype=_acc_dtype(g2)).reshape(-1)


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
