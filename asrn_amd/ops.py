"""torch.autograd wrappers around the HIP entry points (include/asrn_hip.h).

Every op takes device tensors, allocates its outputs and workspaces with torch's caching allocator, and launches on
torch's current stream. They replace the reference's fused-op layer: _CasillerosTriton (asrn/nucleo.py:461-515),
_Escaneo / escaneo (asrn/nucleo.py:188-196, 518-537), the stable argsorts (asrn/estable.py:283, nucleo:693-701) and
the clock cumsum (asrn/estable.py:418).
"""
import ctypes
import math

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import call, ptr, query, stream_of
from .lineal import column_sums, weight_grad

I32 = torch.int32


def _dev(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError('asrn_amd runs on the GPU only: got a CPU tensor (move the layer and inputs to cuda)')
    return ts[0].device


def _c(t, dtype=None):
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _rows_in_place(V, dtype=torch.float32):
    """True when V (B, L, d) of `dtype` can be read in place: unit column stride, rows evenly strided across the batch
    (a column block of a (B, L, n) tensor), a row stride that keeps the 4-element row loads aligned."""
    return (V.dtype == dtype and V.dim() == 3 and V.stride(2) == 1 and V.stride(1) % 4 == 0
            and V.stride(1) >= V.shape[2] and V.stride(0) == V.shape[1] * V.stride(1) and V.data_ptr() % 16 == 0)


def _pad4(t):
    """fp32, contiguous, last dimension zero-padded to a multiple of 4."""
    t = _c(t, torch.float32)
    extra = -t.shape[-1] % 4
    return torch.nn.functional.pad(t, (0, extra)) if extra else t


# ---------------------------------------------------------------------------------------------------------------------
# a1 + a2
# ---------------------------------------------------------------------------------------------------------------------

def bucket_sort(phi, T, nb, C, ids=None):
    """phi (B, L, P) fp32 -> ids (B*T, L), order (B*T, L), ids_sorted (B*T, L), rank (B, L, T) and the recent-mates
    index win (B, L, T) = min(C, mates before) | min(C, mates after) << 8, all int32. ids: the bucket ids the fused
    hash producer already wrote (HashProducer with T, nb): the sort reads them instead of hashing phi again."""
    dev = _dev(phi)
    B, L, P = phi.shape
    if ids is not None:
        if ids.dtype != I32 or tuple(ids.shape) != (B * T, L) or not ids.is_contiguous() or ids.device != dev:
            raise ValueError('bucket_sort: ids must be a contiguous (B*T, L) int32 tensor on the device of phi')
        phi = None
    else:
        phi = _c(phi, torch.float32)
        ids = torch.empty((B * T, L), dtype=I32, device=dev)
    # every entry of order, ids_sorted, rank and win is written by the sort (no fill); the candidate kernels clamp
    # the positions they read from order
    buf = torch.empty((4, B * T * L), dtype=I32, device=dev)
    order, ids_s = buf[0].view(B * T, L), buf[1].view(B * T, L)
    rank, win = buf[2].view(B, L, T), buf[3].view(B, L, T)
    wsb = query('asrn_bucket_sort_workspace', B, L, T)
    ws = torch.empty((wsb,), dtype=torch.uint8, device=dev) if wsb else None
    call('asrn_bucket_sort', ptr(phi) if phi is not None else None, B, L, T, nb, P, C, ptr(ids), ptr(order),
         ptr(ids_s), ptr(rank), ptr(win), ptr(ws), wsb, stream_of(dev))
    return ids, order, ids_s, rank, win


def candidate_lists(sig, order, win, rank, C, K):
    """The candidate windows the kernels walk: pos, ell (B, L, T, C) int32, -1 where a slot is empty."""
    dev = _dev(sig)
    B, L, T = rank.shape
    pos = torch.empty((B, L, T, C), dtype=I32, device=dev)
    ell = torch.empty_like(pos)
    sig32 = _c(sig, torch.float32)            # held until the launch: a converted copy must outlive its pointer
    call('asrn_candidate_lists', ptr(sig32), ptr(order), ptr(win), ptr(rank), B, L, T, C, K, ptr(pos), ptr(ell),
         stream_of(dev))
    return pos, ell


# ---------------------------------------------------------------------------------------------------------------------
# a10
# ---------------------------------------------------------------------------------------------------------------------

def ngram_sort(sig, coef, n):
    """sig (B, L) fp32, coef (n,) fp64 -> keys (B, L, n) fp64, order (B, n, L) int32, repeated (B, n, L) uint8,
    rank_k (B, n, L) int32, vistos (B, L, n) fp32."""
    dev = _dev(sig)
    sig = _c(sig, torch.float32)
    coef = _c(coef, torch.float64)
    B, L = sig.shape
    keys = torch.empty((B, L, n), dtype=torch.float64, device=dev)
    order = torch.empty((B, n, L), dtype=I32, device=dev)
    rep = torch.empty((B, n, L), dtype=torch.uint8, device=dev)
    buf = torch.zeros((2, B * n * L), dtype=I32, device=dev)   # one fill: every index read later is in range
    rank_k = buf[0].view(B, n, L)
    vistos = buf[1].view(torch.float32).view(B, L, n)              # int32 zeros are fp32 zeros
    wsb = query('asrn_ngram_sort_workspace', B, L, n)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    call('asrn_ngram_sort', ptr(sig), ptr(coef), B, L, n, ptr(keys), ptr(order), ptr(rep), ptr(rank_k), ptr(vistos),
         ptr(ws), wsb, stream_of(dev))
    return keys, order, rep, rank_k, vistos


# ---------------------------------------------------------------------------------------------------------------------
# a0 (the context producer's LayerNorm and clock projection)
# ---------------------------------------------------------------------------------------------------------------------

def _context_fwd(h, ln_w, ln_b, w_reloj, b_reloj, meta):
    """asrn_context_fwd: (h32 (BL, d), the fp32 parameters, hh, stats, beta, la)."""
    eps, beta_max, la_min = meta
    dev = _dev(h)
    d = h.shape[-1]
    h32 = _c(h, torch.float32).reshape(-1, d)
    BL = h32.shape[0]
    params = [_c(p, torch.float32) for p in (ln_w, ln_b, w_reloj, b_reloj)]
    hh = torch.empty_like(h32)
    stats = torch.empty((BL, 4), dtype=torch.float32, device=dev)
    beta = torch.empty((BL,), dtype=torch.float64, device=dev)
    la = torch.empty((BL,), dtype=torch.float32, device=dev)
    call('asrn_context_fwd', ptr(h32), *[ptr(p) for p in params], BL, d, eps, beta_max, la_min, ptr(hh),
         ptr(stats), ptr(beta), ptr(la), stream_of(dev))
    return h32, params, hh, stats, beta, la


def _context_bwd(h32, lnw, lnb, wr, stats, beta_max, la_min, dhh, dy, wq, dbeta, dla, dh_add):
    """asrn_context_bwd from dhh (BL, d) or from dy (BL, ny) and wq (ny, d): dh (BL, d) and the 4 d + 2 parameter
    gradients [ln_w | ln_b | w_reloj | b_reloj]."""
    BL, d = h32.shape
    dev = h32.device
    dbeta = (torch.zeros((BL,), dtype=torch.float64, device=dev) if dbeta is None
             else _c(dbeta, torch.float64).reshape(BL))
    dla = torch.zeros((BL,), dtype=torch.float32, device=dev) if dla is None else _c(dla, torch.float32).reshape(BL)
    if dh_add is not None:
        dh_add = _c(dh_add, torch.float32).reshape(BL, d)
    dh = torch.empty_like(h32)
    dp = torch.empty((4 * d + 2,), dtype=torch.float32, device=dev)
    wsb = query('asrn_context_bwd_workspace', BL, d)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    ny = 0 if dy is None else dy.shape[1]
    call('asrn_context_bwd', ptr(h32), ptr(lnw), ptr(lnb), ptr(wr), ptr(stats), BL, d, beta_max, la_min,
         ptr(dhh), ptr(dy), max(ny, 1), ny, ptr(wq), ptr(dbeta), ptr(dla), ptr(dh_add), ptr(dh), ptr(dp), ptr(ws),
         wsb, stream_of(dev))
    return dh, dp


class Context(torch.autograd.Function):
    """hh = LayerNorm(h), beta = min(softplus(u_0), beta_max) fp64, log_alfa = max(logsigmoid(u_1) + log 2, min) with
    u = w_reloj hh + b_reloj in fp32 (asrn/estable.py:153-194), fused in asrn_context_fwd/bwd. hh feeds the Qc/Kc GEMM.
    The fourth output is h itself (fp32, an alias) for the layer's other use of h (the gate): its gradient is added
    to dh inside asrn_context_bwd, so the two paths to h need no separate addition.
    meta = (eps, beta_max or -1, log_alfa_min or -inf)."""

    @staticmethod
    def forward(ctx, h, ln_w, ln_b, w_reloj, b_reloj, meta):
        _, beta_max, la_min = meta
        d, lead = h.shape[-1], h.shape[:-1]
        h32, params, hh, stats, beta, la = _context_fwd(h, ln_w, ln_b, w_reloj, b_reloj, meta)
        ctx.save_for_backward(h32, *params[:3], stats)
        ctx.meta = (beta_max, la_min, h.dtype, lead, [p.shape for p in (ln_w, ln_b, w_reloj, b_reloj)])
        return hh.view(*lead, d), beta.view(lead), la.view(lead), h32.view(*lead, d)

    @staticmethod
    def backward(ctx, dhh, dbeta, dla, dh_add):
        h32, lnw, lnb, wr, stats = ctx.saved_tensors
        beta_max, la_min, hdt, lead, shapes = ctx.meta
        BL, d = h32.shape
        dhh = torch.zeros_like(h32) if dhh is None else _c(dhh, torch.float32).reshape(BL, d)
        dh, dp = _context_bwd(h32, lnw, lnb, wr, stats, beta_max, la_min, dhh, None, None, dbeta, dla, dh_add)
        grads = [t.view(s) for t, s in zip(torch.split(dp, [d, d, 2 * d, 2]), shapes)]
        return (dh.view(*lead, d).to(hdt), *grads, None)


class ContextProj(torch.autograd.Function):
    """Context followed by the Qc/Kc projection y = hh Wq^T, fp32 (asrn/estable.py:153-194): the first output is y
    (.., ny) instead of hh. The backward forms the projection's input gradient dhh = dy Wq inside asrn_context_bwd
    (no GEMM and no dhh buffer: dy is ny <= 32 values a token) and Wq's gradient dy^T hh by token slabs, as lineal
    does. For fp32 layers with d <= 512 and 2 cf <= 32."""

    @staticmethod
    def forward(ctx, h, ln_w, ln_b, w_reloj, b_reloj, Wq, meta):
        _, beta_max, la_min = meta
        d, lead = h.shape[-1], h.shape[:-1]
        h32, params, hh, stats, beta, la = _context_fwd(h, ln_w, ln_b, w_reloj, b_reloj, meta)
        wq = _c(Wq, torch.float32)
        with torch.autocast(device_type=h.device.type, enabled=False):
            y = F.linear(hh, wq)
        ctx.save_for_backward(h32, *params[:3], stats, hh, wq)
        ctx.meta = (beta_max, la_min, h.dtype, lead, [p.shape for p in (ln_w, ln_b, w_reloj, b_reloj)], Wq.dtype)
        return y.view(*lead, wq.shape[0]), beta.view(lead), la.view(lead), h32.view(*lead, d)

    @staticmethod
    def backward(ctx, dy, dbeta, dla, dh_add):
        h32, lnw, lnb, wr, stats, hh, wq = ctx.saved_tensors
        beta_max, la_min, hdt, lead, shapes, wdt = ctx.meta
        BL, d = h32.shape
        ny = wq.shape[0]
        dy = (torch.zeros((BL, ny), dtype=torch.float32, device=h32.device) if dy is None
              else _c(dy, torch.float32).reshape(BL, ny))
        dwq = weight_grad(dy, hh).to(wdt) if ctx.needs_input_grad[5] else None
        dh, dp = _context_bwd(h32, lnw, lnb, wr, stats, beta_max, la_min, None, dy, wq, dbeta, dla, dh_add)
        grads = [t.view(s) for t, s in zip(torch.split(dp, [d, d, 2 * d, 2]), shapes)]
        return (dh.view(*lead, d).to(hdt), *grads, dwq, None)


# ---------------------------------------------------------------------------------------------------------------------
# a0 (the hash MLPs' first layers)
# ---------------------------------------------------------------------------------------------------------------------

class Producer(torch.autograd.Function):
    """y = E W^T by one bias-free GEMM, W's rows [W_p (m) | W_a (mc) | W_b (mc)]; returns the hash MLPs' hidden units
    g (B, L, m + mc) = [gelu(W_p E_t + b_word) | gelu(W_a E_t + W_b E_{t-1} + b_ctx)] (asrn_hidden_fwd;
    asrn/nucleo.py:644-652) and E itself (fp32, an alias) as the rows the candidate kernels gather.

    Backward: asrn_hidden_bwd turns dg into dy; the alias's gradient (from the candidate backward) is the buffer the
    input gradient accumulates into, dE = dE_rows + dy W in one GEMM with beta = 1, so the two paths to E need no
    separate addition. dW by token slabs; the biases' gradients are the column sums of dy. fp32 only."""

    @staticmethod
    def forward(ctx, E, W, b_word, b_ctx, m, mc):
        dev = _dev(E, W)
        B, L, d = E.shape
        n = W.shape[0]
        if n != m + 2 * mc:
            raise ValueError(f'Producer: W has {n} rows, expected m + 2 mc = {m + 2 * mc}')
        E = _c(E, torch.float32)
        bw, bc = _c(b_word, torch.float32), _c(b_ctx, torch.float32)
        y = torch.nn.functional.linear(E, W)
        g = torch.empty((B, L, m + mc), dtype=torch.float32, device=dev)
        call('asrn_hidden_fwd', ptr(y), n, ptr(bw), ptr(bc), B, L, m, mc, ptr(g), stream_of(dev))
        ctx.save_for_backward(E, W, y, bw, bc)
        ctx.meta = (m, mc)
        return g, E.view_as(E)

    @staticmethod
    def backward(ctx, dg, drows):
        E, W, y, bw, bc = ctx.saved_tensors
        m, mc = ctx.meta
        B, L, n = y.shape
        d = E.shape[-1]
        dev = y.device
        dE = dW = dbw = dbc = None
        if dg is None:
            if ctx.needs_input_grad[0] and drows is not None:
                dE = drows
            return dE, None, None, None, None, None
        dg = _c(dg, torch.float32)
        dy = torch.empty((B, L, n), dtype=torch.float32, device=dev)
        call('asrn_hidden_bwd', ptr(y), n, ptr(bw), ptr(bc), B, L, m, mc, ptr(dg), ptr(dy), n, stream_of(dev))
        dy2 = dy.view(B * L, n)
        if ctx.needs_input_grad[0]:
            if drows is None:
                dE = dy2.mm(W).view(B, L, d)
            else:
                # the rows' gradient is a fresh buffer of the candidate backward: accumulate the GEMM into it
                dE = _c(drows, torch.float32) if drows.dtype != torch.float32 or not drows.is_contiguous() else drows
                dE.view(B * L, d).addmm_(dy2, W)
        if ctx.needs_input_grad[1]:
            dW = weight_grad(dy2, E.view(B * L, d))
        if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
            db = column_sums(dy2[:, :m + mc])
            dbw, dbc = db[:m], db[m:]
        return dE, dW, dbw, dbc, None, None


def copy_blocks(blocks):
    """One launch of asrn_copy_blocks: blocks is a list of (src, dst) 2-D fp32 device views of equal shape with unit
    column stride (src None: dst is filled with zeros)."""
    n = len(blocks)
    if n == 0:
        return
    dev = _dev(blocks[0][1])
    for src, dst in blocks:
        if dst.dim() != 2 or dst.dtype != torch.float32 or dst.stride(1) != 1 or (
                src is not None and (src.shape != dst.shape or src.dtype != torch.float32 or src.stride(1) != 1)):
            raise ValueError('copy_blocks: blocks are 2-D fp32 views of one shape with unit column stride')
    arr = lambda ty, xs: (ty * n)(*xs)
    call('asrn_copy_blocks', n, arr(ctypes.c_void_p, [None if s is None else s.data_ptr() for s, _ in blocks]),
         arr(ctypes.c_void_p, [d.data_ptr() for _, d in blocks]),
         arr(ctypes.c_int64, [d.shape[1] if s is None else s.stride(0) for s, d in blocks]),
         arr(ctypes.c_int64, [d.stride(0) for _, d in blocks]), arr(ctypes.c_int64, [d.shape[0] for _, d in blocks]),
         arr(ctypes.c_int64, [d.shape[1] for _, d in blocks]), stream_of(dev))


class HashProducer(torch.autograd.Function):
    """phi (B, L, Pw + Pc) from E through both hash MLPs (asrn/nucleo.py:644-659): y = E W^T by one bias-free GEMM
    (W's rows [W_p (m) | W_a (mc) | W_b (mc)]), then the hidden layer and both second layers in asrn_hash_fwd (the
    second layers on the matrix cores as the two diagonal blocks they are). Also returns E itself (fp32, an alias) as
    the rows the candidate kernels gather. Backward: asrn_hash_bwd writes dy and every second-layer and bias gradient;
    dE = dE_rows + dy W in one GEMM with beta = 1; dW by token slabs. fp32 only. With T > 0 (and T nb = Pw + Pc) the
    kernel also writes the bucket ids (B*T, L) of the phi it stores, returned third (empty otherwise), for
    bucket_sort(..., ids=)."""

    @staticmethod
    def forward(ctx, E, W, b_word, b_ctx, W2w, b2w, W2c, b2c, m, mc, T=0, nb=0):
        dev = _dev(E, W)
        B, L, d = E.shape
        n = W.shape[0]
        Pw, Pc = W2w.shape[0], W2c.shape[0]
        if n != m + 2 * mc or W2w.shape[1] != m or W2c.shape[1] != mc:
            raise ValueError('HashProducer: W must be (m + 2 mc, d), W2w (Pw, m) and W2c (Pc, mc)')
        E = _c(E, torch.float32)
        ps = [_c(t, torch.float32) for t in (b_word, b_ctx, W2w, b2w, W2c, b2c)]
        if B * L <= 256:        # a few tokens (the generation step): one small tile per workgroup beats the library
            W32 = _c(W, torch.float32)
            y = torch.empty((B, L, n), dtype=torch.float32, device=dev)
            call('asrn_small_gemm', ptr(E), d, 0, ptr(W32), d, 1, ptr(y), n, B * L, n, d, stream_of(dev))
        else:
            y = torch.nn.functional.linear(E, W)
        phi = torch.empty((B, L, Pw + Pc), dtype=torch.float32, device=dev)
        con_ids = T > 0 and T * nb == Pw + Pc
        ids = torch.empty((B * T, L) if con_ids else (0,), dtype=I32, device=dev)
        call('asrn_hash_fwd', ptr(y), n, *[ptr(t) for t in ps], B, L, m, mc, Pw, Pc, ptr(phi),
             ptr(ids) if con_ids else None, T if con_ids else 0, nb if con_ids else 0, stream_of(dev))
        ctx.save_for_backward(E, W, y, ps[0], ps[1], ps[2], ps[4])
        ctx.meta = (m, mc, Pw, Pc)
        ctx.set_materialize_grads(False)
        ctx.mark_non_differentiable(ids)
        return phi, E.view_as(E), ids

    @staticmethod
    def backward(ctx, dphi, drows, dids):
        E, W, y, bw, bc, W2w, W2c = ctx.saved_tensors
        m, mc, Pw, Pc = ctx.meta
        B, L, n = y.shape
        d = E.shape[-1]
        dev = y.device
        if dphi is None:
            dphi = torch.zeros((B, L, Pw + Pc), dtype=torch.float32, device=dev)
        dphi = _c(dphi, torch.float32)
        dy = torch.empty((B, L, n), dtype=torch.float32, device=dev)
        dp = torch.empty((Pw * m + Pc * mc + Pw + Pc + m + mc,), dtype=torch.float32, device=dev)
        wsb = query('asrn_hash_bwd_workspace', B, L, m, mc, Pw, Pc)
        ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
        call('asrn_hash_bwd', ptr(y), n, ptr(bw), ptr(bc), ptr(W2w), ptr(W2c), B, L, m, mc, Pw, Pc, ptr(dphi),
             ptr(dy), n, ptr(dp), ptr(ws), wsb, stream_of(dev))
        dW2w, dW2c, db2w, db2c, dbw, dbc = torch.split(dp, [Pw * m, Pc * mc, Pw, Pc, m, mc])
        dy2 = dy.view(B * L, n)
        dE = None
        if ctx.needs_input_grad[0]:
            if drows is None:
                dE = dy2.mm(W).view(B, L, d)
            else:
                # the rows' gradient is a fresh buffer of the candidate backward: accumulate the GEMM into it
                dE = _c(drows, torch.float32) if drows.dtype != torch.float32 or not drows.is_contiguous() else drows
                dE.view(B * L, d).addmm_(dy2, W)
        dW = weight_grad(dy2, E.view(B * L, d)) if ctx.needs_input_grad[1] else None
        return (dE, dW, dbw, dbc, dW2w.view(Pw, m), db2w, dW2c.view(Pc, mc), db2c, None, None, None, None)


# products of more multiply-adds than this go to the library GEMM: the one-tile-per-workgroup kernel wins only while
# the launch, not the arithmetic, is the cost (d = 256: 7 us; d = 768: 70-105 us against about 10 us in the library)
SMALL_GEMM_MAX_MACS = 256 ** 3


def _mm32(A, B):
    """fp32 A @ B on the library GEMM, outside any autocast region (operands may be transposed views)."""
    with torch.autocast(device_type=A.device.type, enabled=False):
        return A.mm(B)


class SmallMatmul(torch.autograd.Function):
    """A @ B for small fp32 matrices (asrn_small_gemm: one workgroup per 16 x 16 tile of the result): the layer's
    W_o W_v. The backward's dA = dC B^T and dB = A^T dC run on the same kernel. Products beyond SMALL_GEMM_MAX_MACS
    multiply-adds (d > 256) run on the library's fp32 GEMM instead, in both directions."""

    @staticmethod
    def forward(ctx, A, B):
        dev = _dev(A, B)
        A32, B32 = _c(A, torch.float32), _c(B, torch.float32)
        (M, K), (K2, N) = A32.shape, B32.shape
        if K != K2:
            raise ValueError(f'SmallMatmul: shapes {tuple(A.shape)} and {tuple(B.shape)} do not chain')
        if M * N * K > SMALL_GEMM_MAX_MACS:
            C = _mm32(A32, B32)
        else:
            C = torch.empty((M, N), dtype=torch.float32, device=dev)
            call('asrn_small_gemm', ptr(A32), K, 0, ptr(B32), N, 0, ptr(C), N, M, N, K, stream_of(dev))
        ctx.save_for_backward(A32, B32)
        ctx.dts = (A.dtype, B.dtype)
        return C

    @staticmethod
    def backward(ctx, dC):
        A, B = ctx.saved_tensors
        (M, K), N = A.shape, B.shape[1]
        dev = A.device
        dC = _c(dC, torch.float32)
        dA = dB = None
        if M * N * K > SMALL_GEMM_MAX_MACS:
            if ctx.needs_input_grad[0]:
                dA = _mm32(dC, B.t()).to(ctx.dts[0])
            if ctx.needs_input_grad[1]:
                dB = _mm32(A.t(), dC).to(ctx.dts[1])
            return dA, dB
        if ctx.needs_input_grad[0]:                # (M, K) = dC (M, N) B^T
            dA = torch.empty((M, K), dtype=torch.float32, device=dev)
            call('asrn_small_gemm', ptr(dC), N, 0, ptr(B), N, 1, ptr(dA), K, M, K, N, stream_of(dev))
            dA = dA.to(ctx.dts[0])
        if ctx.needs_input_grad[1]:                # (K, N) = A^T (K, M) dC (M, N)
            dB = torch.empty((K, N), dtype=torch.float32, device=dev)
            call('asrn_small_gemm', ptr(A), K, 1, ptr(dC), N, 0, ptr(dB), N, K, N, M, stream_of(dev))
            dB = dB.to(ctx.dts[1])
        return dA, dB


# ---------------------------------------------------------------------------------------------------------------------
# a9
# ---------------------------------------------------------------------------------------------------------------------

def _scan_workspace(rows, N, dev):
    """Chunk totals for the scans (asrn_scan_workspace): None for rows that fit one chunk."""
    wsb = query('asrn_scan_workspace', rows, N)
    if wsb < 0:
        raise RuntimeError(f'scan of {rows} rows x {N}: too many chunks')
    return (torch.empty((wsb,), dtype=torch.uint8, device=dev) if wsb else None), wsb


class ClockScan(torch.autograd.Function):
    """Bt = cumsum(beta, 1) in fp64; the backward is the suffix sum. reloj32: each sum rounded to fp32 (kept in an
    fp64 tensor), the core layer's fp32 clock (asrn/nucleo.py:882: an fp32 cumsum, accumulated in double on the CPU);
    its gradient is the same suffix sum."""

    @staticmethod
    def forward(ctx, beta, reloj32=False):
        dev = _dev(beta)
        x = _c(beta, torch.float64)
        y = torch.empty_like(x)
        ws, wsb = _scan_workspace(x.shape[0], x.shape[1], dev)
        call('asrn_clock_scan', ptr(x), ptr(y), x.shape[0], x.shape[1], 2 if reloj32 else 0, ptr(ws), wsb,
             stream_of(dev))
        return y

    @staticmethod
    def backward(ctx, g):
        g = _c(g, torch.float64)
        out = torch.empty_like(g)
        ws, wsb = _scan_workspace(g.shape[0], g.shape[1], g.device)
        call('asrn_clock_scan', ptr(g), ptr(out), g.shape[0], g.shape[1], 1, ptr(ws), wsb, stream_of(g.device))
        return out, None


# ---------------------------------------------------------------------------------------------------------------------
# a12
# ---------------------------------------------------------------------------------------------------------------------

class AffineScan(torch.autograd.Function):
    """S_i = a_i S_{i-1} + b_i over the last axis in fp32 (the reference's escaneo, asrn/nucleo.py:188-196)."""

    @staticmethod
    def forward(ctx, a, b):
        dev = _dev(a, b)
        a, b = torch.broadcast_tensors(a, b)
        shape = a.shape
        N = shape[-1]
        a2, b2 = _c(a, torch.float32).reshape(-1, N), _c(b, torch.float32).reshape(-1, N)
        S = torch.empty_like(a2)
        ws, wsb = _scan_workspace(a2.shape[0], N, dev)
        call('asrn_scan_fwd', ptr(a2), ptr(b2), ptr(S), a2.shape[0], N, ptr(ws), wsb, stream_of(dev))
        ctx.save_for_backward(a2, S)
        ctx.shape = shape
        return S.view(shape)

    @staticmethod
    def backward(ctx, g):
        a2, S = ctx.saved_tensors
        N = a2.shape[-1]
        g2 = _c(g, torch.float32).reshape(-1, N)
        ga, gb = torch.empty_like(g2), torch.empty_like(g2)
        ws, wsb = _scan_workspace(a2.shape[0], N, g.device)
        call('asrn_scan_bwd', ptr(a2), ptr(S), ptr(g2), ptr(ga), ptr(gb), a2.shape[0], N, ptr(ws), wsb,
             stream_of(g.device))
        return ga.view(ctx.shape), gb.view(ctx.shape)


def escaneo(a, b):
    return AffineScan.apply(a, b)


# ---------------------------------------------------------------------------------------------------------------------
# a11
# ---------------------------------------------------------------------------------------------------------------------

class Hawkes(torch.autograd.Function):
    """hawkes (B, L, n) from the clock, log alfa and kappa (n,) along the n-gram key order (asrn/estable.py:313-318).
    order/repeated/rank_k come from ngram_sort and carry no gradient."""

    @staticmethod
    def forward(ctx, Bt, log_alfa, kappa, order, rep, rank_k):
        dev = _dev(Bt)
        B, n, L = order.shape
        Bt = _c(Bt, torch.float64)
        la = _c(log_alfa, torch.float32)
        kap = _c(kappa, torch.float32)
        hawkes = torch.empty((B, L, n), dtype=torch.float32, device=dev)
        S = torch.empty((B, n, L), dtype=torch.float32, device=dev)
        ws, wsb = _scan_workspace(B * n, L, dev)
        call('asrn_hawkes_fwd', ptr(order), ptr(rep), ptr(Bt), ptr(la), ptr(kap), B, L, n, ptr(hawkes), ptr(S),
             ptr(ws), wsb, stream_of(dev))
        ctx.save_for_backward(Bt, la, kap, order, rep, rank_k, S)
        return hawkes

    @staticmethod
    def backward(ctx, g):
        Bt, la, kap, order, rep, rank_k, S = ctx.saved_tensors
        B, n, L = order.shape
        dev = Bt.device
        g = _c(g, torch.float32)
        dBt = torch.empty((B, L), dtype=torch.float64, device=dev)
        dla = torch.empty((B, L), dtype=torch.float32, device=dev)
        dk = torch.empty((B, n), dtype=torch.float32, device=dev)
        wsb = query('asrn_hawkes_bwd_workspace', B, L, n)
        ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
        call('asrn_hawkes_bwd', ptr(order), ptr(rep), ptr(rank_k), ptr(Bt), ptr(la), ptr(kap), ptr(S), ptr(g), B, L,
             n, ptr(dBt), ptr(dla), ptr(dk), ptr(ws), wsb, stream_of(dev))
        return dBt, dla, dk.sum(0), None, None, None


class Streak(torch.autograd.Function):
    """racha (B, L) = scan(r exp(-kappa_r beta), r) with r = vistos[..., n-1] (asrn/estable.py:319-320)."""

    @staticmethod
    def forward(ctx, beta, kappa_r, vistos):
        dev = _dev(beta)
        B, L, n = vistos.shape
        beta = _c(beta, torch.float64)
        kr = _c(kappa_r, torch.float32)
        vistos = _c(vistos, torch.float32)
        racha = torch.empty((B, L), dtype=torch.float32, device=dev)
        ws, wsb = _scan_workspace(B, L, dev)
        call('asrn_streak_fwd', ptr(vistos), ptr(beta), ptr(kr), B, L, n, ptr(racha), ptr(ws), wsb, stream_of(dev))
        ctx.save_for_backward(vistos, beta, kr, racha)
        return racha

    @staticmethod
    def backward(ctx, g):
        vistos, beta, kr, racha = ctx.saved_tensors
        B, L, n = vistos.shape
        dev = beta.device
        g = _c(g, torch.float32)
        dbeta = torch.empty((B, L), dtype=torch.float64, device=dev)
        dkr = torch.empty((B,), dtype=torch.float32, device=dev)
        ws, wsb = _scan_workspace(B, L, dev)
        call('asrn_streak_bwd', ptr(vistos), ptr(beta), ptr(kr), ptr(racha), ptr(g), B, L, n, ptr(dbeta), ptr(dkr),
             ptr(ws), wsb, stream_of(dev))
        return dbeta, dkr.sum().reshape(1), None


class Repeticion(torch.autograd.Function):
    """Hawkes and Streak in one pass (asrn_repetition_fwd/bwd: the B n Hawkes rows and the B streak rows share the
    scans' launches): (hawkes (B, L, n), racha (B, L)), the same values and gradients as the two functions."""

    @staticmethod
    def forward(ctx, Bt, log_alfa, kappa, beta, kappa_r, order, rep, rank_k, vistos):
        dev = _dev(Bt)
        B, n, L = order.shape
        Bt = _c(Bt, torch.float64)
        la = _c(log_alfa, torch.float32)
        kap = _c(kappa, torch.float32)
        beta = _c(beta, torch.float64)
        kr = _c(kappa_r, torch.float32)
        vistos = _c(vistos, torch.float32)
        hawkes = torch.empty((B, L, n), dtype=torch.float32, device=dev)
        S = torch.empty((B, n, L), dtype=torch.float32, device=dev)
        racha = torch.empty((B, L), dtype=torch.float32, device=dev)
        wsb = query('asrn_repetition_workspace', B, L, n)
        if wsb < 0:
            raise RuntimeError(f'repetition scans of {B * (n + 1)} rows x {L}: too many chunks')
        ws = torch.empty((wsb,), dtype=torch.uint8, device=dev) if wsb else None
        call('asrn_repetition_fwd', ptr(order), ptr(rep), ptr(Bt), ptr(la), ptr(kap), ptr(vistos), ptr(beta), ptr(kr),
             B, L, n, ptr(hawkes), ptr(S), ptr(racha), ptr(ws), wsb, stream_of(dev))
        ctx.save_for_backward(Bt, la, kap, order, rep, rank_k, S, vistos, beta, kr, racha)
        return hawkes, racha

    @staticmethod
    def backward(ctx, gh, gr):
        Bt, la, kap, order, rep, rank_k, S, vistos, beta, kr, racha = ctx.saved_tensors
        B, n, L = order.shape
        dev = Bt.device
        gh = torch.zeros((B, L, n), dtype=torch.float32, device=dev) if gh is None else _c(gh, torch.float32)
        gr = torch.zeros((B, L), dtype=torch.float32, device=dev) if gr is None else _c(gr, torch.float32)
        dBt = torch.empty((B, L), dtype=torch.float64, device=dev)
        dla = torch.empty((B, L), dtype=torch.float32, device=dev)
        dk = torch.empty((B, n), dtype=torch.float32, device=dev)
        dbeta = torch.empty((B, L), dtype=torch.float64, device=dev)
        dkr = torch.empty((B,), dtype=torch.float32, device=dev)
        wsb = query('asrn_repetition_bwd_workspace', B, L, n)
        ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
        call('asrn_repetition_bwd', ptr(order), ptr(rep), ptr(rank_k), ptr(Bt), ptr(la), ptr(kap), ptr(S), ptr(gh),
             ptr(vistos), ptr(beta), ptr(kr), ptr(racha), ptr(gr), B, L, n, ptr(dBt), ptr(dla), ptr(dk), ptr(dbeta),
             ptr(dkr), ptr(ws), wsb, stream_of(dev))
        return dBt, dla, dk.sum(0), dbeta, dkr.sum().reshape(1), None, None, None, None


# ---------------------------------------------------------------------------------------------------------------------
# a13
# ---------------------------------------------------------------------------------------------------------------------

GATE_COLS = 64        # the small parameters' block of asrn_gate_bwd's dparams


def gate_step(h, salida, w_o, signals, vistos, hawkes, racha, wg, bg, wc, bc, wv, uh, dr, meta):
    """The generation step's W_o product and gate in one kernel (asrn_gate_step), no autograd: h, salida (B, d)
    fp32, w_o (d, d) -> h' = h + sigmoid(cap(logit)) W_o salida / max(1, peso_total) (B, d), as Gate.apply gives it
    from A = W_o salida. meta as for Gate."""
    T, Tc, paso, mejor_max, tope = meta
    dev = _dev(h, salida)
    B, d = h.shape
    n, nodes = vistos.shape[-1], dr.shape[0]
    ins = [_c(t, torch.float32) for t in (h, salida, w_o, signals, vistos, hawkes, racha)]
    params = [_c(p, torch.float32).reshape(-1) for p in (wg, bg, wc, bc, wv, uh, dr)]
    logit = torch.empty((B,), dtype=torch.float32, device=dev)
    out = torch.empty((B, d), dtype=torch.float32, device=dev)
    call('asrn_gate_step', *[ptr(t) for t in ins], *[ptr(p) for p in params], B, d, n, nodes, T, Tc, paso, mejor_max,
         tope, ptr(logit), ptr(out), stream_of(dev))
    return out


class Gate(torch.autograd.Function):
    """h' = h + sigmoid(cap(logit)) A / max(1, peso_total), A = W_o salida, with the logit of _combinar
    (asrn/estable.py:376-403) and the streak response (asrn/nucleo.py:865-878), fused in asrn_gate_fwd/bwd.
    meta = (T, Tc, racha_paso, mejor_max or -1, tope or 0). signals and vistos carry no gradient."""

    @staticmethod
    def forward(ctx, h, A, signals, vistos, hawkes, racha, wg, bg, wc, bc, wv, uh, dr, meta):
        T, Tc, paso, mejor_max, tope = meta
        dev = _dev(h, A)
        B, L, d = h.shape
        n, nodes = vistos.shape[-1], dr.shape[0]
        h32 = _c(h, torch.float32)
        bf = A.dtype == torch.bfloat16
        A = A.contiguous() if bf else _c(A, torch.float32)
        sig, vis, haw, ra = (_c(t, torch.float32) for t in (signals, vistos, hawkes, racha))
        params = [_c(p, torch.float32).reshape(-1) for p in (wg, bg, wc, bc, wv, uh, dr)]
        logit = torch.empty((B, L), dtype=torch.float32, device=dev)
        out = torch.empty_like(h32)
        call('asrn_gate_fwd', ptr(h32), ptr(A), int(bf), ptr(sig), ptr(vis), ptr(haw), ptr(ra),
             *[ptr(p) for p in params], B * L, d, n, nodes, T, Tc, paso, mejor_max, tope, ptr(logit), ptr(out),
             stream_of(dev))
        ctx.save_for_backward(h32, A, sig, vis, haw, ra, *params, logit)
        ctx.meta = (B, L, d, n, nodes, T, Tc, paso, mejor_max, tope, h.dtype,
                    [p.shape for p in (wg, bg, wc, bc, wv, uh, dr)])
        return out.to(torch.promote_types(h.dtype, A.dtype))

    @staticmethod
    def backward(ctx, g):
        h32, A, sig, vis, haw, ra, *rest = ctx.saved_tensors
        params, logit = rest[:7], rest[7]
        B, L, d, n, nodes, T, Tc, paso, mejor_max, tope, hdt, shapes = ctx.meta
        dev = h32.device
        g = _c(g, torch.float32)
        dh = torch.empty_like(h32)
        dA = torch.empty_like(A)
        dhaw = torch.empty_like(haw)
        dra = torch.empty_like(ra)
        dp = torch.empty((d + GATE_COLS,), dtype=torch.float32, device=dev)
        wsb = query('asrn_gate_bwd_workspace', B * L, d)
        ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
        call('asrn_gate_bwd', ptr(h32), ptr(A), int(A.dtype == torch.bfloat16), ptr(sig), ptr(vis), ptr(haw),
             ptr(ra), *[ptr(p) for p in params], B * L, d, n, nodes, T, Tc, paso, mejor_max, tope, ptr(logit),
             ptr(g), ptr(dh), ptr(dA), ptr(dhaw), ptr(dra), ptr(dp), ptr(ws), wsb, stream_of(dev))
        sizes = [d, 1, 4, 1, n, n, nodes]
        grads = [t.view(s) for t, s in zip(torch.split(dp[:sum(sizes)], sizes), shapes)]
        return (dh.to(hdt), dA, None, None, dhaw, dra, *grads, None)


# ---------------------------------------------------------------------------------------------------------------------
# a3 - a8
# ---------------------------------------------------------------------------------------------------------------------

class Candidates(torch.autograd.Function):
    """Candidate attention of all tables (the drop-in for _CasillerosTriton, asrn/nucleo.py:461-515). Returns salida
    (B, L, d) and the gate signals (B, L, 4) = (peso_total, mejor, pico, peso_ctx), the latter without gradient.
    Saves its inputs and the candidates' attention weights (B, L, T, C, 2 with room for ds), so the backward
    recomputes no score. shape['v_shift'] = 1 takes V as the value projection of every position (the kernels read
    position s + 1 for candidate s, the reference's V[s] = W_v E[s+1]); a column block of a wider fp32 GEMM output is
    read in place through its row stride."""

    @staticmethod
    def forward(ctx, phi, V, Qc, Kc, Bt, log_alfa, w_suf, gamma, sig, order, win, rank, shape):
        T, Tc, C, K = shape['T'], shape['Tc'], shape['C'], shape['K']
        dev = _dev(phi, V)
        B, L, P0 = phi.shape
        d, cf0 = V.shape[-1], Qc.shape[-1]
        sp, sc = float(P0) ** -0.5, float(cf0) ** -0.5
        # the kernels read feature rows as float4: zero columns pad P and cf to multiples of 4 (dot products and the
        # gradients of the real columns are unchanged)
        vs = int(shape.get('v_shift', 0))
        # bf16 rows (autocast) are read as they are, the kernels widening each element exactly: the value rows
        # (mode 1), and the feature rows too when phi, Qc and Kc are all bf16 with widths that need no padding (mode 2)
        bf = torch.bfloat16
        rows16 = V.dtype == bf and d % 4 == 0
        feat16 = (rows16 and phi.dtype == bf and Qc.dtype == bf and Kc.dtype == bf and P0 % 4 == 0
                  and cf0 % 4 == 0)
        if rows16:
            Vk = V if _rows_in_place(V, bf) else _c(V)
        else:
            Vk = V if _rows_in_place(V) else _c(V, torch.float32)
        ft = bf if feat16 else torch.float32
        if (_rows_in_place(Qc, ft) and _rows_in_place(Kc, ft) and Qc.stride(1) == Kc.stride(1)
                and Qc.shape[-1] % 4 == 0):
            Qk, Kk = Qc, Kc                        # column blocks of one projection, read through their row stride
        elif feat16:
            Qk, Kk = _c(Qc), _c(Kc)
        else:
            Qk, Kk = _pad4(Qc), _pad4(Kc)
        mode = 2 if feat16 else int(rows16)
        ins = dict(phi=_c(phi) if feat16 else _pad4(phi), V=Vk, Qc=Qk, Kc=Kk, sig=_c(sig, torch.float32),
                   Bt=_c(Bt, torch.float64), la=_c(log_alfa, torch.float32), w=_c(w_suf.detach(), torch.float32),
                   g=_c(gamma.detach(), torch.float32))
        P, cf = ins['phi'].shape[-1], ins['Qc'].shape[-1]
        # bf16 value rows: salida written in bf16 by the kernel (each fp32 sum rounded once, as a cast would)
        salida = torch.empty((B, L, d), dtype=bf if mode else torch.float32, device=dev)
        signals = torch.empty((B, L, 4), dtype=torch.float32, device=dev)
        ent = torch.empty((B, L, T, C, 2), dtype=torch.float32, device=dev)  # only the valid slots are written
        # each query's deduplicated candidate list, for the backward's query pass (shape['listas'] = False: none)
        listas = (torch.empty((B, L, query('asrn_candidates_record_bytes', T, C)), dtype=torch.uint8, device=dev)
                  if shape.get('listas', True) else None)
        # the core layer (shape['reloj32']): the fp32 clock's score term; shape['fuga']: a device int32 counting the
        # (query, table) pairs where the core layer's -1e9 fill would leak weight
        fuga = shape.get('fuga')
        call('asrn_candidates_fwd', ptr(ins['phi']), ptr(ins['V']), ptr(ins['Qc']), ptr(ins['Kc']), ptr(ins['sig']),
             ptr(ins['Bt']), ptr(ins['la']), ptr(ins['w']), ptr(ins['g']), ptr(order), ptr(win), ptr(rank), B, L, d,
             P, cf, K, T, Tc, C, sp, sc, Vk.stride(1), vs, Qk.stride(1), mode, ptr(salida), ptr(signals),
             ptr(ent), ptr(listas), 1 if shape.get('reloj32') else 0, ptr(fuga), stream_of(dev))
        ctx.save_for_backward(*ins.values(), order, win, rank, ent, listas)
        ctx.meta = (B, L, P, d, cf, K, T, Tc, C, sp, sc, V.dtype, phi.dtype, Qc.dtype, Kc.dtype, log_alfa.dtype,
                    P0, cf0, vs)
        ctx.mark_non_differentiable(signals)
        ctx.set_materialize_grads(False)       # no zero-filled gradient for the signals (none flows back through them)
        return salida.to(V.dtype), signals

    @staticmethod
    def backward(ctx, dsal, _dsig):
        if dsal is None:
            return (None,) * 13
        phi, V, Qc, Kc, sig, Bt, la, w, g, order, win, rank, ent, listas = ctx.saved_tensors
        B, L, P, d, cf, K, T, Tc, C, sp, sc, tv, tp, tq, tk, tl, P0, cf0, vs = ctx.meta
        dev = phi.device
        bf = torch.bfloat16
        mode = (2 if phi.dtype == bf else 1) if V.dtype == bf else 0
        if mode and dsal.dtype != bf:             # an fp32 gradient: the fp32 path throughout
            mode = 0
            V, phi = V.float(), phi.float()
            if Qc.dtype == bf:
                Qc, Kc = Qc.float(), Kc.float()
        dsal = _c(dsal) if mode else _c(dsal, torch.float32)
        dphi = torch.empty(phi.shape, dtype=torch.float32, device=dev)
        # dV takes V's layout: when V is a column block read in place, the same block of a (B, L, ldv) buffer, so the
        # producer whose output V is can take the buffer as its own output gradient without a copy
        ldv = V.stride(1)
        col = V.storage_offset() % ldv
        col = col if col + d <= ldv else 0
        dV = torch.empty((B, L, ldv), dtype=bf if mode else torch.float32, device=dev)[..., col:col + d]
        # dQc and dKc take the layout of Qc and Kc: when both are column blocks of one projection (row stride ldq),
        # the same blocks of one (B, L, ldq) buffer, which _Split2's backward hands on whole
        ldq = Qc.stride(1)
        qo, ko = Qc.storage_offset() % ldq, Kc.storage_offset() % ldq
        if Qc.data_ptr() != Kc.data_ptr() and qo + cf <= ldq and ko + cf <= ldq and (qo + cf <= ko or ko + cf <= qo):
            dq = torch.empty((B, L, ldq), dtype=torch.float32, device=dev)
            dQc, dKc = dq[..., qo:qo + cf], dq[..., ko:ko + cf]
        else:
            dQc = torch.empty((B, L, ldq), dtype=torch.float32, device=dev)[..., :cf]
            dKc = torch.empty((B, L, ldq), dtype=torch.float32, device=dev)[..., :cf]
        dBt = torch.empty_like(Bt)
        dla = torch.empty_like(la)
        partials = torch.empty((B * L, T + K + 1), dtype=torch.float32, device=dev)
        call('asrn_candidates_bwd', ptr(phi), ptr(V), ptr(Qc), ptr(Kc), ptr(sig), ptr(Bt), ptr(la), ptr(w), ptr(g),
             ptr(order), ptr(win), ptr(rank), B, L, d, P, cf, K, T, Tc, C, sp, sc, ldv, vs, Qc.stride(1), mode,
             ptr(dsal), ptr(ent), ptr(listas),
             ptr(dphi), ptr(dV), ptr(dQc), ptr(dKc), ptr(dBt), ptr(dla), ptr(partials), stream_of(dev))
        part = column_sums(partials)          # per-query partials summed over the tokens (no memset-cleared reduction)
        dgamma = part[:T]
        dw = part[T:]
        return (dphi[..., :P0].to(tp), dV.to(tv), dQc[..., :cf0].to(tq), dKc[..., :cf0].to(tk), dBt, dla.to(tl), dw,
                dgamma, None, None, None, None, None)


# ---------------------------------------------------------------------------------------------------------------------
# a14: the O(1) generation step's state
# ---------------------------------------------------------------------------------------------------------------------

def ring_build(phi_prefix, T, nb, C):
    """Rings of the positions of phi_prefix (B, n, P): rings (B*T, 2^nb, C) int32 (-1 empty) and counts (B*T, 2^nb)
    int32; the r-th position to enter a bucket sits in slot r % C (asrn/nucleo.py:1585-1607)."""
    dev = _dev(phi_prefix)
    B, n, _ = phi_prefix.shape
    rings = torch.empty((B * T, 2 ** nb, C), dtype=I32, device=dev)
    counts = torch.empty((B * T, 2 ** nb), dtype=I32, device=dev)
    if n > 0:
        _, order, ids_s, _, _ = bucket_sort(phi_prefix, T, nb, C)
    else:
        order = ids_s = None
    call('asrn_ring_build', ptr(order), ptr(ids_s), B, n, T, nb, C, ptr(rings), ptr(counts), stream_of(dev))
    return rings, counts


def _posicion(t, t_max):
    """The position for the generation entry points: (host int, device pointer). t an int: (t, None); t a one-element
    int64 device tensor (the position as a step captured in a graph reads it): (t_max, its pointer), t_max being the
    largest position it will hold, which the host checks against the capacities."""
    if torch.is_tensor(t):
        if t.dtype != torch.int64 or t.numel() != 1 or not t.is_cuda or t_max is None:
            raise ValueError('a device position is a one-element int64 cuda tensor, with t_max given')
        return int(t_max), ptr(t)
    return int(t), None


def decode_attend(cache, t, rings, counts, w_suf, gamma, shape, insert, t_max=None, hechos=None):
    """The step's candidate attention for position t of the caches (dict of (B, cap, .) tensors phi, V, Qc, Kc, sig,
    Bt, log_alfa) over the rings; with insert, t then enters the rings. Returns salida (B, d), signals (B, 4) and
    the bucket ids (B, T). t: an int, or a one-element int64 device tensor holding it (then t_max: the largest
    position it will hold). hechos: a (B,) int32 device tensor of zeros kept by the caller across calls (the launch
    leaves it zero); with it, a row's value columns are gathered by several workgroups when B leaves CUs idle."""
    T, Tc, C, K, nb = shape['T'], shape['Tc'], shape['C'], shape['K'], shape['nb']
    phi, V = cache['phi'], cache['V']
    dev = _dev(phi)
    B, cap, P = phi.shape
    d, cf = V.shape[-1], cache['Qc'].shape[-1]
    if P != T * nb:
        raise ValueError(f'phi has {P} features, expected T * nb = {T * nb}')
    salida = torch.empty((B, d), dtype=torch.float32, device=dev)
    signals = torch.empty((B, 4), dtype=torch.float32, device=dev)
    ids = torch.empty((B, T), dtype=I32, device=dev)
    w = _c(w_suf.detach(), torch.float32)
    g = _c(gamma.detach(), torch.float32)
    th, tdev = _posicion(t, t_max)
    call('asrn_decode_attend', ptr(phi), ptr(V), ptr(cache['Qc']), ptr(cache['Kc']), ptr(cache['sig']),
         ptr(cache['Bt']), ptr(cache['log_alfa']), ptr(w), ptr(g), ptr(rings), ptr(counts), B, cap, th, tdev, d, nb,
         cf, K, T, Tc, C, float(P) ** -0.5, float(cf) ** -0.5, 1 if insert else 0, ptr(salida), ptr(signals),
         ptr(ids), ptr(shape.get('fuga')), ptr(hechos), stream_of(dev))
    return salida, signals, ids


def decode_attend_repeat(cache, t, rings, counts, w_suf, gamma, shape, insert, tabla, beta_t, coef, kappa, kappa_r,
                         racha, t_max=None, reloj32=False, hechos=None):
    """decode_attend and tabla.step (the repetition step: clock, Hawkes, streak) for position t in one launch
    (asrn_decode_attend_repeat), with the same outputs, bit for bit, as the two calls in the order step, attend (with
    the same hechos, as decode_attend takes it): returns salida (B, d), signals (B, 4), the bucket ids (B, T), vistos
    and hawkes (B, n); Bt[:, t], the Hawkes tables and racha are updated in place as tabla.step does."""
    T, Tc, C, K, nb = shape['T'], shape['Tc'], shape['C'], shape['K'], shape['nb']
    phi, V = cache['phi'], cache['V']
    dev = _dev(phi)
    B, cap, P = phi.shape
    d, cf = V.shape[-1], cache['Qc'].shape[-1]
    if P != T * nb:
        raise ValueError(f'phi has {P} features, expected T * nb = {T * nb}')
    th, tdev = _posicion(t, t_max)
    tabla.reserve(th + 1)
    salida = torch.empty((B, d), dtype=torch.float32, device=dev)
    signals = torch.empty((B, 4), dtype=torch.float32, device=dev)
    ids = torch.empty((B, T), dtype=I32, device=dev)
    vistos = torch.empty((B, tabla.n), dtype=torch.float32, device=dev)
    hawkes = torch.empty((B, tabla.n), dtype=torch.float32, device=dev)
    # the converted inputs are held until the launch (a freed copy's memory could be reused by the next one)
    ins = [_c(w_suf.detach(), torch.float32), _c(gamma.detach(), torch.float32), _c(beta_t, torch.float64),
           _c(coef, torch.float64), _c(kappa.detach(), torch.float32), _c(kappa_r.detach(), torch.float32)]
    call('asrn_decode_attend_repeat', ptr(phi), ptr(V), ptr(cache['Qc']), ptr(cache['Kc']), ptr(cache['sig']),
         ptr(cache['Bt']), ptr(cache['log_alfa']), ptr(ins[0]), ptr(ins[1]), ptr(rings), ptr(counts), B, cap, th, tdev,
         d, nb, cf, K, T, Tc, C, float(P) ** -0.5, float(cf) ** -0.5, 1 if insert else 0, ptr(salida), ptr(signals),
         ptr(ids), ptr(shape.get('fuga')), ptr(ins[2]), ptr(ins[3]), ptr(ins[4]), ptr(ins[5]), tabla.n, tabla.cap,
         ptr(tabla.keys), ptr(tabla.Bu), ptr(tabla.A), ptr(racha), ptr(vistos), ptr(hawkes), 1 if reloj32 else 0,
         ptr(hechos), stream_of(dev))
    return salida, signals, ids, vistos, hawkes


def decode_produce_ok(capa, e):
    """Whether asrn_decode_produce covers this layer and input: fp32 (no autocast) and the widths it takes."""
    pal, ctx = capa.afin_palabra, capa.afin_contexto
    ps = [capa.v.weight, pal[0].weight, ctx[0].weight, pal[0].bias, ctx[0].bias, pal[2].weight, pal[2].bias,
          ctx[2].weight, ctx[2].bias, capa.ln_ctx.weight, capa.ln_ctx.bias, capa.w_reloj, capa.b_reloj, capa.cq.weight,
          capa.ck.weight]
    d = e.shape[-1]
    m, mc, cf = pal[0].out_features, ctx[0].out_features, capa.confirmar
    return (e.is_cuda and e.dtype == torch.float32 and not torch.is_autocast_enabled(e.device.type)
            and all(p.dtype == torch.float32 and p.is_cuda and p.is_contiguous() for p in ps)
            and d % 4 == 0 and d <= 1024 and 1 <= m <= 64 and 1 <= mc <= 64 and 1 <= cf <= 64
            and pal[2].out_features + ctx[2].out_features <= 256)


def embed_step(emb, pieza, texto, pos):
    """The loop step's embedding rows (asrn_embed_step): e_t = emb[pieza] and e_prev = emb[texto[:, pos - 1]], both
    (B, d) fp32; pos a one-element int64 device tensor >= 1."""
    dev = _dev(emb)
    V, d = emb.shape
    B = pieza.shape[0]
    if emb.dtype != torch.float32 or not emb.is_contiguous() or texto.dtype != torch.int64 or texto.stride(1) != 1:
        raise ValueError('embed_step: a contiguous fp32 table and an int64 text with unit column stride')
    ids = _c(pieza, torch.int64)
    e_t = torch.empty((B, d), dtype=torch.float32, device=dev)
    e_prev = torch.empty((B, d), dtype=torch.float32, device=dev)
    call('asrn_embed_step', ptr(emb), V, d, ptr(ids), ptr(texto), texto.stride(0), ptr(pos), B, ptr(e_t), ptr(e_prev),
         stream_of(dev))
    return e_t, e_prev


def decode_produce(capa, cache, e, e_prev, h, pieza, t, t_max=None):
    """The generation step's producers for the new tokens at position t (asrn_decode_produce): V[t-1], phi[t], Qc[t],
    Kc[t], log_alfa[t] and sig[t] written into the caches; returns beta (B,) fp64. t: an int, or a one-element int64
    device tensor holding it (then t_max: the largest position it will hold)."""
    dev = _dev(e)
    B, d = e.shape
    pal, ctx = capa.afin_palabra, capa.afin_contexto
    m, mc = pal[0].out_features, ctx[0].out_features
    Pw, Pc, cf = pal[2].out_features, ctx[2].out_features, capa.confirmar
    cap = cache['phi'].shape[1]
    p = capa.protecciones
    beta_max = -1.0 if p.beta_max is None else float(p.beta_max)
    la_min = -math.inf if p.log_alfa_min is None else float(p.log_alfa_min)
    beta = torch.empty((B,), dtype=torch.float64, device=dev)
    wsb = query('asrn_decode_produce_workspace', B, m, mc)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    th, tdev = _posicion(t, t_max)
    # the converted inputs are held until the launch (a freed copy's memory could be reused by the next one)
    ins = [_c(e, torch.float32), _c(e_prev, torch.float32), _c(h, torch.float32), _c(pieza, torch.int64)]
    call('asrn_decode_produce', ptr(ins[0]), ptr(ins[1]), ptr(ins[2]),
         ptr(ins[3]), B, d, ptr(capa.v.weight), ptr(pal[0].weight), ptr(ctx[0].weight),
         ptr(pal[0].bias), ptr(ctx[0].bias), ptr(pal[2].weight), ptr(pal[2].bias), ptr(ctx[2].weight),
         ptr(ctx[2].bias), m, mc, Pw, Pc, ptr(capa.ln_ctx.weight), ptr(capa.ln_ctx.bias), float(capa.ln_ctx.eps),
         ptr(capa.w_reloj), ptr(capa.b_reloj), beta_max, la_min, ptr(capa.cq.weight), ptr(capa.ck.weight), cf,
         ptr(cache['phi']), ptr(cache['V']), ptr(cache['Qc']), ptr(cache['Kc']), ptr(cache['sig']),
         ptr(cache['log_alfa']), cap, th, tdev, ptr(beta), ptr(ws), wsb, stream_of(dev))
    return beta


def _formas_productor(capa):
    pal, ctx = capa.afin_palabra, capa.afin_contexto
    return pal[0].out_features, ctx[0].out_features, pal[2].out_features, ctx[2].out_features


def decode_produce_e_ok(capas, caches, e):
    """Whether asrn_decode_produce_e takes these layers together: each one decode_produce_ok, at most 8 of them, with
    the same widths and cache capacity."""
    return (1 <= len(capas) <= 8 and all(decode_produce_ok(c, e) for c in capas)
            and len({_formas_productor(c) for c in capas}) == 1 and len({c['phi'].shape[1] for c in caches}) == 1)


def decode_produce_e(capas, caches, e, e_prev, pieza, t, t_max=None):
    """The part of the generation step's producers that acts on the new tokens' embedding rows, for every layer at
    once (asrn_decode_produce_e): V[t-1], phi[t] and sig[t] of each layer written into its caches (capas and caches
    in the same order; decode_produce_e_ok holds). t: as decode_produce's."""
    dev = _dev(e)
    B, d = e.shape
    L = len(capas)
    m, mc, Pw, Pc = _formas_productor(capas[0])
    cap = caches[0]['phi'].shape[1]
    wsb = query('asrn_decode_produce_e_workspace', L, B, m, mc)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    th, tdev = _posicion(t, t_max)
    ins = [_c(e, torch.float32), _c(e_prev, torch.float32), _c(pieza, torch.int64)]
    arr = lambda ts: (ctypes.c_void_p * L)(*[t_.data_ptr() for t_ in ts])
    pal = [c.afin_palabra for c in capas]
    ctx = [c.afin_contexto for c in capas]
    call('asrn_decode_produce_e', L, ptr(ins[0]), ptr(ins[1]), ptr(ins[2]), B, d, arr([c.v.weight for c in capas]),
         arr([p[0].weight for p in pal]), arr([x[0].weight for x in ctx]), arr([p[0].bias for p in pal]),
         arr([x[0].bias for x in ctx]), arr([p[2].weight for p in pal]), arr([p[2].bias for p in pal]),
         arr([x[2].weight for x in ctx]), arr([x[2].bias for x in ctx]), m, mc, Pw, Pc,
         arr([c_['phi'] for c_ in caches]), arr([c_['V'] for c_ in caches]), arr([c_['sig'] for c_ in caches]), cap, th,
         tdev, ptr(ws), wsb, stream_of(dev))


def decode_produce_h(capa, cache, h, t, t_max=None, previo=None):
    """The part of the generation step's producers that acts on the layer input h (asrn_decode_produce_h): Qc[t],
    Kc[t] and log_alfa[t] written into the caches; returns beta (B,) fp64. With decode_produce_e, the same bits as
    decode_produce. previo: a BloquePendiente whose output is the layer input (h is then None): it is formed here, into
    previo.out, as the block step's last kernel forms it (asrn_decode_produce_h_ex)."""
    if previo is not None:
        h = previo.out
    dev = _dev(h)
    B, d = h.shape
    cap = cache['phi'].shape[1]
    p = capa.protecciones
    beta_max = -1.0 if p.beta_max is None else float(p.beta_max)
    la_min = -math.inf if p.log_alfa_min is None else float(p.log_alfa_min)
    beta = torch.empty((B,), dtype=torch.float64, device=dev)
    th, tdev = _posicion(t, t_max)
    tail = (ptr(capa.ln_ctx.weight), ptr(capa.ln_ctx.bias), float(capa.ln_ctx.eps), ptr(capa.w_reloj),
            ptr(capa.b_reloj), beta_max, la_min, ptr(capa.cq.weight), ptr(capa.ck.weight), capa.confirmar,
            ptr(cache['Qc']), ptr(cache['Kc']), ptr(cache['log_alfa']), cap, th, tdev, ptr(beta), stream_of(dev))
    if previo is None:
        hh = _c(h, torch.float32)
        call('asrn_decode_produce_h', ptr(hh), B, d, *tail)
        return beta
    pv = previo
    call('asrn_decode_produce_h_ex', None, ptr(pv.h1), ptr(pv.b2), ptr(pv.z), ptr(pv.anillo), pv.k, pv.ff, ptr(pv.out),
         ptr(pv.pos), ptr(pv.espacio), pv.espacio.numel(), B, d, *tail)
    return beta


def _pow2_at_least(x):
    c = 1
    while c < x:
        c *= 2
    return c


class HawkesTable:
    """Per (b, j) open-addressing tables of the Hawkes memory (asrn/nucleo.py:1634-1714): keys (B*n, cap) uint64
    codes, Bu (B*n, cap) fp64, A (B*n, cap) fp32; cap a power of two kept >= 2x the keys a table can hold."""

    def __init__(self, B, n, cap, dev):
        self.B, self.n, self.cap = B, n, cap
        self.keys = torch.empty((B * n, cap), dtype=torch.int64, device=dev)   # uint64 bits
        self.Bu = torch.empty((B * n, cap), dtype=torch.float64, device=dev)
        self.A = torch.empty((B * n, cap), dtype=torch.float32, device=dev)

    @classmethod
    def load(cls, keys, order, rep, hawkes, Bt, log_alfa, cap=None):
        """The memory after a text of L: keys (B, L, n), order / rep (B, n, L) from ngram_sort, hawkes (B, L, n)."""
        dev = _dev(keys)
        B, L, n = keys.shape
        tab = cls(B, n, _pow2_at_least(max(cap or 0, 2 * L, 2)), dev)
        # the converted inputs are held until the launch (a freed copy's memory could be reused by the next one)
        ins = [_c(keys, torch.float64), _c(hawkes, torch.float32), _c(Bt, torch.float64), _c(log_alfa, torch.float32)]
        call('asrn_hawkes_table_load', ptr(ins[0]), ptr(order), ptr(rep), ptr(ins[1]), ptr(ins[2]), ptr(ins[3]), B, L,
             n, tab.cap, ptr(tab.keys), ptr(tab.Bu), ptr(tab.A), stream_of(dev))
        return tab

    def reserve(self, positions):
        """Grows (rehashes) the tables so they can hold the keys of `positions` positions."""
        if self.cap >= 2 * positions:
            return
        dev = self.keys.device
        new = HawkesTable(self.B, self.n, _pow2_at_least(2 * positions), dev)
        call('asrn_hawkes_table_grow', ptr(self.keys), ptr(self.Bu), ptr(self.A), self.B * self.n, self.cap,
             ptr(new.keys), ptr(new.Bu), ptr(new.A), new.cap, stream_of(dev))
        self.keys, self.Bu, self.A, self.cap = new.keys, new.Bu, new.A, new.cap

    def step(self, cache, t, beta_t, coef, kappa, kappa_r, racha, t_max=None, reloj32=False):
        """Position t: Bt[:, t] = Bt[:, t-1] + beta_t (written into cache['Bt']), vistos and hawkes (B, n); racha (B)
        is updated in place (asrn/nucleo.py:953-960, 1683-1714, 1826). t: an int, or a one-element int64 device
        tensor holding it (then t_max: the largest position it will hold). reloj32: the core layer's fp32 clock (the
        sum in fp32)."""
        dev = _dev(racha)
        th, tdev = _posicion(t, t_max)
        self.reserve(th + 1)
        sig, Bt, la = cache['sig'], cache['Bt'], cache['log_alfa']
        B, stride = sig.shape
        vistos = torch.empty((B, self.n), dtype=torch.float32, device=dev)
        hawkes = torch.empty((B, self.n), dtype=torch.float32, device=dev)
        # the converted inputs are held until the launch (a freed copy's memory could be reused by the next one)
        ins = [_c(beta_t, torch.float64), _c(coef, torch.float64), _c(kappa.detach(), torch.float32),
               _c(kappa_r.detach(), torch.float32)]
        call('asrn_repetition_step', ptr(sig), ptr(Bt), ptr(la), ptr(ins[0]), ptr(ins[1]), ptr(ins[2]), ptr(ins[3]),
             B, stride, th, tdev, self.n, self.cap, ptr(self.keys), ptr(self.Bu), ptr(self.A), ptr(racha),
             ptr(vistos), ptr(hawkes), 1 if reloj32 else 0, stream_of(dev))
        return vistos, hawkes


# ---------------------------------------------------------------------------------------------------------------------
# generation: n-gram sets and the device sampler
# ---------------------------------------------------------------------------------------------------------------------

def bits_por_pieza(V):
    """Bits per token id in a packed n-gram key: the smallest width whose all-ones field exceeds V - 1."""
    return int(query('asrn_sample_bits', int(V)))


class ConjuntoNgramas:
    """Per text row, a device hash set of the n-grams seen and a table of their contexts' distinct successors (the
    first asrn_ngram_set_successors() inline): the device side of the reference's _Ngramas
    (asrn/nucleo.py:1857-1889). A key packs the n token ids into 64 bits when n * bits_por_pieza(V) <= 64, and is a
    64-bit hash of them otherwise (two distinct n-grams share a key with probability 2^-64 per pair). Sized for
    `capacidad` n-grams per row (at most half the slots in use)."""

    def __init__(self, filas, n, V, capacidad, dev):
        w = bits_por_pieza(V)
        if n < 1:
            raise ValueError(f'n-gram sets need n >= 1 (got {n})')
        self.n, self.w, self.V = n, w, V
        self.cap = _pow2_at_least(max(2 * int(capacidad), 2))
        self.slots = torch.full((filas, self.cap), -1, dtype=torch.int64, device=dev)     # all ones: empty
        self.ctx = torch.full((filas, self.cap), -1, dtype=torch.int64, device=dev)
        self.count = torch.zeros((filas, self.cap), dtype=torch.int32, device=dev)
        self.succ = torch.empty((filas, self.cap, int(query('asrn_ngram_set_successors'))), dtype=torch.int32,
                                device=dev)

    def punteros(self):
        return [ptr(self.slots), ptr(self.ctx), ptr(self.count), ptr(self.succ), self.cap, self.n]

    def agregar_texto(self, x):
        """Every n-gram of the rows of x (filas, L) int64."""
        dev = _dev(x)
        if x.dim() != 2 or x.dtype != torch.int64 or x.shape[0] != self.slots.shape[0]:
            raise ValueError('agregar_texto: x is (rows, L) int64 with one row per set')
        x = x if x.stride(1) == 1 else x.contiguous()
        if x.shape[1] > self.cap // 2:
            raise ValueError(f'agregar_texto: {x.shape[1]} n-grams per row exceed the sets\' capacity')
        call('asrn_ngram_set_build', ptr(x), x.stride(0), x.shape[0], x.shape[1], self.n, self.w, ptr(self.slots),
             ptr(self.ctx), ptr(self.count), ptr(self.succ), self.cap, stream_of(dev))


def muestrear(lg, texto, pos, pos_max, L0, piezas, terminado, paso_fin, trabajo, bits_cita, temperatura, top_k,
              top_p, pena, ventana, semilla, cita=None, prohibidas=None, parar_en=None, logits=None, prob=None):
    """One token per row by asrn_sample: lg (B, V) fp32 logits (rows unit-strided), texto (B, cap) int64 (the token
    is written at position pos: a one-element int64 device tensor, at most pos_max), piezas (B,) int64 out,
    terminado (B,) uint8 and paso_fin (B,) int32 (stop flags and the step each row stopped at), trabajo (B, V) fp32 and
    bits_cita (B, ceil(V/32)) int32 scratch; cita / prohibidas: ConjuntoNgramas or None; logits: (B, steps, V) fp32
    receiving lg at step pos - L0; prob: (B, V) fp32 receiving the final probabilities."""
    dev = _dev(lg, texto, pos)
    B, V = lg.shape
    if lg.dtype != torch.float32 or lg.stride(1) != 1 or texto.dtype != torch.int64 or texto.stride(1) != 1:
        raise ValueError('muestrear: lg fp32 and texto int64, both with unit column stride')
    if pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError('muestrear: pos is a one-element int64 device tensor')
    if parar_en is not None and not 0 <= int(parar_en) < V:
        raise ValueError(f'parar_en={parar_en}: a token id in [0, {V})')
    for t, forma, tipo in ((piezas, (B,), torch.int64), (terminado, (B,), torch.uint8), (paso_fin, (B,), torch.int32),
                           (trabajo, (B, V), torch.float32), (bits_cita, (B, (V + 31) // 32), torch.int32)):
        if tuple(t.shape) != forma or t.dtype != tipo or not t.is_contiguous():
            raise ValueError(f'muestrear: a buffer must be contiguous {tipo} of shape {forma}')
    if logits is not None and (logits.dim() != 3 or logits.shape[0] != B or logits.shape[2] != V
                               or logits.dtype != torch.float32 or not logits.is_contiguous()):
        raise ValueError('muestrear: logits is a contiguous (B, steps, V) fp32 tensor')
    if prob is not None and (tuple(prob.shape) != (B, V) or prob.dtype != torch.float32 or not prob.is_contiguous()):
        raise ValueError('muestrear: prob is a contiguous (B, V) fp32 tensor')
    w = bits_por_pieza(V)
    for s in (cita, prohibidas):
        if s is not None and (s.w != w or s.slots.shape[0] != B):
            raise ValueError('muestrear: an n-gram set made for another vocabulary or batch')
    semilla = int(semilla) & 0xFFFFFFFFFFFFFFFF
    call('asrn_sample', ptr(lg), lg.stride(0), ptr(trabajo), ptr(bits_cita), ptr(prob), ptr(logits),
         logits.shape[1] if logits is not None else 0, ptr(texto), texto.stride(0), ptr(pos), int(pos_max), int(L0),
         ptr(piezas), ptr(terminado), ptr(paso_fin),
         *(cita.punteros() if cita else [None, None, None, None, 0, 0]),
         *(prohibidas.punteros() if prohibidas else [None, None, None, None, 0, 0]), w, B, V, float(temperatura), int(top_k), float(top_p), float(pena),
         int(ventana), -1 if parar_en is None else int(parar_en), ctypes.c_uint64(semilla), stream_of(dev))


# ---------------------------------------------------------------------------------------------------------------------
# the model's local block, generation step
# ---------------------------------------------------------------------------------------------------------------------

def paso_bloque_ok(blq, h):
    """Whether asrn_block_step takes this block and state: mezcla 'conv', fp32 parameters and state, no autocast,
    one LayerNorm epsilon, the block's usual feed-forward layout, d up to 4,096."""
    dev = h.device.type
    ps = [blq.ln1.weight, blq.ln1.bias, blq.conv.weight, blq.conv.bias, blq.ln2.weight, blq.ln2.bias, blq.ff[0].weight,
          blq.ff[0].bias, blq.ff[2].weight, blq.ff[2].bias]
    return (blq.mezcla == 'conv' and h.is_cuda and h.dtype == torch.float32 and h.dim() == 2 and h.stride(1) == 1
            and not torch.is_autocast_enabled(dev) and all(p is not None and p.dtype == torch.float32 for p in ps)
            and blq.ln1.eps == blq.ln2.eps and blq.conv.groups == 1 and h.shape[-1] <= 4096)


def espacio_bloque(B, d, ff, dev):
    """The workspace of paso_bloque at these sizes (the products' partial sums); one serves every block of a writer
    whose blocks share d and ff."""
    return torch.empty(int(query('asrn_block_step_workspace', B, d, ff)), dtype=torch.uint8, device=dev)


class BloquePendiente:
    """A block step whose last launch was left to the next block's first (paso_bloque(..., terminar=False)): `out` is
    the (B, d) buffer its output will be written into, and it must be passed as `previo` to the next paso_bloque call,
    with the same workspace, or to decode_produce_h, before anything reads `out` or uses the workspace."""

    def __init__(self, out, h1, b2, z, anillo, k, ff, pos=None, espacio=None):
        self.out, self.h1, self.b2, self.z, self.anillo, self.k, self.ff = out, h1, b2, z, anillo, k, ff
        self.pos, self.espacio = pos, espacio      # its position and its workspace (uint8 device tensor)


def paso_bloque(blq, h, anillo, pos, espacio, previo=None, terminar=True):
    """The block's step for rows h (B, d) at position pos (a one-element int64 device tensor): returns (B, d); the ring
    anillo (B, d, k - 1) of LayerNorm1 rows (position t at slot t mod (k - 1)) takes this position's row.
    previo: a BloquePendiente, the block just before this one, whose output is this block's input (h is then None):
    this block's first kernel finishes it (asrn_block_step_ex). terminar=False: returns this block as a
    BloquePendiente instead of its output, for the next block to finish."""
    if previo is not None:
        h = previo.out
    dev = _dev(h)
    B, d = h.shape
    k = blq.k
    ff = blq.ff[0].weight.shape[0]
    if k > 1 and (anillo is None or tuple(anillo.shape) != (B, d, k - 1) or not anillo.is_contiguous()):
        raise ValueError('paso_bloque: the ring is a contiguous (B, d, k - 1) fp32 tensor')
    ws = [_c(p.detach()) for p in (blq.ln1.weight, blq.ln1.bias, blq.conv.weight, blq.conv.bias, blq.ln2.weight,
                                   blq.ln2.bias, blq.ff[0].weight, blq.ff[0].bias, blq.ff[2].weight, blq.ff[2].bias)]
    z, h1, x2, out = (torch.empty((B, d), dtype=torch.float32, device=dev) for _ in range(4))
    x1 = torch.empty((B, d * k), dtype=torch.float32, device=dev)
    if previo is None and terminar:
        call('asrn_block_step', ptr(h), h.stride(0), ptr(anillo), ptr(pos), B, d, k, ff, *[ptr(w) for w in ws],
             float(blq.ln1.eps), ptr(z), ptr(x1), ptr(h1), ptr(x2), ptr(out), ptr(espacio), espacio.numel(),
             stream_of(dev))
        return out
    pv = previo
    call('asrn_block_step_ex', None if pv else ptr(h), h.stride(0), ptr(pv.h1) if pv else None,
         ptr(pv.b2) if pv else None, ptr(pv.z) if pv else None, ptr(pv.anillo) if pv else None, pv.k if pv else 0,
         pv.ff if pv else 0, ptr(pv.out) if pv else None, ptr(anillo), ptr(pos), B, d, k, ff, *[ptr(w) for w in ws],
         float(blq.ln1.eps), ptr(z), ptr(x1), ptr(h1), ptr(x2), ptr(out), 1 if terminar else 0, ptr(espacio),
         espacio.numel(), stream_of(dev))
    if terminar:
        return out
    return BloquePendiente(out, h1, ws[9], z, anillo, k, ff, pos, espacio)


def norma_pendiente_ok(ln, d, dev):
    """Whether norma_pendiente takes this LayerNorm after blocks of width d on the GPU dev: fp32 affine weights of
    that width on a GPU, outside autocast."""
    return (isinstance(ln, torch.nn.LayerNorm) and ln.elementwise_affine and ln.bias is not None
            and ln.weight.dtype == torch.float32 and ln.weight.is_cuda and torch.device(dev).type == 'cuda'
            and tuple(ln.normalized_shape) == (d,) and d <= 4096 and not torch.is_autocast_enabled('cuda'))


def norma_pendiente(ln, previo, avance=None):
    """ln(previo's output) for a BloquePendiente, its output formed first (into previo.out, its ring row too) as the
    block step's last kernel forms it, in one launch (asrn_block_finish_norm): the last block's end and the final
    norm of the generation step (asrn/nucleo.py:1854). The norm is the row kernels' two-pass LayerNorm (biased
    variance). avance: (pos, count), previo's position tensor and a one-element int32 device tensor of 0 kept across
    calls: the same launch then advances pos by one once every workgroup has used it."""
    pv = previo
    B, d = pv.out.shape
    y = torch.empty((B, d), dtype=torch.float32, device=pv.out.device)
    call('asrn_block_finish_norm', ptr(pv.h1), ptr(pv.b2), ptr(pv.z), ptr(pv.anillo), pv.k, pv.ff, ptr(pv.out),
         ptr(pv.pos), B, d, ptr(_c(ln.weight.detach())), ptr(_c(ln.bias.detach())), float(ln.eps), ptr(y),
         ptr(pv.espacio), pv.espacio.numel(), ptr(avance[0]) if avance else None, ptr(avance[1]) if avance else None,
         stream_of(pv.out.device))
    return y


# ---------------------------------------------------------------------------------------------------------------------
# the model's loss
# ---------------------------------------------------------------------------------------------------------------------

class CrossEntropy(torch.autograd.Function):
    """F.cross_entropy(logits.float().reshape(-1, V), target.reshape(-1), ignore_index, reduction) for 'mean' and
    'sum' (asrn/nucleo.py:1108): asrn_cross_entropy_fwd/bwd compute it in fp32 from fp32 or bf16 logits as they are
    (no fp32 copy), and the gradient comes back in the logits' dtype. The rows are reduced here: the mean divides the
    summed row losses by the count of rows not ignored (NaN when there is none, as PyTorch gives)."""

    @staticmethod
    def forward(ctx, logits, target, ignore_index, reduction):
        dev = _dev(logits)
        V = logits.shape[-1]
        x = logits.reshape(-1, V)
        if x.dtype not in (torch.float32, torch.bfloat16):
            x = x.float()
        bf16 = x.dtype == torch.bfloat16
        step = 8 if bf16 else 4                      # elements per 16 bytes: rows must start 16-byte aligned
        if x.stride(-1) != 1 or x.stride(0) % step or x.data_ptr() % 16:
            if V % step:
                xp = torch.empty((x.shape[0], V + (-V % step)), dtype=x.dtype, device=dev)
                xp[:, :V] = x
                x = xp[:, :V]
            else:
                x = x.contiguous()
        rows, ld = x.shape[0], x.stride(0)
        t = target.reshape(-1).to(torch.int64).contiguous()
        if t.numel() != rows:
            raise ValueError(f'cross_entropy: {rows} rows of logits against {t.numel()} targets')
        lse = torch.empty((rows,), dtype=torch.float32, device=dev)
        per = torch.empty((rows,), dtype=torch.float32, device=dev)
        call('asrn_cross_entropy_fwd', ptr(x), int(bf16), ld, ptr(t), rows, V, int(ignore_index), ptr(lse), ptr(per),
             stream_of(dev))
        total = per.sum()
        if reduction == 'mean':
            count = (t != ignore_index).sum().to(torch.float32)
            out = total / count
        else:
            count = None
            out = total
        ctx.save_for_backward(x, t, lse, count if count is not None else total)
        ctx.meta = (int(ignore_index), reduction, logits.shape, logits.dtype, bf16)
        return out

    @staticmethod
    def backward(ctx, g):
        x, t, lse, count = ctx.saved_tensors
        ignore_index, reduction, shape, dtype, bf16 = ctx.meta
        rows, V = x.shape
        dev = x.device
        scale = (g.float() / count) if reduction == 'mean' else g.float().reshape(())
        scale = scale.reshape(1).contiguous()
        ld = V + (-V % (8 if bf16 else 4))
        dx = torch.empty((rows, ld), dtype=x.dtype, device=dev)
        call('asrn_cross_entropy_bwd', ptr(x), int(bf16), x.stride(0), ptr(t), ptr(lse), rows, V, ignore_index,
             ptr(scale), ptr(dx), ld, stream_of(dev))
        return dx[:, :V].reshape(shape).to(dtype), None, None, None


def cross_entropy(logits, target, ignore_index=-100, reduction='mean'):
    """The model's loss on the GPU (CrossEntropy); 'none' and CPU tensors take F.cross_entropy on the fp32 logits."""
    if logits.is_cuda and reduction in ('mean', 'sum'):
        return CrossEntropy.apply(logits, target, ignore_index, reduction)
    return torch.nn.functional.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), target.reshape(-1),
                                             ignore_index=ignore_index, reduction=reduction)


# ---------------------------------------------------------------------------------------------------------------------
# the local block's convolution window
# ---------------------------------------------------------------------------------------------------------------------

class VentanaCausal(torch.autograd.Function):
    """The columns of a 'conv' local block's causal convolution, cols[b, t, c k + j] = z[b, t + j - (k - 1), c] (zeros
    before a row's start): what pad + unfold + reshape build (asrn/nucleo.py:969-1014), written by asrn_conv_window_fwd
    straight in the dtype the GEMM takes (bf16 under autocast: the same rounding as the cast); the backward folds the
    columns' gradient back (asrn_conv_window_bwd) into an fp32 z gradient. z fp32 (B, L, d)."""

    @staticmethod
    def forward(ctx, z, k, dtype):
        dev = _dev(z)
        B, L, d = z.shape
        zc = z if z.stride(-1) == 1 and z.stride(0) == L * z.stride(1) else z.contiguous()
        cols = torch.empty((B, L, d * k), dtype=dtype, device=dev)
        call('asrn_conv_window_fwd', ptr(zc), zc.stride(1), B, L, d, k, int(dtype == torch.bfloat16), ptr(cols),
             stream_of(dev))
        ctx.meta = (B, L, d, k)
        return cols

    @staticmethod
    def backward(ctx, dcols):
        B, L, d, k = ctx.meta
        dev = dcols.device
        bf16 = dcols.dtype == torch.bfloat16
        dc = _c(dcols) if bf16 else _c(dcols, torch.float32)
        dz = torch.empty((B, L, d), dtype=torch.float32, device=dev)
        call('asrn_conv_window_bwd', ptr(dc), int(bf16), B, L, d, k, ptr(dz), d, stream_of(dev))
        return dz, None, None


def ventana_causal(z, k, dtype):
    return VentanaCausal.apply(z, k, dtype)


class NormaResidual(torch.autograd.Function):
    """A local block's or the model's LayerNorm (asrn/nucleo.py:969-1014, 1047-1125) as torch.nn.LayerNorm computes it
    in fp32, written by asrn_layer_norm_fwd straight in the dtype the next product takes (bf16 under autocast: the same
    rounding as the cast), with (mean, rstd) kept per row. The second output is x itself (fp32, an alias) for the
    residual path: its gradient is added to dx inside asrn_layer_norm_bwd, so autograd adds nothing. x fp32
    (..., d), d a multiple of 4 and at most 1024."""

    @staticmethod
    def forward(ctx, x, gamma, beta, eps, dtype):
        dev = _dev(x)
        d, lead = x.shape[-1], x.shape[:-1]
        x2 = _c(x, torch.float32).reshape(-1, d)
        rows = x2.shape[0]
        g, b = _c(gamma, torch.float32), _c(beta, torch.float32)
        y = torch.empty((rows, d), dtype=dtype, device=dev)
        stats = torch.empty((rows, 2), dtype=torch.float32, device=dev)
        call('asrn_layer_norm_fwd', ptr(x2), d, ptr(g), ptr(b), rows, d, float(eps), int(dtype == torch.bfloat16),
             ptr(y), d, ptr(stats), stream_of(dev))
        ctx.save_for_backward(x2, g, stats)
        ctx.meta = (x.dtype, lead, gamma.shape, beta.shape)
        return y.view(*lead, d), x2.view(*lead, d)

    @staticmethod
    def backward(ctx, dy, dres):
        x2, g, stats = ctx.saved_tensors
        xdt, lead, gshape, bshape = ctx.meta
        rows, d = x2.shape
        dev = x2.device
        if dy is None:
            dy = torch.zeros((rows, d), dtype=torch.float32, device=dev)
        bf16 = dy.dtype == torch.bfloat16
        dyc = (_c(dy) if bf16 else _c(dy, torch.float32)).reshape(rows, d)
        dr = None if dres is None else _c(dres, torch.float32).reshape(rows, d)
        dx = torch.empty_like(x2)
        dp = torch.empty((2 * d,), dtype=torch.float32, device=dev)
        wsb = query('asrn_layer_norm_bwd_workspace', rows, d)
        ws = torch.empty((wsb,), dtype=torch.uint8, device=dev)
        call('asrn_layer_norm_bwd', ptr(x2), d, ptr(g), ptr(stats), rows, d, ptr(dyc), int(bf16), d, ptr(dr), ptr(dx),
             ptr(dp), ptr(ws), wsb, stream_of(dev))
        return dx.view(*lead, d).to(xdt), dp[:d].view(gshape), dp[d:].view(bshape), None, None


def norma_residual(ln, x, dtype):
    """(LayerNorm ln of x in `dtype`, x for the residual path): the library's fused LayerNorm for fp32 x on the GPU
    with d a multiple of 4 up to 1024, else ln(x) (cast to dtype) and x itself."""
    d = x.shape[-1]
    if x.is_cuda and x.dtype == torch.float32 and dtype in (torch.float32, torch.bfloat16) and d % 4 == 0 and \
            d <= 1024 and ln.elementwise_affine and ln.bias is not None and tuple(ln.normalized_shape) == (d,):
        return NormaResidual.apply(x, ln.weight, ln.bias, ln.eps, dtype)
    y = ln(x)
    return (y if y.dtype == dtype else y.to(dtype)), x
