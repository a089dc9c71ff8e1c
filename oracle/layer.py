"""CPU restatement of the reference's stable ASRN layer, stage by stage -- TEST INFRASTRUCTURE ONLY.

Follows asrn/estable.py (CapaASRNEstable with group-A protections, the layer behind asrn.ASRNLayer) and the helpers
of asrn/nucleo.py it inherits. Floating-point stages run in torch on the CPU so autograd supplies the backward;
integer stages (bucket ids, stable sorts, n-gram keys) run in numpy. Nothing here is used by the product path.

Parameters are passed as a plain dict of tensors keyed by the reference's state_dict names (nucleo:591-630).
"""
import dataclasses
import math

import numpy as np
import torch
import torch.nn.functional as F

PROHIBIDO = -1e9          # nucleo:86 (the fp32 "not allowed" score; nucleo:89-91 keeps it for fp32)


@dataclasses.dataclass(frozen=True)
class Shape:
    """Layer hyper-parameters (nucleo:585-586 defaults). P = T*nb, temperatura = sqrt(P) (nucleo:599)."""
    d: int
    T: int = 8
    nb: int = 14
    C: int = 32
    Tc: int = 4
    cf: int = 16
    K: int = 4
    n: int = 4
    nodos: int = 16
    racha_max: int = 256

    @property
    def P(self):
        return self.T * self.nb

    @property
    def racha_paso(self):
        return math.log1p(self.racha_max) / (self.nodos - 1)        # nucleo:629


@dataclasses.dataclass(frozen=True)
class Prot:
    """Group-A protections (estable:57-66) plus the optional group-B ones. ninguna(): none of them, the core layer's
    v89 numerics (estable:68-71; nucleo.CapaASRN computes the same, asrn/__init__.py:84)."""
    beta_max: float = 1e4
    log_alfa_min: float = -30.0
    mejor_max: float = 1e4
    tope_puerta: float = None
    kappa_min: float = None
    mascara_exacta: bool = True
    reloj_64: bool = True

    @classmethod
    def ninguna(cls):
        return cls(beta_max=None, log_alfa_min=None, mejor_max=None, mascara_exacta=False, reloj_64=False)


def shape_from_params(p, d, **kw):
    """Reads T, nb, Tc, cf, K, n and the streak nodes from the parameter shapes (nucleo:591-630)."""
    Tw_nb = p['afin_palabra.2.weight'].shape[0]
    Tc_nb = p['afin_contexto.2.weight'].shape[0]
    nb = kw.pop('n_bits', 14)             # not recoverable from the shapes alone (T*nb is): the reference default
    T = (Tw_nb + Tc_nb) // nb
    return Shape(d=d, T=T, nb=nb, Tc=Tc_nb // nb, cf=p['cq.weight'].shape[0], K=p['w_sufijo'].shape[0] - 1,
                 n=p['w_vistos'].shape[0], nodos=p['d_racha'].shape[0], **kw)


# ----------------------------------------------------------------------------------------------------------------
# small pieces
# ----------------------------------------------------------------------------------------------------------------

def firmas(x):
    """Signature of each token = its id in fp32 (nucleo:161-164)."""
    return x.to(torch.float32)


def previous(sig, n, start=1):
    """(B, L, n): out[t, j] = sig[t - start - j], NaN before the text starts (nucleo:167-172)."""
    B, L = sig.shape
    out = torch.full((B, L, n), float('nan'), dtype=sig.dtype)
    for j in range(n):
        s = start + j
        if s < L:
            out[:, s:, j] = sig[:, :L - s]
    return out


def suffix_len(a, b):
    """Leading run of equal entries of a and b over the last axis (nucleo:98-108); NaN never matches."""
    eq = (a == b)
    return eq.to(torch.int64).cumprod(-1).sum(-1)


# ----------------------------------------------------------------------------------------------------------------
# producers (they stay PyTorch GEMMs in the product as well)
# ----------------------------------------------------------------------------------------------------------------

def _autocast(x):
    """x in autocast's 16-bit type when CPU autocast is on, else x (nucleo:565-571)."""
    if torch.is_autocast_enabled('cpu') and x.is_floating_point():
        return x.to(torch.get_autocast_dtype('cpu'))
    return x


def phi_and_values(p, E):
    """phi (B, L, P) = [word hash(E_t) ; context hash(E_t, E_{t-1})] and V[t] = W_v E[t+1] with V[L-1] = 0.
    The first word-hash layer and W_v share one GEMM, as in nucleo:644-659; under autocast E is converted once and
    the key [E_t; E_{t-1}] is built from the 16-bit E (nucleo:653)."""
    E = _autocast(E)
    B, L, d = E.shape
    W0, b0 = p['afin_palabra.0.weight'], p['afin_palabra.0.bias']
    m = W0.shape[0]
    y = F.linear(E, torch.cat([W0, p['v.weight']]), F.pad(b0, (0, d)))
    hp, v = y.split([m, d], dim=-1)
    word = F.linear(F.gelu(hp), p['afin_palabra.2.weight'], p['afin_palabra.2.bias'])
    key = torch.cat([E, F.pad(E, (0, 0, 1, 0))[:, :L]], dim=-1)
    ctx = F.linear(F.gelu(F.linear(key, p['afin_contexto.0.weight'], p['afin_contexto.0.bias'])),
                   p['afin_contexto.2.weight'], p['afin_contexto.2.bias'])
    return torch.cat([word, ctx], dim=-1), F.pad(v, (0, 0, 0, 1))[:, 1:]


def context(p, h, sh, prot):
    """Qc, Kc (B, L, cf), beta (B, L) fp64 (fp32 without reloj_64), log_alfa (B, L) fp32 (estable:153-194, its CPU
    branches). Without autocast: one GEMM for cq, ck and the clock projection (estable:181-185). Under autocast: Qc, Kc
    from the 16-bit LayerNorm output, the clock projection apart in fp32 with autocast off (estable:176-180); without
    reloj_64 the one GEMM in 16 bits, the clock projection rounded to 16 bits too (estable:181-185, nucleo:702-706)."""
    cf = sh.cf
    hh32 = F.layer_norm(h, (h.shape[-1],), p['ln_ctx.weight'], p['ln_ctx.bias'])
    hh = _autocast(hh32)
    if hh.dtype != hh32.dtype and prot.reloj_64:
        y = F.linear(hh, torch.cat([p['cq.weight'], p['ck.weight']]))
        with torch.autocast(device_type='cpu', enabled=False):
            u = F.linear(hh32.float(), p['w_reloj'].float(), p['b_reloj'].float())
        return _clock(y, u, cf, prot)
    y = F.linear(hh, torch.cat([p['cq.weight'], p['ck.weight'], p['w_reloj']]), F.pad(p['b_reloj'], (2 * cf, 0)))
    return _clock(y, y[..., 2 * cf:].float(), cf, prot)


def _clock(y, u, cf, prot):
    """beta = min(softplus(u_0), beta_max) and log_alfa = max(logsigmoid(u_1) + log 2, min) (estable:186-193); beta
    in fp64 with reloj_64, else fp32 (its cumsum then gives the fp32 clock)."""
    beta = F.softplus(u[..., 0])
    log_alfa = F.logsigmoid(u[..., 1]) + math.log(2)
    if prot.beta_max is not None:
        beta = beta.clamp(max=prot.beta_max)
    if prot.log_alfa_min is not None:
        log_alfa = log_alfa.clamp(min=prot.log_alfa_min)
    return y[..., :cf], y[..., cf:2 * cf], (beta.double() if prot.reloj_64 else beta), log_alfa


# ----------------------------------------------------------------------------------------------------------------
# a1-a2: sign hash and stable bucket sort
# ----------------------------------------------------------------------------------------------------------------

def bucket_ids(phi, T, nb):
    """(B, L, T) int32: id = sum_j 2^j [phi[.., tau*nb + j] > 0] (nucleo:661-664)."""
    bits = (phi.detach().reshape(*phi.shape[:-1], T, nb) > 0).numpy().astype(np.int64)
    return torch.from_numpy((bits << np.arange(nb)).sum(-1).astype(np.int32))


def stable_argsort_rows(keys):
    """Stable argsort of each row (torch.argsort(stable=True) semantics: NaN last, ties in index order), int64."""
    return torch.from_numpy(np.argsort(keys.numpy(), axis=-1, kind='stable').astype(np.int64))


def bucket_rows(phi, T, nb):
    """ids as rows r = b*T + tau (B*T, L) and their stable order (estable:282-283)."""
    B, L, _ = phi.shape
    ids = bucket_ids(phi, T, nb).transpose(1, 2).reshape(B * T, L).contiguous()
    return ids, stable_argsort_rows(ids)


def candidate_lists_bruteforce(ids_rows, C):
    """For each row and text position t: the <= C most recent earlier positions with the same bucket, oldest first.
    The definition the sorted-window band (nucleo:809-812) and the rings (tn:143-157) both realise."""
    R, L = ids_rows.shape
    out = []
    for r in range(R):
        row = ids_rows[r].tolist()
        seen = {}
        lists = []
        for t, k in enumerate(row):
            prev = seen.setdefault(k, [])
            lists.append(prev[-C:] if C > 0 else [])
            prev.append(t)
        out.append(lists)
    return out


# ----------------------------------------------------------------------------------------------------------------
# a3-a8: candidate attention (forward; autograd gives the backward)
# ----------------------------------------------------------------------------------------------------------------

def candidates(phi, V, Qc, Kc, Bt, log_alfa, sig, w_suf, gamma, sh, prot=None):
    """Candidate attention of all tables in bucket-sorted space (estable:204-272, group A: exact mask and the fp64
    clock difference of _TiempoRelativo estable:101-118). Without reloj_64 the clock term is formed as
    (log alfa_k + rate B_k) - rate B_q in the clock's own (fp32) type (estable:266-267, nucleo:815-817); without
    mascara_exacta the invalid keys of the window score -1e9 and the softmax runs over the whole window, so they take
    weight when every valid score sinks toward -1e9 (estable:121-133, nucleo:819-823).

    Each row (b, tau) is stably sorted by bucket, prefixed by one block of C empty slots and cut into blocks of C. A
    query at sorted rank s scores the keys of its own block and of the block before; a key is valid when it has the
    same bucket, is a real position and its rank lies in [s - C, s). Returns salida (B, L, d) summed over tables and
    the per-table signals (B, T, L, 3) = (hay, valid max score, max weight)."""
    B, L, P = phi.shape
    d = V.shape[-1]
    T, C, cf, K = sh.T, sh.C, sh.cf, sh.K
    ids, order = bucket_rows(phi, T, sh.nb)
    nblk = -(-L // C)
    R = nblk + 1
    S = R * C
    BT = B * T
    null = B * L
    base = (torch.arange(B).repeat_interleave(T) * L).unsqueeze(1)
    src = torch.full((BT, S), null, dtype=torch.int64)
    src[:, C:C + L] = order + base
    real = src != null
    ids_s = torch.full((BT, S), -1, dtype=torch.int64)
    ids_s[:, C:C + L] = torch.gather(ids.long(), 1, order)

    def srt(x):
        k = x.shape[-1]
        flat = torch.cat([x.reshape(null, k), x.new_zeros(1, k)])
        return flat.index_select(0, src.reshape(-1)).view(BT, R, C, k)

    def qk(xs):           # (BT, R, C, k) -> queries (BT, R-1, C, k), keys (BT, R-1, 2C, k)
        return xs[:, 1:], torch.cat([xs[:, :-1], xs[:, 1:]], dim=2)

    flatq = lambda t: t.reshape(BT * (R - 1), t.shape[2], t.shape[3])
    phq, phk = qk(srt(phi))
    qcq, _ = qk(srt(Qc))
    _, kck = qk(srt(Kc))
    pfq, pfk = qk(srt(previous(sig, K)))
    vq, vk = qk(srt(V))
    Bq, Bk = qk(srt(Bt.unsqueeze(-1)))
    _, lak = qk(srt(log_alfa.unsqueeze(-1)))

    sc = torch.bmm(flatq(phq), flatq(phk).transpose(1, 2)) / math.sqrt(P)
    sc = sc + torch.bmm(flatq(qcq), flatq(kck).transpose(1, 2)) * cf ** -0.5
    ell = suffix_len(flatq(pfq).unsqueeze(2), flatq(pfk).unsqueeze(1))            # (W, C, 2C)
    sc = sc + w_suf[ell]
    rate = (gamma / C).repeat(B).view(BT, 1, 1, 1).expand(BT, R - 1, 1, 1).reshape(-1, 1, 1)
    if prot is None or prot.reloj_64:
        dt = (flatq(Bk).squeeze(-1).unsqueeze(1) - flatq(Bq).squeeze(-1).unsqueeze(2)).to(torch.float32)
        sc = sc + flatq(lak).squeeze(-1).unsqueeze(1) + dt * rate
    else:
        # formed on each sorted row before it is cut into windows, as the reference does (estable:266-267): the two
        # large sums that make d gamma (sum ds B_k - sum ds B_q) then accumulate in the reference's order
        rate_row = (gamma / C).repeat(B).unsqueeze(1)                            # (BT, 1)
        B_row = srt(Bt.unsqueeze(-1)).reshape(BT, S)
        la_row = srt(log_alfa.unsqueeze(-1)).reshape(BT, S)
        _, keyk = qk((la_row + rate_row * B_row).view(BT, R, C, 1))
        qq, _ = qk((rate_row * B_row).view(BT, R, C, 1))
        sc = sc + flatq(keyk).squeeze(-1).unsqueeze(1) - flatq(qq).squeeze(-1).unsqueeze(2)

    ii = torch.arange(C).unsqueeze(1)
    jj = torch.arange(2 * C)
    band = (jj >= ii) & (jj < C + ii)
    idq, idk = qk(ids_s.view(BT, R, C, 1))
    _, rk = qk(real.view(BT, R, C, 1))
    valid = (flatq(idq).squeeze(-1).unsqueeze(2) == flatq(idk).squeeze(-1).unsqueeze(1)) \
        & flatq(rk).squeeze(-1).unsqueeze(1) & band
    hay = valid.any(-1, keepdim=True)
    att, mx = masked_softmax(sc, valid, hay, prot)
    out = torch.bmm(att, flatq(vk))                                              # (W, C, d)

    # back to text order, summed over the tables (the forward of _DesordenarSumar, nucleo:116-133)
    rank = torch.empty_like(order).scatter_(1, order, torch.arange(L).expand(BT, L))
    row_of = (rank + torch.arange(BT).unsqueeze(1) * ((R - 1) * C)).reshape(-1)   # row in (BT*(R-1)*C, d)
    salida = out.reshape(-1, d).index_select(0, row_of).view(B, T, L, d).sum(1)
    sen = torch.cat([hay.float(), torch.where(hay, mx, torch.full_like(mx, PROHIBIDO)).float(),
                     att.detach().amax(-1, keepdim=True).float()], dim=-1)
    sen = sen.reshape(-1, 3).index_select(0, row_of).view(B, T, L, 3)
    return salida, sen


def masked_softmax(sc, valid, hay, prot):
    """(att, the per-row max score) over the last dimension (estable:121-138). Exact mask: the max over the valid
    scores is subtracted first and invalid keys weigh exactly 0. Without mascara_exacta (v89): invalid keys score
    -1e9 and the softmax and the max run over every key."""
    if prot is None or prot.mascara_exacta:
        mx = sc.detach().masked_fill(~valid, float('-inf')).amax(-1, keepdim=True)
        ref = torch.where(hay, mx, torch.zeros_like(mx))
        return torch.softmax((sc - ref).masked_fill(~valid, PROHIBIDO), dim=-1) * hay, mx
    scm = sc.masked_fill(~valid, max(PROHIBIDO, torch.finfo(sc.dtype).min))
    return torch.softmax(scm, dim=-1) * hay, scm.detach().amax(-1, keepdim=True)


def candidates_at(phi, V, Qc, Kc, Bt, log_alfa, sig, w_suf, gamma, sh, ids, queries, prot=None):
    """The candidate attention of selected queries only, one query at a time (estable:204-272 restated per query, for
    shapes where the sorted-window form above would not fit in memory). ids (B, L, T): the bucket ids; queries
    (nq, 2) int64: (b, t) pairs. A query's candidates in table tau are the <= C most recent earlier positions with
    its bucket (the set the sorted window nucleo:809-812 keeps), found from a stable sort of each (b, tau) row.
    Returns salida (nq, d) summed over tables and the per-table signals (nq, T, 3) = (hay, valid max, max weight);
    autograd reaches every input through the gathers. prot: as in candidates(), except that the C candidates are the
    whole window here, so v89's fill leaks only into empty slots (the block window's other keys are not formed)."""
    B, L, P = phi.shape
    T, C, cf, K = sh.T, sh.C, sh.cf, sh.K
    ids = np.asarray(ids)
    qb, qt = queries[:, 0].numpy(), queries[:, 1].numpy()
    nq = len(qb)
    pos = np.zeros((nq, T, C), dtype=np.int64)
    valid = np.zeros((nq, T, C), dtype=bool)
    for b in np.unique(qb):
        sel = np.nonzero(qb == b)[0]
        for tau in range(T):
            row = ids[b, :, tau]
            order = np.argsort(row, kind='stable')
            rank = np.empty(L, dtype=np.int64)
            rank[order] = np.arange(L)
            s = rank[qt[sel]]
            idx = s[:, None] - np.arange(1, C + 1)[None, :]              # the C sorted ranks before the query's
            ok = (idx >= 0) & (row[order[np.clip(idx, 0, L - 1)]] == row[qt[sel]][:, None])
            pos[sel, tau] = np.where(ok, order[np.clip(idx, 0, L - 1)], 0)
            valid[sel, tau] = ok
    bq = torch.from_numpy(qb)
    tq = torch.from_numpy(qt)
    pk = torch.from_numpy(pos)
    vk = torch.from_numpy(valid)
    bk = bq.view(nq, 1, 1).expand_as(pk)
    Pf = previous(sig, K)
    sc = (phi[bq, tq].unsqueeze(1).unsqueeze(1) * phi[bk, pk]).sum(-1) / math.sqrt(P)
    sc = sc + (Qc[bq, tq].unsqueeze(1).unsqueeze(1) * Kc[bk, pk]).sum(-1) * cf ** -0.5
    ell = suffix_len(Pf[bq, tq].unsqueeze(1).unsqueeze(1), Pf[bk, pk])
    sc = sc + w_suf[ell]
    rate = (gamma / C).view(1, T, 1)
    if prot is None or prot.reloj_64:
        dt = (Bt[bk, pk] - Bt[bq, tq].view(nq, 1, 1)).to(torch.float32)
        sc = sc + log_alfa[bk, pk] + dt * rate
    else:
        sc = sc + (log_alfa[bk, pk] + rate * Bt[bk, pk]) - rate * Bt[bq, tq].view(nq, 1, 1)
    hay = vk.any(-1, keepdim=True)
    att, mx = masked_softmax(sc, vk, hay, prot)
    salida = (att.unsqueeze(-1) * V[bk, pk]).sum(2).sum(1)
    sen = torch.cat([hay.float(), torch.where(hay, mx, torch.full_like(mx, PROHIBIDO)).float(),
                     att.detach().amax(-1, keepdim=True).float()], dim=-1)
    return salida, sen


def gate_signals(salida, sen, T, Tc):
    """(hay, max, peak) per table -> the gate inputs (estable:294-300)."""
    hay_t, sc_max, pico_t = sen[..., 0:1], sen[..., 1:2], sen[..., 2:3]
    mejor = torch.where(hay_t > 0, sc_max, torch.full_like(sc_max, PROHIBIDO)).amax(1).clamp(min=PROHIBIDO)
    return {'salida': salida, 'peso_total': hay_t.sum(1), 'mejor': mejor,
            'pico': (pico_t * hay_t).sum(1), 'peso_ctx': hay_t[:, T - Tc:].sum(1)}


# ----------------------------------------------------------------------------------------------------------------
# a10: n-gram keys and their stable sort
# ----------------------------------------------------------------------------------------------------------------

def ngram_keys(sig, c, n):
    """(B, L, n) fp64 keys of the 1..n-grams ending at each position (nucleo:175-185): k_j = (((0 + s_t c_0) +
    s_{t-1} c_1) + ...), each multiply and add rounded separately (numpy ufuncs never contract to FMA); NaN when
    the group starts before the text."""
    s = sig.double().numpy()
    c = c.double().numpy()
    B, L = s.shape
    prev = np.full((B, L, n), np.nan)
    for j in range(n):
        if j < L:
            prev[:, j:, j] = s[:, :L - j]
    key = np.zeros((B, L))
    keys = []
    for j in range(n):
        key = key + prev[..., j] * c[j]
        keys.append(key)
    return torch.from_numpy(np.stack(keys, -1))


def ngram_sort(keys):
    """keys (B, L, n) -> order (B, n, L) stable by key (NaN last) and repeated (B, n, L) bool in that order:
    repeated[i] = key[i] == key[i-1] (nucleo:693-701)."""
    k = keys.transpose(1, 2).contiguous()
    order = stable_argsort_rows(k.reshape(-1, k.shape[-1])).view(k.shape)
    ks = torch.gather(k, -1, order)
    rep = torch.zeros(k.shape, dtype=torch.bool)
    rep[..., 1:] = ks[..., 1:] == ks[..., :-1]
    return order, rep


# ----------------------------------------------------------------------------------------------------------------
# a11-a12: scans
# ----------------------------------------------------------------------------------------------------------------

class _SeqScan(torch.autograd.Function):
    """S_i = a_i S_{i-1} + b_i (S_{-1} = 0) over the last axis, as a plain sequential loop in fp32; the backward is
    the reverse recurrence l_i = g_i + a_{i+1} l_{i+1}, dL/db = l, dL/da_i = l_i S_{i-1} (nucleo:188-196, 518-537)."""

    @staticmethod
    def forward(ctx, a, b):
        an, bn = a.detach().float().numpy(), b.detach().float().numpy()
        S = np.empty_like(bn)
        acc = np.zeros(bn.shape[:-1], dtype=np.float32)
        for i in range(bn.shape[-1]):
            acc = an[..., i] * acc + bn[..., i]
            S[..., i] = acc
        S = torch.from_numpy(S)
        ctx.save_for_backward(a, S)
        return S

    @staticmethod
    def backward(ctx, g):
        a, S = ctx.saved_tensors
        an, gn, Sn = a.detach().float().numpy(), g.float().numpy(), S.numpy()
        lam = np.empty_like(gn)
        acc = np.zeros(gn.shape[:-1], dtype=np.float32)
        N = gn.shape[-1]
        for i in range(N - 1, -1, -1):
            nxt = an[..., i + 1] if i + 1 < N else np.zeros_like(acc)
            acc = gn[..., i] + nxt * acc
            lam[..., i] = acc
        ga = lam * np.concatenate([np.zeros_like(Sn[..., :1]), Sn[..., :-1]], -1)
        return torch.from_numpy(ga), torch.from_numpy(lam)


def scan(a, b):
    a, b = torch.broadcast_tensors(a, b)
    return _SeqScan.apply(a.contiguous(), b.contiguous())


def kappas(p, prot):
    """Hawkes rates (n,) and the streak rate (1,) with the optional floor (estable:196-200)."""
    k, kr = p['log_kappa'].exp(), p['log_kappa_racha'].exp()
    if prot.kappa_min is not None:
        k, kr = k.clamp(min=prot.kappa_min), kr.clamp(min=prot.kappa_min)
    return k, kr


def repetition(p, sig, beta, Bt, log_alfa, sh, prot):
    """vistos (B, L, n), hawkes (B, L, n), racha (B, L) (estable:304-321). In key order the previous occurrence of
    the same key sits right before; a_i = repeated_i exp(-kappa dB_i) with dB the fp64 clock step clamped at 0,
    lambda = scan(a, a * alfa_{i-1}); the streak is scan(r exp(-kappa_r beta), r) over the text."""
    n = sh.n
    kappa, kappa_r = kappas(p, prot)
    with torch.no_grad():
        order, rep = ngram_sort(ngram_keys(sig, p['c_vistos'], n))
        vistos = torch.zeros_like(rep).scatter(-1, order, rep)
    B_o = torch.gather(Bt.unsqueeze(1).expand(-1, n, -1), -1, order)
    alfa_o = torch.gather(log_alfa.exp().unsqueeze(1).expand(-1, n, -1), -1, order)
    dB = F.pad((B_o[..., 1:] - B_o[..., :-1]).clamp(min=0), (1, 0)).float()
    a = rep * torch.exp(-kappa.unsqueeze(-1) * dB)
    lam = scan(a, a * F.pad(alfa_o[..., :-1], (1, 0)))
    hawkes = torch.zeros_like(lam).scatter(-1, order, lam).transpose(1, 2)
    r = vistos[:, -1].float()
    racha = scan(r * torch.exp(-kappa_r * beta.float()), r)
    return {'vistos': vistos.transpose(1, 2).float(), 'hawkes': hawkes, 'racha': racha}


# ----------------------------------------------------------------------------------------------------------------
# a13: gate and combine
# ----------------------------------------------------------------------------------------------------------------

def streak_response(p, racha, sh):
    """Piecewise-linear response on log1p(racha), flat past the last node (nucleo:865-878)."""
    dr = p['d_racha']
    x = (torch.log1p(racha) / sh.racha_paso).clamp(max=dr.shape[0] - 1)
    i = torch.nan_to_num(x.detach(), nan=0.0).floor().long().clamp(0, dr.shape[0] - 2)
    return dr.cumsum(0)[i] + (x - i) * dr[1:][i]


def combine(p, acc, h, sh, prot):
    """h' = h + sigmoid(logit) W_o (salida / max(1, peso_total)) (estable:376-403)."""
    salida, pt = acc['salida'], acc['peso_total'].detach()
    salida = salida / acc['peso_total'].clamp(min=1)
    mejor = torch.where(pt > 0, acc['mejor'], torch.zeros_like(pt))
    if prot.mejor_max is not None:
        mejor = mejor.clamp(-prot.mejor_max, prot.mejor_max)
    sen = torch.cat([pt / sh.T, mejor, acc['pico'] / pt.clamp(min=1), acc['peso_ctx'].detach() / sh.Tc], dim=-1)
    with torch.autocast(device_type='cpu', enabled=False):
        logit = F.linear(h, p['g.weight'].to(h.dtype), p['g.bias'].to(h.dtype))
    logit = logit + F.linear(sen, p['g_conf.weight'], p['g_conf.bias']).to(logit.dtype)
    logit = logit + (acc['vistos'] * p['w_vistos']).sum(-1, keepdim=True)
    logit = logit + (torch.log1p(acc['hawkes']) * p['u_hawkes']).sum(-1, keepdim=True)
    logit = logit + streak_response(p, acc['racha'], sh).unsqueeze(-1)
    if prot.tope_puerta is not None:
        logit = prot.tope_puerta * torch.tanh(logit / prot.tope_puerta)
    aporte = F.linear(salida, p['o.weight'])
    return h + torch.sigmoid(logit).to(aporte.dtype) * aporte


def layer_forward(p, E, h, x, sh, prot=Prot()):
    """h' = CapaASRNEstable.forward(E, h, x) (estable:407-421); with Prot.ninguna() the core layer's
    (nucleo.CapaASRN.forward, nucleo:880-885)."""
    sig = firmas(x) if x is not None else E.float() @ p['r_firma'].float()
    Qc, Kc, beta, log_alfa = context(p, h, sh, prot)
    Bt = beta.cumsum(1)
    phi, V = phi_and_values(p, E)
    salida, sen = candidates(phi, V, Qc, Kc, Bt, log_alfa, sig, p['w_sufijo'], p['gamma'], sh, prot)
    acc = gate_signals(salida, sen, sh.T, sh.Tc)
    acc.update(repetition(p, sig, beta, Bt, log_alfa, sh, prot))
    return combine(p, acc, h, sh, prot)
