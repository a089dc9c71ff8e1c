"""CPU restatement of the reference's O(1) generation step for one stable layer -- TEST INFRASTRUCTURE ONLY.

Follows asrn/nucleo.py:1585-1854 (_anillo_desde, _anillo_meter, _candidatos, _MemoriaHawkes, the layer part of
_Escritor.inicio / paso), asrn/estable.py:359-372 (_atender_cand, with _softmax_valido estable:121-139) and
asrn/nucleo.py:947-960 (_acc_cand, _repeticion_o1). The rings and the Hawkes memory are written as the plain state
machines the reference's docstrings define (a loop over positions, a dict per (text, group)); the per-position
producers (hashes, context projections, gate) are the whole-text oracle's, applied to one position.

Pinned by (tests/test_oracle_generation.py): the rings against their definition (the C most recent positions of each
bucket, reference test tests/test_nucleo.py:143-157), and the step-by-step layer against the golden-pinned whole-text
oracle (reference test tests/test_nucleo.py:118-140); the memoria_de_lo_ajeno masking against a brute-force scan of
all earlier positions.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

from . import layer as O


# ----------------------------------------------------------------------------------------------------------------
# rings (nucleo:1585-1618)
# ----------------------------------------------------------------------------------------------------------------

def ring_from(ids, n, C, nc):
    """ids (B, L, T) bucket ids -> ring (B, T, nc, C) int32 positions (-1 empty) and count (B, T, nc) int64 of the
    positions 0..n-1: the r-th position to enter a bucket sits in slot r % C (nucleo:1585-1607)."""
    ids = np.asarray(ids)
    B, L, T = ids.shape
    ring = np.full((B, T, nc, C), -1, dtype=np.int32)
    count = np.zeros((B, T, nc), dtype=np.int64)
    for b in range(B):
        for tau in range(T):
            for p in range(max(0, n)):
                k = ids[b, p, tau]
                ring[b, tau, k, count[b, tau, k] % C] = p
                count[b, tau, k] += 1
    return ring, count


def ring_insert(ring, count, ids_t, t):
    """Position t enters its bucket's ring in every table (nucleo:1610-1618). ids_t (B, T)."""
    B, T = ids_t.shape
    C = ring.shape[-1]
    for b in range(B):
        for tau in range(T):
            k = ids_t[b, tau]
            ring[b, tau, k, count[b, tau, k] % C] = t
            count[b, tau, k] += 1


def ring_positions(ring, ids_t):
    """(B, T, C) positions of the query's buckets (-1 empty) (nucleo:1621-1631)."""
    B, T = ids_t.shape
    return torch.from_numpy(ring[np.arange(B)[:, None], np.arange(T)[None, :], np.asarray(ids_t)].astype(np.int64))


def recent_positions_bruteforce(ids, t, C, allowed):
    """(B, T, C) the C most recent positions k < t with ids[k] == ids[t] and allowed[k] (the O(t) path's choice,
    estable:340-352), -1 padded: the definition the rings must reproduce."""
    ids = np.asarray(ids)
    B, _, T = ids.shape
    out = np.full((B, T, C), -1, dtype=np.int64)
    for b in range(B):
        for tau in range(T):
            ks = [k for k in range(t) if allowed[k] and ids[b, k, tau] == ids[b, t, tau]][-C:]
            out[b, tau, :len(ks)] = ks
    return torch.from_numpy(out)


# ----------------------------------------------------------------------------------------------------------------
# the step's candidate attention (estable:359-372, nucleo:947-951)
# ----------------------------------------------------------------------------------------------------------------

def attend(pos, t, phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, sh):
    """Query position t against candidate positions pos (B, T, C) (-1: empty). The caches are (B, >t, .) rows of
    the whole text so far. Returns salida (B, d) summed over tables and signals (B, 4) = (peso_total, mejor, pico,
    peso_ctx) (_acc_cand: mejor = max over tables of the valid max score, at least -1e9)."""
    B = phi.shape[0]
    T, C, K = sh.T, sh.C, sh.K
    valid = pos >= 0
    p = pos.clamp(min=0)
    b = torch.arange(B).view(B, 1, 1)
    Pf = O.previous(sig, K)                                                   # (B, L, K)
    sc = torch.einsum('bp,btkp->btk', phi[:, t], phi[b, p]) / math.sqrt(sh.P)
    sc = sc + torch.einsum('bp,btkp->btk', Qc[:, t], Kc[b, p]) * sh.cf ** -0.5
    sc = sc + w_suf[O.suffix_len(Pf[:, t].view(B, 1, 1, K), Pf[b, p])]
    dB = (Bt[:, t].view(B, 1, 1) - Bt[b, p]).float()
    sc = sc + (log_alfa[b, p] - (gamma / C).view(1, T, 1) * dB)
    hay = valid.any(-1, keepdim=True)                                         # exact mask (estable:121-139)
    mx = sc.masked_fill(~valid, float('-inf')).amax(-1, keepdim=True)
    ref = torch.where(hay, mx, torch.zeros_like(mx))
    att = torch.softmax((sc - ref).masked_fill(~valid, O.PROHIBIDO), dim=-1) * hay
    sc_max = torch.where(hay, mx, torch.full_like(mx, O.PROHIBIDO))
    out = torch.einsum('btk,btkd->bd', att, V[b, p])
    hayf = hay.float()
    signals = torch.cat([hayf.sum(1), sc_max.amax(1).clamp(min=O.PROHIBIDO), (att.amax(-1, keepdim=True) * hayf).sum(1),
                         hayf[:, T - sh.Tc:].sum(1)], -1)
    return out, signals


# ----------------------------------------------------------------------------------------------------------------
# Hawkes memory (nucleo:1634-1714) and the streak (nucleo:953-960)
# ----------------------------------------------------------------------------------------------------------------

class HawkesMemory:
    """Per (text b, group j): a dict key -> [Bu, A], Bu the clock of the key's last occurrence (fp64) and A = lambda +
    alfa there (fp32). Python float keys: -0.0 and 0.0 are one key; NaN keys are skipped."""

    def __init__(self, B, n):
        self.n = n
        self.maps = [{} for _ in range(B * n)]

    def load(self, keys, hawkes, Bt, log_alfa):
        """keys (B, L, n) fp64, hawkes (B, L, n), Bt (B, L) fp64, log_alfa (B, L): every key's last occurrence
        (nucleo:1656-1681)."""
        B, L, n = keys.shape
        A_all = (hawkes + log_alfa.exp().unsqueeze(-1)).float()              # A = lambda + alfa, per position
        for b in range(B):
            Bb = Bt[b].tolist()
            for j in range(n):
                m = self.maps[b * n + j] = {}
                ks, As = keys[b, :, j].tolist(), A_all[b, :, j]
                for t in range(L):
                    k = ks[t]
                    if k != k:
                        continue
                    m[k] = [Bb[t], t]
                for v in m.values():                        # the last occurrence's A, as a 0-d fp32 tensor
                    v[1] = As[v[1]].clone()

    def step(self, keys_t, B_t, log_alfa_t, kappa):
        """keys_t (B, n) fp64, B_t (B,) fp64, log_alfa_t (B,), kappa (n,) -> vistos, hawkes (B, n) fp32
        (nucleo:1683-1714): lambda = exp(-kappa fp32(B_t - Bu)) A for a known key (0 and not seen for a new one),
        then A <- lambda + alfa_t and Bu <- B_t."""
        B, n = keys_t.shape
        vistos = torch.zeros(B, n)
        hawkes = torch.zeros(B, n)
        for b in range(B):
            for j in range(n):
                k = float(keys_t[b, j])
                if k != k:
                    continue
                m = self.maps[b * n + j]
                lam = torch.zeros((), dtype=torch.float32)
                if k in m:
                    Bu, A = m[k]
                    dB = torch.tensor(B_t[b].item() - Bu, dtype=torch.float64).float()
                    lam = torch.exp(-kappa[j] * dB) * A
                    vistos[b, j] = 1.0
                hawkes[b, j] = lam
                m[k] = [B_t[b].item(), lam + log_alfa_t[b].float().exp()]
        return vistos, hawkes


def streak_step(vistos_t, beta_t, racha_prev, kappa_r):
    """racha = r (exp(-kappa_r fp32(beta)) racha_prev + 1), r = vistos[:, n-1] (nucleo:953-960)."""
    r = vistos_t[:, -1]
    return r * (torch.exp(-kappa_r * beta_t.float()) * racha_prev + 1)


# ----------------------------------------------------------------------------------------------------------------
# one layer written step by step (the layer part of _Escritor, nucleo:1751-1854)
# ----------------------------------------------------------------------------------------------------------------

def decode_layer(p, E, h, x, L0, sh, prot=O.Prot(), ajeno=False, rings='ring'):
    """The layer's outputs at positions L0..L-1 of E, h (B, L, d), x (B, L), computed one position at a time from
    the state after the prompt x[:, :L0] (L0 >= 1). ajeno: the keys are only prompt positions k with k + 1 < L0
    (memoria_de_lo_ajeno, nucleo:1808, 1789). rings='ring' reads the per-bucket rings; 'bruteforce' scans all earlier
    positions (the O(t) path). Returns y (B, L - L0, d) and the per-step (salida, signals, vistos, hawkes, racha)."""
    B, L, d = E.shape
    T, C, nb, n = sh.T, sh.C, sh.nb, sh.n
    with torch.no_grad():
        sig = O.firmas(x)
        Qc, Kc, beta, log_alfa = O.context(p, h, sh, prot)                  # per position: causal
        phi_all = torch.stack([O.phi_and_values(p, E[:, max(0, t - 1):t + 1])[0][:, -1] for t in range(L)], 1)
        Bt = torch.zeros(B, L, dtype=torch.float64)
        Bt[:, :L0] = beta[:, :L0].cumsum(1)
        V = torch.zeros(B, L, d)
        V[:, :L0 - 1] = F.linear(E[:, 1:L0], p['v.weight'])
        ids = O.bucket_ids(phi_all, T, nb).numpy()
        n_ring = L0 - 1 if ajeno else L0
        ring, count = ring_from(ids, n_ring, C, 2 ** nb)
        kappa, kappa_r = O.kappas(p, prot)
        keys = O.ngram_keys(sig, p['c_vistos'], n)
        rep0 = O.repetition(p, sig[:, :L0], beta[:, :L0], Bt[:, :L0], log_alfa[:, :L0], sh, prot)
        mem = HawkesMemory(B, n)
        mem.load(keys[:, :L0], rep0['hawkes'], Bt[:, :L0], log_alfa[:, :L0])
        racha = rep0['racha'][:, -1]
        ys, steps = [], []
        allowed = np.array([(k + 1 < L0) if ajeno else True for k in range(L)])
        for t in range(L0, L):
            V[:, t - 1] = F.linear(E[:, t], p['v.weight'])
            Bt[:, t] = Bt[:, t - 1] + beta[:, t]
            if rings == 'ring':
                pos = ring_positions(ring, ids[:, t])
            else:
                pos = recent_positions_bruteforce(ids, t, C, allowed)
            salida, sen = attend(pos, t, phi_all, V, Qc, Kc, sig, Bt, log_alfa, p['w_sufijo'], p['gamma'], sh)
            vistos, hawkes = mem.step(keys[:, t], Bt[:, t], log_alfa[:, t], kappa)
            racha = streak_step(vistos, beta[:, t], racha, kappa_r)
            acc = {'salida': salida[:, None], 'peso_total': sen[:, None, 0:1], 'mejor': sen[:, None, 1:2],
                   'pico': sen[:, None, 2:3], 'peso_ctx': sen[:, None, 3:4], 'vistos': vistos[:, None],
                   'hawkes': hawkes[:, None], 'racha': racha[:, None]}
            ys.append(O.combine(p, acc, h[:, t:t + 1], sh, prot)[:, 0])
            steps.append((salida, sen, vistos, hawkes, racha.clone()))
            if not ajeno:
                ring_insert(ring, count, ids[:, t], t)
    return torch.stack(ys, 1), steps
