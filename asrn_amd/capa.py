"""CapaASRNEstable on MI355X: the reference's stable ASRN layer with its hot path on HIP kernels.

Same constructor arguments, parameter and buffer names, construction order (so the same seed gives the same weights)
and forward contract as asrn.estable.CapaASRNEstable (asrn/estable.py:141-421, inheriting asrn/nucleo.py:574-886):
forward(E (B, L, d), h (B, L, d), piezas (B, L) int64 | None) -> h' (B, L, d). The dense projections (hash MLPs, V,
LayerNorm, Qc/Kc, the clock projection, the gate and W_o) stay hipBLASLt GEMMs, with their weight gradients split
over slabs of tokens (asrn_amd.lineal); the bucket sort, the candidate attention forward and backward, the n-gram
sort, the clock, Hawkes and streak scans run in libasrn_hip.so. There is no CPU path: CPU tensors or unsupported
shapes raise.
"""
import dataclasses
import math
import os

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .lineal import _rows, column_sums, lineal, weight_grad

PROHIBIDO = -1e9          # the "not allowed" score (asrn/nucleo.py:86)
ANCHO_FUSIONADO = 1024    # widest layer the fused context and gate kernels take; wider ones use PyTorch ops there


@dataclasses.dataclass(frozen=True)
class Protecciones:
    """Numerical protections (asrn/estable.py:57-77). Protecciones() = group A, the default of asrn.ASRNLayer."""
    mascara_exacta: bool = True
    reloj_64: bool = True
    beta_max: float = 1e4
    log_alfa_min: float = -30.0
    mejor_max: float = 1e4
    tope_puerta: float = None
    kappa_min: float = None

    @classmethod
    def ninguna(cls):
        return cls(mascara_exacta=False, reloj_64=False, beta_max=None, log_alfa_min=None, mejor_max=None)

    @classmethod
    def textos_largos(cls, largo_entrenamiento=1024):
        return cls(tope_puerta=10.0, kappa_min=1.0 / (4 * largo_entrenamiento))


Protections = Protecciones


def firmas_de_piezas(piezas):
    """Token signature = its id in fp32, exact for ids < 2**24 (asrn/nucleo.py:161-164)."""
    return piezas.to(torch.float32)


class CapaASRNEstable(nn.Module):
    """The ASRN layer with group-A protections (asrn.ASRNLayer). See the module docstring."""

    def __init__(self, d, protecciones=None, n_tablas=8, n_bits=14, afin_oculto=128, chunk=32, tablas_contexto=4,
                 confirmar=16, sufijo=4, vistos=4, dropout=0.0, nodos_racha=16, racha_max=256):
        super().__init__()
        assert 0 < tablas_contexto < n_tablas and nodos_racha >= 2
        self.n_tablas, self.n_bits, self.chunk = n_tablas, n_bits, chunk
        self.tablas_contexto, self.confirmar, self.sufijo, self.vistos = tablas_contexto, confirmar, sufijo, vistos
        # construction order = the reference's (asrn/nucleo.py:591-630): it fixes the weights a seed produces
        mitad = max(8, afin_oculto // 2)
        self.afin_palabra = nn.Sequential(nn.Linear(d, mitad), nn.GELU(),
                                          nn.Linear(mitad, (n_tablas - tablas_contexto) * n_bits))
        self.afin_contexto = nn.Sequential(nn.Linear(2 * d, mitad), nn.GELU(),
                                           nn.Linear(mitad, tablas_contexto * n_bits))
        self.v = nn.Linear(d, d, bias=False)
        self.o = nn.Linear(d, d, bias=False)
        self.g = nn.Linear(d, 1)
        self.temperatura = (n_tablas * n_bits) ** 0.5
        self.register_buffer('pot', 2 ** torch.arange(n_bits))
        self.g_conf = nn.Linear(4, 1)
        nn.init.zeros_(self.g_conf.weight)
        nn.init.zeros_(self.g_conf.bias)
        self.cq = nn.Linear(d, confirmar, bias=False)
        nn.init.zeros_(self.cq.weight)
        self.ck = nn.Linear(d, confirmar, bias=False)
        self.ln_ctx = nn.LayerNorm(d)
        self.w_vistos = nn.Parameter(torch.zeros(vistos))
        g_v = torch.Generator().manual_seed(12345)
        self.register_buffer('c_vistos', torch.rand(vistos, generator=g_v, dtype=torch.float64) + 0.5)
        self.w_sufijo = nn.Parameter(torch.zeros(sufijo + 1))
        self.register_buffer('r_firma', torch.randn(d))
        self.drop = nn.Dropout(dropout)
        self.w_reloj = nn.Parameter(torch.zeros(2, d))
        self.b_reloj = nn.Parameter(torch.tensor([math.log(math.e - 1), 0.0]))
        self.gamma = nn.Parameter(torch.zeros(n_tablas))
        self.log_kappa = nn.Parameter(-torch.log(chunk * 4.0 ** torch.arange(vistos)))
        self.log_kappa_racha = nn.Parameter(torch.tensor([-math.log(8.0 * chunk)]))
        self.u_hawkes = nn.Parameter(torch.zeros(vistos))
        self.racha_paso = math.log1p(racha_max) / (nodos_racha - 1)
        self.d_racha = nn.Parameter(torch.zeros(nodos_racha))
        self.protecciones = protecciones or Protecciones()

    # --- checks -----------------------------------------------------------------------------------------------------

    def _revisar(self, E):
        p = self.protecciones
        if not E.is_cuda:
            raise RuntimeError('asrn_amd.ASRNLayer runs on the GPU only (HIP kernels for gfx950): move the layer and '
                               'its inputs to a cuda device')
        if not 1 <= self.n_bits <= 14:
            raise ValueError(f'n_bits={self.n_bits}: the HIP bucket sort supports 1..14 bits per table')
        if not 1 <= self.chunk <= 64 or self.n_tablas * self.chunk > 256:
            raise ValueError(f'chunk={self.chunk}, n_tablas={self.n_tablas}: the HIP candidate kernels support 1..64 '
                             'candidates per table and n_tablas * chunk <= 256')
        d = E.shape[-1]
        if d % 4:
            raise ValueError(f'd={d}: the HIP candidate kernels read rows as float4: d must be a multiple of 4')
        if self.n_tablas * self.n_bits + self.confirmar > 256 or self.sufijo > 16 or self.n_tablas > 32:
            raise ValueError('n_tablas*n_bits + confirmar must be <= 256, sufijo <= 16, n_tablas <= 32')

    # --- producers (PyTorch GEMMs, asrn/nucleo.py:634-664 and asrn/estable.py:153-194) --------------------------------

    def _firma(self, E):
        with torch.autocast(device_type=E.device.type, enabled=False):
            return E.float() @ self.r_firma.float()

    def _phi(self, E):
        llave = torch.cat([E, F.pad(E, (0, 0, 1, 0))[:, :E.shape[1]]], dim=-1)
        return torch.cat([self.afin_palabra(E), self.afin_contexto(llave)], dim=-1)

    def _hash_fusionado(self, E):
        """Whether phi comes from the fused hash kernels (ops.HashProducer): fp32 outside autocast and the widths
        asrn_hash_fwd supports; otherwise the first layers' GEMM, the hidden-layer kernel or PyTorch ops, and one
        block-diagonal GEMM."""
        pal, ctx = self.afin_palabra, self.afin_contexto
        m, mc = pal[0].out_features, ctx[0].out_features
        pw, pc = pal[2].out_features, ctx[2].out_features
        return (E.dtype == torch.float32 and not torch.is_autocast_enabled(E.device.type) and m % 4 == 0
                and mc % 4 == 0 and 4 <= m <= 64 and 4 <= mc <= 64 and 256 % ((m + mc) // 4) == 0
                and 1 <= pw <= 64 and 1 <= pc <= 64 and pal[0].weight.dtype == torch.float32)

    def _pesos(self, E):
        """The fused GEMMs' weights assembled in one launch (_Pesos): a dict with W and Wq, and W2, b2 unless the hash
        kernels take the second layers' parameters directly; None when a parameter is not fp32 (the methods below
        then assemble them with PyTorch ops)."""
        pal, ctx = self.afin_palabra, self.afin_contexto
        ps = [pal[0].weight, ctx[0].weight, self.cq.weight, self.ck.weight]
        if not self._hash_fusionado(E):
            ps += [pal[2].weight, ctx[2].weight, pal[2].bias, ctx[2].bias]
        if not all(p.dtype == torch.float32 and p.is_cuda and p.is_contiguous() for p in ps):
            return None
        out = _Pesos.apply(*ps)
        return dict(zip(('W', 'Wq', 'W2', 'b2'), out))

    def _phi_y_valores(self, E, pesos=None):
        """phi (B, L, P) and the rows the candidate kernels gather for the values (see _phi_filas)."""
        phi, filas, _ = self._phi_filas(E, pesos)
        return phi, filas

    def _phi_filas(self, E, pesos=None, ids=False):
        """phi (B, L, P), the rows the candidate kernels gather for the values (asrn/nucleo.py:644-659) and, with ids
        and the fused fp32 producer, the bucket ids of phi (B*T, L) its kernel wrote with it (else None).

        The reference's values are V[s] = W_v E[s+1] and the layer adds W_o (sum over tables of att V). Both maps are
        linear, so the kernels gather E[s+1] itself (read in place, shifted) and the layer applies W_o W_v once to the
        gathered sum (_combinar): the same result up to fp32 reassociation, without the W_v projection of every
        position in the forward and its two GEMMs in the backward. One GEMM over E gives the word MLP's first layer
        and the context MLP's first layer split by linearity (W [E_t; E_{t-1}] = W_a E_t + W_b E_{t-1}: the key
        [E_t; E_{t-1}] is never materialized). In fp32 the biases, the shift of the W_b product and the GELU are one
        kernel (ops.Producer); under autocast they are PyTorch ops on the GEMM's output."""
        d = E.shape[-1]
        pal, ctx = self.afin_palabra, self.afin_contexto
        m, mc = pal[0].out_features, ctx[0].out_features
        W = (torch.cat([pal[0].weight, ctx[0].weight.view(mc, 2, d).transpose(0, 1).reshape(2 * mc, d)])
             if pesos is None else pesos['W'])
        if self._hash_fusionado(E):
            phi, filas, idv = ops.HashProducer.apply(E, W, pal[0].bias, ctx[0].bias, pal[2].weight, pal[2].bias,
                                                     ctx[2].weight, ctx[2].bias, m, mc,
                                                     self.n_tablas if ids else 0, self.n_bits)
            return phi, filas, (idv if idv.numel() else None)
        if pesos is None or 'W2' not in pesos:
            W2 = torch.block_diag(pal[2].weight, ctx[2].weight)    # both second layers as one GEMM: phi comes whole
            b2 = torch.cat([pal[2].bias, ctx[2].bias])
        else:
            W2, b2 = pesos['W2'], pesos['b2']
        if (E.dtype == torch.float32 and not torch.is_autocast_enabled(E.device.type) and m % 4 == 0
                and mc % 4 == 0 and W.dtype == torch.float32):
            g, filas = ops.Producer.apply(E, W, pal[0].bias, ctx[0].bias, m, mc)
        elif torch.is_autocast_enabled(E.device.type):
            # 16-bit: the reference's own products (nucleo:644-659): the word MLP's first layer on E, and the context
            # MLP's on the key [E_t; E_{t-1}] built from the 16-bit E, each rounded once. Split by linearity, the
            # context layer would round W_a E_t and W_b E_{t-1} apart: one 16-bit rounding more, which moves phi
            # values near 0 to the other sign and their positions to other buckets than the reference's
            E16 = _a_autocast(E)
            llave = torch.cat([E16, F.pad(E16, (0, 0, 1, 0))[:, :E16.shape[1]]], dim=-1)
            g = F.gelu(torch.cat([lineal(E16, pal[0].weight, pal[0].bias), lineal(llave, ctx[0].weight, ctx[0].bias)],
                                 dim=-1))
            filas = E16
        else:
            y = lineal(E, W, F.pad(pal[0].bias, (0, 2 * mc)))
            hp, za, zb = y.split([m, mc, mc], dim=-1)
            g = F.gelu(torch.cat([hp, _ShiftAdd.apply(za, zb, ctx[0].bias)], dim=-1))
            filas = E
        phi = lineal(g, W2, b2)
        return phi, filas, None

    def _contexto(self, h, con_h=False, pesos=None):
        """Qc, Kc (B, L, cf), beta (B, L) fp64 and log_alfa (B, L) (asrn/estable.py:153-194 with the GPU branch's clock
        projection in true fp32, estable:171-175): LayerNorm, the clock projection and its softplus / logsigmoid /
        clamps fused in asrn_context_fwd/bwd; Qc, Kc on hipBLASLt. con_h: also h as the gate should take it (an
        alias whose gradient the context backward adds to its own)."""
        p = self.protecciones
        meta = (float(self.ln_ctx.eps), -1.0 if p.beta_max is None else float(p.beta_max),
                -math.inf if p.log_alfa_min is None else float(p.log_alfa_min))
        cf = self.confirmar
        Wq = torch.cat([self.cq.weight, self.ck.weight]) if pesos is None else pesos['Wq']
        if h.shape[-1] > ANCHO_FUSIONADO:
            return self._contexto_ancho(h, Wq, con_h)
        if not torch.is_autocast_enabled(h.device.type) and h.shape[-1] <= 512 and 2 * cf <= 32:
            # fp32: the projection's input gradient formed inside the context backward (no GEMM, no dhh buffer)
            y, beta, log_alfa, h_puerta = ops.ContextProj.apply(h, self.ln_ctx.weight, self.ln_ctx.bias,
                                                                self.w_reloj, self.b_reloj, Wq, meta)
        else:
            hh32, beta, log_alfa, h_puerta = ops.Context.apply(h, self.ln_ctx.weight, self.ln_ctx.bias,
                                                               self.w_reloj, self.b_reloj, meta)
            y = lineal(_a_autocast(hh32), Wq)
        Qc, Kc = _Split2.apply(y, cf)
        return (Qc, Kc, beta, log_alfa, h_puerta) if con_h else (Qc, Kc, beta, log_alfa)

    def fugas(self):
        """The number of (query, table) pairs of the last forward whose best valid score lay within reach of the -1e9
        fill (without mascara_exacta; None otherwise). There the reference's unprotected layer gives the invalid keys
        of its block window weight (asrn/estable.py:20-24, asrn/nucleo.py:337-339, 813) and its output depends on how
        it cuts each sorted row into blocks; this layer only ever weighs the valid candidates, so its output there
        differs from the reference's. Everywhere else the two agree. Reading it waits for the GPU."""
        f = getattr(self, '_fuga', None)
        return None if f is None else int(f.item())

    def _contexto_ancho(self, h, Wq, con_h):
        """_contexto for widths past the fused context kernels (d > 1024), as PyTorch ops on the GPU, with the same
        math (asrn/estable.py:153-194): LayerNorm in fp32, Qc and Kc from its output in the autocast dtype, the clock
        projection in true fp32 (no TF32: a sum of products), softplus / logsigmoid and the clamps."""
        p = self.protecciones
        hh32 = F.layer_norm(h.float(), (h.shape[-1],), self.ln_ctx.weight.float(), self.ln_ctx.bias.float(),
                            self.ln_ctx.eps)
        y = lineal(_a_autocast(hh32), Wq)
        with torch.autocast(device_type=h.device.type, enabled=False):
            w = self.w_reloj.float()
            u = torch.stack([(hh32 * w[0]).sum(-1), (hh32 * w[1]).sum(-1)], -1) + self.b_reloj.float()
        beta = F.softplus(u[..., 0])
        log_alfa = F.logsigmoid(u[..., 1]) + math.log(2)
        if p.beta_max is not None:
            beta = beta.clamp(max=p.beta_max)
        if p.log_alfa_min is not None:
            log_alfa = log_alfa.clamp(min=p.log_alfa_min)
        Qc, Kc = _Split2.apply(y, self.confirmar)
        out = (Qc, Kc, beta.double(), log_alfa)
        return out + (h,) if con_h else out

    def _kappas(self):
        k, kr = self.log_kappa.exp(), self.log_kappa_racha.exp()
        m = self.protecciones.kappa_min
        return (k, kr) if m is None else (k.clamp(min=m), kr.clamp(min=m))

    # --- hot path (HIP) ---------------------------------------------------------------------------------------------

    def _cubetas(self, E, partes=None, pesos=None):
        """The hash producers and the bucket sort (asrn/estable.py:204-236): phi, the rows the values gather, and the
        sorted order, windows and ranks of every table."""
        phi, filas, ids = self._phi_filas(E, pesos, ids=True)
        if partes is not None:                                              # the generation step's value cache
            v = F.linear(_a_autocast(E), self.v.weight)
            partes.update(phi=phi, V=F.pad(v, (0, 0, 0, 1))[:, 1:])         # V[t] = W_v E[t+1], 0 at the end
        _, order, _, rank, win = ops.bucket_sort(phi.detach(), self.n_tablas, self.n_bits, self.chunk, ids=ids)
        return phi, filas, order, win, rank

    def _acumular(self, E, Qc, Kc, Bt, log_alfa, sig, partes=None, pesos=None, esperar=None, cubetas=None):
        """Candidate attention of all tables -> salida and the gate signals (asrn/estable.py:204-300). esperar: called
        before the candidate kernels, after the producers and the bucket sort (the point where the context inputs
        must be ready); cubetas: what _cubetas returned, when it already ran."""
        phi, filas, order, win, rank = self._cubetas(E, partes, pesos) if cubetas is None else cubetas
        p = self.protecciones
        shape = dict(T=self.n_tablas, Tc=self.tablas_contexto, C=self.chunk, K=self.sufijo, v_shift=1,
                     reloj32=not p.reloj_64)
        if not p.mascara_exacta:           # the reference's -1e9 fill: count where it would leak (fugas())
            self._fuga = torch.zeros(1, dtype=torch.int32, device=E.device)
            shape['fuga'] = self._fuga
        if esperar is not None:
            esperar()
        suma, sen = ops.Candidates.apply(phi, filas, Qc, Kc, Bt, log_alfa, self.w_sufijo, self.gamma, sig, order,
                                         win, rank, shape)
        # sum over tables of att E[s+1]: W_v and W_o are applied together after it (see _phi_y_valores)
        return {'salida': suma, 'senales': sen}

    def _repeticion(self, sig, beta, Bt, log_alfa, partes=None, ngram=None):
        """vistos, hawkes (B, L, n) and racha (B, L) (asrn/estable.py:304-321); ngram: ops.ngram_sort(sig, ...) when
        it already ran."""
        kappa, kappa_r = self._kappas()
        if ngram is None:
            with torch.no_grad():
                ngram = ops.ngram_sort(sig, self.c_vistos, self.vistos)
        claves, order, rep, rank_k, vistos = ngram
        hawkes, racha = ops.Repeticion.apply(Bt, log_alfa, kappa, beta, kappa_r, order, rep, rank_k, vistos)
        if partes is not None:
            partes.update(claves=claves, orden_k=order, repetido=rep)
        return {'vistos': vistos, 'hawkes': hawkes, 'racha': racha}

    # --- gate (asrn/estable.py:376-403 and asrn/nucleo.py:865-878) ---------------------------------------------------

    def _combinar(self, acc, h):
        """h' = h + sigmoid(logit) W_o (salida / max(1, peso_total)): W_o on hipBLASLt, the rest fused in asrn_gate_*
        (the division by the table count is applied after W_o, per token). acc['w_salida'], when present, replaces W_o
        (the whole-text path passes W_o W_v with the gathered sum of E rows); acc['gemelo'], when present, takes the
        projection's weight gradient (_Gemelo), and the GEMM here computes only the input gradient."""
        p = self.protecciones
        w = acc.get('w_salida', self.o.weight)
        gemelo = acc.get('gemelo')
        if gemelo is None:
            aporte = lineal(acc['salida'], w)
        else:
            aporte = _ConPeso.apply(lineal(acc['salida'], w.detach()), gemelo)
        aporte = self.drop(aporte)
        if h.shape[-1] > ANCHO_FUSIONADO:
            return self._compuerta_ancha(h, aporte, acc)
        meta = (self.n_tablas, self.tablas_contexto, self.racha_paso,
                -1.0 if p.mejor_max is None else float(p.mejor_max), 0.0 if p.tope_puerta is None else float(p.tope_puerta))
        return ops.Gate.apply(h, aporte, acc['senales'], acc['vistos'], acc['hawkes'], acc['racha'], self.g.weight,
                               self.g.bias, self.g_conf.weight, self.g_conf.bias, self.w_vistos, self.u_hawkes,
                               self.d_racha, meta)

    def _combinar_paso(self, salida, h, sen, vistos, hawkes, racha):
        """The generation step's _combinar for B tokens, h and salida (B, d): W_o and the gate in one kernel
        (ops.gate_step), or None where that does not apply (16-bit or wide layers, autograd, an active dropout), and
        then _combinar runs."""
        if (torch.is_grad_enabled() or h.dtype != torch.float32 or salida.dtype != torch.float32
                or torch.is_autocast_enabled(h.device.type) or h.shape[-1] > ANCHO_FUSIONADO or h.shape[-1] % 4
                or (self.drop.training and self.drop.p > 0) or self.o.weight.dtype != torch.float32):
            return None
        p = self.protecciones
        meta = (self.n_tablas, self.tablas_contexto, self.racha_paso,
                -1.0 if p.mejor_max is None else float(p.mejor_max), 0.0 if p.tope_puerta is None else float(p.tope_puerta))
        return ops.gate_step(h, salida, self.o.weight, sen, vistos, hawkes, racha, self.g.weight, self.g.bias,
                             self.g_conf.weight, self.g_conf.bias, self.w_vistos, self.u_hawkes, self.d_racha, meta)

    def _compuerta_ancha(self, h, aporte, acc):
        """The gate for widths past the fused gate kernels (d > 1024), as PyTorch ops on the GPU with the same math
        (asrn/estable.py:376-403, asrn/nucleo.py:865-878; the division by the table count after W_o, per token):
        h' = h + sigmoid(cap(logit)) A / max(1, peso_total), the logit in fp32."""
        p = self.protecciones
        sen = acc['senales']
        pt = sen[..., 0:1]
        mejor = torch.where(pt > 0, sen[..., 1:2], torch.zeros_like(pt))
        if p.mejor_max is not None:
            mejor = mejor.clamp(-p.mejor_max, p.mejor_max)
        senales = torch.cat([pt / self.n_tablas, mejor, sen[..., 2:3] / pt.clamp(min=1),
                             sen[..., 3:4] / self.tablas_contexto], dim=-1)
        with torch.autocast(device_type=h.device.type, enabled=False):
            hf = h.float()
            logit = F.linear(hf, self.g.weight.float(), self.g.bias.float())
            logit = logit + F.linear(senales, self.g_conf.weight.float(), self.g_conf.bias.float())
            logit = logit + (acc['vistos'].float() * self.w_vistos.float()).sum(-1, keepdim=True)
            logit = logit + (torch.log1p(acc['hawkes'].float()) * self.u_hawkes.float()).sum(-1, keepdim=True)
            racha = acc['racha'].float()
            nodos = self.d_racha.shape[0]
            x = (torch.log1p(racha) / self.racha_paso).clamp(max=nodos - 1)
            i = torch.nan_to_num(x.detach(), nan=0.0).floor().long().clamp(0, nodos - 2)
            dr = self.d_racha.float()
            logit = logit + (dr.cumsum(0)[i] + (x - i) * dr[1:][i]).unsqueeze(-1)
            if p.tope_puerta is not None:
                logit = p.tope_puerta * torch.tanh(logit / p.tope_puerta)
            return hf + torch.sigmoid(logit) * (aporte.float() / pt.clamp(min=1))

    # --- all together -----------------------------------------------------------------------------------------------

    def forward(self, E, h, piezas=None, ngramas=None):
        """E (B, L, d), h (B, L, d), piezas (B, L) or None -> h' (B, L, d) (asrn/estable.py:407-421).

        ngramas: what `ngramas(piezas, capa)` returned for these token ids, to share one n-gram sort between every ASRN
        layer of a model (it depends on the tokens only; the reference sorts again in each layer, nucleo:688-701).
        Without it the layer sorts itself."""
        return self._adelante(E, h, piezas, ngramas=ngramas)

    def _adelante(self, E, h, piezas=None, partes=None, ngramas=None):
        """forward; with a dict `partes`, also keeps what the generation step starts from (the prompt's phi, V,
        Qc, Kc, sig, beta, Bt, log_alfa, n-gram keys and their sort, hawkes and racha)."""
        self._revisar(E)
        if ngramas is not None:
            if piezas is None:
                raise ValueError('ngramas: the shared n-gram sort is for token ids (piezas); without them the '
                                 'signatures come from E and differ per layer')
            _revisar_ngramas(ngramas, piezas, self)
        # Two streams: the context producer (LayerNorm, Qc/Kc, the clock), the token signatures, W_o W_v and the
        # repetition branch (n-gram sort, Hawkes and streak scans: small, latency-bound kernels) run on the second
        # one, beside the hash producers and the bucket sort; the candidate attention waits for the context only.
        # Autograd runs each op's backward on the stream of its forward, so the backward overlaps the same way, and
        # the W_o W_v projection's weight gradient (_Gemelo) runs there too.
        principal, lado = torch.cuda.current_stream(E.device), _lateral(E.device)
        pesos = self._pesos(E)
        lado.wait_stream(principal)
        with torch.cuda.stream(lado):
            # signatures carry no gradient (they are only compared); a detached E keeps E's gradient accumulation
            # on the main stream, where its gradient is made
            sig = self._firma(E.detach()) if piezas is None else firmas_de_piezas(piezas)
            w_salida = ops.SmallMatmul.apply(self.o.weight, self.v.weight)
            Qc, Kc, beta, log_alfa, h = self._contexto(h, con_h=True, pesos=pesos)
            # the clock: fp64 (reloj_64), or the core layer's fp32 clock, each sum rounded to fp32 (kept in fp64)
            Bt = ops.ClockScan.apply(beta, not self.protecciones.reloj_64)
            contexto_listo = torch.cuda.Event()
            contexto_listo.record(lado)
            if ngramas is None:
                with torch.no_grad():
                    ngram = ops.ngram_sort(sig, self.c_vistos, self.vistos)
            else:
                ngram = ngramas[1:]
            rep = self._repeticion(sig, beta, Bt, log_alfa, partes, ngram)
        if pesos is not None:
            pesos['Wq'].record_stream(lado)            # made here, used there: not reused before both are done
        acc = self._acumular(E, Qc, Kc, Bt, log_alfa, sig, partes, pesos,
                             esperar=lambda: principal.wait_event(contexto_listo))
        with torch.cuda.stream(lado):
            gemelo = _Gemelo.apply(acc['salida'], w_salida)    # launches nothing
        principal.wait_stream(lado)
        for t in [Qc, Kc, beta, Bt, log_alfa, h, sig, w_salida] + list(rep.values()) + list(ngram):
            t.record_stream(principal)
        acc.update(rep, w_salida=w_salida, gemelo=gemelo)
        if partes is not None:
            partes.update(Qc=Qc, Kc=Kc, sig=sig, beta=beta, Bt=Bt, log_alfa=log_alfa, hawkes=acc['hawkes'],
                          racha=acc['racha'])
        return self._combinar(acc, h)


_LATERAL = {}


def _lateral(device):
    """The second stream of a device (default priority), made once. With ASRN_ONE_STREAM=1 in the environment the
    branches run one after the other on the current stream instead (a profiler's kernel trace then times each kernel
    alone, without the waits of kernels that share the CUs)."""
    if os.environ.get('ASRN_ONE_STREAM') == '1':
        return torch.cuda.current_stream(device)
    i = torch.device(device).index
    if i is None:
        i = torch.cuda.current_device()
    s = _LATERAL.get(i)
    if s is None:
        s = _LATERAL[i] = torch.cuda.Stream(device=i)
    return s


class _Gemelo(torch.autograd.Function):
    """Stands in for the projection A = x W^T in W's part of the autograd graph: no value and no memory (a stride-0
    view of an uninitialized scalar), and it reads nothing in the forward. Its backward receives dA (from _ConPeso)
    and returns dW = dA^T x, cast and summed over token slabs as lineal's own backward does, on the stream the forward
    was called on: the weight gradient's GEMM runs there, beside the input gradient's."""

    @staticmethod
    def forward(ctx, x, w):
        dev = x.device.type
        ctx.dt = torch.get_autocast_dtype(dev) if torch.is_autocast_enabled(dev) else x.dtype
        ctx.wdt = w.dtype
        ctx.save_for_backward(x)
        return torch.empty((), dtype=ctx.dt, device=x.device).expand(*x.shape[:-1], w.shape[0])   # A's dtype

    @staticmethod
    def backward(ctx, g):
        x, = ctx.saved_tensors
        s = torch.cuda.current_stream(g.device)
        g.record_stream(s)                             # both made on the other stream and read here
        x.record_stream(s)
        with torch.autocast(device_type=g.device.type, enabled=False):
            gw = weight_grad(_rows(g.to(ctx.dt)), _rows(x.to(ctx.dt)))
        return None, gw.to(ctx.wdt)


class _ConPeso(torch.autograd.Function):
    """A itself (an alias); the backward hands dA to A's producer and to the _Gemelo that takes its weight
    gradient."""

    @staticmethod
    def forward(ctx, a, gemelo):
        return a.view_as(a)

    @staticmethod
    def backward(ctx, g):
        return g, g


class _ShiftAdd(torch.autograd.Function):
    """out[:, t] = za[:, t] + zb[:, t - 1] + bias (zb's term absent at t = 0): the context MLP's first layer on the key
    [E_t; E_{t-1}], from the two halves' products. No zero-padded copies in either direction."""

    @staticmethod
    def forward(ctx, za, zb, bias):
        out = za + bias
        out[:, 1:] += zb[:, :-1]
        return out

    @staticmethod
    def backward(ctx, g):
        dzb = torch.empty_like(g)
        dzb[:, :-1] = g[:, 1:]
        dzb[:, -1] = 0
        return g, dzb, column_sums(g.reshape(-1, g.shape[-1]))


class _Pesos(torch.autograd.Function):
    """The fused GEMMs' weights, assembled from the parameters in one launch (ops.copy_blocks):
    W = [W_p; W_a; W_b] (the word MLP's first layer and the context MLP's split into its E_t and E_{t-1} halves) and
    Wq = [cq; ck]; with the second layers given, also W2 = blockdiag(word second layer, context second layer) and
    b2 = [b_word2; b_ctx2]. The backward scatters the gradients back to the parameters in one launch. fp32 only."""

    @staticmethod
    def forward(ctx, p0w, c0w, cqw, ckw, p2w=None, c2w=None, p2b=None, c2b=None):
        (m, d), mc, cf = p0w.shape, c0w.shape[0], cqw.shape[0]
        dev = p0w.device
        con2 = p2w is not None
        W = torch.empty((m + 2 * mc, d), dtype=torch.float32, device=dev)
        Wq = torch.empty((2 * cf, d), dtype=torch.float32, device=dev)
        W2 = b2 = None
        params = [p0w, c0w, cqw, ckw]
        if con2:
            (o1, h1), (o2, h2) = p2w.shape, c2w.shape
            W2 = torch.empty((o1 + o2, h1 + h2), dtype=torch.float32, device=dev)
            b2 = torch.empty((1, o1 + o2), dtype=torch.float32, device=dev)
            params += [p2w, c2w, p2b.view(1, -1), c2b.view(1, -1)]
        ops.copy_blocks(_Pesos.bloques(W, Wq, W2, b2, params, ida=True))
        ctx.meta = [t.shape for t in (p0w, c0w, cqw, ckw)] + ([t.shape for t in (p2w, c2w, p2b, c2b)] if con2 else [])
        ctx.set_materialize_grads(False)
        return (W, Wq, W2, b2.view(-1)) if con2 else (W, Wq)

    @staticmethod
    def bloques(W, Wq, W2, b2, params, ida):
        """(source, destination) pairs: parameters -> assembled weights (ida), or the reverse for the gradients."""
        p0w, c0w, cqw, ckw = params[:4]
        m, d, mc, cf = p0w.shape[0], p0w.shape[1], c0w.shape[0], cqw.shape[0]
        pares = [(p0w, W[:m]), (c0w[:, :d], W[m:m + mc]), (c0w[:, d:], W[m + mc:]), (cqw, Wq[:cf]), (ckw, Wq[cf:])]
        ceros = []
        if W2 is not None:
            p2w, c2w, p2b, c2b = params[4:]
            o1, h1 = p2w.shape
            pares += [(p2w, W2[:o1, :h1]), (c2w, W2[o1:, h1:]), (p2b, b2[:, :o1]), (c2b, b2[:, o1:])]
            ceros = [(None, W2[:o1, h1:]), (None, W2[o1:, :h1])]
        return pares + ceros if ida else [(b, a) for a, b in pares]

    @staticmethod
    def backward(ctx, dW, dWq, dW2=None, db2=None):
        shapes = ctx.meta
        con2 = len(shapes) == 8
        dev = next(g for g in (dW, dWq, dW2, db2) if g is not None).device
        (m, d), mc, cf = shapes[0], shapes[1][0], shapes[2][0]
        formas = [(m + 2 * mc, d), (2 * cf, d)]
        if con2:
            (o1, h1), (o2, h2) = shapes[4], shapes[5]
            formas += [(o1 + o2, h1 + h2), (o1 + o2,)]
        gs = [torch.zeros(f, dtype=torch.float32, device=dev) if g is None else g.to(torch.float32).contiguous()
              for g, f in zip((dW, dWq, dW2, db2), formas)]
        grads = [torch.empty(sh, dtype=torch.float32, device=dev) for sh in shapes]
        destinos = grads[:4] + ([grads[4], grads[5], grads[6].view(1, -1), grads[7].view(1, -1)] if con2 else [])
        ops.copy_blocks(_Pesos.bloques(gs[0], gs[1], gs[2] if con2 else None,
                                       gs[3].view(1, -1) if con2 else None, destinos, ida=False))
        return tuple(grads) + ((None,) * 4 if not con2 else ())


class _Split2(torch.autograd.Function):
    """y[..., :k] and y[..., k:] as views (the candidate kernels read both in place through their row stride). The
    backward hands on the buffer both gradients live in when they arrive as its two column blocks (the candidate
    backward writes them so), and otherwise joins them with one concatenation; slicing's own backward would zero-fill
    a copy of y per part and add them."""

    @staticmethod
    def forward(ctx, y, k):
        ctx.k, ctx.shape, ctx.dtype = k, y.shape, y.dtype
        return y[..., :k], y[..., k:]

    @staticmethod
    def backward(ctx, ga, gb):
        k, n = ctx.k, ctx.shape[-1]
        if (ga is not None and gb is not None and ga.dim() == 3 and ga.dtype == gb.dtype and ga.stride() == gb.stride()
                and ga.stride(-1) == 1 and ga.stride(1) == n and ga.stride(0) == ga.shape[1] * n
                and gb.storage_offset() == ga.storage_offset() + k and ga.untyped_storage().data_ptr()
                == gb.untyped_storage().data_ptr()
                and ga.untyped_storage().nbytes() >= ga.element_size() * (ga.storage_offset() + ga.shape[0] * ga.stride(0))):
            return ga.as_strided(ctx.shape, (ga.stride(0), n, 1), ga.storage_offset()), None
        ref = ga if ga is not None else gb
        if ga is None:
            ga = torch.zeros(ctx.shape[:-1] + (k,), dtype=ref.dtype, device=ref.device)
        if gb is None:
            gb = torch.zeros(ctx.shape[:-1] + (n - k,), dtype=ref.dtype, device=ref.device)
        return torch.cat([ga, gb], dim=-1), None


def _a_autocast(x):
    disp = x.device.type
    if torch.is_autocast_enabled(disp) and x.is_floating_point():
        return x.to(torch.get_autocast_dtype(disp))
    return x


ASRNLayer = CapaASRNEstable


class CapaASRN(CapaASRNEstable):
    """The unprotected core ASRN layer (asrn.ASRNCoreLayer = asrn.nucleo.CapaASRN, asrn/nucleo.py:574-886): the same
    constructor arguments (without protecciones), parameters, buffers and construction order, and the v89 numerics
    that CapaASRNEstable computes under Protecciones.ninguna() (asrn/estable.py:68-71): an fp32 clock (the cumsum
    rounded to fp32; the writer's step adds in fp32), the score's clock term formed as (log alfa_k + rate B_k) -
    rate B_q, no clamps on beta, log alfa or the gate's 'mejor', no kappa floor.

    Two differences, both declared: (1) the reference's -1e9 fill gives weight to invalid keys when every valid score
    of a (query, table) sinks within ~100 of -1e9 (the leak the protected layer exists for); this layer weighs only the
    valid candidates there and counts such pairs (fugas()). (2) Under autocast the reference computes the clock
    projection in the 16-bit GEMM with Qc and Kc; here it stays fp32, as in the protected layer."""

    def __init__(self, d, n_tablas=8, n_bits=14, afin_oculto=128, chunk=32, tablas_contexto=4, confirmar=16,
                 sufijo=4, vistos=4, dropout=0.0, nodos_racha=16, racha_max=256):
        super().__init__(d, Protecciones.ninguna(), n_tablas=n_tablas, n_bits=n_bits, afin_oculto=afin_oculto,
                         chunk=chunk, tablas_contexto=tablas_contexto, confirmar=confirmar, sufijo=sufijo,
                         vistos=vistos, dropout=dropout, nodos_racha=nodos_racha, racha_max=racha_max)


ASRNCoreLayer = CapaASRN


@torch.no_grad()
def ngramas(piezas, capa):
    """The n-gram keys of token ids `piezas` (B, L), their stable sort per (b, j) row, the repeated flags, the ranks
    and the seen flags, for every ASRN layer of a model at once: they depend on the tokens, on the buffer c_vistos
    (the same constants in every layer, drawn from a fixed generator, nucleo:609-610) and on the group count n only.
    Pass the result to each layer's forward(..., ngramas=...). Launched on the current stream."""
    if not piezas.is_cuda:
        raise RuntimeError('asrn_amd.ngramas runs on the GPU only')
    return (piezas,) + tuple(ops.ngram_sort(firmas_de_piezas(piezas), capa.c_vistos, capa.vistos))


def _revisar_ngramas(ng, piezas, capa):
    """Checks that a shared n-gram sort was made for these tokens and this layer's group count and constants."""
    src, claves = ng[0], ng[1]
    if src is not piezas and not (src.shape == piezas.shape and src.data_ptr() == piezas.data_ptr()):
        raise ValueError('ngramas: computed for other token ids than this call\'s piezas')
    if claves.shape[-1] != capa.vistos:
        raise ValueError(f'ngramas: {claves.shape[-1]} groups, this layer has vistos={capa.vistos}')


def convertir(modelo, protecciones=None):
    """Swaps, in place, every ASRN layer of a model (its `largos` ModuleList, as in the reference's ModeloASRN,
    asrn/nucleo.py:1072) for this package's CapaASRNEstable with the same hyper-parameters, weights, device and
    train/eval mode, and returns the model: the counterpart of asrn/estable.py:424-442 for the HIP layer."""
    base = getattr(modelo, '_orig_mod', modelo)
    for j, vieja in enumerate(base.largos):
        d = vieja.v.weight.shape[1]
        nodos = vieja.d_racha.shape[0]
        racha_max = int(round(math.expm1(vieja.racha_paso * (nodos - 1))))
        drop = vieja.drop.p if isinstance(vieja.drop, nn.Dropout) else 0.0
        nueva = CapaASRNEstable(d, protecciones or getattr(vieja, 'protecciones', None), n_tablas=vieja.n_tablas,
                                n_bits=vieja.n_bits, afin_oculto=2 * vieja.afin_palabra[0].out_features,
                                chunk=vieja.chunk, tablas_contexto=vieja.tablas_contexto,
                                confirmar=vieja.confirmar, sufijo=vieja.sufijo, vistos=vieja.vistos, dropout=drop,
                                nodos_racha=nodos, racha_max=racha_max)
        nueva = nueva.to(vieja.v.weight.device)
        nueva.load_state_dict(vieja.state_dict())
        nueva.train(vieja.training)
        base.largos[j] = nueva
    return modelo
