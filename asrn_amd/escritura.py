"""The O(1) generation step of one stable ASRN layer on MI355X: the layer part of the reference's _Escritor
(asrn/nucleo.py:1717-1854) with its state on the device.

EscritorCapa(capa, memoria_de_lo_ajeno) keeps, per layer:
  caches      (B, cap, .) rows of phi, V, Qc, Kc, sig, Bt (fp64) and log_alfa, written in place; cap doubles when
              the text outgrows it (asrn/nucleo.py:1733-1745);
  rings       (B*T, 2^nb, C) int32 positions and (B*T, 2^nb) int32 counts: each bucket's C most recent positions
              (asrn/nucleo.py:1585-1618), built from the prompt's stable bucket sort;
  Hawkes      per (text, group) open-addressing tables of (key code, Bu, A) (asrn/nucleo.py:1634-1714);
  racha       (B,) the streak.
inicio() runs the layer over the prompt (its ordinary forward) and builds that state; paso() processes one new token
with two HIP kernels: asrn_repetition_step (clock advance, n-gram keys, Hawkes lookup/update, streak) and
asrn_decode_attend (the T*C ring candidates: score, exact softmax, copy-gather, and the ring insert when every
position may become a key). The per-token producers (hash MLPs, V, context projections) and the gate stay PyTorch,
as in the whole-text layer. Every step reads a fixed amount, T*C candidates, whatever the text length.

memoria_de_lo_ajeno=True (the reference default): the keys are only prompt positions k with k + 1 < L0 (their V rows
are values of prompt tokens), so the rings hold positions 0..L0-2 and never change. False: every earlier position is
a key, and the step equals the whole-text layer position by position.
"""
import torch

from . import ops


def _reservar(x, cap):
    buf = x.new_zeros((x.shape[0], cap) + tuple(x.shape[2:]))
    buf[:, :x.shape[1]] = x
    return buf


class EscritorCapa:
    """Step-by-step writer for one CapaASRNEstable (see the module docstring)."""

    def __init__(self, capa, memoria_de_lo_ajeno=True):
        self.capa, self.ajeno = capa, memoria_de_lo_ajeno

    def _forma(self):
        c = self.capa
        return dict(T=c.n_tablas, Tc=c.tablas_contexto, C=c.chunk, K=c.sufijo, nb=c.n_bits)

    def bytes_anillos(self, B):
        """Device bytes of the rings and counts (asrn/nucleo.py:1747-1748 sizes them the same way)."""
        c = self.capa
        return B * c.n_tablas * 2 ** c.n_bits * (4 * c.chunk + 4)

    @torch.no_grad()
    def inicio(self, E, h, piezas, capacidad=0):
        """The prompt: E, h (B, L0, d), piezas (B, L0) (L0 >= 1) -> the layer's output (B, L0, d); builds the state."""
        capa = self.capa
        B, L0 = piezas.shape
        if L0 < 1:
            raise ValueError('the prompt needs at least one token')
        if (capa.n_tablas * capa.n_bits) % 4 or capa.confirmar % 4:
            raise ValueError('the generation step reads its caches as float4 rows: n_tablas * n_bits and confirmar '
                             'must be multiples of 4')
        partes = {}
        y = capa._adelante(E, h, piezas, partes)
        self.cap = max(L0 + 1, capacidad)
        f32 = torch.float32
        self.cache = {
            'phi': _reservar(partes['phi'].to(f32), self.cap), 'V': _reservar(partes['V'].to(f32), self.cap),
            'Qc': _reservar(partes['Qc'].to(f32), self.cap), 'Kc': _reservar(partes['Kc'].to(f32), self.cap),
            'sig': _reservar(partes['sig'].to(f32), self.cap), 'Bt': _reservar(partes['Bt'].double(), self.cap),
            'log_alfa': _reservar(partes['log_alfa'].to(f32), self.cap)}
        n = L0 - 1 if self.ajeno else L0
        self.anillos, self.cuentas = ops.ring_build(partes['phi'][:, :n].to(f32).contiguous(), capa.n_tablas,
                                                    capa.n_bits, capa.chunk)
        self.hawkes = ops.HawkesTable.load(partes['claves'], partes['orden_k'], partes['repetido'], partes['hawkes'],
                                           partes['Bt'], partes['log_alfa'], cap=2 * self.cap)
        self.racha = partes['racha'][:, -1].to(f32).contiguous().clone()
        self.e_ult = E[:, -1]
        self.t = L0
        return y

    def _crecer(self):
        self.cap *= 2
        self.cache = {k: _reservar(v, self.cap) for k, v in self.cache.items()}

    @torch.no_grad()
    def paso(self, e_t, h_t, pieza_t):
        """One new token at position t: e_t, h_t (B, d) its embedding and layer input, pieza_t (B,) its id ->
        the layer's output (B, d) (the layer part of asrn/nucleo.py:1797-1854)."""
        capa = self.capa
        # rows of a (B, L, d) text are strided views; the GEMMs below want dense (B, d) operands (a batch stride
        # above 2^25 elements is outside what hipBLASLt accepts, and its fallback costs ~20 ms per call)
        e_t, h_t = e_t.contiguous(), h_t.contiguous()
        if self.t >= self.cap:
            self._crecer()
        c, t = self.cache, self.t
        c['sig'][:, t] = pieza_t.to(torch.float32)
        c['V'][:, t - 1] = capa.v(e_t)                                        # V[t-1] = W_v e_t
        c['phi'][:, t] = capa._phi(torch.stack([self.e_ult, e_t], 1))[:, -1]
        Qc, Kc, beta, log_alfa = capa._contexto(h_t.unsqueeze(1))
        c['Qc'][:, t], c['Kc'][:, t], c['log_alfa'][:, t] = Qc[:, 0], Kc[:, 0], log_alfa[:, 0]
        kappa, kappa_r = capa._kappas()
        vistos, hawkes = self.hawkes.step(c, t, beta[:, 0], capa.c_vistos, kappa, kappa_r, self.racha)
        salida, sen, _ = ops.decode_attend(c, t, self.anillos, self.cuentas, capa.w_sufijo, capa.gamma, self._forma(),
                                           insert=not self.ajeno)
        acc = {'salida': salida.unsqueeze(1).to(e_t.dtype), 'senales': sen[:, None],
               'vistos': vistos.unsqueeze(1), 'hawkes': hawkes.unsqueeze(1), 'racha': self.racha.unsqueeze(1).clone()}
        y = capa._combinar(acc, h_t.unsqueeze(1))[:, 0]
        self.e_ult = e_t
        self.t += 1
        return y


LayerWriter = EscritorCapa
