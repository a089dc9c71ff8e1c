"""The O(1) generation step of one stable ASRN layer on MI355X: the layer part of the reference's _Escritor
(asrn/nucleo.py:1717-1854) with its state on the device.

EscritorCapa(capa, memoria_de_lo_ajeno) keeps, per layer:
  caches      (B, cap, .) rows of phi, V, Qc, Kc, sig, Bt (fp64) and log_alfa, written in place; cap doubles when
              the text outgrows it (asrn/nucleo.py:1733-1745);
  rings       (B*T, 2^nb, C) int32 positions and (B*T, 2^nb) int32 counts: each bucket's C most recent positions
              (asrn/nucleo.py:1585-1618), built from the prompt's stable bucket sort;
  Hawkes      per (text, group) open-addressing tables of (key code, Bu, A) (asrn/nucleo.py:1634-1714);
  racha       (B,) the streak.
inicio() runs the layer over the prompt (its ordinary forward) and builds that state; paso() processes one new token:
asrn_decode_produce writes the token's V, phi, Qc, Kc, log_alfa and signature rows into the caches and returns its
beta (fp32 layers within its widths; otherwise the layer's own producers, PyTorch GEMMs, write those rows);
asrn_decode_attend_repeat then runs, in one launch, the repetition step (the clock advance, the n-gram keys, the
Hawkes lookup/update and the streak) and the attention, which scores the T*C ring candidates (exact softmax,
copy-gather) and inserts the token into the rings when every position may become a key; the gate is the layer's fused
gate kernel with W_o (or the W_o GEMM and the gate kernel). Every step reads a fixed amount, T*C candidates, whatever
the text length.

memoria_de_lo_ajeno=True (the reference default): the keys are only prompt positions k with k + 1 < L0 (their V rows
are values of prompt tokens), so the rings hold positions 0..L0-2 and never change. False: every earlier position is
a key, and the step equals the whole-text layer position by position.

grafo=True: the step is captured once in a HIP graph and replayed, since launching its small kernels from Python
costs several times their GPU time. The position then lives in a one-element device buffer that the kernels read: one
asrn_copy_blocks launch before each replay copies the token's inputs into the graph's input buffers and the position
from a device table of positions (0, 1, ..., cap - 1) into that buffer, so nothing inside the graph advances it. The
first step runs eagerly (it initializes the GEMM libraries' handles), the second is captured, and a capacity doubling
(new cache tensors) captures again. The graph holds the layer's parameters and this writer's state by address:
replacing a parameter tensor (rather than updating it in place) needs a new writer.
"""
import torch

from . import ops


def _reservar(x, cap):
    buf = x.new_zeros((x.shape[0], cap) + tuple(x.shape[2:]))
    buf[:, :x.shape[1]] = x
    return buf


class EscritorCapa:
    """Step-by-step writer for one CapaASRNEstable (see the module docstring)."""

    def __init__(self, capa, memoria_de_lo_ajeno=True, grafo=False):
        self.capa, self.ajeno, self.grafo = capa, memoria_de_lo_ajeno, grafo
        self._g = None

    def _forma(self):
        c = self.capa
        return dict(T=c.n_tablas, Tc=c.tablas_contexto, C=c.chunk, K=c.sufijo, nb=c.n_bits)

    def bytes_anillos(self, B):
        """Device bytes of the rings and counts: (B*T, 2^nb) buckets of C int32 slots and an int32 count. The
        reference sizes its rings as B*T*2^nb*(4*chunk + 8) bytes (int32 slots, int64 counts; asrn/nucleo.py:1747)."""
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
        # the attention's per-row count of column workgroups past their ring reads (zero between launches)
        self.hechos = torch.zeros(self.cuentas.shape[0] // capa.n_tablas, dtype=torch.int32, device=self.cuentas.device)
        self.hawkes = ops.HawkesTable.load(partes['claves'], partes['orden_k'], partes['repetido'], partes['hawkes'],
                                           partes['Bt'], partes['log_alfa'], cap=2 * self.cap)
        self.racha = partes['racha'][:, -1].to(f32).contiguous().clone()
        # both decay rates (capa._kappas' values, without autograd), once: the weights do not change while writing, so
        # a step (and its graph) reads them instead of launching the exponential again
        kappa, kappa_r = torch._foreach_exp([capa.log_kappa, capa.log_kappa_racha])
        if capa.protecciones.kappa_min is not None:
            kappa, kappa_r = kappa.clamp(min=capa.protecciones.kappa_min), kappa_r.clamp(min=capa.protecciones.kappa_min)
        self.kappas = (kappa, kappa_r)
        # (query, table) pairs of the steps where the unprotected layer's -1e9 fill would leak (CapaASRN.fugas)
        self.fugas_t = torch.zeros(1, dtype=torch.int32, device=E.device)
        self.e_ult = E[:, -1]
        self.t = L0
        self._g = None
        self._calentado = False
        return y

    def _crecer(self):
        self.cap *= 2
        self.cache = {k: _reservar(v, self.cap) for k, v in self.cache.items()}

    def _escribir(self, nombre, pos, valor):
        """valor (B, ...) into row pos of cache[nombre]: pos an int, or a one-element device tensor."""
        c = self.cache[nombre]
        if torch.is_tensor(pos):
            c.index_copy_(1, pos, valor.unsqueeze(1).to(c.dtype))
        else:
            c[:, pos] = valor

    def _cuerpo(self, e_t, e_ult, h_t, pieza_t, pos, t_max=None, producido=False, previo=None):
        """One step's work at position pos (an int, or a one-element device buffer holding it, t_max its largest value) ->
        the layer's output (B, d) (the layer part of asrn/nucleo.py:1797-1854). producido: the rows that act on e_t
        (V, phi, sig) are already in the caches (ops.decode_produce_e, for every layer of a model at once). previo
        (with producido): the local block step left pending whose output is h_t (h_t is then None); the producer
        forms it (ops.decode_produce_h)."""
        capa = self.capa
        c = self.cache
        if previo is not None and not producido:
            raise ValueError('EscritorCapa: a pending block step is finished by the producer of decode_produce_e')
        if producido:
            beta_t = ops.decode_produce_h(capa, c, h_t, pos, t_max=t_max, previo=previo)
            if previo is not None:
                h_t = previo.out
        elif ops.decode_produce_ok(capa, e_t):
            # fp32: the token's V, phi, Qc, Kc, log_alfa and id rows in two kernels (asrn_decode_produce)
            beta_t = ops.decode_produce(capa, c, e_t, e_ult, h_t, pieza_t, pos, t_max=t_max)
        else:
            self._escribir('sig', pos, pieza_t.to(torch.float32))
            self._escribir('V', pos - 1, capa.v(e_t))                      # V[t-1] = W_v e_t
            # the token's phi from its own row and the previous one (the context MLP's key), by the whole-text
            # producer
            self._escribir('phi', pos, capa._phi_y_valores(torch.stack([e_ult, e_t], 1))[0][:, -1])
            Qc, Kc, beta, log_alfa = capa._contexto(h_t.unsqueeze(1))
            self._escribir('Qc', pos, Qc[:, 0])
            self._escribir('Kc', pos, Kc[:, 0])
            self._escribir('log_alfa', pos, log_alfa[:, 0])
            beta_t = beta[:, 0]
        kappa, kappa_r = self.kappas
        forma = self._forma()
        if not capa.protecciones.mascara_exacta:          # the -1e9 fill's leak case, counted over the steps
            forma['fuga'] = self.fugas_t
        # the repetition step (clock, Hawkes, streak) and the attention in one launch
        salida, sen, _, vistos, hawkes = ops.decode_attend_repeat(
            c, pos, self.anillos, self.cuentas, capa.w_sufijo, capa.gamma, forma, not self.ajeno, self.hawkes, beta_t,
            capa.c_vistos, kappa, kappa_r, self.racha, t_max=t_max, reloj32=not capa.protecciones.reloj_64,
            hechos=self.hechos)
        if e_t.dtype == torch.float32:
            y = capa._combinar_paso(salida, h_t, sen, vistos, hawkes, self.racha)   # W_o and the gate, one kernel
            if y is not None:
                return y
        acc = {'salida': salida.unsqueeze(1).to(e_t.dtype), 'senales': sen[:, None],
               'vistos': vistos.unsqueeze(1), 'hawkes': hawkes.unsqueeze(1), 'racha': self.racha.unsqueeze(1)}
        return capa._combinar(acc, h_t.unsqueeze(1))[:, 0]

    @torch.no_grad()
    def paso(self, e_t, h_t, pieza_t):
        """One new token at position t: e_t, h_t (B, d) its embedding and layer input, pieza_t (B,) its id ->
        the layer's output (B, d) (the layer part of asrn/nucleo.py:1797-1854)."""
        if self.t >= self.cap:
            self._crecer()
            self._g = None
        if self.grafo and self._calentado:
            return self._paso_grafo(e_t, h_t, pieza_t)     # its dense input buffers take strided rows in one copy
        # rows of a (B, L, d) text are strided views; the GEMMs below want dense (B, d) operands (a batch stride
        # above 2^25 elements is outside what hipBLASLt accepts, and its fallback costs ~20 ms per call)
        e_t, h_t = e_t.contiguous(), h_t.contiguous()
        y = self._cuerpo(e_t, self.e_ult, h_t, pieza_t, self.t)
        self.e_ult = e_t
        self.t += 1
        self._calentado = True
        return y

    def _paso_grafo(self, e_t, h_t, pieza_t):
        if self._g is None:
            self._capturar(e_t, h_t, pieza_t)
        k = self._k
        dev = self._h.device
        if (all(v.device == dev for v in (e_t, h_t, pieza_t)) and e_t.dtype == h_t.dtype == torch.float32
                and pieza_t.dtype == torch.int64 and e_t.shape == self._eb[k].shape and h_t.shape == self._h.shape
                and pieza_t.shape == self._p.shape and e_t.stride(1) == 1 and h_t.stride(1) == 1
                and e_t.stride(0) >= e_t.shape[1] and h_t.stride(0) >= h_t.shape[1] and pieza_t.stride(0) >= 1):
            # the three inputs and the position into the graph's buffers in one launch (the int64 ids and position
            # as pairs of 32-bit words, moved as bits)
            ops.copy_blocks([(e_t, self._eb[k]), (h_t, self._h),
                             (pieza_t.unsqueeze(1).view(torch.float32), self._p.view(torch.float32).view(-1, 2)),
                             (self._posiciones[self.t:self.t + 1].unsqueeze(1).view(torch.float32),
                              self._pos.view(torch.float32).view(1, 2))])
        else:
            self._eb[k].copy_(e_t)
            self._h.copy_(h_t)
            self._p.copy_(pieza_t)
            self._pos.copy_(self._posiciones[self.t:self.t + 1])
        self._g[k].replay()
        self.t += 1
        self.e_ult = self._eb[k]
        self._k = 1 - k
        return self._y[k].clone()

    def _capturar(self, e_t, h_t, pieza_t):
        """Captures the step twice, with the two embedding buffers in swapped roles: graph k reads the token's
        embedding from buffer k and the previous one from buffer 1 - k, so consecutive steps alternate and no copy
        carries e_t over. Its position is the device scalar _pos (valid for positions < cap, the caches' capacity),
        set before each replay from the device table _posiciones = 0, 1, ..., cap - 1."""
        self.hawkes.reserve(self.cap)          # tables sized for every position the graph will see: no growth inside
        self._eb = [torch.empty(e_t.shape, dtype=e_t.dtype, device=e_t.device) for _ in range(2)]
        self._h, self._p = (torch.empty(v.shape, dtype=v.dtype, device=v.device) for v in (h_t, pieza_t))
        self._eb[1].copy_(self.e_ult)
        self._k = 0
        self._posiciones = torch.arange(self.cap, dtype=torch.int64, device=e_t.device)
        self._pos = torch.full((1,), self.t, dtype=torch.int64, device=e_t.device)
        torch.cuda.current_stream(e_t.device).synchronize()
        self._g, self._y = [], []
        for k in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._y.append(self._cuerpo(self._eb[k], self._eb[1 - k], self._h, self._p, self._pos,
                                            t_max=self.cap - 1))
            self._g.append(g)


LayerWriter = EscritorCapa
