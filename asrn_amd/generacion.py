"""Generation with the whole model on the device: the model's O(1) step and the generation loop. The drop-in for the
reference's _Escritor (model part) and escribir (asrn/nucleo.py:1717-1854, 1965-2043).

EscritorModelo keeps, besides each ASRN layer's EscritorCapa state, each local block's last k - 1 LayerNorm rows (the
causal convolution's window) and, for mezcla='memoria', its per-channel memory, so one new token costs the same work
whatever the text length. A 'conv' block's step in fp32 is three fused kernels (asrn_block_step) that stream its
three weight matrices once for all rows, its window a ring indexed by the position. (The reference's step leaves the
'memoria' blocks' memory out, nucleo:1811-1814; here the step equals the whole-text model for both block kinds.)

escribir keeps the text, the n-gram sets behind the quote mask and the no-repeat bans, and the stop flags on the
device, and makes each token's choice with one kernel (ops.muestrear: penalty, bans, quote mask, temperature, top-k,
top-p, the quote-mass correction, the draw). After one eager step, a whole loop step (the choice, the model's step,
the position's advance) is captured in one HIP graph and replayed, so the host only launches replays: no per-token
sync, no host dictionaries. The draws come from a counter-based generator seeded by `semilla` (the reference draws
with a CPU torch.Generator): token streams equal the reference's where the choice is deterministic (greedy, top_k=1);
sampled ones follow the same distribution, not the same random stream.
"""
import torch
import torch.nn.functional as F

from . import ops
from .escritura import EscritorCapa
from .modelo import _base, revisar_precision


def _ventana_inicial(z, k):
    """(B, d, k - 1): the last k - 1 rows of z (B, L, d), zeros before the text's start."""
    return F.pad(z, (0, 0, k - 1, 0))[:, z.shape[1]:].transpose(1, 2).contiguous()


class EscritorModelo:
    """Step-by-step writer of a ModeloASRN (see the module docstring). inicio(x0) runs the prompt and returns the last
    position's logits (B, V); paso(pieza) takes the next token ids (B,) and returns the logits after it."""

    def __init__(self, modelo, memoria_de_lo_ajeno=True):
        self.m = _base(modelo)
        self.ajeno = memoria_de_lo_ajeno
        self.capas = [EscritorCapa(c, memoria_de_lo_ajeno) for c in self.m.largos]

    def bytes_anillos(self, B):
        return sum(c.bytes_anillos(B) for c in self.capas)

    @torch.no_grad()
    def inicio(self, x0, capacidad=0):
        m = self.m
        B, L0 = x0.shape
        if L0 < 1:
            raise ValueError('the prompt needs at least one token')
        self.cap = max(L0 + 1, capacidad)
        E = m.emb(x0)
        h = E
        self.ventanas, self.memorias, self.anillos, self.fusion = [], [], [], []
        if hasattr(self, 'espacio'):
            del self.espacio
        capas = iter(self.capas)
        for i, blq in enumerate(m.bloques):
            z = blq.ln1(h)
            ventana = _ventana_inicial(z, blq.k)
            # the fused step keeps the window as a ring: position t at slot t mod (k - 1)
            fusion = ops.paso_bloque_ok(blq, h[:, -1])
            anillo = None
            if fusion and blq.k > 1:
                anillo = torch.empty_like(ventana)
                anillo[:, :, (L0 + torch.arange(blq.k - 1, device=x0.device)) % (blq.k - 1)] = ventana
            self.ventanas.append(None if fusion else ventana)
            self.anillos.append(anillo)
            self.fusion.append(fusion)
            if fusion and not hasattr(self, 'espacio'):
                self.espacio = ops.espacio_bloque(B, blq.ln1.weight.shape[0], blq.ff[0].weight.shape[0], x0.device)
            if blq.mezcla == 'memoria':
                u, f = blq.mem(z).float().chunk(2, dim=-1)
                f = torch.sigmoid(f) * blq.f_max
                mem = ops.escaneo(f.transpose(1, 2).contiguous(), ((1 - f) * u).transpose(1, 2).contiguous())
                self.memorias.append(mem[..., -1].contiguous())
            h = blq(h)
            if i in m.pos_largo:
                h = next(capas).inicio(E, h, x0, capacidad=self.cap)
        self.e_ult = E[:, -1].contiguous()
        # the last block's end and the final norm in one launch (ops.norma_pendiente) when that block is fused
        self.norma_final = bool(self.fusion) and self.fusion[-1] and ops.norma_pendiente_ok(m.ln_f, h.shape[-1],
                                                                                              x0.device)
        self.cuenta_pos = torch.zeros(1, dtype=torch.int32, device=x0.device)   # the final norm's advance count
        self.avanzado = False
        self.t = L0
        self.pos = torch.full((1,), L0, dtype=torch.int64, device=x0.device)
        return m.head(m.ln_f(h[:, -1]))

    def _bloque(self, i, blq, h, mem_i, pos, previo=None, terminar=True):
        """Block i's step on the new token's state h (B, d) at position pos: six fused kernels for 'conv' blocks in
        fp32 (asrn_block_step, the window a ring), else PyTorch ops on a window that shifts by one row. previo and
        terminar (fused blocks): the pending block before this one and whether to leave this one pending, as
        ops.paso_bloque takes them."""
        if self.fusion[i]:
            if not ops.paso_bloque_ok(blq, h if previo is None else previo.out):
                raise ValueError('EscritorModelo: the prompt ran the fused block step (fp32, no autocast); every step '
                                 'must run the same way')
            return ops.paso_bloque(blq, h, self.anillos[i], pos, self.espacio, previo=previo, terminar=terminar)
        z = blq.ln1(h)
        ventana = torch.cat([self.ventanas[i], z.unsqueeze(-1)], dim=-1)            # (B, d, k)
        if blq.mezcla == 'conv':
            c = F.linear(ventana.flatten(1), blq.conv.weight.flatten(1), blq.conv.bias)
        else:
            c = (ventana * blq.conv.weight[:, 0, :]).sum(-1) + blq.conv.bias
        self.ventanas[i].copy_(ventana[..., 1:])
        c = F.gelu(c)
        if blq.mezcla == 'memoria':
            u, f = blq.mem(z).float().chunk(2, dim=-1)
            f = torch.sigmoid(f) * blq.f_max
            mem = self.memorias[mem_i]
            mem.copy_(f * mem + (1 - f) * u)
            c = c + blq.mem_o(mem.to(z.dtype))
        h = h + c
        return h + blq.ff(blq.ln2(h))

    def _cuerpo(self, pieza, pos, t_max, texto=None, out=None, avanzar=False):
        """The token ids pieza (B,) at position pos (a one-element device tensor, at most t_max) -> logits (B, V).
        texto: the loop's text (B, >= pos) holding the previous tokens: the previous row is looked up from it
        (asrn_embed_step, with this step's) instead of being copied from the last step, and e_ult is then not kept.
        out: a (B, V) fp32 buffer the head's product writes into. avanzar: advance pos by one in the final norm's
        launch when it takes the last block (self.avanzado then says it did)."""
        m = self.m
        emb = m.emb.weight
        if (texto is not None and torch.is_tensor(pos) and emb.dtype == torch.float32 and emb.is_contiguous()
                and m.emb.padding_idx is None and m.emb.max_norm is None):
            e_t, e_prev = ops.embed_step(emb, pieza, texto, pos)
        else:
            e_t, e_prev = m.emb(pieza), None
        h = e_t
        e_ant = self.e_ult if e_prev is None else e_prev
        # every ASRN layer's rows that act on the embedding rows, in one launch pair before the first block
        ls, cs = [c.capa for c in self.capas], [c.cache for c in self.capas]
        producido = bool(ls) and torch.is_tensor(pos) and ops.decode_produce_e_ok(ls, cs, e_t)
        if producido:
            ops.decode_produce_e(ls, cs, e_t, e_ant, pieza, pos, t_max=t_max)
        capas = iter(self.capas)
        k = 0
        pendiente = None
        nb = len(m.bloques)
        for i, blq in enumerate(m.bloques):
            # a fused block's last launch is done by the next kernel that reads its output: the next block's first
            # when that is fused too, the ASRN layer's producer when one follows (with the embedding rows produced),
            # the final norm after the last block
            if i in m.pos_largo:
                encadenar = self.fusion[i] and producido
            elif i + 1 < nb:
                encadenar = self.fusion[i] and self.fusion[i + 1]
            else:
                encadenar = self.fusion[i] and self.norma_final
            r = self._bloque(i, blq, h, k, pos, previo=pendiente, terminar=not encadenar)
            pendiente, h = (r, None) if encadenar else (None, r)
            k += blq.mezcla == 'memoria'
            if i in m.pos_largo:
                h = next(capas)._cuerpo(e_t, e_ant, h, pieza, pos, t_max=t_max, producido=producido, previo=pendiente)
                pendiente = None
        if e_prev is None:
            self.e_ult.copy_(e_t)
        self.avanzado = avanzar and pendiente is not None
        x = m.ln_f(h) if pendiente is None else ops.norma_pendiente(
            m.ln_f, pendiente, avance=(pos, self.cuenta_pos) if self.avanzado else None)
        if (out is not None and m.head.bias is None and x.dtype == out.dtype == m.head.weight.dtype
                and not torch.is_autocast_enabled(x.device.type)):
            return torch.mm(x, m.head.weight.t(), out=out)
        return m.head(x)

    def reservar(self, posiciones):
        """Caches and tables sized for `posiciones` positions (what a captured step must not outgrow)."""
        while self.cap < posiciones:
            self.cap *= 2
            for c in self.capas:
                c._crecer()
        for c in self.capas:
            c.cap = self.cap
            c.hawkes.reserve(self.cap)

    @torch.no_grad()
    def paso(self, pieza):
        """Eager step: the next token ids (B,) -> logits (B, V); caches grow as needed."""
        if self.t >= self.cap:
            self.reservar(self.t + 1)
        self.pos.fill_(self.t)
        lg = self._cuerpo(pieza.view(-1), self.pos, self.cap - 1)
        self.t += 1
        return lg


class _Bucle:
    """The generation loop's state on the device and its step: choose a token from the current logits, run the
    model's step on it, advance the position. The step is captured once in a HIP graph (after one eager step) and
    replayed."""

    def __init__(self, esc, x, n_nuevos, temperatura, top_k, semilla, pena, ventana, no_repetir, parar_en, top_p,
                 devolver_logits, conservar_cita, grafo):
        m = esc.m
        dev = x.device
        B, L0 = x.shape
        V = m.config['V']
        self.esc, self.B, self.V, self.L0, self.n = esc, B, V, L0, n_nuevos
        self.total = L0 + n_nuevos
        self.texto = torch.empty((B, self.total), dtype=torch.int64, device=dev)
        self.texto[:, :L0] = x
        self.piezas = torch.zeros(B, dtype=torch.int64, device=dev)
        self.terminado = torch.zeros(B, dtype=torch.uint8, device=dev)
        self.paso_fin = torch.full((B,), -1, dtype=torch.int32, device=dev)
        self.trabajo = torch.empty((B, V), dtype=torch.float32, device=dev)
        self.bits = torch.empty((B, (V + 31) // 32), dtype=torch.int32, device=dev)
        self.logits = torch.empty((B, n_nuevos, V), dtype=torch.float32, device=dev) if devolver_logits else None
        self.cita = None
        if conservar_cita:
            self.cita = ops.ConjuntoNgramas(B, m.largos[0].vistos, V, self.total, dev)
            self.cita.agregar_texto(x)
        self.prohibidas = ops.ConjuntoNgramas(B, no_repetir, V, n_nuevos, dev) if no_repetir else None
        self.args = dict(temperatura=temperatura, top_k=top_k, top_p=top_p, pena=pena, ventana=ventana,
                         semilla=semilla, parar_en=parar_en)
        self.lg = torch.empty((B, V), dtype=torch.float32, device=dev)
        self.grafo = grafo
        self.g = None

    def elegir(self):
        ops.muestrear(self.lg, self.texto, self.esc.pos, self.total - 1, self.L0, self.piezas, self.terminado,
                      self.paso_fin, self.trabajo, self.bits, cita=self.cita, prohibidas=self.prohibidas,
                      logits=self.logits, **self.args)

    def _paso_completo(self):
        self.elegir()
        lg = self.esc._cuerpo(self.piezas, self.esc.pos, self.esc.cap - 1, texto=self.texto, out=self.lg,
                              avanzar=True)
        if lg.data_ptr() != self.lg.data_ptr():
            self.lg.copy_(lg)
        if not self.esc.avanzado:                  # else the final norm's launch advanced it
            self.esc.pos.add_(1)

    def paso(self, k):
        """Step k: choose token k, then (k < n - 1) run the model on it."""
        esc = self.esc
        if k == self.n - 1:
            self.elegir()
            return
        if not self.grafo or k == 0:
            self._paso_completo()
        else:
            if self.g is None:
                torch.cuda.current_stream().synchronize()
                self.g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.g):
                    self._paso_completo()
            self.g.replay()
        esc.t += 1


@torch.no_grad()
def escribir(modelo, inicio, n_nuevos=200, temperatura=0.8, top_k=40, semilla=0, memoria_de_lo_ajeno=True,
             pena_repeticion=1.0, ventana_pena=64, no_repetir_ngramas=0, parar_en=None, top_p=1.0,
             devolver_logits=True, conservar_cita=True, grafo=True):
    """Writes n_nuevos tokens after `inicio` (batch, length) or (length,), with the reference's arguments and return
    value (asrn/nucleo.py:1965-1991): (full sequences, logits of every step (batch, steps, V)) on the CPU, or
    (sequences, None) with devolver_logits=False. memoria_de_lo_ajeno: the ASRN layers copy only from the prompt.
    parar_en: the token that ends a text (later positions are filled with it; generation stops when every text has
    ended). top_p < 1: nucleus sampling (the most probable token always stays). no_repetir_ngramas=n: no n-gram is
    written twice (a step where that bans every token goes unbanned). conservar_cita: temperature and top-k/top-p do
    not change the probability of following a quote (closing an n-gram of the text, n = the first layer's vistos),
    which stays the model's at temperature 1. grafo=False launches every step from the host (the same arithmetic)."""
    modelo = _base(modelo)
    estaba = modelo.training
    try:
        return _escribir(modelo, inicio, n_nuevos, temperatura, top_k, semilla, memoria_de_lo_ajeno, pena_repeticion,
                         ventana_pena, no_repetir_ngramas, parar_en, top_p, devolver_logits, conservar_cita, grafo)
    finally:
        modelo.train(estaba)


def _escribir(modelo, inicio, n_nuevos, temperatura, top_k, semilla, ajeno, pena, ventana, no_repetir, parar_en, top_p,
              devolver_logits, conservar_cita, grafo):
    modelo.eval()
    revisar_precision(modelo)
    disp = next(modelo.parameters()).device
    if disp.type != 'cuda':
        raise RuntimeError('asrn_amd.escribir runs on the GPU only: move the model to a cuda device')
    x = torch.as_tensor(inicio).to(disp)
    if x.dim() == 1:
        x = x.unsqueeze(0)
    x = x.long().contiguous()
    B, L0 = x.shape
    if L0 < 1:
        raise AssertionError('at least one prompt token is needed')
    V = modelo.config['V']
    lo, hi = int(x.min()), int(x.max())
    if lo < 0 or hi >= V:
        raise ValueError(f'inicio: token ids outside [0, {V}) (min {lo}, max {hi}): check that the tokenizer is the '
                         'model\'s')
    if parar_en is not None and not 0 <= int(parar_en) < V:
        raise ValueError(f'parar_en={parar_en}: a token id in [0, {V})')
    if n_nuevos < 0 or no_repetir_ngramas_invalido(no_repetir):
        raise ValueError(f'n_nuevos={n_nuevos} and no_repetir_ngramas={no_repetir} must be >= 0')
    esc = EscritorModelo(modelo, ajeno)
    lg = esc.inicio(x, capacidad=L0 + n_nuevos)
    if n_nuevos == 0:
        return x.cpu(), (torch.zeros(B, 0, V) if devolver_logits else None)
    esc.reservar(L0 + n_nuevos)
    bucle = _Bucle(esc, x, n_nuevos, temperatura, top_k, semilla, pena, ventana, no_repetir, parar_en, top_p,
                   devolver_logits, conservar_cita, grafo)
    bucle.lg.copy_(lg)
    hechos = n_nuevos
    for k in range(n_nuevos):
        bucle.paso(k)
        # every text ended: the reference stops after that step; checked every 16 steps (one sync), the length is
        # then cut back to the step where the last text ended
        if parar_en is not None and (k % 16 == 15 or k == n_nuevos - 1) and bool(bucle.terminado.all()):
            hechos = int(bucle.paso_fin.max()) + 1
            break
    texto = bucle.texto[:, :L0 + hechos]
    if not devolver_logits:
        return texto.cpu(), None
    return texto.cpu(), bucle.logits[:, :hechos].cpu()


def no_repetir_ngramas_invalido(n):
    return not isinstance(n, int) or isinstance(n, bool) or n < 0


generate = escribir
