"""The language model around the HIP ASRN layers: local blocks, tied head, configuration. The drop-in for the
reference's ModeloASRN and its constructors (asrn/nucleo.py:969-1130, 1131-1300, 1384-1397; asrn/__init__.py:60-69).

ModeloASRN(V, d, n_capas, largo_cada, ...) takes the reference's arguments and has its parameter and buffer names
and construction order, so crear_modelo(..., semilla=s) holds the reference's weights for seed s and state_dicts
move between the two. Its ASRN layers are asrn_amd.CapaASRNEstable (group-A protections unless told otherwise), and
one n-gram sort per forward serves all of them (asrn_amd.ngramas). The local blocks and the head are dense work on
hipBLASLt: the causal convolution is one GEMM over the k shifted copies of the block input rather than a convolution
call. Weights stay fp32; 16-bit work goes through autocast, as in the reference (nucleo:1025-1032).
"""
import dataclasses
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .capa import CapaASRNEstable, ngramas
from . import ops
from .ops import escaneo
from .lineal import lineal

MEZCLAS = ('conv', 'memoria')
OPCIONES_CAPA = ('n_tablas', 'n_bits', 'afin_oculto', 'chunk', 'tablas_contexto', 'confirmar', 'sufijo', 'vistos',
                 'nodos_racha', 'racha_max')
MODOS_CHECKPOINT = ('no', 'asrn', 'todo')


def _base(modelo):
    """The module itself when wrapped by torch.compile."""
    return getattr(modelo, '_orig_mod', modelo)


def modo_checkpoint(valor):
    """Recomputation mode of ModeloASRN (asrn/nucleo.py:1017-1022): False and None mean 'no', True means 'asrn'."""
    if not isinstance(valor, str):
        valor = 'asrn' if valor is True else 'no' if valor in (False, None) else valor
    if valor not in MODOS_CHECKPOINT:
        raise ValueError(f"checkpoint: one of 'no', 'asrn', 'todo' (got {valor!r})")
    return valor


def conv_causal(z, peso, sesgo):
    """out[:, t] = sesgo + sum_j peso[:, :, j] z[:, t - k + 1 + j] (positions before 0 read zeros): nn.Conv1d's
    weight layout (d_out, d_in, k) over the left-padded sequence, as one GEMM of (B L, k d_in) by (k d_in, d_out).
    z (B, L, d_in) -> (B, L, d_out)."""
    k = peso.shape[-1]
    if z.is_cuda and z.dtype == torch.float32 and 1 <= k <= 16:
        # the columns written once, in the dtype the GEMM computes in (ops.VentanaCausal)
        dt = torch.get_autocast_dtype('cuda') if torch.is_autocast_enabled('cuda') else torch.float32
        cols = ops.ventana_causal(z, k, dt if dt in (torch.float32, torch.bfloat16) else torch.float32)
    else:
        zp = F.pad(z, (0, 0, k - 1, 0))
        cols = zp.unfold(1, k, 1)                        # (B, L, d_in, k): [b, t, c, j] = zp[b, t + j, c]
        cols = cols.reshape(z.shape[0], z.shape[1], -1)  # (B, L, d_in * k), column c * k + j (one copy)
    return lineal(cols, peso.reshape(peso.shape[0], -1), sesgo)


def conv_canal_causal(z, peso, sesgo):
    """The per-channel (depthwise) version: peso (d, 1, k). k fused multiply-adds over shifted views."""
    k = peso.shape[-1]
    w = peso[:, 0, :].to(z.dtype)
    zp = F.pad(z, (0, 0, k - 1, 0))
    L = z.shape[1]
    out = zp[:, k - 1:k - 1 + L] * w[:, k - 1]
    for j in range(k - 1):
        out = out + zp[:, j:j + L] * w[:, j]
    return out + sesgo.to(z.dtype)


def _dtype_producto(x):
    """The dtype the next product takes x in: autocast's on x's device when enabled, else x's own."""
    dev = x.device.type
    return torch.get_autocast_dtype(dev) if torch.is_autocast_enabled(dev) else x.dtype


class BloqueLocal(nn.Module):
    """Causal local context (asrn/nucleo.py:969-1014): h += GELU(causal conv of LayerNorm(h) over the current and
    k - 1 previous tokens); h += FF(LayerNorm(h)). mezcla='memoria': the convolution is per channel, plus a forgetting
    memory per channel m_t = f_t m_{t-1} + (1 - f_t) u_t, f < f_max = 1 - 1/memoria_max, computed by the library's
    affine scan; channel c starts with a time scale of 10**(c log10(memoria_max) / (d - 1)) tokens."""

    def __init__(self, d, k=4, ff=128, dropout=0.0, mezcla='conv', memoria_max=1024):
        super().__init__()
        if mezcla not in MEZCLAS or memoria_max < 2:
            raise ValueError(f'mezcla={mezcla!r} (one of {MEZCLAS}), memoria_max={memoria_max} (>= 2)')
        self.k, self.mezcla = k, mezcla
        self.f_max = 1.0 - 1.0 / memoria_max
        # creation order fixes what a seed produces: ln1, conv, [mem, mem_o], ln2, ff
        self.ln1 = nn.LayerNorm(d)
        self.conv = nn.Conv1d(d, d, k, groups=d if mezcla == 'memoria' else 1)
        if mezcla == 'memoria':
            self.mem = nn.Linear(d, 2 * d)
            self.mem_o = nn.Linear(d, d, bias=False)
            self._olvido_inicial(d, memoria_max)
        self.ln2 = nn.LayerNorm(d)
        self.ff = nn.Sequential(nn.Linear(d, ff), nn.GELU(), nn.Linear(ff, d))
        self.drop = nn.Dropout(dropout)

    @torch.no_grad()
    def _olvido_inicial(self, d, memoria_max):
        """Forget-gate biases such that f_max * sigmoid(b_c) = 1 - 1/tau_c, tau geometric from 1 to memoria_max."""
        tau = torch.logspace(0, math.log10(memoria_max), d)
        q = ((1 - 1 / tau) / self.f_max).clamp(1e-3, 1 - 1e-3)
        self.mem.bias[d:] = torch.log(q / (1 - q))

    def _memoria(self, z):
        u, f = self.mem(z).float().chunk(2, dim=-1)
        f = torch.sigmoid(f) * self.f_max
        m = escaneo(f.transpose(1, 2).contiguous(), ((1 - f) * u).transpose(1, 2).contiguous())
        return self.mem_o(m.transpose(1, 2).to(z.dtype))

    def forward(self, h):
        # the LayerNorms run fused (ops.norma_residual): ln2's output comes out in the feed-forward's dtype, and the
        # residual path's gradient joins each LayerNorm's backward
        z, h = ops.norma_residual(self.ln1, h, torch.float32)
        if self.mezcla == 'conv':
            c = conv_causal(z, self.conv.weight, self.conv.bias)
        else:
            c = conv_canal_causal(z, self.conv.weight, self.conv.bias)
        c = F.gelu(c)
        if self.mezcla == 'memoria':
            c = c + self._memoria(z)
        h = h + self.drop(c)
        y, h = ops.norma_residual(self.ln2, h, _dtype_producto(h))
        return h + self.drop(self._ff(y))

    def _ff(self, y):
        """self.ff on the library's Linear (lineal: the bias gradients as the library's fixed-order column sums)."""
        f0, act, f2 = self.ff
        return lineal(act(lineal(y, f0.weight, f0.bias)), f2.weight, f2.bias)


@torch.no_grad()
def _escalar_profundo(bloques, largos, n_capas):
    """Deep-model start (asrn/nucleo.py:1036-1046): every projection that writes into the residual stream shrinks by
    1/sqrt(2 n_capas)."""
    f = 1.0 / (2 * n_capas) ** 0.5
    for b in bloques:
        salidas = [b.conv.weight, b.ff[2].weight] + ([b.mem_o.weight] if b.mezcla == 'memoria' else [])
        for w in salidas:
            w.mul_(f)
    for c in largos:
        c.o.weight.mul_(f)


def revisar_precision(modelo):
    """Weights must stay fp32: the layer mixes fp32 and fp64 arithmetic (clock, signatures, n-gram keys)."""
    if modelo.emb.weight.dtype in (torch.float16, torch.bfloat16):
        raise ValueError(f'the model holds {modelo.emb.weight.dtype} weights; ASRN needs fp32 weights. For bf16/fp16 '
                         'work use autocast and keep the model in float32')


class ModeloASRN(nn.Module):
    """Token ids -> n_capas local blocks, with an ASRN layer after block i when i % largo_cada == 0 and i is not the
    last block -> logits through the head, which is the embedding matrix (asrn/nucleo.py:1047-1125). No position table.
    checkpoint: 'asrn' recomputes the ASRN layers in the backward, 'todo' the local blocks too. protecciones: the ASRN
    layers' Protecciones (group A by default); the remaining keywords are CapaASRNEstable's."""

    def __init__(self, V, d=64, n_capas=2, largo_cada=2, ff=None, k=4, init_profundo=None, checkpoint=False,
                 dropout=0.0, mezcla='conv', memoria_max=1024, protecciones=None, **opciones_capa):
        super().__init__()
        if n_capas < 2 or largo_cada < 1:
            raise ValueError(f'n_capas={n_capas} (>= 2), largo_cada={largo_cada} (>= 1)')
        if V > 2 ** 24:
            raise ValueError(f'V={V}: token signatures are exact only up to 2**24 tokens')
        ff = ff or 2 * d
        self.config = dict(V=V, d=d, n_capas=n_capas, largo_cada=largo_cada, ff=ff, k=k, dropout=dropout,
                           mezcla=mezcla, memoria_max=memoria_max, opciones_capa=dict(opciones_capa))
        self.n_capas = n_capas
        self.checkpoint = checkpoint
        self.init_profundo = (n_capas >= 8) if init_profundo is None else bool(init_profundo)
        self.pos_largo = list(range(0, n_capas - 1, largo_cada))
        # creation order fixes what a seed produces: emb (normal, std 0.02), ln_f, head (then tied), blocks, layers
        self.emb = nn.Embedding(V, d)
        nn.init.normal_(self.emb.weight, std=0.02)
        self.ln_f = nn.LayerNorm(d)
        self.head = nn.Linear(d, V, bias=False)
        self.head.weight = self.emb.weight
        self.bloques = nn.ModuleList(BloqueLocal(d, k, ff, dropout, mezcla, memoria_max) for _ in range(n_capas))
        self.largos = nn.ModuleList(CapaASRNEstable(d, protecciones, dropout=dropout, **opciones_capa)
                                    for _ in self.pos_largo)
        if self.init_profundo:
            _escalar_profundo(self.bloques, self.largos, n_capas)

    @property
    def checkpoint(self):
        return self._checkpoint

    @checkpoint.setter
    def checkpoint(self, valor):
        self._checkpoint = modo_checkpoint(valor)

    def estado(self, x):
        """The last block's output, before ln_f and the head: (B, L, d)."""
        revisar_precision(self)
        E = self.emb(x)
        recalcular = self.training and torch.is_grad_enabled()
        ck_bloque = recalcular and self.checkpoint == 'todo'
        ck_capa = recalcular and self.checkpoint != 'no'
        # the n-gram sort depends on the token ids only: one for every ASRN layer
        ng = ngramas(x, self.largos[0]) if len(self.largos) and x.is_cuda else None
        capas = iter(self.largos)
        h = E
        for i, bloque in enumerate(self.bloques):
            h = torch.utils.checkpoint.checkpoint(bloque, h, use_reentrant=False) if ck_bloque else bloque(h)
            if i in self.pos_largo:
                capa = next(capas)
                if ck_capa:
                    h = torch.utils.checkpoint.checkpoint(capa, E, h, x, use_reentrant=False, ngramas=ng)
                else:
                    h = capa(E, h, x, ngramas=ng)
        return h

    def forward(self, x):
        h = self.estado(x)
        y, _ = ops.norma_residual(self.ln_f, h, _dtype_producto(h))
        return self.head(y)

    def perdida(self, x, y, ignorar=-100):
        """Mean fp32 cross-entropy of predicting y from x, both (B, L) (asrn/nucleo.py:1122-1125)."""
        logits = self(x)
        return ops.cross_entropy(logits, y, ignore_index=ignorar)

    def num_parametros(self):
        return sum(p.numel() for p in self.parameters())


def crear_modelo(V, d=64, n_capas=2, largo_cada=2, semilla=None, protecciones=None, **kw):
    """ModeloASRN with the final recipe (asrn/__init__.py:60-64). semilla seeds torch's generator right before the
    construction, so the weights equal the reference's for that seed."""
    if semilla is not None:
        torch.manual_seed(semilla)
    return ModeloASRN(V, d, n_capas, largo_cada, protecciones=protecciones, **kw)


# ---------------------------------------------------------------------------------------------------------------------
# configuration (asrn/nucleo.py:1131-1300)
# ---------------------------------------------------------------------------------------------------------------------

def _entero(v):
    return isinstance(v, int) and not isinstance(v, bool)


@dataclasses.dataclass(frozen=True)
class ConfigASRN:
    """Every choice that defines a ModeloASRN; the defaults are the final recipe. The model fields are ModeloASRN's,
    the rest CapaASRNEstable's."""
    V: int
    d: int = 64
    n_capas: int = 2
    largo_cada: int = 2
    ff: int = None
    k: int = 4
    dropout: float = 0.0
    init_profundo: bool = None
    checkpoint: str = 'no'
    mezcla: str = 'conv'
    memoria_max: int = 1024
    n_tablas: int = 8
    n_bits: int = 14
    afin_oculto: int = 128
    chunk: int = 32
    tablas_contexto: int = 4
    confirmar: int = 16
    sufijo: int = 4
    vistos: int = 4
    nodos_racha: int = 16
    racha_max: int = 256

    def __post_init__(self):
        object.__setattr__(self, 'checkpoint', modo_checkpoint(self.checkpoint))
        self.validar()

    def _problemas(self):
        """What is wrong, as messages; the integer check runs first, since the others compare numbers."""
        no_enteros = [n for n in ('V', 'd', 'n_capas', 'largo_cada', 'k') + OPCIONES_CAPA if not _entero(getattr(self, n))]
        if no_enteros:
            return [f'{n} must be an integer (got {getattr(self, n)!r})' for n in no_enteros]
        reglas = [
            (2 <= self.V <= 2 ** 24, f'V={self.V}: between 2 and 2**24 tokens (signatures are exact up to 2**24)'),
            (self.d >= 1 and self.k >= 1, 'd and k must be >= 1'),
            (self.n_capas >= 2, f'n_capas={self.n_capas}: at least 2 (the ASRN layer sits between blocks)'),
            (self.largo_cada >= 1, 'largo_cada must be >= 1'),
            (self.ff is None or (_entero(self.ff) and self.ff >= 1), f'ff={self.ff!r}: None (= 2d) or an integer >= 1'),
            (0.0 <= self.dropout < 1.0, f'dropout={self.dropout}: in [0, 1)'),
            (0 < self.tablas_contexto < self.n_tablas,
             f'tablas_contexto={self.tablas_contexto}: between 1 and n_tablas-1 (n_tablas={self.n_tablas})'),
            (1 <= self.n_bits <= 30, f'n_bits={self.n_bits}: between 1 and 30'),
        ]
        reglas += [(getattr(self, n) >= 1, f'{n} must be >= 1')
                   for n in ('afin_oculto', 'chunk', 'confirmar', 'sufijo', 'vistos', 'racha_max')]
        reglas += [
            (self.nodos_racha >= 2, 'nodos_racha must be >= 2'),
            (self.mezcla in MEZCLAS, f"mezcla={self.mezcla!r}: one of {', '.join(MEZCLAS)}"),
            (_entero(self.memoria_max) and self.memoria_max >= 2, f'memoria_max={self.memoria_max!r}: an integer >= 2'),
        ]
        return [msg for ok, msg in reglas if not ok]

    def validar(self):
        """Raises ValueError with the first problem found; returns self."""
        problemas = self._problemas()
        if problemas:
            raise ValueError(f'ConfigASRN: {problemas[0]}')
        return self

    def con(self, **cambios):
        """A checked copy with some fields changed: TALLAS['125m'].con(V=8000)."""
        return dataclasses.replace(self, **cambios)

    def opciones_capa(self):
        return {n: getattr(self, n) for n in OPCIONES_CAPA}

    def a_dict(self):
        return dataclasses.asdict(self)

    @classmethod
    def desde_dict(cls, dic):
        campos = {c.name for c in dataclasses.fields(cls)}
        extra = sorted(set(dic) - campos)
        if extra:
            raise ValueError(f'ConfigASRN: unknown fields {extra}')
        return cls(**dic)

    @classmethod
    def desde_modelo(cls, modelo):
        base = _base(modelo)
        return cls.desde_config_guardada(base.config, init_profundo=base.init_profundo, checkpoint=base.checkpoint)

    @classmethod
    def desde_config_guardada(cls, c, **extra):
        """From a model's `config` dict, the one checkpoints hold (asrn/nucleo.py:1233-1239). Layer options the dict
        lacks take their defaults; ff equal to 2d becomes None."""
        capa = dict(cls(V=2).opciones_capa())
        capa.update(c['opciones_capa'])
        modelo = dict(V=c['V'], d=c['d'], n_capas=c['n_capas'], largo_cada=c['largo_cada'], k=c['k'],
                      ff=None if c['ff'] == 2 * c['d'] else c['ff'], dropout=c.get('dropout', 0.0),
                      mezcla=c.get('mezcla', 'conv'), memoria_max=c.get('memoria_max', 1024))
        return cls(**modelo, **extra, **capa)

    def argumentos_modelo(self):
        """ModeloASRN's keyword arguments for this configuration (V, d, n_capas, largo_cada aside)."""
        return dict(ff=self.ff, k=self.k, init_profundo=self.init_profundo, checkpoint=self.checkpoint,
                    dropout=self.dropout, mezcla=self.mezcla, memoria_max=self.memoria_max, **self.opciones_capa())

    def contar_parametros(self, desglose=False):
        """The exact parameter count, from the model built on the 'meta' device (shapes only, no memory).
        desglose=True: {'vocabulario', 'bloques_locales', 'capas_asrn', 'otros', 'total'}; the tied embedding and
        head count once."""
        with torch.device('meta'):
            m = ModeloASRN(self.V, self.d, self.n_capas, self.largo_cada,
                           **{**self.argumentos_modelo(), 'init_profundo': False})
        total = m.num_parametros()
        if not desglose:
            return total
        partes = {'vocabulario': m.emb.weight.numel(),
                  'bloques_locales': sum(p.numel() for p in m.bloques.parameters()),
                  'capas_asrn': sum(p.numel() for p in m.largos.parameters())}
        return {**partes, 'otros': total - sum(partes.values()), 'total': total}


def _reducida(**kw):
    """The small models' ASRN layer: 2 tables of 6 bits, a hash MLP 16 wide."""
    return ConfigASRN(n_tablas=2, tablas_contexto=1, n_bits=6, afin_oculto=16, confirmar=4, vistos=2, nodos_racha=4,
                      **kw)


# the reference's named sizes (asrn/nucleo.py:1285-1294). The HIP layer needs d % 4 == 0, so 'nano-3k' (d = 10)
# builds and loads, but its ASRN layers refuse to run.
TALLAS = {
    'nano-3k': _reducida(V=48, d=10, n_capas=2, ff=24, k=3),
    '12m': ConfigASRN(V=8000, d=256, n_capas=16),
    '30m': ConfigASRN(V=32768, d=384, n_capas=13),
    '125m': ConfigASRN(V=32768, d=768, n_capas=18),
    '350m': ConfigASRN(V=32768, d=1024, n_capas=31),
    '1b': ConfigASRN(V=32768, d=2048, n_capas=27),
    '7b': ConfigASRN(V=32768, d=4096, n_capas=44),
    '27b': ConfigASRN(V=32768, d=8192, n_capas=44),
}


def crear_desde_config(cfg, semilla=None, dispositivo=None, protecciones=None):
    """ModeloASRN from a ConfigASRN or a TALLAS name (asrn/nucleo.py:1384-1397; asrn/__init__.py:67-69).
    dispositivo='meta': shapes only."""
    cfg = TALLAS[cfg] if isinstance(cfg, str) else cfg
    cfg.validar()
    kw = dict(cfg.argumentos_modelo(), protecciones=protecciones)
    if dispositivo is not None and torch.device(dispositivo).type == 'meta':
        with torch.device('meta'):
            return ModeloASRN(cfg.V, cfg.d, cfg.n_capas, cfg.largo_cada, **kw)
    m = crear_modelo(cfg.V, cfg.d, cfg.n_capas, cfg.largo_cada, semilla=semilla, **kw)
    return m if dispositivo is None else m.to(dispositivo)


ASRNModel, LocalBlock, ASRNConfig = ModeloASRN, BloqueLocal, ConfigASRN
create_model, create_from_config = crear_modelo, crear_desde_config
