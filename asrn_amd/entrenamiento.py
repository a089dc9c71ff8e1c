"""Training around the HIP ASRN layers: AdamW groups, the learning-rate curve, the graphed training step, evaluation
and the training loop. The drop-in for the reference's crear_optimizador / tasa_aprendizaje / PasoGrafado / evaluar /
entrenar (asrn/nucleo.py:2143-2642) on one MI355X.

Same arguments, same batches for the same seed (windows drawn by a CPU generator), same optimizer groups and
numbering, same training-state files (they resume in either implementation). One process only: FSDP and the other
multi-GPU options are not part of this package, and torch.compile is not used (the hot path is HIP already).
PasoGrafado replays the whole step (forward, backward, clipping, fused AdamW) as one HIP graph.
"""
import math
import numbers
import os
import time
import warnings

import torch

from . import archivo, ops
from .modelo import _base

# the suffix and gate parameters of each ASRN layer learn this many times faster (asrn/nucleo.py:2188-2189)
PESOS_SUFIJO_Y_PUERTA = ('w_sufijo', 'g.bias', 'g_conf.weight', 'g_conf.bias')
MULT_SUFIJO_Y_PUERTA = 3.0


def _rapidos(base):
    """ids of the PESOS_SUFIJO_Y_PUERTA parameters of every ASRN layer of `base`."""
    return {id(p) for capa in getattr(base, 'largos', ()) for n, p in capa.named_parameters()
            if n in PESOS_SUFIJO_Y_PUERTA}


def grupos_optimizador(base, mult=MULT_SUFIJO_Y_PUERTA):
    """[(names, parameters, with weight decay, rate multiplier)] in the optimizer's numbering order
    (asrn/nucleo.py:2203-2218): matrices, then the rest; with mult != 1 the suffix and gate parameters form their own
    groups after those (their matrices, then the rest). Parameters without gradients are left out."""
    rapidos = _rapidos(base) if float(mult) != 1.0 else set()
    claves = [(True, False), (False, False), (True, True), (False, True)]
    grupos = {c: ([], []) for c in claves}
    for n, p in base.named_parameters():
        if p.requires_grad:
            nombres, ps = grupos[(p.dim() >= 2, id(p) in rapidos)]
            nombres.append(n)
            ps.append(p)
    return [(nombres, ps, decae, float(mult) if rapido else 1.0)
            for (decae, rapido), (nombres, ps) in ((c, grupos[c]) for c in claves) if ps or not rapido]


def nombres_en_optimizador(modelo, mult=MULT_SUFIJO_Y_PUERTA):
    """The parameter names in the order crear_optimizador numbers them."""
    return [n for nombres, _, _, _ in grupos_optimizador(_base(modelo), mult) for n in nombres]


def crear_optimizador(modelo, lr=1e-3, decaimiento=0.1, betas=(0.9, 0.95), capturable=False,
                      mult_sufijo_y_puerta=MULT_SUFIJO_Y_PUERTA):
    """AdamW (asrn/nucleo.py:2234-2250): weight decay on matrices only; the suffix and gate parameters at
    mult_sufijo_y_puerta times the rate. Every group carries its 'mult' (a schedule sets lr * mult). Fused on the GPU;
    capturable=True for PasoGrafado."""
    base = _base(modelo)
    grupos = [dict(params=ps, weight_decay=decaimiento if decae else 0.0, mult=m, lr=lr * m)
              for _, ps, decae, m in grupos_optimizador(base, mult_sufijo_y_puerta)]
    opciones = {}
    if capturable:
        opciones['capturable'] = True
    if next(base.parameters()).is_cuda:
        opciones['fused'] = True
    try:
        return torch.optim.AdamW(grupos, lr=lr, betas=betas, **opciones)
    except (RuntimeError, TypeError):
        return torch.optim.AdamW(grupos, lr=lr, betas=betas)


def tasa_aprendizaje(paso, lr, pasos, calentamiento, lr_min):
    """Linear warm-up over `calentamiento` steps, then a half cosine from lr down to lr_min at `pasos`
    (asrn/nucleo.py:2346-2352)."""
    if paso < calentamiento:
        return lr * (paso + 1) / calentamiento
    x = min(1.0, (paso - calentamiento) / max(1, pasos - calentamiento))
    return lr_min + (lr - lr_min) * 0.5 * (1.0 + math.cos(math.pi * x))


def elegir_precision(precision, disp):
    """'auto' -> bf16 on the GPU (fp16 where bf16 is missing), fp32 on the CPU."""
    if precision == 'auto':
        if disp.type != 'cuda':
            return 'fp32'
        return 'bf16' if torch.cuda.is_bf16_supported() else 'fp16'
    if precision not in ('fp32', 'bf16', 'fp16'):
        raise ValueError(f"precision={precision!r}: 'auto', 'fp32', 'bf16' or 'fp16'")
    return precision


def autocast(precision, disp, cache=True):
    tipo = dict(bf16=torch.bfloat16, fp16=torch.float16).get(precision)
    return torch.autocast(device_type=disp.type, dtype=tipo, enabled=tipo is not None, cache_enabled=cache)


def entropia(logits, y, reduccion='mean'):
    """fp32 cross-entropy of logits (..., V) against y (...) (asrn/nucleo.py:2301): on the GPU by ops.cross_entropy,
    which reads bf16 logits as they are."""
    return ops.cross_entropy(logits, y, reduction=reduccion)


class PasoGrafado:
    """The whole training step (forward, backward, gradient clipping, AdamW) on batches of one fixed shape, replayed
    as one HIP graph (asrn/nucleo.py:2253-2343):

        opt = crear_optimizador(modelo, lr, capturable=True)
        paso = PasoGrafado(modelo, opt, lote, largo)
        perdida, norma, salto = paso(x, y, lr=...)       # device tensors; read them only when logging

    The first `calentar` calls are ordinary steps, run on a side stream (they build AdamW's state and the layers'
    workspaces); the next call captures one step and every later call replays it. A step with a non-finite loss or
    gradient norm changes nothing (the fused AdamW's found_inf), salto = 1. bf16 or fp32; no checkpointing, no
    torch.compile, no accumulation. grabar=False runs every step eagerly (the same arithmetic; also on the CPU)."""

    def __init__(self, modelo, optimizador, lote, largo, precision='bf16', recorte=1.0, calentar=3, grabar=None):
        base = _base(modelo)
        disp = next(base.parameters()).device
        grabar = (disp.type == 'cuda') if grabar is None else bool(grabar)
        if grabar and disp.type != 'cuda':
            raise ValueError('PasoGrafado: a graph needs the model on the GPU (or grabar=False)')
        if precision == 'fp16':
            raise ValueError("PasoGrafado: fp16 needs a gradient scaler; use 'bf16' or 'fp32'")
        if modelo is not base or getattr(base, 'checkpoint', 'no') != 'no':
            raise ValueError('PasoGrafado: no checkpointing and no torch.compile')
        if grabar and not all(g.get('capturable') and g.get('fused') for g in optimizador.param_groups):
            raise ValueError('PasoGrafado: the optimizer must be crear_optimizador(..., capturable=True) on the GPU')
        self.modelo, self.opt, self.precision, self.disp, self.grabar = base, optimizador, precision, disp, grabar
        self.recorte = recorte or float('inf')
        self.calentar, self.hechos, self.grafo, self.salida = calentar, 0, None, None
        self.params = [p for p in base.parameters() if p.requires_grad]
        self.x = torch.zeros((lote, largo), dtype=torch.long, device=disp)
        self.y = torch.zeros_like(self.x)
        self.lrs = []
        if grabar:
            # the rate lives in device tensors, so a schedule needs no new capture
            base_lr = float(optimizador.param_groups[0]['lr']) / optimizador.param_groups[0].get('mult', 1.0)
            for g in optimizador.param_groups:
                g['lr'] = torch.tensor(base_lr * g.get('mult', 1.0), device=disp)
                self.lrs.append((g['lr'], g.get('mult', 1.0)))
            self.lr = self.lrs[0][0]

    def _uno(self):
        with autocast(self.precision, self.disp, cache=not self.grabar):
            logits = self.modelo(self.x)
        perdida = entropia(logits, self.y)
        perdida.backward()
        norma = torch.nn.utils.clip_grad_norm_(self.params, self.recorte)
        salto = (~(torch.isfinite(perdida) & torch.isfinite(norma))).float()
        if self.opt.param_groups[0].get('fused'):
            self.opt.found_inf = salto               # read by the fused kernel on the device: no host sync
            try:
                self.opt.step()
            finally:
                del self.opt.found_inf
        elif not bool(salto):
            self.opt.step()
        return perdida.detach(), norma.detach(), salto

    def _poner_lr(self, lr):
        if self.grabar:
            for t, m in self.lrs:
                t.fill_(lr * m)
        else:
            for g in self.opt.param_groups:
                g['lr'] = lr * g.get('mult', 1.0)

    def _calentando(self):
        lado = torch.cuda.Stream()
        lado.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(lado):
            self.opt.zero_grad(set_to_none=True)
            r = self._uno()
        torch.cuda.current_stream().wait_stream(lado)
        self.hechos += 1
        return r

    def _capturar(self):
        # gradients start as None: inside the graph they are assigned, not accumulated
        self.opt.zero_grad(set_to_none=True)
        self.grafo = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.grafo):
            self.salida = self._uno()

    def __call__(self, x, y, lr=None):
        """x, y (lote, largo) -> (loss, gradient norm, skipped) as device tensors."""
        self.x.copy_(x, non_blocking=True)
        self.y.copy_(y, non_blocking=True)
        if lr is not None:
            self._poner_lr(lr)
        if not self.grabar:
            self.opt.zero_grad(set_to_none=True)
            return self._uno()
        if self.hechos < self.calentar:
            return self._calentando()
        if self.grafo is None:
            self._capturar()
        self.grafo.replay()
        return self.salida


# ---------------------------------------------------------------------------------------------------------------------
# data, evaluation, the training loop
# ---------------------------------------------------------------------------------------------------------------------

def _revisar_enteros(minimo=1, **valores):
    for n, v in valores.items():
        if isinstance(v, bool) or not isinstance(v, numbers.Integral) or v < minimo:
            raise ValueError(f'{n}={v!r}: an integer >= {minimo} is needed')


def preparar_datos(datos, V, largo, disp):
    """A 1-D tensor of token ids in [0, V), stored as int32; moved to the GPU when it holds under 2**31 bytes."""
    datos = torch.as_tensor(datos)
    if datos.dim() != 1 or datos.is_floating_point() or datos.dtype == torch.bool:
        raise ValueError(f'datos: a 1-D tensor of token ids is needed (got {datos.dtype} {tuple(datos.shape)})')
    if datos.numel() <= largo + 1:
        raise ValueError(f'more than {largo + 1} tokens are needed (got {datos.numel()})')
    lo, hi = int(datos.min()), int(datos.max())
    if lo < 0 or hi >= V:
        raise ValueError(f'token ids outside [0, {V}): min {lo}, max {hi}')
    datos = datos.to(torch.int32)
    if disp.type == 'cuda' and datos.numel() * 4 < 2 ** 31:
        datos = datos.to(disp)
    return datos


def lote_al_azar(datos, largo, lote, g, disp):
    """`lote` windows of largo + 1 tokens at starts drawn by the CPU generator g: (x, y), y shifted by one
    (asrn/nucleo.py:2173-2179)."""
    ini = torch.randint(0, datos.numel() - largo, (lote,), generator=g)
    idx = ini[:, None] + torch.arange(largo + 1)
    w = datos[idx.to(datos.device)].to(disp, non_blocking=True).long()
    return w[:, :-1], w[:, 1:]


@torch.no_grad()
def evaluar(modelo, datos, largo=512, lote=16, max_lotes=50, precision='auto'):
    """Mean loss and perplexity over consecutive windows from the start of `datos` (asrn/nucleo.py:2355-2378)."""
    _revisar_enteros(largo=largo, lote=lote, max_lotes=max_lotes)
    base = _base(modelo)
    disp = next(base.parameters()).device
    datos = preparar_datos(datos, base.config['V'], largo, disp)
    precision = elegir_precision(precision, disp)
    estaba = base.training
    base.eval()
    inicios = torch.arange(0, datos.numel() - largo, largo)[:lote * max_lotes]
    suma = torch.zeros((), dtype=torch.float64, device=disp)
    n = 0
    for grupo in inicios.split(lote):
        w = datos[(grupo[:, None] + torch.arange(largo + 1)).to(datos.device)].to(disp).long()
        with autocast(precision, disp):
            logits = base(w[:, :-1])
        suma += entropia(logits, w[:, 1:], 'sum').double()
        n += w[:, 1:].numel()
    base.train(estaba)
    perdida = float(suma) / max(n, 1)
    return {'perdida': perdida, 'perplejidad': math.exp(min(perdida, 50)), 'piezas': n}


def entrenar(modelo, datos, validacion=None, largo=512, lote=16, pasos=10000, lr=1e-3, lr_min=None,
             calentamiento=None, decaimiento=0.1, betas=(0.9, 0.95), recorte=1.0, acumular=1, precision='auto',
             compilar=False, evaluar_cada=500, lotes_eval=50, guardar_en=None, guardar_cada=1000, reanudar=None,
             semilla=0, registrar_cada=50, registro=print, max_saltos=20, mult_sufijo_y_puerta=None):
    """Trains `modelo` on its device with random windows of `datos` (1-D token ids), with the reference's arguments
    and behaviour (asrn/nucleo.py:2453-2642) in one process: per step `acumular` batches of `lote` windows of `largo`
    tokens; linear warm-up (default 2% of the steps, at most 2000) then a cosine to lr_min (default lr/10); precision
    'auto' / 'fp32' / 'bf16' / 'fp16' (with a gradient scaler); a step with a non-finite loss or norm is skipped (more
    than max_saltos in a row stop the run); recorte is a max norm (0/None: none) or a callable that clips after each
    backward and returns the norm; validacion is evaluated every evaluar_cada steps. guardar_en='m.pt' writes the
    training state every guardar_cada steps and at the end (loadable by cargar(), resumable with reanudar=) and the
    best model by validation to 'm.mejor.pt'. Ctrl+C saves and returns. Returns the history."""
    base = _base(modelo)
    disp = next(base.parameters()).device
    if compilar:
        warnings.warn('entrenar: compilar is ignored; the ASRN layers run as HIP kernels', stacklevel=2)
    if torch.distributed.is_available() and torch.distributed.is_initialized() and torch.distributed.get_world_size() > 1:
        raise ValueError('entrenar: one process per model; several processes are not supported by this package')
    _revisar_enteros(largo=largo, lote=lote, acumular=acumular, evaluar_cada=evaluar_cada, lotes_eval=lotes_eval,
                     guardar_cada=guardar_cada, registrar_cada=registrar_cada)
    _revisar_enteros(minimo=0, pasos=pasos, max_saltos=max_saltos)
    V = base.config['V']
    datos = preparar_datos(datos, V, largo, disp)
    if validacion is not None:
        validacion = preparar_datos(validacion, V, largo, disp)
    precision = elegir_precision(precision, disp)
    if disp.type == 'cuda':
        torch.backends.cuda.matmul.allow_tf32 = True
        torch.backends.cudnn.allow_tf32 = True
    lr_min = lr / 10 if lr_min is None else lr_min
    calentamiento = max(1, calentamiento) if calentamiento is not None else min(2000, max(1, pasos // 50))
    mult = MULT_SUFIJO_Y_PUERTA if mult_sufijo_y_puerta is None else float(mult_sufijo_y_puerta)
    previo = None
    if reanudar:
        previo = archivo.leer(reanudar)
        if 'optimizador' not in previo and 'optimizador_nombres' not in previo:
            raise ValueError(f'{reanudar} holds weights only (written by guardar()); resuming needs the guardar_en '
                             'file of entrenar(), which also holds AdamW and the step. To start a new run from those '
                             'weights: entrenar(cargar(file), ...) without reanudar')
        del_archivo = float(previo.get('ajustes', {}).get('mult_sufijo_y_puerta', 1.0))
        if mult_sufijo_y_puerta is None:
            mult = del_archivo
        elif mult != del_archivo:
            raise ValueError(f'{reanudar} was trained with mult_sufijo_y_puerta={del_archivo:g} and {mult:g} was '
                             'asked: the AdamW groups differ. Resume without mult_sufijo_y_puerta or start anew')
    opt = crear_optimizador(base, lr, decaimiento, betas, mult_sufijo_y_puerta=mult)
    escalador = torch.amp.GradScaler(disp.type, enabled=precision == 'fp16')
    g = torch.Generator(device='cpu').manual_seed(semilla)
    ajustes = dict(pasos=pasos, lr=lr, lr_min=lr_min, calentamiento=calentamiento, largo=largo, lote=lote,
                   acumular=acumular, decaimiento=decaimiento, mult_sufijo_y_puerta=mult)
    paso, mejor_val, historial = 0, float('inf'), []
    if previo is not None:
        paso, mejor_val, historial = archivo.reanudar_entrenamiento(base, opt, escalador, g, previo)
        distintos = {k: (previo['ajustes'][k], v) for k, v in ajustes.items()
                     if k in previo.get('ajustes', {}) and previo['ajustes'][k] != v}
        if distintos:
            registro('warning: these settings differ from the file (then -> now): '
                     + ', '.join(f'{k} {a} -> {b}' for k, (a, b) in distintos.items())
                     + '. The learning-rate curve follows the new ones')
        if paso >= pasos:
            registro(f'warning: the file is at step {paso} and pasos={pasos}: nothing left to train')
        registro(f'resuming from step {paso} ({reanudar})')
        previo = None
    registro(f'ASRN (HIP): {base.num_parametros():,} parameters | {datos.numel():,} tokens | precision {precision} | '
             f'{lote * acumular * largo:,} tokens per step | {disp}')
    mejor_archivo = None
    if guardar_en:
        raiz, ext = os.path.splitext(guardar_en)
        mejor_archivo = f'{raiz}.mejor{ext or ".pt"}'

    def guardar_estado(paso_):
        if guardar_en:
            archivo.guardar_entrenamiento(guardar_en, base, opt, escalador, paso_, mejor_val, g, historial, ajustes)

    base.train()
    saltos, t0, vistas, suma, cuenta = 0, time.time(), 0, 0.0, 0
    try:
        while paso < pasos:
            lr_t = tasa_aprendizaje(paso, lr, pasos, calentamiento, lr_min)
            for grupo in opt.param_groups:
                grupo['lr'] = lr_t * grupo.get('mult', 1.0)
            acumulada = torch.zeros((), device=disp)
            for _ in range(acumular):
                x, y = lote_al_azar(datos, largo, lote, g, disp)
                with autocast(precision, disp):
                    logits = base(x)
                p = entropia(logits, y)
                escalador.scale(p / acumular).backward()
                acumulada += p.detach() / acumular
            perdida = float(acumulada)
            norma = float('nan')
            if math.isfinite(perdida):
                escalador.unscale_(opt)
                if callable(recorte):
                    norma = float(recorte())
                else:
                    norma = float(torch.nn.utils.clip_grad_norm_(base.parameters(), recorte or float('inf')))
            if not math.isfinite(perdida) or (precision != 'fp16' and not math.isfinite(norma)):
                opt.zero_grad(set_to_none=True)
                saltos += 1
                registro(f'step {paso}: loss {perdida}, norm {norma}: step skipped ({saltos} in a row)')
                if saltos > max_saltos:
                    raise RuntimeError('too many NaN/inf steps in a row: lower lr or check the data')
                paso += 1
                continue
            saltos = 0
            escalador.step(opt)
            escalador.update()
            opt.zero_grad(set_to_none=True)
            paso += 1
            vistas += lote * acumular * largo
            suma, cuenta = suma + perdida, cuenta + 1
            if paso % registrar_cada == 0 or paso == pasos:
                dt = max(time.time() - t0, 1e-9)
                fila = {'paso': paso, 'perdida': suma / cuenta, 'lr': lr_t, 'norma': norma, 'piezas_s': vistas / dt}
                historial.append(fila)
                registro(f"step {paso:>7} | loss {fila['perdida']:.4f} | lr {lr_t:.2e} | norm {norma:.2f} | "
                         f"{fila['piezas_s']:,.0f} tokens/s")
                t0, vistas, suma, cuenta = time.time(), 0, 0.0, 0
            if validacion is not None and (paso % evaluar_cada == 0 or paso == pasos):
                ev = evaluar(base, validacion, largo, lote, lotes_eval, precision)
                historial.append({'paso': paso, 'val_perdida': ev['perdida'], 'val_perplejidad': ev['perplejidad']})
                mejor = ev['perdida'] < mejor_val
                if mejor:
                    mejor_val = ev['perdida']
                    if mejor_archivo:
                        archivo.guardar(base, mejor_archivo)
                registro(f"   validation: loss {ev['perdida']:.4f} | perplexity {ev['perplejidad']:.2f}"
                         + ('  (best)' if mejor else ''))
            if guardar_en and paso % guardar_cada == 0:
                guardar_estado(paso)
    except KeyboardInterrupt:
        registro(f'interrupted at step {paso}' + (f': saved to {guardar_en}' if guardar_en else ''))
    guardar_estado(paso)
    base.eval()
    return historial


train, evaluate = entrenar, evaluar
