"""Model and training-state files in the reference's format (asrn/nucleo.py:2050-2133, 2396-2450), so checkpoints
move both ways between this package and the reference.

A model file is torch.save({'config': modelo.config, 'pesos': state_dict}); a training-state file (entrenar's
guardar_en) adds 'optimizador' (AdamW's numbered state_dict), 'escalador', 'paso', 'mejor_val', 'azar' (the batch
generator's state), 'historial', 'ajustes' and 'version'. Files are read with weights_only=True (nothing in them
runs); confiar=True is an explicit opt-in for one's own older files that need more.

Loading migrates files from v83 on. v86 kept the streak response per node ('u_racha'); later versions keep its
increments ('d_racha', the same function, converted exactly). Files from before v86/v87 lack the parameters added
then (NUEVOS_V87); those keep their neutral initial values, so the model computes what it computed in its version.
"""
import os
import tempfile

import torch

from .modelo import ModeloASRN, _base

NUEVOS_V87 = ('w_reloj', 'b_reloj', 'gamma', 'log_kappa', 'log_kappa_racha', 'u_hawkes', 'd_racha')
VERSION = 'asrn_v89'


def escribir_seguro(obj, ruta):
    """torch.save into a unique temporary file in the target's folder, fsync, rename over `ruta`, fsync the folder:
    an interrupted write leaves the previous file whole, and concurrent writers never share a temporary."""
    carpeta = os.path.dirname(os.path.abspath(ruta))
    os.makedirs(carpeta, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=os.path.basename(ruta) + '.', suffix='.tmp', dir=carpeta)
    try:
        with os.fdopen(fd, 'wb') as f:
            torch.save(obj, f)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, ruta)
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise
    try:
        dfd = os.open(carpeta, os.O_RDONLY)
    except OSError:
        return
    try:
        os.fsync(dfd)
    except OSError:
        pass
    finally:
        os.close(dfd)


def guardar(modelo, ruta):
    """Writes the model's config and weights (asrn/nucleo.py:2068-2074)."""
    base = _base(modelo)
    escribir_seguro({'config': base.config, 'pesos': base.state_dict()}, ruta)


def leer(ruta, confiar=False):
    """The dict stored in `ruta`, on the CPU, read with weights_only=True; confiar=True falls back to a full load."""
    if not os.path.isfile(ruta):
        raise FileNotFoundError(f'no such file: {ruta}')
    try:
        return torch.load(ruta, map_location='cpu', weights_only=True)
    except Exception as e:
        if not confiar:
            raise ValueError(f'{ruta}: not readable in safe mode ({type(e).__name__}: {e}). For a file of your own, '
                             'confiar=True loads it in full (it may run code stored in the file)') from e
    return torch.load(ruta, map_location='cpu', weights_only=False)


def _racha_por_incrementos(pesos):
    """v86 -> v87: every '*.u_racha' (per-node values u) becomes '*.d_racha' = (u_0, u_1 - u_0, u_2 - u_1, ...)."""
    convertidos = {}
    for n in [n for n in pesos if n.endswith('.u_racha') or n == 'u_racha']:
        u = pesos.pop(n)
        nuevo = n[:-len('u_racha')] + 'd_racha'
        pesos[nuevo] = torch.diff(u, prepend=torch.zeros_like(u[:1]))
        convertidos[nuevo] = n
    return list(convertidos)


# (what it does, function(pesos) -> names it changed), applied in order to a copy of the weights
MIGRACIONES = [('v86 streak nodes -> v87 increments', _racha_por_incrementos)]


def migrar(pesos):
    """A migrated copy of `pesos` and the names whose meaning changed (their AdamW moments do not carry over)."""
    pesos = dict(pesos)
    cambiados = []
    for _, f in MIGRACIONES:
        cambiados += f(pesos)
    return pesos, cambiados


def cargar_pesos(modelo, pesos):
    """Loads v83+ weights into `modelo`. Only NUEVOS_V87 parameters may be missing; anything else missing or any
    unexpected name raises ValueError."""
    pesos, _ = migrar(pesos)
    faltan, sobran = modelo.load_state_dict(pesos, strict=False)
    ajenos = [n for n in faltan if n.rsplit('.', 1)[-1] not in NUEVOS_V87]
    if ajenos or sobran:
        raise ValueError(f'weights that are not ASRN v83-v89: missing {ajenos}, unexpected {list(sobran)}')
    return modelo


def modelo_de_config(c, protecciones=None):
    """An untrained ModeloASRN for a stored `config` dict, built without touching torch's global generator."""
    with torch.random.fork_rng(devices=[]):
        return ModeloASRN(c['V'], c['d'], c['n_capas'], c['largo_cada'], c['ff'], c['k'], init_profundo=False,
                          dropout=c.get('dropout', 0.0), mezcla=c.get('mezcla', 'conv'),
                          memoria_max=c.get('memoria_max', 1024), protecciones=protecciones, **c['opciones_capa'])


def cargar(ruta, dispositivo=None, confiar=False, protecciones=None):
    """A model written by guardar() or entrenar() (this package's or the reference's, v83 to v89), with the HIP
    layers, in eval mode on `dispositivo` (default: the GPU when there is one) (asrn/nucleo.py:2122-2133;
    asrn/__init__.py:72-74)."""
    r = leer(ruta, confiar)
    if not isinstance(r, dict) or 'config' not in r or 'pesos' not in r:
        raise ValueError(f'{ruta}: not a model written by guardar() or entrenar()')
    m = cargar_pesos(modelo_de_config(dict(r['config']), protecciones), r['pesos'])
    return m.to(dispositivo or ('cuda' if torch.cuda.is_available() else 'cpu')).eval()


# ---------------------------------------------------------------------------------------------------------------------
# training state (asrn/nucleo.py:2396-2450)
# ---------------------------------------------------------------------------------------------------------------------

def _nombres_de(base, opt):
    nombre = {id(p): n for n, p in base.named_parameters()}
    return [nombre[id(p)] for g in opt.param_groups for p in g['params']]


def guardar_entrenamiento(ruta, base, opt, escalador, paso, mejor_val, g, historial, ajustes):
    """Everything entrenar() needs to resume, in the reference's layout."""
    escribir_seguro({'config': base.config, 'pesos': base.state_dict(), 'optimizador': opt.state_dict(),
                     'escalador': escalador.state_dict(), 'paso': paso, 'mejor_val': mejor_val, 'azar': g.get_state(),
                     'historial': historial, 'version': VERSION, 'ajustes': ajustes or {}}, ruta)


def reanudar_entrenamiento(base, opt, escalador, g, r):
    """Restores weights, AdamW, the scaler and the batch generator from a training-state dict `r` (written by one
    process, or by several with the optimizer state by parameter name). Returns (step, best validation loss,
    history)."""
    pesos, migrados = migrar(r['pesos'])
    nombres = _nombres_de(base, opt)
    numero = {n: i for i, n in enumerate(nombres)}
    if 'optimizador_nombres' in r:
        por_nombre = r['optimizador_nombres']
        estado = {numero[n]: st for n, st in por_nombre['state'].items() if n not in migrados}
        grupos = [{**pg, 'params': [numero[n] for n in pg['params']]} for pg in por_nombre['param_groups']]
    else:
        numerado = r['optimizador']
        estado = {i: st for i, st in numerado['state'].items() if nombres[i] not in migrados}
        grupos = numerado['param_groups']
    base.load_state_dict(pesos)
    opt.load_state_dict({'state': estado, 'param_groups': grupos})
    if r.get('escalador'):
        escalador.load_state_dict(r['escalador'])
    azares = r.get('azar_procesos')
    g.set_state(azares[0] if azares and len(azares) == 1 else r['azar'])
    return r['paso'], r['mejor_val'], list(r.get('historial', []))


save, load = guardar, cargar
