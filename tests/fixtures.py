"""Loader for the golden fixtures under tests/golden (data only: inputs, state_dict, stage outputs, gradients)."""
import glob
import json
import os

from safetensors import safe_open

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def names(autocast=None):
    """Fixture names; autocast=None: all, False: the fp32 ones, 'bf16': those written under bf16 autocast."""
    out = []
    for f in sorted(glob.glob(os.path.join(GOLDEN, '*.safetensors'))):
        with safe_open(f, framework='pt') as fh:
            mode = json.loads(fh.metadata()['extra']).get('autocast', False)
        if autocast is None or mode == autocast:
            out.append(os.path.basename(f)[:-len('.safetensors')])
    return out


def load(name):
    path = os.path.join(GOLDEN, name + '.safetensors')
    with safe_open(path, framework='pt') as f:
        t = {k: f.get_tensor(k) for k in f.keys()}
        meta = f.metadata()
    meta = {'d': int(meta['d']), 'B': int(meta['B']), 'L': int(meta['L']), 'V': int(meta['V']),
            'kw': json.loads(meta['kw']), 'extra': json.loads(meta['extra'])}
    params = {k[2:]: v for k, v in t.items() if k.startswith('p.')}
    return t, params, meta


def shape_of(params, meta):
    from oracle.layer import shape_from_params
    kw = dict(meta['kw'])
    extra = {}
    if 'chunk' in kw:
        extra['C'] = kw['chunk']
    return shape_from_params(params, meta['d'], n_bits=kw.get('n_bits', 14), **extra)


def nucleo(meta):
    """Whether a fixture was written by the unprotected core layer (nucleo.CapaASRN, asrn.ASRNCoreLayer)."""
    return meta['extra'].get('clase') == 'nucleo'


def prot(meta):
    """The oracle's protections for a fixture: group A, plus group B (estable:72-77) for a 'textos_largos' case, none
    for a core-layer case."""
    from oracle.layer import Prot
    if nucleo(meta):
        return Prot.ninguna()
    if meta['extra'].get('prot') == 'textos_largos':
        return Prot(tope_puerta=10.0, kappa_min=1.0 / (4 * meta['extra']['largo']))
    return Prot()


def protecciones(meta):
    """The HIP layer's Protecciones for a fixture (the same choice as prot)."""
    from asrn_amd.capa import Protecciones
    if nucleo(meta):
        return Protecciones.ninguna()
    if meta['extra'].get('prot') == 'textos_largos':
        return Protecciones.textos_largos(meta['extra']['largo'])
    return Protecciones()


def cpu_autocast(meta):
    """torch.autocast('cpu', bfloat16) for a fixture written under it, else a no-op context."""
    import contextlib

    import torch
    if meta['extra'].get('autocast') == 'bf16':
        return torch.autocast('cpu', dtype=torch.bfloat16)
    return contextlib.nullcontext()


def stage_input(g, k):
    """A candidate-stage input of a fixture: the stage output of that name, except the clock when the fixture ran its
    candidate stage on a moved clock (acc.Bt)."""
    return g['acc.Bt'] if k == 'Bt' and 'acc.Bt' in g else g[k]
