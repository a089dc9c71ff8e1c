"""Loader for the golden fixtures under tests/golden (data only: inputs, state_dict, stage outputs, gradients)."""
import glob
import json
import os

from safetensors import safe_open

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def names():
    return sorted(os.path.basename(f)[:-len('.safetensors')] for f in glob.glob(os.path.join(GOLDEN, '*.safetensors')))


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
