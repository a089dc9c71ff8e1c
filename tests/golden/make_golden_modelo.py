"""Writes the model-level fixtures under tests/golden/modelo/.

The reference (KIROKOWA/ASRN) is imported here, in the build container only, for what only its own code pins:
the weights create_model(semilla) produces (its generator consumption order), the parameter counts of its named
sizes, its AdamW groups, learning-rate curve and batch draws, one whole-model training step's loss and gradients
on the CPU, and checkpoint files written by its guardar()/entrenar() with what its cargar() makes of them. Every
fixture is data (JSON, safetensors, or torch.save files of tensors and plain values); nothing from the reference's
source is stored.

Run from the repository root:  python tests/golden/make_golden_modelo.py /root/reference
"""
import hashlib
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'modelo')
ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

REDUCIDA = dict(n_tablas=2, tablas_contexto=1, n_bits=6, afin_oculto=16, confirmar=4, vistos=2, nodos_racha=4)

# (name, create_model kwargs): constructions whose state_dict hashes are stored
CONSTRUCCIONES = [
    ('cfg0', dict(V=256, d=64, n_capas=4, semilla=0)),
    ('profundo', dict(V=64, d=32, n_capas=8, semilla=3, **REDUCIDA)),
    ('memoria', dict(V=64, d=32, n_capas=3, largo_cada=1, semilla=5, mezcla='memoria', memoria_max=64, **REDUCIDA)),
    ('opciones', dict(V=100, d=48, n_capas=5, largo_cada=3, semilla=7, ff=40, k=3, chunk=16, n_bits=10, sufijo=3,
                      racha_max=100)),
]

# (name, create_model kwargs, B, L, seed of the token stream): one training step each
PASOS = [
    ('paso_cfg0', dict(V=256, d=64, n_capas=4, semilla=0), 8, 256, 0),
    ('paso_memoria', dict(V=64, d=32, n_capas=3, largo_cada=1, semilla=5, mezcla='memoria', memoria_max=64), 2, 96, 1),
]

CKPT = dict(V=32, d=16, n_capas=3, largo_cada=1, semilla=1, **REDUCIDA)


def sha(t):
    return hashlib.sha256(t.detach().contiguous().cpu().numpy().tobytes()).hexdigest()


def huellas(sd):
    return {k: {'shape': list(v.shape), 'dtype': str(v.dtype), 'sha256': sha(v)} for k, v in sd.items()}


def mover(modelo, nuevos, seed):
    """Moves every parameter off its initial value (the new ones more), so migrations are not vacuous."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for n, p in modelo.named_parameters():
            p.add_(torch.randn(p.shape, generator=g) * (0.5 if n.rsplit('.', 1)[-1] in nuevos else 0.05))
        for c in modelo.largos:
            c.gamma.abs_()


def build(ref_root):
    sys.path.insert(0, ref_root)
    sys.path.insert(0, ROOT)
    os.environ['ASRN_TRITON'] = '0'
    import asrn
    import asrn.nucleo as v89
    from asrn_amd import synth

    os.makedirs(HERE, exist_ok=True)
    out = {'construccion': {}, 'tallas': {}, 'grupos': {}, 'tasa': [], 'lotes': {}}

    for name, kw in CONSTRUCCIONES:
        m = asrn.crear_modelo(**kw)
        out['construccion'][name] = {'kw': kw, 'config': m.config, 'num_parametros': m.num_parametros(),
                                     'pos_largo': m.pos_largo, 'init_profundo': m.init_profundo,
                                     'estado': huellas(m.state_dict())}

    for name, cfg in asrn.TALLAS.items():
        out['tallas'][name] = {'config': cfg.a_dict(), 'desglose': cfg.contar_parametros(desglose=True)}

    m = asrn.crear_modelo(V=256, d=64, n_capas=4, semilla=0)
    for mult in (3.0, 1.0, 2.5):
        opt = asrn.crear_optimizador(m, lr=2e-3, decaimiento=0.05, mult_sufijo_y_puerta=mult)
        out['grupos'][str(mult)] = {
            'nombres': v89._nombres_en_optimizador(m, mult),
            'grupos': [{'n': len(g['params']), 'lr': g['lr'], 'weight_decay': g['weight_decay'], 'mult': g['mult'],
                        'betas': list(g['betas']), 'eps': g['eps']} for g in opt.param_groups]}

    for args in [(0, 1e-3, 1000, 20, 1e-4), (19, 1e-3, 1000, 20, 1e-4), (20, 1e-3, 1000, 20, 1e-4),
                 (500, 1e-3, 1000, 20, 1e-4), (999, 1e-3, 1000, 20, 1e-4), (1000, 1e-3, 1000, 20, 1e-4),
                 (5000, 3e-4, 1000, 20, 0.0), (0, 1.0, 1, 1, 0.5), (3, 6e-4, 3, 5, 6e-5), (7, 6e-4, 10, 2, 6e-5)]:
        out['tasa'].append({'args': list(args), 'valor': v89.tasa_aprendizaje(*args)})

    datos = torch.randint(0, 50, (5000,), generator=torch.Generator().manual_seed(11))
    g = torch.Generator(device='cpu').manual_seed(4)
    lotes = [v89._lote(v89._preparar_datos(datos, 50, 64, torch.device('cpu')), 64, 3, g, torch.device('cpu'))
             for _ in range(2)]
    save_file({k: v.contiguous() for k, v in dict(datos=datos, x0=lotes[0][0], y0=lotes[0][1], x1=lotes[1][0],
                                                   y1=lotes[1][1]).items()},
              os.path.join(HERE, 'lotes.safetensors'), metadata={'seed': '4', 'largo': '64', 'lote': '3', 'V': '50'})

    with open(os.path.join(HERE, 'modelo.json'), 'w') as f:
        json.dump(out, f, indent=1, sort_keys=True)

    # one training step: loss, pre-clip norm, every gradient (fp32, on the CPU, the reference's PyTorch path)
    for name, kw, B, L, seed in PASOS:
        m = asrn.crear_modelo(**kw)
        m.train()
        w = synth.tokens(B, L + 1, kw['V'], seed=seed)
        x, y = w[:, :-1].contiguous(), w[:, 1:].contiguous()
        perdida = m.perdida(x, y)
        perdida.backward()
        norma = torch.nn.utils.clip_grad_norm_(m.parameters(), float('inf'))
        t = {'x': x, 'y': y, 'perdida': perdida.detach().reshape(1), 'norma': norma.detach().reshape(1)}
        for n, p in m.named_parameters():
            t['g.' + n] = p.grad.clone()
        save_file(t, os.path.join(HERE, name + '.safetensors'), metadata={'kw': json.dumps(kw)})
        print(name, float(perdida.detach()), float(norma))

    # checkpoints: v89 (guardar), v86 (streak per node), v83 (no v86/v87 parameters), entrenar's training state
    torch.manual_seed(0)
    m = asrn.crear_modelo(**CKPT)
    mover(m, v89._NUEVOS_V87, 9)
    if True:
        p89 = os.path.join(HERE, 'ckpt_v89.pt')
        asrn.guardar(m, p89)
        r = torch.load(p89, map_location='cpu', weights_only=True)
        pesos86 = {}
        for k, v in r['pesos'].items():
            if k.endswith('.d_racha'):
                pesos86[k[:-len('d_racha')] + 'u_racha'] = v.cumsum(0)
            else:
                pesos86[k] = v
        torch.save({'config': r['config'], 'pesos': pesos86}, os.path.join(HERE, 'ckpt_v86.pt'))
        pesos83 = {k: v for k, v in r['pesos'].items() if k.rsplit('.', 1)[-1] not in v89._NUEVOS_V87}
        torch.save({'config': r['config'], 'pesos': pesos83}, os.path.join(HERE, 'ckpt_v83.pt'))
        datos = synth.tokens(1, 4000, CKPT['V'], seed=3)[0]
        pe = os.path.join(HERE, 'ckpt_entrenar.pt')
        asrn.entrenar(m, datos, largo=32, lote=2, pasos=2, lr=1e-3, precision='fp32', guardar_en=pe,
                      registrar_cada=1, registro=lambda *a, **k: None, semilla=5)
        for cual in ('v89', 'v86', 'v83', 'entrenar'):
            cargado = asrn.cargar(os.path.join(HERE, f'ckpt_{cual}.pt'), dispositivo='cpu')
            save_file({k: v.clone().contiguous() for k, v in cargado.state_dict().items()},
                      os.path.join(HERE, f'ckpt_{cual}_cargado.safetensors'))
        est = torch.load(pe, map_location='cpu', weights_only=True)
        with open(os.path.join(HERE, 'ckpt_entrenar.json'), 'w') as f:
            json.dump({'claves': sorted(est), 'paso': est['paso'], 'version': est['version'],
                       'ajustes': est['ajustes'], 'n_estado_opt': len(est['optimizador']['state']),
                       'grupos': [{k: v for k, v in g.items() if k != 'params'} | {'params': g['params']}
                                  for g in est['optimizador']['param_groups']]}, f, indent=1, sort_keys=True)
    escritura(asrn, v89)
    for fn in sorted(os.listdir(HERE)):
        print(fn, os.path.getsize(os.path.join(HERE, fn)) // 1024, 'KiB')


ESCRITURA = dict(V=60, d=32, n_capas=3, largo_cada=1, semilla=1, chunk=8, n_bits=3)


def escritura(asrn, v89):
    """The reference's O(1) writer (asrn/nucleo.py:1717-1854) on a teacher-forced text, with and without
    memoria_de_lo_ajeno, the whole-text logits beside it, and one greedy escribir() (top_k=1, nucleo:1965-2043):
    its tokens and the logits of every step."""
    torch.manual_seed(0)
    m = asrn.crear_modelo(**ESCRITURA)
    mover(m, v89._NUEVOS_V87, 7)
    m.eval()
    B, L0, n = 2, 40, 24
    g = torch.Generator().manual_seed(0)
    x = torch.randint(0, ESCRITURA['V'], (B, L0 + n), generator=g)
    x[:, 20:36] = x[:, 2:18].clone()
    out = {'x': x}
    with torch.no_grad():
        for ajeno in (True, False):
            esc = v89._Escritor(m, memoria_de_lo_ajeno=ajeno, o1=True)
            lgs = [esc.inicio(x[:, :L0], capacidad=L0 + 3)] + [esc.paso(x[:, t]) for t in range(L0, L0 + n - 1)]
            out['paso_ajeno' if ajeno else 'paso_todo'] = torch.stack(lgs, 1)
        out['entero'] = m(x[:, :L0 + n - 1])[:, L0 - 1:].contiguous()
        sec, pasos = asrn.escribir(m, x[:, :L0], n_nuevos=n, top_k=1, semilla=0)
    out['greedy'] = sec
    out['greedy_logits'] = pasos
    save_file({k: v.contiguous() for k, v in out.items()}, os.path.join(HERE, 'escritura.safetensors'),
              metadata={'kw': json.dumps(ESCRITURA), 'L0': str(L0), 'n': str(n)})
    torch.manual_seed(0)
    m2 = asrn.crear_modelo(**ESCRITURA)
    mover(m2, v89._NUEVOS_V87, 7)
    for k, v in m2.state_dict().items():
        assert torch.equal(v, m.state_dict()[k])


if __name__ == '__main__':
    build(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
