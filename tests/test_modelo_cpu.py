"""The model API on the CPU against fixtures the reference wrote (tests/golden/make_golden_modelo.py): the weights
create_model(semilla) gives (asrn/nucleo.py:1047-1120, asrn/__init__.py:60-64), the named sizes' parameter counts
(nucleo:1285-1294), the AdamW groups and their numbering (nucleo:2192-2250), the learning-rate curve
(nucleo:2346-2352), the training batches (nucleo:2173-2179), and checkpoints in the v89, v86, v83 and training-state
layouts loaded as the reference's cargar() loads them (nucleo:2050-2133). No GPU: nothing here runs an ASRN layer."""
import hashlib
import json
import os
import tempfile

import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import load_file

import asrn_amd
from asrn_amd import archivo, entrenamiento
from asrn_amd.modelo import ConfigASRN, conv_canal_causal, conv_causal

AQUI = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'modelo')
with open(os.path.join(AQUI, 'modelo.json')) as _f:
    FIX = json.load(_f)
REDUCIDA = dict(n_tablas=2, tablas_contexto=1, n_bits=6, afin_oculto=16, confirmar=4, vistos=2, nodos_racha=4)


def _sha(t):
    return hashlib.sha256(t.detach().contiguous().numpy().tobytes()).hexdigest()


def _json(x):
    return json.loads(json.dumps(x))


@pytest.mark.parametrize('nombre', sorted(FIX['construccion']))
def test_construction_matches_reference_bit_for_bit(nombre):
    caso = FIX['construccion'][nombre]
    m = asrn_amd.crear_modelo(**caso['kw'])
    sd = m.state_dict()
    assert sorted(sd) == sorted(caso['estado']), 'state_dict names differ'
    for k, v in sd.items():
        ref = caso['estado'][k]
        assert list(v.shape) == ref['shape'] and str(v.dtype) == ref['dtype'], k
        assert _sha(v) == ref['sha256'], f'{k}: weights differ from the reference for this seed'
    assert _json(m.config) == caso['config']
    assert m.num_parametros() == caso['num_parametros']
    assert m.pos_largo == caso['pos_largo'] and m.init_profundo == caso['init_profundo']
    assert m.head.weight is m.emb.weight


def test_construction_leaves_the_same_generator_state():
    """A seed's later draws (dropout, data) follow the construction: the generator must end where the reference's
    does, which the weights of a second model built right after show."""
    torch.manual_seed(0)
    asrn_amd.crear_modelo(V=256, d=64, n_capas=4)
    a = torch.rand(4)
    torch.manual_seed(0)
    ModeloSinSemilla = asrn_amd.ModeloASRN(256, 64, 4, 2)
    b = torch.rand(4)
    assert torch.equal(a, b) and ModeloSinSemilla.num_parametros() == FIX['construccion']['cfg0']['num_parametros']


@pytest.mark.parametrize('nombre', sorted(FIX['tallas']))
def test_named_sizes_and_parameter_counts(nombre):
    ref = FIX['tallas'][nombre]
    cfg = asrn_amd.TALLAS[nombre]
    assert _json(cfg.a_dict()) == ref['config']
    assert cfg.contar_parametros(desglose=True) == ref['desglose']
    assert cfg.contar_parametros() == ref['desglose']['total']
    meta = asrn_amd.crear_desde_config(nombre, dispositivo='meta')
    assert meta.num_parametros() == ref['desglose']['total']


@pytest.mark.parametrize('mult', sorted(FIX['grupos']))
def test_optimizer_groups_and_numbering(mult):
    ref = FIX['grupos'][mult]
    m = asrn_amd.crear_modelo(V=256, d=64, n_capas=4, semilla=0)
    assert entrenamiento.nombres_en_optimizador(m, float(mult)) == ref['nombres']
    opt = asrn_amd.crear_optimizador(m, lr=2e-3, decaimiento=0.05, mult_sufijo_y_puerta=float(mult))
    got = [{'n': len(g['params']), 'lr': g['lr'], 'weight_decay': g['weight_decay'], 'mult': g['mult'],
            'betas': list(g['betas']), 'eps': g['eps']} for g in opt.param_groups]
    assert got == ref['grupos']
    nombre = {id(p): n for n, p in m.named_parameters()}
    assert [nombre[id(p)] for g in opt.param_groups for p in g['params']] == ref['nombres']


def test_learning_rate_curve():
    for caso in FIX['tasa']:
        assert asrn_amd.tasa_aprendizaje(*caso['args']) == caso['valor'], caso['args']


def test_training_batches_follow_the_seed():
    t = load_file(os.path.join(AQUI, 'lotes.safetensors'))
    cpu = torch.device('cpu')
    datos = entrenamiento.preparar_datos(t['datos'], 50, 64, cpu)
    g = torch.Generator(device='cpu').manual_seed(4)
    for i in range(2):
        x, y = entrenamiento.lote_al_azar(datos, 64, 3, g, cpu)
        assert torch.equal(x, t[f'x{i}']) and torch.equal(y, t[f'y{i}'])


def test_data_checks():
    cpu = torch.device('cpu')
    with pytest.raises(ValueError, match='1-D'):
        entrenamiento.preparar_datos(torch.zeros(3, 3, dtype=torch.long), 10, 2, cpu)
    with pytest.raises(ValueError, match='more than'):
        entrenamiento.preparar_datos(torch.zeros(5, dtype=torch.long), 10, 8, cpu)
    with pytest.raises(ValueError, match='outside'):
        entrenamiento.preparar_datos(torch.tensor([0, 1, 12, 3, 4, 5]), 10, 2, cpu)
    with pytest.raises(ValueError, match='1-D'):
        entrenamiento.preparar_datos(torch.rand(100), 10, 2, cpu)


# ---------------------------------------------------------------------------------------------------------------------
# checkpoints
# ---------------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize('cual', ['v89', 'v86', 'v83', 'entrenar'])
def test_reference_checkpoints_load_as_the_reference_loads_them(cual):
    m = asrn_amd.cargar(os.path.join(AQUI, f'ckpt_{cual}.pt'), dispositivo='cpu')
    ref = load_file(os.path.join(AQUI, f'ckpt_{cual}_cargado.safetensors'))
    sd = m.state_dict()
    assert set(sd) == set(ref)
    for k in sd:
        assert sd[k].dtype == ref[k].dtype and torch.equal(sd[k], ref[k]), k
    assert not m.training
    assert isinstance(m.largos[0], asrn_amd.CapaASRNEstable)


def test_v86_streak_migration_is_the_increments():
    r = archivo.leer(os.path.join(AQUI, 'ckpt_v86.pt'))
    pesos, cambiados = archivo.migrar(r['pesos'])
    assert sorted(cambiados) == sorted(k[:-len('u_racha')] + 'd_racha' for k in r['pesos'] if k.endswith('u_racha'))
    for n in cambiados:
        u = r['pesos'][n[:-len('d_racha')] + 'u_racha']
        assert torch.equal(pesos[n][0], u[0]) and torch.equal(pesos[n][1:], u[1:] - u[:-1])
    assert 'u_racha' not in ''.join(pesos)


def test_save_load_round_trip_and_layout():
    m = asrn_amd.crear_modelo(V=40, d=16, n_capas=3, largo_cada=1, semilla=2, **REDUCIDA)
    with tempfile.TemporaryDirectory() as tmp:
        ruta = os.path.join(tmp, 'sub', 'm.pt')
        asrn_amd.guardar(m, ruta)
        assert os.listdir(os.path.dirname(ruta)) == ['m.pt']
        r = torch.load(ruta, map_location='cpu', weights_only=True)
        assert set(r) == {'config', 'pesos'} and r['config'] == m.config
        ref = torch.load(os.path.join(AQUI, 'ckpt_v89.pt'), map_location='cpu', weights_only=True)
        assert set(r['config']) == set(ref['config'])
        m2 = asrn_amd.cargar(ruta, 'cpu')
        for k, v in m.state_dict().items():
            assert torch.equal(v, m2.state_dict()[k]), k
        assert m2.head.weight is m2.emb.weight
        # loading does not move torch's generator
        torch.manual_seed(5)
        a = torch.rand(3)
        torch.manual_seed(5)
        asrn_amd.cargar(ruta, 'cpu')
        assert torch.equal(torch.rand(3), a)


def test_load_errors():
    with tempfile.TemporaryDirectory() as tmp:
        with pytest.raises(FileNotFoundError):
            asrn_amd.cargar(os.path.join(tmp, 'nada.pt'), 'cpu')
        ruta = os.path.join(tmp, 'x.pt')
        torch.save({'otra': 1}, ruta)
        with pytest.raises(ValueError, match='not a model'):
            asrn_amd.cargar(ruta, 'cpu')
        r = torch.load(os.path.join(AQUI, 'ckpt_v89.pt'), map_location='cpu', weights_only=True)
        r['pesos']['largos.0.extra'] = torch.zeros(2)
        torch.save(r, ruta)
        with pytest.raises(ValueError, match='unexpected'):
            asrn_amd.cargar(ruta, 'cpu')
        r['pesos'].pop('largos.0.extra')
        r['pesos'].pop('bloques.0.conv.weight')
        torch.save(r, ruta)
        with pytest.raises(ValueError, match='missing'):
            asrn_amd.cargar(ruta, 'cpu')


def test_training_state_layout_and_resume_from_reference_file():
    with open(os.path.join(AQUI, 'ckpt_entrenar.json')) as f:
        ref = json.load(f)
    r = archivo.leer(os.path.join(AQUI, 'ckpt_entrenar.pt'))
    m = archivo.modelo_de_config(dict(r['config']))
    opt = asrn_amd.crear_optimizador(m, lr=1e-3, mult_sufijo_y_puerta=r['ajustes']['mult_sufijo_y_puerta'])
    esc = torch.amp.GradScaler('cpu', enabled=False)
    g = torch.Generator(device='cpu').manual_seed(123)
    paso, mejor, hist = archivo.reanudar_entrenamiento(m, opt, esc, g, r)
    assert paso == ref['paso'] == 2 and mejor == float('inf') and len(hist) == 2
    for k, v in r['pesos'].items():
        assert torch.equal(m.state_dict()[k], v), k
    assert torch.equal(g.get_state(), r['azar'])
    assert len(opt.state) == ref['n_estado_opt']
    sd = opt.state_dict()
    for i, st in r['optimizador']['state'].items():
        for k, v in st.items():
            assert torch.equal(sd['state'][i][k], v), (i, k)
    with tempfile.TemporaryDirectory() as tmp:
        ruta = os.path.join(tmp, 'e.pt')
        archivo.guardar_entrenamiento(ruta, m, opt, esc, paso, mejor, g, hist, r['ajustes'])
        propio = torch.load(ruta, map_location='cpu', weights_only=True)
        assert sorted(propio) == ref['claves']
        assert propio['version'] == ref['version'] and propio['ajustes'] == ref['ajustes']
        assert _json(propio['optimizador']['param_groups']) == ref['grupos']
        m2 = asrn_amd.cargar(ruta, 'cpu')
        for k, v in m.state_dict().items():
            assert torch.equal(m2.state_dict()[k], v)


# ---------------------------------------------------------------------------------------------------------------------
# configuration, blocks, argument checks
# ---------------------------------------------------------------------------------------------------------------------

def test_config_validation_and_round_trips():
    cfg = ConfigASRN(V=1000, d=128, n_capas=6)
    assert cfg.con(d=256).d == 256 and cfg.con(d=256).ff is None
    assert ConfigASRN.desde_dict(cfg.a_dict()) == cfg
    assert ConfigASRN(V=2, checkpoint=True).checkpoint == 'asrn'
    m = asrn_amd.crear_desde_config(ConfigASRN(V=50, d=16, n_capas=3, largo_cada=1, **REDUCIDA), semilla=0)
    assert ConfigASRN.desde_modelo(m) == ConfigASRN(V=50, d=16, n_capas=3, largo_cada=1, init_profundo=False,
                                                    **REDUCIDA)
    viejo = dict(m.config, opciones_capa={'n_tablas': 2, 'tablas_contexto': 1})
    c = ConfigASRN.desde_config_guardada(viejo)
    assert c.n_tablas == 2 and c.n_bits == 14 and c.ff is None
    malos = [dict(V=1), dict(V=10, d=0), dict(V=10, n_capas=1), dict(V=10, ff=0), dict(V=10, dropout=1.0),
             dict(V=10, tablas_contexto=8), dict(V=10, n_bits=31), dict(V=10, chunk=0), dict(V=10, nodos_racha=1),
             dict(V=10, mezcla='otra'), dict(V=10, memoria_max=1), dict(V=10.0), dict(V=10, d=True),
             dict(V=10, checkpoint='a veces')]
    for kw in malos:
        with pytest.raises(ValueError):
            ConfigASRN(**kw)
    with pytest.raises(ValueError, match='unknown'):
        ConfigASRN.desde_dict({'V': 10, 'otro': 1})


@pytest.mark.parametrize('k', [1, 3, 4])
def test_causal_convolution_as_one_gemm(k):
    torch.manual_seed(k)
    z = torch.randn(3, 11, 8, dtype=torch.float64, requires_grad=True)
    conv = torch.nn.Conv1d(8, 8, k).double()
    ref = conv(F.pad(z.transpose(1, 2), (k - 1, 0))).transpose(1, 2)
    out = conv_causal(z, conv.weight, conv.bias)
    assert torch.allclose(out, ref, rtol=0, atol=1e-13)
    g = torch.randn_like(ref)
    a = torch.autograd.grad((ref * g).sum(), [z, conv.weight, conv.bias])
    b = torch.autograd.grad((out * g).sum(), [z, conv.weight, conv.bias])
    for x, y in zip(a, b):
        assert torch.allclose(x, y, rtol=0, atol=1e-12)
    dw = torch.nn.Conv1d(8, 8, k, groups=8).double()
    ref = dw(F.pad(z.transpose(1, 2), (k - 1, 0))).transpose(1, 2)
    assert torch.allclose(conv_canal_causal(z, dw.weight, dw.bias), ref, rtol=0, atol=1e-13)


def test_model_argument_checks():
    with pytest.raises(ValueError):
        asrn_amd.ModeloASRN(10, n_capas=1)
    with pytest.raises(ValueError):
        asrn_amd.ModeloASRN(2 ** 24 + 1, d=4)
    with pytest.raises(ValueError):
        asrn_amd.BloqueLocal(8, mezcla='otra')
    m = asrn_amd.crear_modelo(V=20, d=8, n_capas=2, **REDUCIDA)
    m.checkpoint = True
    assert m.checkpoint == 'asrn'
    with pytest.raises(ValueError):
        m.checkpoint = 'x'
    m.to(torch.bfloat16)
    with pytest.raises(ValueError, match='fp32 weights'):
        m(torch.zeros(1, 4, dtype=torch.long))
    m2 = asrn_amd.crear_modelo(V=20, d=8, n_capas=2, **REDUCIDA)
    with pytest.raises(RuntimeError, match='GPU only'):
        m2(torch.zeros(1, 4, dtype=torch.long))


def test_graphed_step_argument_checks():
    m = asrn_amd.crear_modelo(V=20, d=8, n_capas=2, **REDUCIDA)
    opt = asrn_amd.crear_optimizador(m)
    with pytest.raises(ValueError, match='fp16'):
        asrn_amd.PasoGrafado(m, opt, 2, 8, precision='fp16', grabar=False)
    with pytest.raises(ValueError, match='GPU'):
        asrn_amd.PasoGrafado(m, opt, 2, 8, grabar=True)
    m.checkpoint = 'asrn'
    with pytest.raises(ValueError, match='checkpoint'):
        asrn_amd.PasoGrafado(m, opt, 2, 8, grabar=False)


def test_public_names_mirror_the_reference():
    for n in ['ASRNLayer', 'ASRNModel', 'ASRNConfig', 'LocalBlock', 'Protections', 'create_model',
              'create_from_config', 'convert', 'train', 'evaluate', 'save', 'load', 'CapaASRNEstable',
              'BloqueLocal', 'ModeloASRN', 'ConfigASRN', 'TALLAS', 'Protecciones', 'PasoGrafado', 'crear_modelo',
              'crear_desde_config', 'cargar', 'guardar', 'convertir', 'crear_optimizador', 'tasa_aprendizaje',
              'entrenar', 'evaluar', 'firmas_de_piezas', 'escaneo', 'MULT_SUFIJO_Y_PUERTA',
              'PESOS_SUFIJO_Y_PUERTA']:
        assert hasattr(asrn_amd, n), n
    assert asrn_amd.load is asrn_amd.cargar and asrn_amd.train is asrn_amd.entrenar
    assert asrn_amd.MULT_SUFIJO_Y_PUERTA == 3.0
