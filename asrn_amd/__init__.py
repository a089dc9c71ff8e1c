"""asrn_amd: the ASRN layer's data-parallel hot path, MI355X-native (HIP kernels for gfx950 behind a C ABI).

The public names mirror the reference package (KIROKOWA/ASRN, asrn/__init__.py:83-97) for the layer this build
replaces: ASRNLayer / CapaASRNEstable, Protecciones / Protections, convertir / convert, firmas_de_piezas and
escaneo, plus EscritorCapa / LayerWriter, the layer's O(1) generation step, and ngramas, one n-gram sort shared by
every layer of a model.
"""
from . import ops, synth
from ._lib import ASRNHipError, LIB_PATH, load
from .capa import ASRNLayer, CapaASRNEstable, Protecciones, Protections, convertir, firmas_de_piezas, ngramas
from .escritura import EscritorCapa, LayerWriter
from .ops import escaneo

__version__ = '0.1.0'

convert = convertir

__all__ = ['ASRNLayer', 'CapaASRNEstable', 'EscritorCapa', 'LayerWriter', 'Protecciones', 'Protections', 'convertir',
           'convert', 'firmas_de_piezas', 'ngramas', 'escaneo', 'ops', 'load', 'LIB_PATH', 'ASRNHipError', '__version__']
