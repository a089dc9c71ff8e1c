"""asrn_amd: the ASRN layer's data-parallel hot path, MI355X-native (HIP kernels for gfx950 behind a C ABI), and the
model, training and checkpoint API around it.

The public names mirror the reference package (KIROKOWA/ASRN, asrn/__init__.py:41-97):
  - the layer: ASRNLayer / CapaASRNEstable, ASRNCoreLayer / CapaASRN (the unprotected core layer, v89 numerics),
    Protecciones / Protections, convertir / convert, firmas_de_piezas, escaneo;
  - the model: ModeloASRN / ASRNModel, BloqueLocal / LocalBlock, ConfigASRN / ASRNConfig, TALLAS,
    crear_modelo / create_model, crear_desde_config / create_from_config;
  - training: crear_optimizador, tasa_aprendizaje, PasoGrafado, entrenar / train, evaluar / evaluate;
  - files: guardar / save, cargar / load (the reference's format, v83 on);
  - generation: escribir / generate (the loop on the device), EscritorModelo / ModelWriter (the model's O(1) step),
    EscritorCapa / LayerWriter (one layer's);
  - ngramas, one n-gram sort shared by every layer of a model.
cargar_biblioteca() opens the HIP library (the product has no CPU fallback).
"""
from . import ops, synth
from ._lib import ASRNHipError, LIB_PATH
from ._lib import load as cargar_biblioteca
from .archivo import cargar, guardar
from .capa import (ASRNCoreLayer, ASRNLayer, CapaASRN, CapaASRNEstable, Protecciones, Protections, convertir,
                   firmas_de_piezas, ngramas)
from .entrenamiento import (MULT_SUFIJO_Y_PUERTA, PESOS_SUFIJO_Y_PUERTA, PasoGrafado, crear_optimizador, entrenar,
                            evaluar, tasa_aprendizaje)
from .escritura import EscritorCapa, LayerWriter
from .generacion import EscritorModelo, escribir
from .modelo import TALLAS, BloqueLocal, ConfigASRN, ModeloASRN, crear_desde_config, crear_modelo
from .ops import escaneo

__version__ = '0.2.0'

ASRNModel, ASRNConfig, LocalBlock = ModeloASRN, ConfigASRN, BloqueLocal
create_model, create_from_config, convert = crear_modelo, crear_desde_config, convertir
train, evaluate, save, load, generate = entrenar, evaluar, guardar, cargar, escribir
ModelWriter = EscritorModelo
load_library = cargar_biblioteca

__all__ = ['ASRNLayer', 'CapaASRNEstable', 'ASRNCoreLayer', 'CapaASRN', 'Protecciones', 'Protections', 'convertir', 'convert', 'firmas_de_piezas',
           'ngramas', 'escaneo', 'ModeloASRN', 'ASRNModel', 'BloqueLocal', 'LocalBlock', 'ConfigASRN', 'ASRNConfig',
           'TALLAS', 'crear_modelo', 'create_model', 'crear_desde_config', 'create_from_config', 'crear_optimizador',
           'tasa_aprendizaje', 'PasoGrafado', 'entrenar', 'train', 'evaluar', 'evaluate', 'guardar', 'save',
           'cargar', 'load', 'escribir', 'generate', 'EscritorModelo', 'ModelWriter', 'EscritorCapa', 'LayerWriter',
           'MULT_SUFIJO_Y_PUERTA', 'PESOS_SUFIJO_Y_PUERTA', 'ops', 'cargar_biblioteca', 'load_library', 'LIB_PATH', 'ASRNHipError', '__version__']
