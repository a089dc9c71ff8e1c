"""Loads libasrn_hip.so (the C ABI declared in include/asrn_hip.h) and calls it with torch device tensors.

torch is imported first so the HIP runtime the library links against is the one torch already loaded (both carry
the soname libamdhip64.so.7): kernels and torch tensors then share one runtime, one device context and its streams.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get('ASRN_HIP_LIB') or os.path.join(_HERE, 'libasrn_hip.so')   # override: another build

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/asrn_hip.h
SIGNATURES = {
    'asrn_hip_last_error': (ctypes.c_char_p, []),
    'asrn_hip_abi_version': (_I32, []),
    'asrn_bucket_sort_workspace': (_I64, [_I64, _I64, _I32]),
    'asrn_bucket_sort': (ctypes.c_int, [_P, _I64, _I64, _I32, _I32, _I64, _I32, _P, _P, _P, _P, _P, _P, _I64, _P]),
    'asrn_candidates_fwd': (ctypes.c_int, [_P] * 12 + [_I64, _I64] + [_I32] * 7
                            + [_F32, _F32, _I64, _I32, _I64, _I32] + [_P] * 4 + [_I32, _P, _P]),
    'asrn_candidates_record_bytes': (_I64, [_I32, _I32]),
    'asrn_candidate_lists': (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P]),
    'asrn_candidates_bwd': (ctypes.c_int, [_P] * 12 + [_I64, _I64] + [_I32] * 7
                            + [_F32, _F32, _I64, _I32, _I64, _I32] + [_P] * 11),
    'asrn_scan_workspace': (_I64, [_I64, _I64]),
    'asrn_clock_scan': (ctypes.c_int, [_P, _P, _I64, _I64, _I32, _P, _I64, _P]),
    'asrn_ngram_sort_workspace': (_I64, [_I64, _I64, _I32]),
    'asrn_ngram_sort': (ctypes.c_int, [_P, _P, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _I64, _P]),
    'asrn_scan_fwd': (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _I64, _P]),
    'asrn_scan_bwd': (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _P, _I64, _P]),
    'asrn_scan_static_scratch_bytes': (_I64, []),
    'asrn_scan_fwd_static': (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P]),
    'asrn_hawkes_fwd': (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _P]),
    'asrn_hawkes_bwd_workspace': (_I64, [_I64, _I64, _I32]),
    'asrn_hawkes_bwd': (ctypes.c_int, [_P] * 8 + [_I64, _I64, _I32] + [_P] * 4 + [_I64, _P]),
    'asrn_streak_fwd': (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I32, _P, _P, _I64, _P]),
    'asrn_streak_bwd': (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _P]),
    'asrn_repetition_workspace': (_I64, [_I64, _I64, _I32]),
    'asrn_repetition_fwd': (ctypes.c_int, [_P] * 8 + [_I64, _I64, _I32] + [_P] * 4 + [_I64, _P]),
    'asrn_repetition_bwd_workspace': (_I64, [_I64, _I64, _I32]),
    'asrn_repetition_bwd': (ctypes.c_int, [_P] * 13 + [_I64, _I64, _I32] + [_P] * 6 + [_I64, _P]),
    'asrn_context_fwd': (ctypes.c_int, [_P] * 5 + [_I64, _I32] + [_F32] * 3 + [_P] * 5),
    'asrn_context_bwd_workspace': (_I64, [_I64, _I32]),
    'asrn_context_bwd': (ctypes.c_int, [_P] * 5 + [_I64, _I32] + [_F32] * 2 + [_P] * 2 + [_I64, _I32] + [_P] * 7
                         + [_I64, _P]),
    'asrn_hidden_fwd': (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I64, _I32, _I32, _P, _P]),
    'asrn_hidden_bwd': (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I64, _I32, _I32, _P, _P, _I64, _P]),
    'asrn_hash_fwd': (ctypes.c_int, [_P, _I64] + [_P] * 6 + [_I64, _I64] + [_I32] * 4 + [_P, _P, _I32, _I32, _P]),
    'asrn_hash_bwd_workspace': (_I64, [_I64, _I64] + [_I32] * 4),
    'asrn_hash_bwd': (ctypes.c_int, [_P, _I64] + [_P] * 4 + [_I64, _I64] + [_I32] * 4 + [_P, _P, _I64, _P, _P, _I64, _P]),
    'asrn_column_sums_workspace': (_I64, [_I64, _I64]),
    'asrn_column_sums': (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _P, _P, _I64, _P]),
    'asrn_small_gemm': (ctypes.c_int, [_P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I32, _I32, _I32, _P]),
    'asrn_copy_blocks': (ctypes.c_int, [_I32] + [_P] * 7),
    'asrn_gate_fwd': (ctypes.c_int, [_P, _P, _I32] + [_P] * 11 + [_I64] + [_I32] * 5 + [_F32] * 3 + [_P] * 3),
    'asrn_gate_step': (ctypes.c_int, [_P] * 14 + [_I64] + [_I32] * 5 + [_F32] * 3 + [_P] * 3),
    'asrn_gate_bwd_workspace': (_I64, [_I64, _I32]),
    'asrn_gate_bwd': (ctypes.c_int, [_P, _P, _I32] + [_P] * 11 + [_I64] + [_I32] * 5 + [_F32] * 3 + [_P] * 8
                      + [_I64, _P]),
    'asrn_ring_build': (ctypes.c_int, [_P, _P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P]),
    'asrn_decode_attend': (ctypes.c_int, [_P] * 11 + [_I64, _I64, _I64, _P] + [_I32] * 7 + [_F32, _F32, _I32]
                           + [_P] * 6),
    'asrn_hawkes_table_load': (ctypes.c_int, [_P] * 6 + [_I64, _I64, _I32, _I64] + [_P] * 4),
    'asrn_hawkes_table_grow': (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _P, _P, _I64, _P]),
    'asrn_repetition_step': (ctypes.c_int, [_P] * 7 + [_I64, _I64, _I64, _P, _I32, _I64] + [_P] * 6 + [_I32, _P]),
    'asrn_decode_attend_repeat': (ctypes.c_int, [_P] * 11 + [_I64, _I64, _I64, _P] + [_I32] * 7 + [_F32, _F32, _I32]
                                  + [_P] * 8 + [_I32, _I64] + [_P] * 6 + [_I32, _P, _P]),
    'asrn_sample_bits': (_I32, [_I64]),
    'asrn_ngram_set_successors': (_I32, []),
    'asrn_ngram_set_build': (ctypes.c_int, [_P, _I64, _I64, _I64, _I32, _I32, _P, _P, _P, _P, _I64, _P]),
    'asrn_sample': (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _P, _P, _P]
                    + [_P, _P, _P, _P, _I64, _I32] * 2
                    + [_I32, _I64, _I64, _F32, _I32, _F32, _F32, _I32, _I64, ctypes.c_uint64, _P]),
    'asrn_cross_entropy_fwd': (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _I64, _I64, _P, _P, _P]),
    'asrn_cross_entropy_bwd': (ctypes.c_int, [_P, _I32, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P]),
    'asrn_conv_window_fwd': (ctypes.c_int, [_P, _I64, _I64, _I64, _I32, _I32, _I32, _P, _P]),
    'asrn_conv_window_bwd': (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _I32, _P, _I64, _P]),
    'asrn_layer_norm_fwd': (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I32, _F32, _I32, _P, _I64, _P, _P]),
    'asrn_layer_norm_bwd_workspace': (_I64, [_I64, _I32]),
    'asrn_layer_norm_bwd': (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I32, _P, _I32, _I64, _P, _P, _P, _P, _I64, _P]),
    'asrn_block_step_workspace': (_I64, [_I64, _I32, _I32]),
    'asrn_block_step': (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I32, _I32, _I32] + [_P] * 10 + [_F32] + [_P] * 6
                        + [_I64, _P]),
    'asrn_block_step_ex': (ctypes.c_int, [_P, _I64] + [_P] * 4 + [_I32, _I32] + [_P] * 3 + [_I64, _I32, _I32, _I32]
                           + [_P] * 10 + [_F32] + [_P] * 5 + [_I32, _P, _I64, _P]),
    'asrn_block_finish_norm': (ctypes.c_int, [_P] * 4 + [_I32, _I32, _P, _P, _I64, _I32, _P, _P, _F32, _P, _P, _I64,
                                                     _P, _P, _P]),
    'asrn_embed_step': (ctypes.c_int, [_P, _I64, _I32, _P, _P, _I64, _P, _I64, _P, _P, _P]),
    'asrn_decode_produce_workspace': (ctypes.c_int64, [_I64, _I32, _I32]),
    'asrn_decode_produce_e_workspace': (_I64, [_I32, _I64, _I32, _I32]),
    'asrn_decode_produce_e': (ctypes.c_int, [_I32, _P, _P, _P, _I64, _I32] + [_P] * 9 + [_I32] * 4 + [_P] * 3
                              + [_I64, _I64, _P, _P, _I64, _P]),
    'asrn_decode_produce_h': (ctypes.c_int, [_P, _I64, _I32, _P, _P, _F32, _P, _P, _F32, _F32, _P, _P, _I32, _P, _P, _P,
                                             _I64, _I64, _P, _P, _P]),
    'asrn_decode_produce_h_ex': (ctypes.c_int, [_P] * 5 + [_I32, _I32, _P, _P, _P, _I64, _I64, _I32, _P, _P, _F32, _P,
                                                      _P, _F32, _F32, _P, _P, _I32, _P, _P, _P, _I64, _I64, _P, _P,
                                                      _P]),
    'asrn_decode_produce': (ctypes.c_int, [_P] * 4 + [_I64, _I32] + [_P] * 9 + [_I32] * 4 + [_P, _P, _F32, _P, _P, _F32,
                                                                                              _F32, _P, _P, _I32]
                            + [_P] * 6 + [_I64, _I64, _P, _P, _P, _I64, _P]),
}

_lib = None


class ASRNHipError(RuntimeError):
    pass


def load(path=LIB_PATH):
    """Opens the library once (raises if it is missing: the product has no CPU fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ASRNHipError(f'{path} is missing: build it with `python -m asrn_amd.build` (hipcc, gfx950)')
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# entry point name -> list of (start, end) torch.cuda.Event pairs; filled only for the names being timed
_TIMED = {}


def time_calls(names):
    """Starts timing the given entry points with device events recorded on torch's current stream (the stream the
    library launches on). Returns the dict that collects (start, end) event pairs per name."""
    _TIMED.clear()
    for n in names:
        _TIMED[n] = []
    return _TIMED


def stop_timing():
    out = dict(_TIMED)
    _TIMED.clear()
    return out


def call(name, *args):
    lib = load()
    ev = _TIMED.get(name)
    if ev is not None:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        rc = getattr(lib, name)(*args)
        e.record()
        ev.append((s, e))
    else:
        rc = getattr(lib, name)(*args)
    if rc != 0:
        raise ASRNHipError(f'{name}: {lib.asrn_hip_last_error().decode(errors="replace")}')
    return rc


def query(name, *args):
    return getattr(load(), name)(*args)
