"""GEMM solution picks for the layer's and the model's dense products on MI355X.

They run on hipBLASLt / rocBLAS through torch, whose default heuristics leave time on the table at the benchmarks'
shapes (the layer: 32768 tokens, d = 256, fp32; the d = 768 model's bf16 training step: 16384 tokens, its blocks,
layers and the 50,304-row head; the quick-start model). The package ships the picks torch's TunableOp measured on
MI355X for those shapes (data/gemm_picks_mi355x.csv: one line per GEMM shape, the solution and its time, headed by the
torch / HIP / hipBLASLt / rocBLAS versions and the GPU arch they are valid for). use_tuned_gemms() loads them with
tuning off: shapes in the file run the measured solution, every other shape the library default, and a version
mismatch makes TunableOp ignore the file. Nothing is tuned at run time.
"""
import os
import tempfile

PICKS = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'data', 'gemm_picks_mi355x.csv')


def use_tuned_gemms(path=PICKS):
    """Turns TunableOp on in lookup-only mode with the shipped picks. Returns True when the file was read."""
    import torch.cuda.tunable as tunable
    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    # results are only written back when something new is tuned (never here); point the output away from the tree
    tunable.set_filename(os.path.join(tempfile.gettempdir(), 'asrn_tunableop_unused.csv'))
    return bool(tunable.read_file(path))
