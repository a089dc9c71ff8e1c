"""Builds libasrn_hip.so (the C-ABI library of HIP kernels for gfx950) in-tree with hipcc.

    python -m asrn_amd.build            # or asrn_amd.build.build()

Every source is compiled with packed-fp32 instructions disabled; ngram.hip and decode.hip also with -ffp-contract=off
because the n-gram keys must round each fp64 multiply and add separately, exactly as the reference does.
"""
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
LIB = os.path.join(HERE, 'libasrn_hip.so')
SOURCES = ['errors.hip', 'bucket_sort.hip', 'ngram.hip', 'scan.hip', 'candidates.hip', 'decode.hip',
           'decode_produce.hip', 'gate.hip', 'context.hip', 'hidden.hip', 'reduce.hip', 'small_gemm.hip', 'blocks.hip',
           'phi.hip', 'sampling.hip', 'block_step.hip', 'cross_entropy.hip', 'conv_window.hip',
           'layernorm.hip']
ARCH = os.environ.get('ASRN_OFFLOAD_ARCH', 'gfx950')
INCLUDE = os.path.join(os.path.dirname(HERE), 'include')
COMMON = ['-O3', '-fPIC', '-std=c++17', f'--offload-arch={ARCH}', '-Xclang', '-target-feature', '-Xclang',
          '-packed-fp32-ops', '-Wno-unused-command-line-argument', f'-I{INCLUDE}']
PER_FILE = {'ngram.hip': ['-ffp-contract=off'], 'decode.hip': ['-ffp-contract=off']}


def hipcc():
    for cand in (shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError('hipcc not found: the ASRN HIP library needs ROCm')


def build(verbose=False, jobs=None):
    """Compiles every source (in parallel) and links the shared library atomically. Raises on any error."""
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix='asrn_build_') as tmp:
        procs = []
        objs = []
        for src in SOURCES:
            obj = os.path.join(tmp, src.replace('.hip', '.o'))
            cmd = [cc, *COMMON, *PER_FILE.get(src, []), '-c', os.path.join(CSRC, src), '-o', obj]
            if verbose:
                print(' '.join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
        errors = []
        for src, p in procs:
            out, _ = p.communicate()
            if p.returncode != 0:
                errors.append(f'--- {src} ---\n{out}')
            elif verbose and out.strip():
                print(out)
        if errors:
            raise RuntimeError('hipcc failed:\n' + '\n'.join(errors))
        tmp_lib = os.path.join(tmp, 'libasrn_hip.so')
        cmd = [cc, '-shared', '-fPIC', f'--offload-arch={ARCH}', *objs, '-o', tmp_lib]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise RuntimeError('link failed:\n' + r.stdout)
        shutil.copyfile(tmp_lib, LIB + '.tmp')
        os.replace(LIB + '.tmp', LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
