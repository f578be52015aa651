"""Build det_amd/libdet_hip.so: every HIP source under det_amd/csrc, for gfx950, with the numerics flags the
spec needs (no FMA contraction, no fast math, fp32 denormals kept, correctly rounded fp32 div/sqrt).

    python -m det_amd.build          (or __graft_entry__.build())
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
LIB = os.path.join(HERE, 'libdet_hip.so')
ARCH = os.environ.get('DET_HIP_ARCH', 'gfx950')

HIPFLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared',
    '-ffp-contract=off', '-fno-fast-math', '-fno-gpu-flush-denormals-to-zero',
    '-fhip-fp32-correctly-rounded-divide-sqrt',
    # packed fp32 VALU ops are kept out of the generated code
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    # MFMA results in architectural VGPRs (the VALU scales them every 128-group; AGPRs would need copies)
    '-mllvm', '-amdgpu-mfma-vgpr-form=1',
    '-Wall', '-Wno-unused-function',
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith('.hip'))


def build(verbose=False):
    hipcc = os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'bin', 'hipcc')
    cmd = [hipcc] + HIPFLAGS + ['-o', LIB + '.tmp'] + sources()
    if verbose:
        print(' '.join(cmd), flush=True)
    subprocess.check_call(cmd)
    os.replace(LIB + '.tmp', LIB)
    return LIB


if __name__ == '__main__':
    build(verbose='-v' in sys.argv)
