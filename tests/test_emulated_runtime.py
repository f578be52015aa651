"""GPU parity tests run on the CPU through the shipped library: det_amd/libdet_hip.so's own host code, unchanged, with
its HIP runtime calls served by a stand-in (tests/emu_runtime/hip_on_emulator.cpp) and every kernel it launches
executed instruction by instruction by the gfx950 emulator (tests/emulated_hip.py, tests/gfx950_emu.py).

The selected `-m gpu` tests call the C ABI exactly as on an MI355X and compare with the oracle bit for bit, so they
cover what the kernel-level emulation tests cannot: argument checks, the choice of kernel per batch size, grid and
K-slice sizes, the library's partial-result buffers and their reuse across calls, and the part routing of fused
outputs.  The stand-in reports 4 compute units, so the slicing and stream-K splitting the library does for a large
chip happen at these small shapes.  The stream-K prefill kernel (DET_PREFILL=streamk) runs through the same tests in
a second process.

Tests that start their own processes (unless the child installs the stand-in itself, as the runtime test's does)
or whose emulation takes minutes are not in the selection; they run on the GPU.
"""
import os
import shutil
import subprocess
import sys

import pytest

from tests import emulated_hip

ROOT = emulated_hip.ROOT
HIPCC = os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'bin', 'hipcc')

SELECTED = [
    'tests/test_runtime.py',
    'tests/test_prim_parity.py',
    'tests/test_quant_parity.py::test_conformance_norms',
    'tests/test_quant_parity.py::test_scale_underflow_rows',
    'tests/test_quantizer_parity.py::test_quantizer_bytes[37-128-6]',
    'tests/test_quantizer_parity.py::test_quantizer_tie_takes_the_first[4]',
    'tests/test_quantizer_parity.py::test_repack_layout[6]',
    'tests/test_mixer_parity.py::test_argmax_first_of_ties',
    'tests/test_mixer_parity.py::test_argmax_nan_and_signed_zero',
    'tests/test_mixer_parity.py::test_gdn_small_shapes[1-2-4-4]',
    'tests/test_mixer_parity.py::test_attention_small_heads_clamped_values_zero_key',
    'tests/test_ffn_decode.py::test_gemv_silu0[widths2-1024-6]',
    'tests/test_gemm_parity.py::test_conformance_fused_parts',
    'tests/test_gemm_parity.py::test_four_parts_and_accumulate_edges[6]',
]
STREAMK = ['tests/test_gemm_parity.py::test_four_parts_and_accumulate_edges[4]',
           'tests/test_quantizer_parity.py::test_prefill_planes[8]']


@pytest.fixture(scope='module')
def emu_env(tmp_path_factory):
    if not (os.path.exists(HIPCC) and shutil.which('g++')):
        pytest.skip('hipcc and g++ are needed')
    if not emulated_hip.library_is_current():
        pytest.skip('det_amd/libdet_hip.so is missing or older than its sources: run __graft_entry__.build()')
    d = str(tmp_path_factory.mktemp('emu'))
    env = dict(os.environ, DET_EMU_SHIM=emulated_hip.build_shim(d), DET_EMU_ASM=d, DET_EMU_CUS='4')
    emulated_hip.build_asm(d)
    env.pop('DET_PREFILL', None)
    return env


def run_selected(env, ids, log, workers=1):
    """The ids in one pytest run under the stand-in (workers > 1: that many processes, each with its own stand-in
    and emulator); returns the device symbols launched."""
    env = dict(env, DET_EMU_LOG=str(log))
    # when this test itself runs in an xdist worker, the child run must not inherit that worker's name: its controller
    # would write the per-worker log of its own worker of the same name (empty), racing with it
    for k in [k for k in env if k.startswith('PYTEST_XDIST')]:
        del env[k]
    par = ['-n', str(workers)] if workers > 1 else []
    r = subprocess.run([sys.executable, '-m', 'pytest', '-p', 'tests.emulated_hip', '-m', 'gpu', '-q', '-x',
                        '-p', 'no:cacheprovider', *par, *ids], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=1500)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert ' passed' in r.stdout and 'skipped' not in r.stdout, r.stdout[-2000:]
    names = set()
    for p in log.parent.glob(log.name + '*'):
        names.update(p.read_text().split())
    return sorted(names)


def launched(names, part):
    return any(part in n for n in names)


def test_gpu_tests_through_the_library(emu_env, tmp_path):
    names = run_selected(emu_env, SELECTED, tmp_path / 'kernels', workers=4)
    for k in ('k_decodeILi', 'k_decode_ms', 'k_prefill2', 'k_repackE', 'k_qrow', 'k_quantize',
              'k_attn', 'k_gdn', 'k_argmax'):
        assert launched(names, k), (k, names)
    # without DET_PREFILL=streamk no linear carries prefill planes, so their repack never runs
    assert not launched(names, 'k_repack_pf'), names


def test_streamk_prefill_through_the_library(emu_env, tmp_path):
    names = run_selected(dict(emu_env, DET_PREFILL='streamk'), STREAMK, tmp_path / 'kernels')
    assert launched(names, 'k_prefillILi') and not launched(names, 'k_prefill2'), names
    assert launched(names, 'k_repack_pf'), names
