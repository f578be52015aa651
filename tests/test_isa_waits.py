"""Every kernel of the library waits for its vector-memory loads before touching their registers, proved on the
generated gfx950 code (tests/isa_waits.py).

The checker matters for k_prefill, whose code loads are inline assembly the compiler cannot see: a copy of a load's
destination that the compiler places before the explicit wait reads the register before the data has arrived (the
hardware has no interlock).  The synthetic cases pin the checker itself: it must flag an early read, a read on one
of two merging paths, an overwrite of a pending register and a read that a too-weak wait leaves exposed, and accept
the waited forms.
"""
import os
import re

import pytest

from tests import isa_waits as w

HIPCC = os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'bin', 'hipcc')
needs_hipcc = pytest.mark.skipif(not os.path.exists(HIPCC), reason='hipcc not available')


def body(text):
    return [l for l in text.strip().splitlines()]


def test_flags_read_before_wait():
    v = w.check_kernel(body("""
        buffer_load_dwordx4 v[4:7], v1, s[0:3], 0 offen
        v_mov_b32_e32 v8, v5
        s_waitcnt vmcnt(0)
        s_endpgm
    """))
    assert [x[2] for x in v] == [[5]]


def test_accepts_waited_read():
    assert w.check_kernel(body("""
        buffer_load_dwordx4 v[4:7], v1, s[0:3], 0 offen
        buffer_load_dwordx4 v1, s[0:3], 0 offen lds
        s_waitcnt vmcnt(1)
        v_mov_b32_e32 v8, v5
        s_endpgm
    """)) == []


def test_flags_weak_wait():
    # two newer operations, but vmcnt(2) lets the load itself stay outstanding
    v = w.check_kernel(body("""
        buffer_load_dword v4, v1, s[0:3], 0 offen
        buffer_load_dword v5, v1, s[0:3], 0 offen
        s_waitcnt vmcnt(2)
        v_add_u32_e32 v8, v4, v4
        s_endpgm
    """))
    assert len(v) == 1 and v[0][2] == [4]


def test_flags_overwrite_of_pending_register():
    v = w.check_kernel(body("""
        global_load_dword v4, v[2:3], off
        v_mov_b32_e32 v4, 0
        s_waitcnt vmcnt(0)
        s_endpgm
    """))
    assert len(v) == 1


def test_flags_read_on_one_merging_path():
    # the wait sits on the taken branch only; the fall-through path reaches the read with the load outstanding
    v = w.check_kernel(body("""
        buffer_load_dword v4, v1, s[0:3], 0 offen
        s_cbranch_scc1 .LBB0_2
        s_nop 0
        s_branch .LBB0_3
    .LBB0_2:
        s_waitcnt vmcnt(0)
    .LBB0_3:
        v_add_u32_e32 v8, v4, v4
        s_endpgm
    """))
    assert len(v) == 1 and v[0][2] == [4]


def test_loop_carried_load():
    # a load issued at the end of a loop body is read at the top of the next iteration: safe only behind the wait
    good = body("""
        buffer_load_dword v4, v1, s[0:3], 0 offen
    .LBB0_1:
        s_waitcnt vmcnt(0)
        v_add_u32_e32 v8, v4, v8
        buffer_load_dword v4, v1, s[0:3], 0 offen
        s_cbranch_scc1 .LBB0_1
        s_endpgm
    """)
    bad = [l for l in good if 's_waitcnt' not in l]
    assert w.check_kernel(good) == []
    assert len(w.check_kernel(bad)) == 1


def test_register_ranges_parse():
    assert w.vregs('v[52:53], v12, s[4:5], vcc') == {12, 52, 53}
    assert w.waitcnt_vm('vmcnt(4) lgkmcnt(0)') == 4 and w.waitcnt_vm('lgkmcnt(0)') is None and w.waitcnt_vm('0') == 0


SOURCES = sorted(f for f in os.listdir(w.CSRC) if f.endswith('.hip'))


@needs_hipcc
@pytest.mark.parametrize('source', SOURCES)
def test_kernels_wait_for_their_loads(source):
    asm = w.asm_of(os.path.join(w.CSRC, source))
    ks = w.kernels(asm)
    if source == 'prefill.hip':
        assert sum('k_prefillILi' in n for n in ks) == 3, sorted(ks)
    bad = {n: v for n, b in ks.items() for v in [w.check_kernel(b)] if v}
    assert not bad, {n: v[:4] for n, v in bad.items()}


@needs_hipcc
@pytest.mark.parametrize('bits', [4, 6])
def test_prefill_group_loop_keeps_its_prefetch(bits):
    """The group loop of k_prefill<4|6> holds no spill reload and no full drain: either would make the compiler wait
    for every copy in flight (vmcnt(0)), including the activation copies two groups ahead."""
    asm = w.asm_of(os.path.join(w.CSRC, 'prefill.hip'))
    name = [n for n in w.kernels(asm) if f'k_prefillILi{bits}E' in n][0]
    items = w.parse(w.kernels(asm)[name])
    labels = {it[1]: i for i, it in enumerate(items) if it[0] == 'label'}
    w4 = [i for i, (mn, ops) in enumerate(items) if mn == 's_waitcnt' and 'vmcnt(4)' in ops][0]
    loops = [(labels[ops.split()[0]], i) for i, (mn, ops) in enumerate(items)
             if w.BRANCH.match(mn) and labels.get(ops.split()[0], len(items)) <= w4 <= i]
    a, b = min(loops, key=lambda x: x[1] - x[0])
    loop = items[a:b + 1]
    assert sum(mn == 'v_mfma_i32_32x32x32_i8' for mn, _ in loop) >= 16
    assert not [mn for mn, _ in loop if mn.startswith('scratch_')]
    assert not [ops for mn, ops in loop if mn == 's_waitcnt' and re.search(r'vmcnt\(0\)|^0$', ops)]
