"""libvault_amd loads, exports every symbol include/vault_amd.h declares, and its host-side
argument validation returns the documented codes (no GPU needed: these calls return before any
HIP call)."""
import ctypes as C

import pytest

from vault_amd import _lib as L


@pytest.fixture(scope="module")
def lib():
    return L.load()


def test_exports_every_declared_symbol(lib):
    declared = L.declared_symbols()
    assert len(declared) >= 10
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared) == set(L._SIGS), "ctypes signatures and header disagree"


def test_abi_version(lib):
    assert lib.vgx_abi_version() == 2


@pytest.mark.parametrize("dt,rows,cols,expect", [
    (L.Q4_0, 13, 96, 256 + 16 * 3 * 2),          # rows padded to 16: quants 16*3*16=768 -> 768, scales 96 B
    (L.Q8_0, 4, 32, 256 + 8),
    (L.F32, 5, 64, 8 * 64 * 4),
])
def test_packed_bytes(lib, dt, rows, cols, expect):
    if dt == L.Q4_0:
        q = 16 * 3 * 16
        expect = (q + 255) // 256 * 256 + 16 * 3 * 2
    elif dt == L.Q8_0:
        q = 4 * 1 * 32
        expect = (q + 255) // 256 * 256 + 4 * 1 * 2
    assert lib.vgx_qweight_packed_bytes(dt, rows, cols) == expect


def test_host_validation_codes(lib):
    assert lib.vgx_qweight_packed_bytes(L.Q4_0, 4, 33) == -7
    assert lib.vgx_qweight_packed_bytes(3, 4, 32) == -5
    assert lib.vgx_qweight_packed_bytes(L.Q8_0, 0, 32) == -1
    assert lib.vgx_qlinear(L.Q4_0, None, 4, 32, None, 32, 1, None, None, 4, 0, None) == -31
    p = C.c_void_p(64)   # never dereferenced: validation fails first
    assert lib.vgx_qlinear(L.Q4_0, p, 4, 33, p, 33, 1, None, p, 4, 0, None) == -7
    assert lib.vgx_qlinear(L.Q4_0, p, 4, 32, p, 16, 1, None, p, 4, 0, None) == -1
    assert lib.vgx_qlinear(L.Q4_0, p, 4, 32, p, 32, 1, None, p, 4, 2, None) == -31
    assert lib.vgx_qlinear_swiglu(L.Q4_0, p, 3, 32, p, 32, 1, p, 3, None) == -7
    assert lib.vgx_qlinear(L.Q4_0, p, 4, 32, p, 32, 0, None, p, 4, 0, None) == 0   # empty batch: no-op


def test_state_has_no_reference_cycle():
    """A decode state must be freed by reference counting alone: a state left to the cyclic garbage
    collector can be collected while a decode graph is being captured, and its destructors (pinned
    host buffers, events, graphs) are not allowed during a capture."""
    import gc
    import weakref

    from tests import modelgen
    from vault_amd.model import VAULTv3State

    cfg = modelgen.tiny_cfg()
    gc.disable()
    try:
        st = VAULTv3State(cfg, 1, "cpu")
        _ = st.layers[0].k_cur
        ref = weakref.ref(st)
        del st, _
        assert ref() is None
    finally:
        gc.enable()


def test_score_side_rejects_bad_jobs(lib):
    """vgx_qlinear_side checks its scorer job before any launch: unknown phase, feature widths past the
    prologue's 5120 or not whole blocks, misaligned rows, null pointers."""
    p = 1 << 20
    job = L.ScoreSide(1, p, 4608, p, 0, p, 256, p, p, p, 1e-5, p, p, p, p, None)
    call = lambda j: lib.vgx_qlinear_side(L.Q4_0, p, 1536, 8960, p, 8960, 1, None, 0.0, None, p, 1536, 1,
                                          C.byref(j), None)
    for field, val, code in [("phase", 3, -31), ("fd", 5152, -10), ("fd", 100, -1), ("feat", p + 4, -11),
                             ("ema", None, -31), ("eps", 0.0, -1)]:
        bad = L.ScoreSide.from_buffer_copy(job)
        setattr(bad, field, val)
        assert call(bad) == code, field
    bad = L.ScoreSide.from_buffer_copy(job)
    bad.phase = 2
    bad.h = None
    assert call(bad) == -31
