"""The C-ABI library: builds, loads without a GPU, exports every symbol the
header declares, and its struct layouts match the Python mirrors."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "scao_amd.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(scao_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    from scao_amd import _lib as L
    lib = L.lib()
    names = _declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), f"{n} declared in scao_amd.h but not exported"
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"
    assert sorted(L.SIGNATURES) == names


def test_abi_version_and_layouts():
    from scao_amd import _lib as L
    lib = L.lib()
    assert lib.scao_abi_version() == L.ABI_VERSION
    L.check_layout(lib)


def test_error_path_without_gpu():
    """Argument validation runs on the host: bad shapes are rejected with a
    message before anything touches a device."""
    from scao_amd import _lib as L
    lib = L.lib()
    rc = lib.scao_fused_kronecker_precond(None, None, None, None, None, 0, None, 0, 0, 0, None, None)
    assert rc == 1
    assert b"null pointer" in lib.scao_last_error()
    assert lib.scao_fused_kronecker_workspace(10, 20, 4) == (4 * 20 + 16 + 10 * 4) * 4
    assert lib.scao_int8_ema_scratch_bytes(5000) == (5000 + 2) * 4
    with pytest.raises(L.ScaoLibError):
        L.call("scao_kron_project", None, -1, None, None, None, 0, None)
    # the no-allocation operator rejects a block whose scratch exceeds its
    # static array (8192 x 8192 at k = 256 needs 16.25 MiB) before any launch
    rc = lib.scao_fused_kronecker_precond_noalloc(16, 16, 16, 16, 16, 8192, 16, 8192, 8192, 256,
                                                  None)
    assert rc == 1 and b"maximum" in lib.scao_last_error()
    assert L.NOALLOC_SCRATCH_BYTES == 16 << 20


def test_eig_entry_points_reject_oversized_n():
    """Every scao_eig_* entry point checks n <= 4096 + SCAO_EIG_BAND on the
    host (larger factors go to the library solver), so a direct C-ABI caller
    gets SCAO_ERR_INVALID instead of a kernel whose progress counters would
    overflow."""
    from scao_amd import _lib as L
    lib = L.lib()
    p, big = 16, 1 << 40   # non-null dummies and strides: nothing is launched
    for n in (4096 + L.EIG_BAND + 1, 40000):
        calls = {
            "scao_eig_panel_qr": (p, big, n, 0, 1, p, p, big, None),
            "scao_eig_sy2sb_panel_w": (p, big, n, 0, 1, p, p, p, 1, None),
            "scao_eig_sy2sb_update": (p, big, n, n, 1, p, big, 16, p, big, 16, p, big, 16, p,
                                      big, p, None),
            "scao_eig_band_finish": (p, big, n, 1, p, big, p, big, p, None),
            "scao_eig_sb2st": (p, n, 1, p, p, None),
            "scao_eig_bisect": (p, p, n, 1, 8, p, p, p, None),
            "scao_eig_vectors": (p, big, n, 1, 8, p, p, big, p, None),
            "scao_eig_back_transform": (p, big, n, 1, p, p, big, 8, None),
            "scao_eig_diag": (p, 1, n, 8, p, p, big, p, None),
        }
        for name, args in calls.items():
            rc = getattr(lib, name)(*args)
            assert rc == 1, (name, n, rc)
    from scao_amd import engine
    assert engine.DIAG_MAX_DIM == 4096 + L.EIG_BAND


def test_missing_library_raises(monkeypatch, tmp_path):
    from scao_amd import _lib as L
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(L.ScaoLibError, match="no CPU or torch fallback"):
        L.lib()


def test_header_constants_match_the_python_binding():
    """Every integer #define SCAO_<NAME> of include/scao_amd.h that scao_amd._lib
    mirrors as <NAME> has the same value there."""
    import re

    from scao_amd import _lib as L
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "include", "scao_amd.h")).read()
    seen = 0
    for name, val in re.findall(r"^#define SCAO_([A-Z0-9_]+)[ \t]+(\d+)[ \t]*(?:/\*|$)", text,
                                re.M):
        if hasattr(L, name) and isinstance(getattr(L, name), int):
            assert getattr(L, name) == int(val), name
            seen += 1
    assert seen >= 5


# One call per status-returning entry point whose arguments fail the host-side
# validation (a negative count, or null pointers with a non-zero size): it
# returns 1 and names itself in scao_last_error(), before any device call.
N = None
BAD_ARGS = {
    "scao_low_rank_precond_mm": (N, N, N, N, 4, 4, 4, 1, N, N),
    "scao_fused_kronecker_precond": (N, N, N, N, N, 4, N, 4, 4, 2, N, N),
    "scao_fused_kronecker_precond_noalloc": (N, N, N, N, N, 4, N, 4, 4, 2, N),
    "scao_int8_ema_update": (N, 1.0, N, 0.9, 4, N, N, N),
    "scao_kron_project": (N, -1, N, N, N, 1, N),
    "scao_kron_delta": (N, -1, N, N, N, N),
    "scao_kron_lift": (N, -1, N, N),
    "scao_diag_reduce": (N, -1, N, N, N),
    "scao_step_finalize": (N, -1, N, N, N, 0, 0, 0, N),
    "scao_kron_apply": (N, -1, N, N, N, N, 0, N),
    "scao_diag_apply": (N, -1, N, N, N, N),
    "scao_lars_write": (N, -1, N, N, N),
    "scao_adam_step": (N, -1, N, N, N),
    "scao_gram_ema": (N, -1, N, N),
    "scao_requant": (N, -1, N, N, N),
    "scao_eig_prep": (N, -1, N, 0, N),
    "scao_eig_offdiag": (N, -1, 8, 0, N, N),
    "scao_eig_diag": (N, 1, 8, 4, N, N, 32, N, N),
    "scao_diag_ema": (N, -1, N, N, N),
    "scao_sparse_filter": (N, -1, N, 0, N),
    "scao_eig_panel_qr": (N, 64, 8, 0, 1, N, N, 8 * 33, N),
    "scao_eig_band_finish": (N, 64, 8, 1, N, 8 * 33, N, 8 * 17, N, N),
    "scao_eig_sy2sb_panel_w": (N, 64, 8, 0, 1, N, N, N, 0, N),
    "scao_eig_sy2sb_update": (N, 64, 8, 8, 1, N, 64, 8, N, 16, 16, N, 64, 8, N, 128, N, N),
    "scao_eig_sb2st": (N, 8, 1, N, N, N),
    "scao_eig_bisect": (N, N, 8, 1, 4, N, N, N, N),
    "scao_eig_vectors": (N, 8 * 17, 8, 1, 4, N, N, 32, N, N),
    "scao_eig_back_transform": (N, 64, 8, 1, N, N, 32, 4, N),
    "scao_lookahead": (N, -1, N, 0.5, N),
}


def test_bad_argument_table_covers_every_entry_point():
    from scao_amd import _lib as L
    status = {name for name, (res, _) in L.SIGNATURES.items()
              if res is ctypes.c_int and name not in ("scao_abi_version", "scao_struct_layout")}
    assert status == set(BAD_ARGS)


@pytest.mark.parametrize("name", sorted(BAD_ARGS))
def test_entry_point_rejects_bad_arguments(name):
    from scao_amd import _lib as L
    lib = L.lib()
    assert getattr(lib, name)(*BAD_ARGS[name]) == 1
    assert lib.scao_last_error().decode().startswith(name + ":")
