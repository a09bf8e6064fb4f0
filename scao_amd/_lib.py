"""ctypes binding of the gfx950 C ABI (include/scao_amd.h).

The shared object is built in-tree by ``scao_amd.build`` into
``scao_amd/_lib/libscao_amd.so``.  It links the HIP runtime by soname; torch
is imported first so the process holds exactly one HIP runtime (torch's),
and the streams torch hands out are valid for the library.

There is no fallback: if the library is missing, ``lib()`` raises.  Set
``SCAO_AMD_LIB`` to load a library from another path.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np
import torch  # noqa: F401  -- loads torch's HIP runtime before ours

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SCAO_AMD_LIB", os.path.join(HERE, "_lib", "libscao_amd.so"))

ABI_VERSION = 12
SLOT_WIDTH = 3
FLAT_CHUNK = 4096
PROJ_COLS = 256
APPLY_TILE = 64
APPLY_WIDE_ROWS = 16
APPLY_WIDE_COLS = 256
APPLY_GROUP = 8
GRAM_TILE = 128
NOALLOC_SCRATCH_BYTES = 16 << 20
EIG_BAND = 16
EIG_BANDW = 2 * EIG_BAND + 1

F32, BF16, F16 = 0, 1, 2
PF_DECAY, PF_LARS, PF_CLIP, PF_GSNR, PF_DIAG, PF_NORM, PF_GF32, PF_ALIGNED = (
    1, 2, 4, 8, 16, 32, 64, 128)
PF_FMASK, PF_FNOISE = 256, 512
FILTER_THR_WORD = 2 * 2048 + 7
LF_SINV4, LF_VEC4, LF_DIAG = 1, 2, 4

DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

# numpy mirrors of the C structs (field order = declaration order)
PARAM_DESC = np.dtype([
    ("p", "u8"), ("g", "u8"), ("graw", "u8"), ("exp_avg", "u8"), ("exp_avg_sq", "u8"),
    ("exp_avg_diff", "u8"), ("prev_grad", "u8"), ("upd", "u8"), ("diag_ema", "u8"),
    ("fema", "u8"), ("fthr", "u8"), ("fseed", "u8"),
    ("numel", "i8"), ("cols", "i8"), ("lr", "f8"), ("decay", "f4"),
    ("beta1", "f4"), ("omb1", "f4"), ("beta2", "f4"), ("omb2", "f4"), ("beta3", "f4"),
    ("omb3", "f4"), ("bc1", "f4"), ("bc2", "f4"), ("bc3", "f4"), ("blend", "f4"),
    ("omblend", "f4"), ("eps", "f4"), ("tau", "f4"), ("lars", "f4"), ("wd", "f4"),
    ("gsnr", "f4"), ("diag_bias", "f4"), ("adam_sqrt_bc2", "f4"), ("adam_alpha", "f4"),
    ("dtype", "i4"), ("flags", "i4"), ("pre_begin", "i4"), ("pre_end", "i4"),
    ("post_begin", "i4"), ("post_end", "i4"), ("norm_index", "i4"), ("fnoise", "f4"),
], align=True)

LEAF_DESC = np.dtype([
    ("Ul", "u8"), ("Ur", "u8"), ("Sl", "u8"), ("Sr", "u8"), ("T", "u8"), ("Delta", "u8"),
    ("W", "u8"), ("off", "i8"), ("ld", "i8"), ("param", "i4"), ("m", "i4"), ("n", "i4"),
    ("k", "i4"), ("flags", "i4"), ("dbias", "f4"), ("Wb", "u8"),
], align=True)

TASK = np.dtype([("idx", "i4"), ("a", "i4"), ("b", "i4"), ("slot", "i4")], align=True)

PARAM_STAT = np.dtype([
    ("g2", "f8"), ("p2", "f8"), ("nu2", "f8"), ("u2", "f8"), ("gnorm", "f4"), ("pnorm", "f4"),
    ("nu", "f4"), ("clip", "f4"), ("unorm", "f4"), ("trust", "f4"), ("alpha", "f4"),
    ("pad0", "f4"),
], align=True)

GRAM_DESC = np.dtype([
    ("g", "u8"), ("off", "i8"), ("ld", "i8"), ("q", "u8"), ("scale", "u8"), ("ema", "u8"),
    ("amax", "u8"), ("rows", "i4"), ("cols", "i4"), ("side", "i4"), ("dtype", "i4"),
    ("ntiles", "i4"), ("flags", "i4"), ("rho", "f4"), ("alpha", "f4"),
], align=True)
GRAM_SYM = 1

PREP_DESC = np.dtype([
    ("q", "u8"), ("scale", "u8"), ("ema", "u8"), ("out", "u8"), ("shift", "u8"), ("dim", "i4"),
    ("bias", "f4"),
], align=True)

FILTER_DESC = np.dtype([
    ("g", "u8"), ("ema", "u8"), ("out", "u8"), ("work", "u8"), ("seed", "u8"), ("numel", "i8"),
    ("decay", "f4"), ("omd", "f4"), ("q", "f4"), ("noise", "f4"), ("dtype", "i4"),
    ("flags", "i4"), ("cand", "u8"), ("cap", "i8"),
], align=True)
FILTER_MASK, FILTER_FIRST = 1, 2

LOOKAHEAD_DESC = np.dtype([
    ("p", "u8"), ("slow", "u8"), ("numel", "i8"), ("dtype", "i4"), ("pad0", "i4"),
], align=True)
FILTER_WORK_WORDS = 2 * 2048 + 16
FILTER_COMPACT_WORD = 2 * 2048 + 11   # 1 when the refinement passes read the candidates
FILTER_REGION = 2048                  # candidate slots per chunk (SCAO_FLAT_CHUNK / 2)

STRUCTS = {0: (PARAM_DESC, [n for n in PARAM_DESC.names if n != "pad0"]),
           1: (LEAF_DESC, list(LEAF_DESC.names)),
           2: (TASK, list(TASK.names)),
           3: (PARAM_STAT, [n for n in PARAM_STAT.names if n != "pad0"]),
           4: (GRAM_DESC, list(GRAM_DESC.names)),
           5: (PREP_DESC, list(PREP_DESC.names)),
           6: (FILTER_DESC, list(FILTER_DESC.names)),
           7: (LOOKAHEAD_DESC, [n for n in LOOKAHEAD_DESC.names if n != "pad0"])}

_VP, _I, _I64, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double

SIGNATURES = {
    "scao_abi_version": (_I, []),
    "scao_last_error": (ctypes.c_char_p, []),
    "scao_struct_layout": (_I, [_I, _VP, _I]),
    "scao_low_rank_precond_mm_workspace": (_I64, [_I64, _I64, _I64, _I]),
    "scao_low_rank_precond_mm": (_I, [_VP, _VP, _VP, _VP, _I64, _I64, _I64, _I, _VP, _VP]),
    "scao_fused_kronecker_workspace": (_I64, [_I64, _I64, _I64]),
    "scao_fused_kronecker_precond": (_I, [_VP, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I64, _I64,
                                          _VP, _VP]),
    "scao_fused_kronecker_precond_noalloc": (_I, [_VP, _VP, _VP, _VP, _VP, _I64, _VP, _I64,
                                                  _I64, _I64, _VP]),
    "scao_int8_ema_scratch_bytes": (_I64, [_I64]),
    "scao_int8_ema_update": (_I, [_VP, _D, _VP, _D, _I64, _VP, _VP, _VP]),
    "scao_kron_project": (_I, [_VP, _I, _VP, _VP, _VP, _I, _VP]),
    "scao_kron_delta": (_I, [_VP, _I, _VP, _VP, _VP, _VP]),
    "scao_kron_lift": (_I, [_VP, _I, _VP, _VP]),
    "scao_diag_reduce": (_I, [_VP, _I, _VP, _VP, _VP]),
    "scao_step_finalize": (_I, [_VP, _I, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "scao_kron_apply": (_I, [_VP, _I, _VP, _VP, _VP, _VP, _I, _VP]),
    "scao_diag_apply": (_I, [_VP, _I, _VP, _VP, _VP, _VP]),
    "scao_lars_write": (_I, [_VP, _I, _VP, _VP, _VP]),
    "scao_adam_step": (_I, [_VP, _I, _VP, _VP, _VP]),
    "scao_gram_ema": (_I, [_VP, _I, _VP, _VP]),
    "scao_requant": (_I, [_VP, _I, _VP, _VP, _VP]),
    "scao_eig_prep": (_I, [_VP, _I, _VP, _I, _VP]),
    "scao_eig_offdiag": (_I, [_VP, _I, _I, _I, _VP, _VP]),
    "scao_eig_diag": (_I, [_VP, _I, _I, _I, _VP, _VP, _I64, _VP, _VP]),
    "scao_diag_ema": (_I, [_VP, _I, _VP, _VP, _VP]),
    "scao_sparse_filter": (_I, [_VP, _I, _VP, _I, _VP]),
    "scao_eig_panel_qr": (_I, [_VP, _I64, _I, _I, _I, _VP, _VP, _I64, _VP]),
    "scao_eig_band_finish": (_I, [_VP, _I64, _I, _I, _VP, _I64, _VP, _I64, _VP, _VP]),
    "scao_eig_sy2sb_work": (_I64, [_I, _I]),
    "scao_eig_sy2sb_panel_w": (_I, [_VP, _I64, _I, _I, _I, _VP, _VP, _VP, _I, _VP]),
    "scao_eig_sy2sb_update": (_I, [_VP, _I64, _I, _I, _I, _VP, _I64, _I, _VP, _I64, _I, _VP,
                                   _I64, _I, _VP, _I64, _VP, _VP]),
    "scao_eig_sb2st": (_I, [_VP, _I, _I, _VP, _VP, _VP]),
    "scao_eig_bisect_work": (_I64, [_I, _I]),
    "scao_eig_bisect": (_I, [_VP, _VP, _I, _I, _I, _VP, _VP, _VP, _VP]),
    "scao_eig_vectors_work": (_I64, [_I, _I, _I]),
    "scao_eig_vectors": (_I, [_VP, _I64, _I, _I, _I, _VP, _VP, _I64, _VP, _VP]),
    "scao_eig_back_transform": (_I, [_VP, _I64, _I, _I, _VP, _VP, _I64, _I, _VP]),
    "scao_lookahead": (_I, [_VP, _I, _VP, ctypes.c_float, _VP]),
}


class ScaoLibError(RuntimeError):
    pass


_lock = threading.Lock()
_lib = None


def _load():
    if not os.path.exists(LIB_PATH):
        raise ScaoLibError(
            f"scao_amd: HIP library not found at {LIB_PATH}. Build it with "
            "`python -m scao_amd.build` (hipcc, gfx950). There is no CPU or torch fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.scao_abi_version() != ABI_VERSION:
        raise ScaoLibError(f"scao_amd: ABI version {lib.scao_abi_version()} != {ABI_VERSION}")
    check_layout(lib)
    return lib


def check_layout(lib) -> None:
    """Compare the numpy struct mirrors with the library's own offsets."""
    buf = (ctypes.c_int64 * 64)()
    for which, (dt, names) in STRUCTS.items():
        n = lib.scao_struct_layout(which, buf, 64)
        got = list(buf[:n])
        want = [dt.itemsize] + [dt.fields[f][1] for f in names]
        if got != want:
            raise ScaoLibError(f"scao_amd: struct {which} layout mismatch: lib {got} != py {want}")


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                _lib = _load()
    return _lib


def call(name: str, *args) -> None:
    """Call a C-ABI entry point and raise on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().scao_last_error().decode(errors="replace")
        raise ScaoLibError(f"{name} failed ({rc}): {msg}")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """Copy a numpy record array to the device on the current stream.

    The staging buffer is pinned host memory from torch's caching host
    allocator, which keeps it alive until the copy has completed."""
    raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    host = torch.empty(raw.size, dtype=torch.uint8, pin_memory=True)
    host.numpy()[:] = raw
    return host.to(device, non_blocking=True)
