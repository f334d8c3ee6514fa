"""ctypes binding of libssalaad_amd.so (the C ABI in include/ssalaad_amd.h).

The library is loaded once, after torch, so that it resolves the HIP runtime
torch already holds. There is no fallback: if the library is missing or cannot
be loaded, every call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads torch's libamdhip64 before ours)

# SSALAAD_AMD_LIB selects another build of the same library, e.g. the device
# bounds-check variant libssalaad_amd_checked.so next to this file.
LIB_PATH = Path(os.environ.get("SSALAAD_AMD_LIB") or
                Path(__file__).resolve().parent / "libssalaad_amd.so").resolve()

SSL_OK = 0
SSL_ERR_INVALID = 1
SSL_ERR_UNSUPPORTED = 2
SSL_ERR_WORKSPACE = 3
SSL_ERR_HIP = 4
SSL_ERR_CAPACITY = 5

SSL_F32, SSL_BF16, SSL_F16 = 0, 1, 2
PLAN_STRIDE = 8

# ssl_debug_set knobs (test hooks)
DEBUG_PREFILL_TILE = 0
DEBUG_WAIT_POLLS = 1
DEBUG_WAIT_UNREACHABLE = 2
DEBUG_PREFILL_SPLIT = 3
DEBUG_CHAIN_FRAG = 4
DEBUG_TOPK_GROUPS = 5

_DTYPE_CODE = {torch.float32: SSL_F32, torch.bfloat16: SSL_BF16, torch.float16: SSL_F16}

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_p = ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "ssl_version": (ctypes.c_int, []),
    "ssl_last_error": (ctypes.c_char_p, []),
    "ssl_debug_set": (ctypes.c_int, [_c_i32, _c_i64]),
    "ssl_status_word_alloc": (ctypes.c_int, [_c_p, _c_p]),
    "ssl_device_checks": (_c_i32, []),
    "ssl_debug_check_word": (_c_i64, []),
    "ssl_plan_build": (
        ctypes.c_int,
        [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_p, _c_i64, _c_p,
         _c_p],
    ),
    "ssl_bsr_addmm_workspace_size": (_c_i64, [_c_i64, _c_i64, _c_i32, _c_i64]),
    "ssl_bsr_addmm_counter_count": (_c_i64, [_c_i64, _c_i64]),
    "ssl_bsr_addmm_inplace": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p,
         _c_i64, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_p,
         _c_i64, _c_p],
    ),
    "ssl_prefill_step_ints": (_c_i32, [_c_i32, _c_i32, _c_i32]),
    "ssl_prefill_step_cols": (_c_i32, [_c_i32]),
    "ssl_prefill_plan_build": (
        ctypes.c_int,
        [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_p,
         _c_i64, _c_p, _c_p],
    ),
    "ssl_prefill_min_rows": (_c_i64, []),
    "ssl_prefill_parts_build": (ctypes.c_int, [_c_p, _c_i64, _c_i32, _c_p, _c_i64, _c_p, _c_p]),
    "ssl_prefill_parts_bytes": (_c_i64, [_c_i64, _c_i64]),
    "ssl_nm24_block_bytes": (_c_i64, []),
    "ssl_nm24_prefill_block_bytes": (_c_i64, []),
    "ssl_nm24_takes_prefill": (_c_i32, [_c_i64, _c_i64, _c_i32]),
    "ssl_prefill_group": (_c_i32, [_c_i64, _c_i64, _c_i32, _c_i32]),
    "ssl_slr_takes_prefill": (_c_i32, [_c_i64, _c_i64, _c_i32, _c_i32, _c_i32]),
    "ssl_bsr_addmm_takes_prefill": (_c_i32, [_c_i64, _c_i64, _c_i32, _c_i32, _c_i32]),
    "ssl_slr_workspace_size": (_c_i64, [_c_i64, _c_i64, _c_i32, _c_i64, _c_i64, _c_i64, _c_i32]),
    "ssl_slr_counter_count": (_c_i64, [_c_i64, _c_i64]),
    "ssl_slr_exchange_size": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i32]),
    "ssl_slr_forward": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64,
         _c_p, _c_i64, _c_p, _c_i64, _c_p],
    ),
    "ssl_slr_noalloc_scratch_bytes": (_c_i64, []),
    "ssl_slr_forward_noalloc": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p],
    ),
    "ssl_block_topk_workspace_size": (_c_i64, [_c_i64]),
    "ssl_block_topk": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i64, _c_p, _c_p, _c_p, _c_i64,
         _c_p, _c_i64, _c_p],
    ),
    "ssl_project_nm": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_p, _c_i64, _c_p],
    ),
    "ssl_bsr_encode_count": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p],
    ),
    "ssl_bsr_encode_fill": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p],
    ),
    "ssl_add_rmsnorm": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_i32,
         _c_p],
    ),
    "ssl_embed_rmsnorm": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_i32, _c_p],
    ),
    "ssl_rope_kv_append": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, ctypes.c_float, _c_p,
         _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_p],
    ),
    "ssl_decode_attention_splits": (_c_i32, [_c_i64, _c_i32, _c_i32, _c_i64]),
    "ssl_decode_attention_workspace_size": (_c_i64, [_c_i64, _c_i32, _c_i32, _c_i32]),
    "ssl_decode_attention_counter_count": (_c_i64, [_c_i64, _c_i32, _c_i32]),
    "ssl_decode_attention": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i64,
         ctypes.c_float, _c_i32, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_p],
    ),
    "ssl_decode_rope_attention": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, ctypes.c_float, _c_p,
         _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i64, ctypes.c_float,
         _c_i32, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_p],
    ),
    "ssl_silu_mul": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p],
    ),
}



class SlrMember(ctypes.Structure):
    """ssl_slr_member: one linear of a fused (grouped) call."""

    _fields_ = [
        ("y", _c_p), ("ldy", _c_i64), ("A", _c_p), ("B", _c_p), ("bias", _c_p),
        ("col", _c_p), ("values", _c_p), ("plan", _c_p), ("n_chunks", _c_i64),
        ("n_slots", _c_i64), ("lr_wgs", _c_i64), ("NB", _c_i64), ("r_pad", _c_i64),
        ("counters", _c_p), ("n_counters", _c_i64), ("exchange", _c_p),
        ("exchange_bytes", _c_i64), ("workspace", _c_p), ("workspace_bytes", _c_i64),
        ("pf_groups", _c_p), ("pf_steps", _c_p), ("pf_n_groups", _c_i64), ("pf_group", _c_i32),
        ("nnz", _c_i64), ("values_pq", _c_p), ("s_format", _c_i32), ("status", _c_p),
        ("pf_parts", _c_p), ("pf_n_parts", _c_i64), ("pf_split_parts", _c_i64),
    ]


_SIGNATURES["ssl_slr_forward_group"] = (
    ctypes.c_int,
    [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, ctypes.POINTER(SlrMember),
     _c_i32, _c_p],
)



class SlrStage(ctypes.Structure):
    """ssl_slr_stage: one stage of a chained launch."""

    _fields_ = [
        ("x", _c_p), ("ldx", _c_i64), ("m", _c_i64), ("m_pad", _c_i64), ("first", _c_i32),
        ("count", _c_i32), ("src", _c_i32), ("sync", _c_p), ("n_sync", _c_i64),
        ("xf", _c_p), ("xf_bytes", _c_i64),
    ]


_SIGNATURES["ssl_slr_chain_sync_count"] = (_c_i64, [_c_i64])
_SIGNATURES["ssl_slr_chain_frag_bytes"] = (_c_i64, [_c_i64, _c_i64])
_SIGNATURES["ssl_slr_chain_table_bytes"] = (_c_i64, [])
_SIGNATURES["ssl_slr_chain_table_build"] = (
    ctypes.c_int,
    [_c_i64, _c_i32, _c_i32, _c_i32, ctypes.POINTER(SlrStage), _c_i32, ctypes.POINTER(SlrMember),
     _c_i32, _c_p, _c_i64],
)
_SIGNATURES["ssl_slr_chain_table_launch"] = (ctypes.c_int, [_c_p, _c_p, _c_p])
_SIGNATURES["ssl_slr_forward_chain"] = (
    ctypes.c_int,
    [_c_i64, _c_i32, _c_i32, _c_i32, ctypes.POINTER(SlrStage), _c_i32, ctypes.POINTER(SlrMember),
     _c_i32, _c_p],
)

MAX_GROUP = 4
MAX_CHAIN = 8
MAX_CHAIN_STAGES = 4
MAX_CHAIN_TABLE = 256

_lib = None


def load() -> ctypes.CDLL:
    """Load the library (once); raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH.name} is not built; run `python s-salaad_amd/build.py` "
            "(or __graft_entry__.build()) first. There is no non-HIP fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _check_single_hip_runtime()
    _lib = lib
    return lib


def _check_single_hip_runtime() -> None:
    """Two HIP runtimes in one process would split device state; refuse that."""
    try:
        maps = Path("/proc/self/maps").read_text()
    except OSError:
        return
    paths = {
        os.path.realpath(line.split()[-1])
        for line in maps.splitlines()
        if "libamdhip64" in line and line.split()[-1].startswith("/")
    }
    if len(paths) > 1:
        raise RuntimeError(f"more than one HIP runtime is loaded: {sorted(paths)}")


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def dtype_code(dtype: torch.dtype) -> int:
    code = _DTYPE_CODE.get(dtype)
    if code is None:
        raise TypeError(f"SLR kernels support float32/bfloat16/float16, got {dtype}")
    return code


def check(rc: int, what: str) -> None:
    """Map a C-ABI status to the exception type the reference raises."""
    if rc == SSL_OK:
        return
    msg = f"{what}: {load().ssl_last_error().decode(errors='replace')}"
    if rc in (SSL_ERR_INVALID, SSL_ERR_CAPACITY):
        raise ValueError(msg)
    if rc == SSL_ERR_UNSUPPORTED:
        raise TypeError(msg)
    raise RuntimeError(msg)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_ptr(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on `device`."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
