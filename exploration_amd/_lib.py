"""ctypes binding of ``libst_attn.so`` (declared in ``include/st_attn.h``).

torch is imported first so that the library binds to the HIP runtime torch
already mapped (both carry the SONAME ``libamdhip64.so.7``). Status codes
map to the reference's exceptions: invalid or unsupported arguments raise
``ValueError`` (reference ``st/ops/attention.py:155-162,171-172``), launch
failures ``RuntimeError``; nothing falls back to another implementation.
"""
import ctypes
import os

import torch  # noqa: F401  (binds the HIP runtime before the library loads)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libst_attn.so")

ST_OK, ST_EINVAL, ST_EUNSUPPORTED, ST_ELAUNCH = 0, 1, 2, 3
DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_i64, _p, _f32p, _i64p, _i32p, _sz = (ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t)

SIGNATURES = {
    "st_abi_version": (ctypes.c_int, []),
    "st_last_error": (ctypes.c_char_p, []),
    "st_launch_report": (_sz, [ctypes.c_char_p, _sz]),
    "st_dense_supported": (ctypes.c_int, [ctypes.c_int, _i64, _i64]),
    "st_dense_fwd_workspace_bytes": (_sz, [ctypes.c_int] + [_i64] * 6),
    "st_dense_fwd": (ctypes.c_int, [ctypes.c_int] + [_i64] * 6 + [_p] * 3 + [_i64p, _p] + [_f32p] * 4
                     + [_p, _sz, _p]),
    "st_dense_bwd_workspace_bytes": (_sz, [ctypes.c_int] + [_i64] * 6),
    "st_dense_bwd": (ctypes.c_int, [ctypes.c_int] + [_i64] * 6 + [_p] * 3 + [_i64p, _p] + [_f32p] * 4
                     + [_p] * 4 + [_p, _sz, _p]),
    "st_sparse_scores": (ctypes.c_int, [ctypes.c_int] + [_i64] * 5 + [_p, _i64p, _p, _i32p] + [_i64] * 4
                         + [_f32p, _i64, _p]),
    "st_sparse_select": (ctypes.c_int, [_i64] * 4 + [_f32p, _i64p, _f32p, _f32p, _p]),
    "st_sparse_workspace_bytes": (_sz, [_i64] * 6),
    "st_sparse_pop": (ctypes.c_int, [ctypes.c_int] + [_i64] * 5 + [_p, _i64p, _p, _p, _i32p] + [_i64] * 4
                      + [_i64p, _f32p, _f32p, _i64, ctypes.c_int, _p, _f32p, _p, _sz, _p]),
    "st_sparse_fwd": (ctypes.c_int, [ctypes.c_int] + [_i64] * 6 + [_p, _i64p, _p, _p, _i32p] + [_i64] * 4
                      + [_p, _i64p, _f32p, _f32p, _f32p, _p, _sz, _p]),
    "st_sparse_noalloc_scratch_bytes": (_sz, []),
    "st_sparse_fwd_noalloc": (ctypes.c_int, [ctypes.c_int] + [_i64] * 6 + [_p, _i64p, _p, _p, _i32p]
                              + [_i64] * 4 + [_p, _i64p, _f32p, _f32p, _f32p, _p]),
    "st_paged_kv_write": (ctypes.c_int, [ctypes.c_int] + [_i64] * 4 + [_p, _p, _i32p] + [_i64] * 3
                          + [_p, _p, _i64, _p]),
    "st_halo_supported": (ctypes.c_int, [ctypes.c_int, _i64, _i64]),
    "st_halo_attn_fwd": (ctypes.c_int, [ctypes.c_int] + [_i64] * 8 + [_p, _f32p, _f32p, _p, _p]),
    "st_halo_attn_bwd": (ctypes.c_int, [ctypes.c_int] + [_i64] * 8 + [_p, _f32p, _f32p, _p, _p, _p, _p]),
}

ABI_VERSION = 5
_lib = None


def load():
    """Load the library once; raises RuntimeError if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run `python -m exploration_amd.build` "
                           "(or __graft_entry__.build()); there is no fallback implementation")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.st_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libst_attn ABI {lib.st_abi_version()} != {ABI_VERSION}; rebuild")
    _lib = lib
    return lib


def hip_runtimes_mapped():
    """Paths of every libamdhip64 mapped into this process (expected: one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(os.path.realpath(line.split()[-1]))
    return sorted(paths)


def check(status, lib=None):
    if status == ST_OK:
        return
    msg = (lib or load()).st_last_error().decode(errors="replace")
    if status in (ST_EINVAL, ST_EUNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


def native_launch_report():
    """The library's launch records (``st_launch_report``) as a list of dicts."""
    import json

    lib = load()
    need = lib.st_launch_report(None, 0)
    buf = ctypes.create_string_buffer(need)
    lib.st_launch_report(buf, need)
    codes = {v: str(k) for k, v in DTYPE_CODES.items()}
    records = json.loads(buf.value.decode())
    for r in records:
        r["dtype"] = codes.get(r["dtype"], r["dtype"])
    return records


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
