"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker and CPU baseline. The product (leanstream_amd) never imports this package.
See oracle.c for the reference file:line each function restates.
"""
import ctypes as C
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = _HERE / "liboracle.so"
_lib = None


class OraDesc(C.Structure):
    _fields_ = [("logical_group", C.c_uint32), ("physical_group", C.c_uint32), ("source_slot", C.c_uint32),
                ("dest_slot", C.c_uint32), ("source_kind", C.c_uint32)]


def lib():
    global _lib
    if _lib is None:
        if not _LIB.is_file():
            raise RuntimeError("oracle/liboracle.so missing: run make -C oracle")
        l = C.CDLL(str(_LIB))
        p = C.c_void_p
        for name, args, res in [
            ("ora_f16_to_f32", [C.c_uint16], C.c_float), ("ora_f32_to_f16", [C.c_float], C.c_uint16),
            ("ora_f64_to_f16", [C.c_double], C.c_uint16), ("ora_stream", [C.c_uint64, C.c_uint64], C.c_uint64),
            ("ora_normal", [C.c_uint64, C.c_uint64], C.c_double),
            ("ora_fill_bytes", [p, C.c_uint64, C.c_uint64], None),
            ("ora_fill_uniform_f16", [p, C.c_uint64, C.c_uint64, C.c_double, C.c_double], None),
            ("ora_fill_normal_f16", [p, C.c_uint64, C.c_uint64], None),
            ("ora_weight", [p, p, C.c_uint32], C.c_float),
            ("ora_compute", [p, p, p, p, p, C.c_uint32, C.c_uint32, p, p], C.c_int),
            ("ora_reduce", [p, C.c_uint32, C.c_uint32, p, p], None),
            ("ora_layer", [p, C.c_uint32, C.c_uint32, p, p, p, p, C.c_uint32, C.c_uint32, C.c_int, p, p, p, p],
             C.c_int),
            ("ora_rank", [p, C.c_uint32, C.c_uint32, p], C.c_int),
            ("ora_publish_hidden", [p, p, C.c_uint32, p], None),
            ("ora_rmsnorm", [p, p, C.c_float, C.c_uint32, p], C.c_int),
        ]:
            f = getattr(l, name)
            f.argtypes = args
            f.restype = res
        _lib = l
    return _lib


def _addr(a):
    return None if a is None else a.ctypes.data


def fill_bytes(n, seed):
    out = np.empty(n, dtype=np.uint8)
    lib().ora_fill_bytes(_addr(out), n, seed)
    return out


def fill_uniform_f16(n, seed, lo, hi):
    out = np.empty(n, dtype=np.float16)
    lib().ora_fill_uniform_f16(_addr(out), n, seed, lo, hi)
    return out


def fill_normal_f16(n, seed):
    out = np.empty(n, dtype=np.float16)
    lib().ora_fill_normal_f16(_addr(out), n, seed)
    return out


def layer(descs, rows, cache, scales, x, width, group_size, staging=None, threads=1, want_partial=False):
    """Reference layer output. descs: uint32 [n, 5]. Returns dict(y32, y16, h, partial)."""
    descs = np.ascontiguousarray(np.asarray(descs, dtype=np.uint32).reshape(-1, 5))
    cache = np.ascontiguousarray(cache, dtype=np.uint8)
    staging = cache if staging is None else np.ascontiguousarray(staging, dtype=np.uint8)
    scales = np.ascontiguousarray(scales).view(np.uint16)
    x = np.ascontiguousarray(x).view(np.uint16)
    y32 = np.zeros(width, dtype=np.float32)
    y16 = np.zeros(width, dtype=np.uint16)
    h = np.zeros(max(1, rows) * group_size, dtype=np.float32)
    partial = np.zeros(max(1, rows) * width, dtype=np.float32)
    rc = lib().ora_layer(_addr(descs), len(descs), rows, _addr(cache), _addr(staging), _addr(scales), _addr(x), width,
                         group_size, threads, _addr(y32), _addr(y16), _addr(h), _addr(partial))
    if rc:
        raise ValueError(f"oracle layer failed: {rc}")
    out = dict(y32=y32, y16=y16.view(np.float16), h=h[: rows * group_size].reshape(rows, group_size))
    if want_partial:
        out["partial"] = partial[: rows * width].reshape(rows, width)
    return out


def rank(scores, k):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros(max(1, k), dtype=np.int32)
    rc = lib().ora_rank(_addr(s), len(s), k, _addr(out))
    if rc:
        raise ValueError(f"oracle rank failed: {rc}")
    return out[:k].astype(np.int64)


def publish_hidden(residual, y16):
    """fp16(fp32 residual + fp32 y) per element (the next layer's hidden state)."""
    r = np.ascontiguousarray(residual, dtype=np.float16).view(np.uint16)
    y = np.ascontiguousarray(y16, dtype=np.float16).view(np.uint16)
    out = np.zeros(r.size, dtype=np.uint16)
    lib().ora_publish_hidden(_addr(r), _addr(y), r.size, _addr(out))
    return out.view(np.float16)


def rmsnorm(x, weight, eps):
    """RMSNorm of one fp16 row with an fp16 weight; fp16 out."""
    xv = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    w = np.ascontiguousarray(weight, dtype=np.float16).view(np.uint16)
    out = np.zeros(xv.size, dtype=np.uint16)
    rc = lib().ora_rmsnorm(_addr(xv), _addr(w), float(eps), xv.size, _addr(out))
    if rc:
        raise ValueError("oracle rmsnorm failed")
    return out.view(np.float16)
