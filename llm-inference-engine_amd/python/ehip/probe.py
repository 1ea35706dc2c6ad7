"""ctypes front for ``lib/libehip_probe.so``: the read-bandwidth probes that
price the decode kernels' HBM roofline on the running device (benchmark
infrastructure, declared in ``probe/ehip_probe.h``; not part of the attention
C ABI)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import PKG, EhipError, lib

LIB_PATH = PKG / "lib" / "libehip_probe.so"
_lib = None


def plib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"probe library not built: {LIB_PATH}")
        lib()  # the HIP runtime and device the attention library uses
        L = C.CDLL(str(LIB_PATH))
        vp, i32, i64, fp = C.c_void_p, C.c_int32, C.c_int64, C.POINTER(C.c_float)
        L.ehip_probe_stream_read.argtypes = [vp, i64, i32, i32, fp]
        L.ehip_probe_tile_gather.argtypes = [vp, vp, i64, vp, i64, i32, i32, i64, i32, i32,
                                             i32, fp]
        L.ehip_probe_stream_read.restype = C.c_int
        L.ehip_probe_tile_gather.restype = C.c_int
        _lib = L
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise EhipError(rc, what)


def stream_read(buf, nbytes: int, nt: bool, reps: int = 3) -> float:
    """Best-of-reps streaming read rate (GB/s) of a device buffer."""
    g = C.c_float()
    _check(plib().ehip_probe_stream_read(buf.ptr, nbytes, int(nt), reps, C.byref(g)),
           "stream-read probe")
    return float(g.value)


def tile_gather(k_slab, v_slab, slab_blocks: int, blocks: np.ndarray, tiles_per_item: int,
                kv_heads: int, block_bytes: int, tile_bytes: int, nt: bool,
                reps: int = 3) -> float:
    """Best-of-reps rate (GB/s) of the decode access pattern alone."""
    b = np.ascontiguousarray(blocks, np.int32)
    g = C.c_float()
    _check(plib().ehip_probe_tile_gather(k_slab.ptr, v_slab.ptr, slab_blocks, b.ctypes.data,
                                         b.size, tiles_per_item, kv_heads, block_bytes,
                                         tile_bytes, int(nt), reps, C.byref(g)),
           "tile-gather probe")
    return float(g.value)
