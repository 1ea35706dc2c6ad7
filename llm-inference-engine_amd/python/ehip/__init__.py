"""ctypes front for ``lib/libehip.so`` — the gfx950 paged-attention C ABI
declared in ``include/ehip.h``.

Host arrays are numpy; device memory is held by :class:`DeviceBuffer`
(allocated with ``ehip_malloc``). Every call goes straight to the HIP library:
there is no CPU fallback, and loading fails loudly if the library was not
built (``make -C llm-inference-engine_amd``).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parents[2]
LIB_PATH = PKG / "lib" / "libehip.so"
HEADER = PKG.parent / "include" / "ehip.h"

OK = 0
INVALID_ARGUMENT = 2
FAILED_PRECONDITION = 5
RESOURCE_EXHAUSTED = 7
OUT_OF_MEMORY = 8
UNIMPLEMENTED = 9
INTERNAL = 11

KV_F32 = 0
KV_BF16 = 1
KV_INT8 = 2
KV_FP8 = 3

WEIGHT_F32 = 0
WEIGHT_BF16 = 1
WEIGHT_F16 = 2

_i32 = C.c_int32
_i64 = C.c_int64
_vp = C.c_void_p
_I64P = C.POINTER(C.c_int64)


class EhipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"ehip status {code}: {msg}")
        self.code = code


class Geometry(C.Structure):
    _fields_ = [("heads", _i32), ("kv_heads", _i32), ("head_dim", _i32), ("block_size", _i32),
                ("kv_dtype", _i32), ("reserved", _i32), ("slab_blocks", _i64),
                ("block_stride", _i64), ("scale", C.c_float)]


class StepDesc(C.Structure):
    _fields_ = [("num_seqs", _i32), ("reserved", _i32), ("h_query_lens", _vp),
                ("h_context_lens", _vp), ("h_table_offsets", _vp), ("h_table_ids", _vp),
                ("h_slot_mapping", _vp)]


_lib = None


def lib():
    """Load libehip.so (raises if it is missing: there is no fallback)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"HIP library not built: {LIB_PATH} "
                               "(run make -C llm-inference-engine_amd)")
        L = C.CDLL(str(LIB_PATH))
        sig = {
            "ehip_init": [C.c_int, C.POINTER(_vp)],
            "ehip_destroy": [_vp],
            "ehip_last_error": [_vp, C.c_char_p, C.c_size_t],
            "ehip_device_count": [C.POINTER(C.c_int)],
            "ehip_sync": [_vp],
            "ehip_malloc": [_vp, _i64, C.POINTER(_vp)],
            "ehip_free": [_vp, _vp],
            "ehip_copy_to_device": [_vp, _vp, _vp, _i64],
            "ehip_copy_to_host": [_vp, _vp, _vp, _i64],
            "ehip_copy_device": [_vp, _vp, _vp, _i64],
            "ehip_fill_normal": [_vp, _vp, _i64, _i32, C.c_float, C.c_float, C.c_uint64],
            "ehip_event_create": [_vp, C.POINTER(_vp)],
            "ehip_event_destroy": [_vp, _vp],
            "ehip_event_record": [_vp, _vp],
            "ehip_event_elapsed_ms": [_vp, _vp, _vp, C.POINTER(C.c_float)],
            "ehip_kv_scatter_f32": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
            "ehip_kv_scatter_bf16": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
            "ehip_kv_gather_f32": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
            "ehip_paged_decode_attention_f32": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                                _i64, _i64, _i64, _i64, C.c_float, _vp],
            "ehip_prefill_attention_f32": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                           _i64, C.c_float],
            "ehip_decode_attention_f32": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                          C.c_float],
            "ehip_prefill_attention_varlen_f32": [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                                                  _i64, _i64, _i64, C.c_float],
            "ehip_pack_weight_panels": [_vp, _vp, _i32, _i64, _i64, _vp],
            "ehip_packed_gemm": [_vp, _vp, _i64, _i64, _vp, _i32, _i64, _vp, _vp],
            "ehip_paged_decode_attention_f32_noalloc": [_vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                                        _i64, _i64, _i64, _i64, _i64, _i64,
                                                        C.c_float, _vp],
            "ehip_paged_decode_attention_batched_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                                        _i64, _i64, _i64, _i64, _i64, _i64,
                                                        C.c_float, _vp],
            "ehip_paged_decode_attention_batched_bf16": [_vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                                         _i64, _i64, _i64, _i64, _i64, _i64,
                                                         C.c_float, _vp],
            "ehip_set_stream": [_vp, _vp],
            "ehip_step_upload": [_vp, C.POINTER(Geometry), C.POINTER(StepDesc)],
            "ehip_step_kv_append": [_vp, _vp, _vp, _vp, _vp],
            "ehip_step_rope_kv_append": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp],
            "ehip_step_kv_append_int8": [_vp, _vp, _vp, _vp, _vp, _vp, _vp],
            "ehip_step_attention_int8": [_vp, _vp, _vp, _vp, _vp, _vp, _vp],
            "ehip_step_kv_append_fp8": [_vp, _vp, _vp, _vp, _vp, _vp, _vp],
            "ehip_step_attention_fp8": [_vp, _vp, _vp, _vp, _vp, _vp, _vp],
            "ehip_step_attention": [_vp, _vp, _vp, _vp, _vp],
            "ehip_step_append_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _vp],
            "ehip_step_info": [_vp, _I64P, _I64P, _I64P],
            "ehip_plan_counts": [C.POINTER(Geometry), C.POINTER(StepDesc), _I64P, _I64P, _I64P,
                                 C.POINTER(C.c_int32), _I64P, _I64P],
            "ehip_plan_items": [C.POINTER(Geometry), C.POINTER(StepDesc), _vp, _i64, _I64P],
            "ehip_rng_u64": [C.c_uint64, C.c_uint64, _vp, _i64],
            "ehip_host_fill_normal": [_vp, _i64, C.c_double, C.c_double, C.c_uint64],
            "ehip_host_fp32_to_bf16": [_vp, _vp, _i64],
            "ehip_plan_prefill_items": [C.POINTER(Geometry), C.POINTER(StepDesc), _vp, _i64,
                                        _I64P],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = C.c_int
        _lib = L
    return _lib


def header_symbols() -> list[str]:
    """Every function include/ehip.h declares."""
    import re
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*int\s+(ehip_\w+)\s*\(", text, flags=re.M)))


def device_count() -> int:
    n = C.c_int(0)
    lib().ehip_device_count(C.byref(n))
    return n.value


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


class StepArrays:
    """Host arrays of one step, kept alive while a StepDesc points at them."""

    def __init__(self, query_lens, context_lens, tables, slot_mapping=None):
        self.query_lens = np.ascontiguousarray(query_lens, np.int32)
        self.context_lens = np.ascontiguousarray(context_lens, np.int64)
        tabs = [np.ascontiguousarray(t, np.int32) for t in tables]
        self.offsets = np.zeros(len(tabs) + 1, np.int32)
        if tabs:
            self.offsets[1:] = np.cumsum([len(t) for t in tabs])
        self.ids = np.ascontiguousarray(np.concatenate(tabs) if tabs else np.zeros(1, np.int32),
                                        np.int32)
        self.slots = None if slot_mapping is None else np.ascontiguousarray(slot_mapping,
                                                                             np.int64)
        self.desc = StepDesc(len(tabs), 0, _ptr(self.query_lens), _ptr(self.context_lens),
                             _ptr(self.offsets), _ptr(self.ids), _ptr(self.slots))


def geometry(heads, kv_heads, head_dim, block_size, kv_dtype, slab_blocks, scale,
             block_stride=0) -> Geometry:
    return Geometry(heads, kv_heads, head_dim, block_size, kv_dtype, 0, slab_blocks,
                    block_stride, scale)


def plan_counts(geom: Geometry, step: StepArrays, joint: bool = False):
    """Host-only planning (no GPU): (status, rows, items, partials, split_tokens)
    and, with joint=True, also (joint_items, shared_tokens)."""
    r, i, p, j, sh = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64()
    s = C.c_int32()
    rc = lib().ehip_plan_counts(C.byref(geom), C.byref(step.desc), C.byref(r), C.byref(i),
                                C.byref(p), C.byref(s), C.byref(j), C.byref(sh))
    out = (rc, r.value, i.value, p.value, s.value)
    return out + (j.value, sh.value) if joint else out


def plan_items(geom: Geometry, step: StepArrays):
    """Host-only planning: (status, items [n, 8] int32) with columns row, the
    joint rows 2..4 (-1 where absent), key_begin, key_end, kv_head, split, in
    dispatch order."""
    n = C.c_int64()
    rc = lib().ehip_plan_items(C.byref(geom), C.byref(step.desc), None, 0, C.byref(n))
    if rc != 0:
        return rc, np.zeros((0, 8), np.int32)
    out = np.zeros((n.value, 8), np.int32)
    rc = lib().ehip_plan_items(C.byref(geom), C.byref(step.desc), out.ctypes.data, n.value,
                               C.byref(n))
    return rc, out


class DeviceBuffer:
    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = _vp()
        ctx._check(lib().ehip_malloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.ctx._check(lib().ehip_free(self.ctx.h, self.ptr))
            self.ptr = None

    def upload(self, arr: np.ndarray):
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        self.ctx._check(lib().ehip_copy_to_device(self.ctx.h, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        self.ctx._check(lib().ehip_copy_to_host(self.ctx.h, out.ctypes.data, self.ptr,
                                                out.nbytes))
        return out


class Context:
    """One ehip_ctx (device + stream + step descriptor + workspace)."""

    def __init__(self, device: int = 0):
        h = _vp()
        rc = lib().ehip_init(device, C.byref(h))
        if rc != OK:
            raise EhipError(rc, f"ehip_init(device={device}) failed")
        self.h = h.value

    def close(self):
        if self.h:
            lib().ehip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def last_error(self) -> str:
        buf = C.create_string_buffer(512)
        lib().ehip_last_error(self.h, buf, 512)
        return buf.value.decode()

    def _check(self, rc: int):
        if rc != OK:
            raise EhipError(rc, self.last_error())

    def status(self, rc: int) -> int:
        return rc

    # -------------------------------------------------------------- memory
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        return DeviceBuffer(self, max(a.nbytes, 1)).upload(a)

    def sync(self):
        self._check(lib().ehip_sync(self.h))

    def fill_normal(self, buf: DeviceBuffer, n: int, dtype: int, mean: float, std: float,
                    seed: int):
        self._check(lib().ehip_fill_normal(self.h, buf.ptr, n, dtype, mean, std, seed))

    # -------------------------------------------------------------- events
    def event(self):
        e = _vp()
        self._check(lib().ehip_event_create(self.h, C.byref(e)))
        return e.value

    def record(self, ev):
        self._check(lib().ehip_event_record(self.h, ev))

    def elapsed_ms(self, e0, e1) -> float:
        ms = C.c_float()
        self._check(lib().ehip_event_elapsed_ms(self.h, e0, e1, C.byref(ms)))
        return float(ms.value)

    # ------------------------------------------------- reference kernels
    def kv_scatter(self, src_k, src_v, slots, t_dim, kv_heads, d, bs, slab_blocks, k_slab,
                   v_slab, bf16: bool) -> int:
        fn = lib().ehip_kv_scatter_bf16 if bf16 else lib().ehip_kv_scatter_f32
        return fn(self.h, src_k.ptr, src_v.ptr, slots.ptr, t_dim, kv_heads, d, bs, slab_blocks,
                  k_slab.ptr, v_slab.ptr)

    def kv_gather(self, k_slab, v_slab, table, bs, length, kv_heads, d, slab_blocks, out_k,
                  out_v) -> int:
        return lib().ehip_kv_gather_f32(self.h, k_slab.ptr, v_slab.ptr, table.ptr, bs, length,
                                        kv_heads, d, slab_blocks, out_k.ptr, out_v.ptr)

    def paged_decode(self, q, k_slab, v_slab, table, num_blocks, length, heads, kv_heads, d,
                     bs, block_stride, slab_blocks, scale, out) -> int:
        return lib().ehip_paged_decode_attention_f32(
            self.h, q.ptr, k_slab.ptr, v_slab.ptr, table.ptr, num_blocks, length, heads,
            kv_heads, d, bs, block_stride, slab_blocks, scale, out.ptr)

    def prefill_attention_varlen(self, q, cu_seqlens, k_seqs, v_seqs, l_dims, out, heads,
                                 kv_heads, d, scale) -> int:
        """q/out device buffers [sum T, H, d]; cu_seqlens, l_dims host arrays;
        k_seqs / v_seqs lists of device buffers ([Hkv, L_b, d] each)."""
        cu = np.ascontiguousarray(cu_seqlens, np.int32)
        ls = np.ascontiguousarray(l_dims, np.int64)
        ks = (_vp * max(1, len(k_seqs)))(*[k.ptr for k in k_seqs])
        vs = (_vp * max(1, len(v_seqs)))(*[v.ptr for v in v_seqs])
        return lib().ehip_prefill_attention_varlen_f32(
            self.h, q.ptr if q else None, cu.ctypes.data, len(k_seqs), C.cast(ks, _vp),
            C.cast(vs, _vp), ls.ctypes.data, out.ptr if out else None, heads, kv_heads, d,
            scale)

    def pack_weight_panels(self, w, weight_dtype, n, k, wp) -> int:
        """Device buffers: w [n, k] -> wp [ceil(n/16), k, 16] (same dtype)."""
        return lib().ehip_pack_weight_panels(self.h, w.ptr, weight_dtype, n, k, wp.ptr)

    def packed_gemm(self, x, m, k, wp, weight_dtype, n, bias, y) -> int:
        """Device buffers: y [m, n] = x [m, k] W^T (+ bias) over the packed wp."""
        return lib().ehip_packed_gemm(self.h, x.ptr, m, k, wp.ptr, weight_dtype, n,
                                      bias.ptr if bias is not None else None, y.ptr)

    def paged_decode_batched(self, q, k_slab, v_slab, tables, lengths, heads, kv_heads, d, bs,
                             block_stride, slab_blocks, scale, out, bf16=False) -> int:
        tabs = [np.ascontiguousarray(t, np.int32) for t in tables]
        arr = (_vp * max(1, len(tabs)))(*[t.ctypes.data for t in tabs])
        lens = np.ascontiguousarray(lengths, np.int64)
        fn = (lib().ehip_paged_decode_attention_batched_bf16 if bf16
              else lib().ehip_paged_decode_attention_batched_f32)
        rc = fn(self.h, q.ptr if q else None, k_slab.ptr if k_slab else None,
                v_slab.ptr if v_slab else None, C.cast(arr, _vp), lens.ctypes.data, len(tabs),
                heads, kv_heads, d, bs, block_stride, slab_blocks, scale,
                out.ptr if out else None)
        del tabs
        return rc

    # ---------------------------------------------------------- step path
    def step_upload(self, geom: Geometry, step: StepArrays) -> int:
        return lib().ehip_step_upload(self.h, C.byref(geom), C.byref(step.desc))

    def step_kv_append(self, src_k, src_v, k_slab, v_slab) -> int:
        return lib().ehip_step_kv_append(self.h, src_k.ptr, src_v.ptr, k_slab.ptr, v_slab.ptr)

    def step_rope_kv_append(self, q, src_k, src_v, cos, sin, table_positions, k_slab,
                            v_slab) -> int:
        return lib().ehip_step_rope_kv_append(self.h, q.ptr, src_k.ptr, src_v.ptr, cos.ptr,
                                              sin.ptr, table_positions, k_slab.ptr, v_slab.ptr)

    def step_kv_append_int8(self, src_k, src_v, k_slab, v_slab, k_scale, v_scale) -> int:
        return lib().ehip_step_kv_append_int8(self.h, src_k.ptr, src_v.ptr, k_slab.ptr,
                                              v_slab.ptr, k_scale.ptr, v_scale.ptr)

    def step_attention_int8(self, q, k_slab, v_slab, k_scale, v_scale, out) -> int:
        return lib().ehip_step_attention_int8(self.h, q.ptr, k_slab.ptr, v_slab.ptr,
                                              k_scale.ptr, v_scale.ptr, out.ptr)

    def step_kv_append_fp8(self, src_k, src_v, k_slab, v_slab, k_scale, v_scale) -> int:
        return lib().ehip_step_kv_append_fp8(self.h, src_k.ptr, src_v.ptr, k_slab.ptr,
                                             v_slab.ptr, k_scale.ptr, v_scale.ptr)

    def step_attention_fp8(self, q, k_slab, v_slab, k_scale, v_scale, out) -> int:
        return lib().ehip_step_attention_fp8(self.h, q.ptr, k_slab.ptr, v_slab.ptr,
                                             k_scale.ptr, v_scale.ptr, out.ptr)

    def step_append_attention(self, src_k, src_v, q, k_slab, v_slab, out) -> int:
        return lib().ehip_step_append_attention(self.h, src_k.ptr, src_v.ptr, q.ptr, k_slab.ptr,
                                                v_slab.ptr, out.ptr)

    def step_attention(self, q, k_slab, v_slab, out) -> int:
        return lib().ehip_step_attention(self.h, q.ptr, k_slab.ptr, v_slab.ptr, out.ptr)

    def step_info(self):
        r, i, p = C.c_int64(), C.c_int64(), C.c_int64()
        self._check(lib().ehip_step_info(self.h, C.byref(r), C.byref(i), C.byref(p)))
        return r.value, i.value, p.value
