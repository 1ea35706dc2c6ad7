"""CPU ORACLE — TEST INFRASTRUCTURE ONLY.

ctypes front for ``oracle/liboracle.so`` (the C restatement of the reference's
paged-attention path, see ``oracle/oracle.h``) and, where it was built, for
``oracle/_ref/libref.so`` (the reference's own kernels compiled from its
sources). Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``; the product never touches it.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libref.so"

ISA_SCALAR = 0
ISA_AVX2 = 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_PP = C.POINTER(C.c_void_p)

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = C.CDLL(str(LIB_PATH))
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_get_threads.restype = C.c_int
        L.orc_mt64_seed.argtypes = [C.c_void_p, C.c_uint64]
        L.orc_mt64_next.argtypes = [C.c_void_p]
        L.orc_mt64_next.restype = C.c_uint64
        L.orc_fill_normal.argtypes = [_f32p, _i64, C.c_double, C.c_double, C.c_uint64]
        L.orc_fill_uniform.argtypes = [_f32p, _i64, C.c_double, C.c_double, C.c_uint64]
        L.orc_fp32_to_bf16_bits.argtypes = [C.c_float]
        L.orc_fp32_to_bf16_bits.restype = C.c_uint16
        L.orc_fp32_to_bf16_array.argtypes = [_f32p, _u16p, _i64]
        L.orc_bf16_to_fp32_array.argtypes = [_u16p, _f32p, _i64]
        L.orc_exp_scalar.argtypes = [C.c_float]
        L.orc_exp_scalar.restype = C.c_float
        L.orc_exp_avx2_array.argtypes = [_f32p, _f32p, _i64]
        L.orc_paged_decode_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _i32p, _i64, _i64,
                                           _i64, _i64, _i64, _i64, _i64, C.c_float, _f32p]
        L.orc_paged_decode_f32.restype = C.c_int
        L.orc_paged_decode_batched_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _PP, _i64p,
                                                   _i64, _i64, _i64, _i64, _i64, _i64,
                                                   C.c_float, _f32p]
        L.orc_paged_decode_batched_f32.restype = C.c_int
        L.orc_decode_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64,
                                     _i64, C.c_float]
        L.orc_prefill_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64,
                                      _i64, _i64, C.c_float]
        L.orc_prefill_varlen_f32.argtypes = [C.c_int, _f32p, _i32p, _i64, _PP, _PP, _i64p,
                                             _f32p, _i64, _i64, _i64, C.c_float]
        L.orc_kv_scatter_f32.argtypes = [_f32p, _f32p, _i64p, _i64, _i64, _i64, _i64,
                                         _f32p, _f32p]
        L.orc_kv_scatter_bf16.argtypes = [_f32p, _f32p, _i64p, _i64, _i64, _i64, _i64,
                                          _u16p, _u16p]
        L.orc_kv_gather_f32.argtypes = [_f32p, _f32p, _i32p, _i64, _i64, _i64, _i64,
                                        _f32p, _f32p]
        L.orc_kv_append_int8.argtypes = [_f32p, _f32p, _i64p, _i64, _i64, _i64, _i64, _i8p,
                                         _i8p, _f32p, _f32p]
        L.orc_kv_append_int8.restype = None
        L.orc_int8_dequant.argtypes = [_i8p, _f32p, _i64, _i64, _i64, _i64, _f32p]
        L.orc_int8_dequant.restype = None
        L.orc_e4m3_to_fp32.argtypes = [C.c_uint8]
        L.orc_e4m3_to_fp32.restype = C.c_float
        L.orc_fp32_to_e4m3.argtypes = [C.c_float]
        L.orc_fp32_to_e4m3.restype = C.c_uint8
        L.orc_kv_append_fp8.argtypes = [_f32p, _f32p, _i64p, _i64, _i64, _i64, _i64, _u8p,
                                        _u8p, _f32p, _f32p]
        L.orc_kv_append_fp8.restype = None
        L.orc_fp8_dequant.argtypes = [_u8p, _f32p, _i64, _i64, _i64, _i64, _f32p]
        L.orc_fp8_dequant.restype = None
        L.orc_rope_apply_f32.argtypes = [C.c_int, _f32p, _i64, _i64, _i64, _i32p, _f32p, _f32p]
        L.orc_rope_apply_f32.restype = None
        L.orc_cpu_attention.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                        C.c_float, _f32p]
        L.orc_cpu_attention.restype = C.c_int
        L.orc_pack_weight_panels_u16.argtypes = [_u16p, _i64, _i64, _u16p]
        L.orc_pack_weight_panels_u16.restype = None
        L.orc_pack_weight_panels_f32.argtypes = [_f32p, _i64, _i64, _f32p]
        L.orc_pack_weight_panels_f32.restype = None
        L.orc_fp16_bits_to_fp32.argtypes = [C.c_uint16]
        L.orc_fp16_bits_to_fp32.restype = C.c_float
        L.orc_packed_gemm.argtypes = [_f32p, _i64, _i64, C.c_void_p, C.c_int, _i64, C.c_void_p,
                                      _f32p]
        L.orc_packed_gemm.restype = C.c_int
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_PATH.exists()


def ref():
    """The reference's own kernels (compiled from its sources), or None."""
    global _ref
    if _ref is None and REF_PATH.exists():
        R = C.CDLL(str(REF_PATH))
        R.ref_selected_isa.restype = C.c_int
        R.ref_exp_scalar.argtypes = [C.c_float]
        R.ref_exp_scalar.restype = C.c_float
        R.ref_paged_decode_batched_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _PP, _i64p,
                                                   _i64, _i64, _i64, _i64, _i64, _i64,
                                                   C.c_float, _f32p]
        R.ref_paged_decode_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _i32p, _i64, _i64,
                                           _i64, _i64, _i64, _i64, _i64, C.c_float, _f32p]
        R.ref_prefill_varlen_f32.argtypes = [C.c_int, _f32p, _i32p, _i64, _PP, _PP, _i64p,
                                             _f32p, _i64, _i64, _i64, C.c_float]
        R.ref_decode_f32.argtypes = [C.c_int, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64,
                                     _i64, C.c_float]
        R.ref_kv_scatter_f32.argtypes = [_f32p, _f32p, _i64p, _i64, _i64, _i64, _i64,
                                         _f32p, _f32p]
        R.ref_rope_apply_f32.argtypes = [C.c_int, _f32p, _i64, _i64, _i64, _i32p, _f32p, _f32p]
        R.ref_rope_apply_f32.restype = None
        R.ref_kv_gather_f32.argtypes = [_f32p, _f32p, _i32p, _i64, _i64, _i64, _i64,
                                        _f32p, _f32p]
        R.ref_pack_weight_panels_u16.argtypes = [_u16p, _i64, _i64, _u16p]
        R.ref_pack_weight_panels_u16.restype = None
        R.ref_pack_weight_panels_f32.argtypes = [_f32p, _i64, _i64, _f32p]
        R.ref_pack_weight_panels_f32.restype = None
        R.ref_packed_gemm.argtypes = [C.c_int, C.c_int, _f32p, _i64, _i64, C.c_void_p, _i64,
                                      C.c_void_p, _f32p]
        R.ref_packed_gemm.restype = None
        _ref = R
    return _ref


def _ptr_array(arrs):
    a = (C.c_void_p * len(arrs))(*[x.ctypes.data for x in arrs])
    return C.cast(a, _PP), a


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ---------------------------------------------------------------- generators
class Mt64:
    """mt19937_64 (restated in C)."""

    def __init__(self, seed: int):
        self._buf = C.create_string_buffer(312 * 8 + 16)
        lib().orc_mt64_seed(self._buf, C.c_uint64(seed))

    def next(self) -> int:
        return int(lib().orc_mt64_next(self._buf))

    def unit(self) -> float:
        return (self.next() >> 11) * 2.0 ** -53


def fill_normal(n: int, mean: float, stddev: float, seed: int) -> np.ndarray:
    out = np.empty(int(n), np.float32)
    lib().orc_fill_normal(out, n, mean, stddev, seed)
    return out


# ---------------------------------------------------------------- bf16 / exp
def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_fp32_to_bf16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_fp32_array(b.reshape(-1), out.reshape(-1), b.size)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(to_bf16_bits(x))


def exp_scalar(x: float) -> float:
    return float(lib().orc_exp_scalar(x))


def exp_avx2(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    assert x.size % 8 == 0
    out = np.empty_like(x)
    lib().orc_exp_avx2_array(x, out, x.size)
    return out


# ---------------------------------------------------------------- attention
def paged_decode(q, k_slab, v_slab, block_table, length, heads, kv_heads, d, bs, scale,
                 isa=ISA_SCALAR):
    """PagedDecodeAttentionF32: q [H,d] -> out [H,d]."""
    out = np.empty((heads, d), np.float32)
    rc = lib().orc_paged_decode_f32(isa, np.ascontiguousarray(q, np.float32).reshape(-1),
                                    k_slab.reshape(-1), v_slab.reshape(-1),
                                    np.ascontiguousarray(block_table, np.int32),
                                    len(block_table), length, heads, kv_heads, d, bs,
                                    kv_heads * bs * d, scale, out.reshape(-1))
    if rc != 0:
        raise ValueError(f"orc_paged_decode_f32 rejected the call (status {rc})")
    return out


def paged_decode_batched(q, k_slab, v_slab, tables, lengths, heads, kv_heads, d, bs, scale,
                         isa=ISA_SCALAR, use_ref=False, ref_isa=None):
    """PagedDecodeAttentionBatchedF32: q [B,H,d] -> out [B,H,d]; tables: list of int32."""
    B = len(lengths)
    out = np.zeros((B, heads, d), np.float32)
    tabs = [np.ascontiguousarray(t, np.int32) for t in tables]
    pp, keep = _ptr_array(tabs) if B else (C.cast((C.c_void_p * 1)(), _PP), None)
    lens = np.ascontiguousarray(lengths, np.int64)
    args = (np.ascontiguousarray(q, np.float32).reshape(-1), k_slab.reshape(-1),
            v_slab.reshape(-1), pp, lens, B, heads, kv_heads, d, bs, kv_heads * bs * d,
            scale, out.reshape(-1))
    if use_ref:
        ref().ref_paged_decode_batched_f32(isa if ref_isa is None else ref_isa, *args)
    else:
        rc = lib().orc_paged_decode_batched_f32(isa, *args)
        if rc != 0:
            raise ValueError(f"orc_paged_decode_batched_f32 rejected the call (status {rc})")
    del keep
    return out


def decode_contig(q, k, v, heads, kv_heads, d, scale, isa=ISA_SCALAR, use_ref=False):
    l_dim = k.shape[1]
    out = np.empty((heads, d), np.float32)
    fn = ref().ref_decode_f32 if use_ref else lib().orc_decode_f32
    fn(isa, np.ascontiguousarray(q, np.float32).reshape(-1),
       np.ascontiguousarray(k, np.float32).reshape(-1),
       np.ascontiguousarray(v, np.float32).reshape(-1), out.reshape(-1), heads, kv_heads, d,
       l_dim, scale)
    return out


def prefill(q, k, v, heads, kv_heads, d, scale, isa=ISA_SCALAR):
    """PrefillAttentionF32: q [T,H,d], k/v [Hkv,L,d] -> out [T,H,d]."""
    t_dim = q.shape[0]
    l_dim = k.shape[1]
    out = np.empty((t_dim, heads, d), np.float32)
    lib().orc_prefill_f32(isa, np.ascontiguousarray(q, np.float32).reshape(-1),
                          np.ascontiguousarray(k, np.float32).reshape(-1),
                          np.ascontiguousarray(v, np.float32).reshape(-1), out.reshape(-1),
                          t_dim, heads, kv_heads, d, l_dim, scale)
    return out


def prefill_varlen(q, cu_seqlens, k_seqs, v_seqs, heads, kv_heads, d, scale,
                   isa=ISA_SCALAR, use_ref=False):
    B = len(k_seqs)
    out = np.zeros((int(cu_seqlens[-1]), heads, d), np.float32)
    ks = [np.ascontiguousarray(x, np.float32) for x in k_seqs]
    vs = [np.ascontiguousarray(x, np.float32) for x in v_seqs]
    kp, k_keep = _ptr_array(ks)
    vp, v_keep = _ptr_array(vs)
    l_dims = np.array([x.shape[1] for x in ks], np.int64)
    fn = ref().ref_prefill_varlen_f32 if use_ref else lib().orc_prefill_varlen_f32
    fn(isa, np.ascontiguousarray(q, np.float32).reshape(-1),
       np.ascontiguousarray(cu_seqlens, np.int32), B, kp, vp, l_dims, out.reshape(-1), heads,
       kv_heads, d, scale)
    del k_keep, v_keep
    return out


def cpu_attention(q, k, v, heads, kv_heads, d, scale):
    """The two-pass oracle cpu::attention: q [T,H,d], k/v [Hkv,L,d]."""
    t_dim = q.shape[0]
    l_dim = k.shape[1]
    out = np.empty((t_dim, heads, d), np.float32)
    rc = lib().orc_cpu_attention(np.ascontiguousarray(q, np.float32).reshape(-1),
                                 np.ascontiguousarray(k, np.float32).reshape(-1),
                                 np.ascontiguousarray(v, np.float32).reshape(-1), t_dim,
                                 heads, kv_heads, d, l_dim, scale, out.reshape(-1))
    if rc != 0:
        raise ValueError(f"orc_cpu_attention rejected the call (status {rc})")
    return out


def rope_apply(x, positions, cos, sin, isa=1, use_ref=False):
    """RopeApplyF32 on a copy of x [t, hx, d] (fp32); returns the rotated copy.
    isa 1 = the AVX2 row kernel's FMA form, 0 = the scalar form."""
    y = np.array(x, np.float32, copy=True, order="C")
    t, hx, d = y.shape
    pos = np.ascontiguousarray(positions, np.int32)
    c = np.ascontiguousarray(cos, np.float32).reshape(-1)
    s = np.ascontiguousarray(sin, np.float32).reshape(-1)
    fn = ref().ref_rope_apply_f32 if use_ref else lib().orc_rope_apply_f32
    fn(isa, y.reshape(-1), t, hx, d, pos, c, s)
    return y


def rope_tables(d, positions, theta=10000.0):
    """cos/sin tables [P, d/2] the way the reference's Rope module builds them
    for the default scaling (src/model/modules.cpp BaseInvFreq: inv_freq in
    double, stored fp32; angle = position * inv_freq in fp32). Test data for
    the RoPE kernels, which take the tables as inputs."""
    half = d // 2
    inv = (1.0 / np.power(float(theta), np.arange(half, dtype=np.float64) * 2.0 / d)).astype(np.float32)
    ang = np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def kv_scatter(src_k, src_v, slot_mapping, kv_heads, d, bs, k_slab, v_slab, use_ref=False):
    """KvScatterF32 in place into fp32 slabs, or the bf16 variant into uint16 slabs."""
    t_dim = len(slot_mapping)
    sm = np.ascontiguousarray(slot_mapping, np.int64)
    sk = np.ascontiguousarray(src_k, np.float32).reshape(-1)
    sv = np.ascontiguousarray(src_v, np.float32).reshape(-1)
    if k_slab.dtype == np.uint16:
        lib().orc_kv_scatter_bf16(sk, sv, sm, t_dim, kv_heads, d, bs, k_slab.reshape(-1),
                                  v_slab.reshape(-1))
    elif use_ref:
        ref().ref_kv_scatter_f32(sk, sv, sm, t_dim, kv_heads, d, bs, k_slab.reshape(-1),
                                 v_slab.reshape(-1))
    else:
        lib().orc_kv_scatter_f32(sk, sv, sm, t_dim, kv_heads, d, bs, k_slab.reshape(-1),
                                 v_slab.reshape(-1))


def kv_append_int8(src_k, src_v, slot_mapping, kv_heads, d, bs, k_slab, v_slab, k_scale,
                   v_scale):
    """INT8 append in place: slabs int8 [blocks, Hkv, bs, d], scales fp32 [blocks, Hkv]."""
    sm = np.ascontiguousarray(slot_mapping, np.int64)
    for a, dt in ((k_slab, np.int8), (v_slab, np.int8), (k_scale, np.float32),
                  (v_scale, np.float32)):
        assert a.dtype == dt and a.flags.c_contiguous
    lib().orc_kv_append_int8(np.ascontiguousarray(src_k, np.float32).reshape(-1),
                             np.ascontiguousarray(src_v, np.float32).reshape(-1), sm, len(sm),
                             kv_heads, d, bs, k_slab.reshape(-1), v_slab.reshape(-1),
                             k_scale.reshape(-1), v_scale.reshape(-1))


def e4m3_to_f32(codes):
    """fp32 values of OCP E4M3 codes (uint8 array)."""
    c = np.ascontiguousarray(codes, np.uint8)
    return np.array([lib().orc_e4m3_to_fp32(int(x)) for x in c.reshape(-1)],
                    np.float32).reshape(c.shape)


def f32_to_e4m3(x):
    """OCP E4M3 codes of fp32 values (round to nearest even, saturating)."""
    a = np.ascontiguousarray(x, np.float32)
    return np.array([lib().orc_fp32_to_e4m3(float(v)) for v in a.reshape(-1)],
                    np.uint8).reshape(a.shape)


def kv_append_fp8(src_k, src_v, slot_mapping, kv_heads, d, bs, k_slab, v_slab, k_scale,
                  v_scale):
    """FP8 (E4M3) append in place: slabs uint8 [blocks, Hkv, bs, d], scales fp32 [blocks, Hkv]."""
    sm = np.ascontiguousarray(slot_mapping, np.int64)
    for a, dt in ((k_slab, np.uint8), (v_slab, np.uint8), (k_scale, np.float32),
                  (v_scale, np.float32)):
        assert a.dtype == dt and a.flags.c_contiguous
    lib().orc_kv_append_fp8(np.ascontiguousarray(src_k, np.float32).reshape(-1),
                            np.ascontiguousarray(src_v, np.float32).reshape(-1), sm, len(sm),
                            kv_heads, d, bs, k_slab.reshape(-1), v_slab.reshape(-1),
                            k_scale.reshape(-1), v_scale.reshape(-1))


def fp8_dequant(slab, scale):
    """fp32 copy of an FP8 slab [blocks, Hkv, bs, d]: e4m3(q) * scale[block, head]."""
    nb, hkv, bs, d = slab.shape
    out = np.empty(slab.shape, np.float32)
    lib().orc_fp8_dequant(np.ascontiguousarray(slab, np.uint8).reshape(-1),
                          np.ascontiguousarray(scale, np.float32).reshape(-1), nb, hkv, bs, d,
                          out.reshape(-1))
    return out


def int8_dequant(slab, scale):
    """fp32 copy of an INT8 slab [blocks, Hkv, bs, d]: q * scale[block, head]."""
    nb, hkv, bs, d = slab.shape
    out = np.empty(slab.shape, np.float32)
    lib().orc_int8_dequant(np.ascontiguousarray(slab).reshape(-1),
                           np.ascontiguousarray(scale, np.float32).reshape(-1), nb, hkv, bs, d,
                           out.reshape(-1))
    return out


def kv_gather(k_slab, v_slab, block_table, bs, length, kv_heads, d, use_ref=False):
    out_k = np.zeros((kv_heads, length, d), np.float32)
    out_v = np.zeros((kv_heads, length, d), np.float32)
    fn = ref().ref_kv_gather_f32 if use_ref else lib().orc_kv_gather_f32
    fn(k_slab.reshape(-1), v_slab.reshape(-1), np.ascontiguousarray(block_table, np.int32),
       bs, length, kv_heads, d, out_k.reshape(-1), out_v.reshape(-1))
    return out_k, out_v


def paged_to_contig(slab, table, length, kv_heads, d, bs):
    """[Hkv, L, d] view of one sequence's cache (numpy indexing, independent of
    the gather kernel): slab is [NB, Hkv, bs, d]."""
    nb = (length + bs - 1) // bs
    blocks = slab[np.asarray(table[:nb], np.int64)]          # [nb, Hkv, bs, d]
    full = blocks.transpose(1, 0, 2, 3).reshape(kv_heads, nb * bs, d)
    return np.ascontiguousarray(full[:, :length])


# ---- packed linear layer (o_proj) -------------------------------------------
WEIGHT_F32, WEIGHT_BF16, WEIGHT_F16 = 0, 1, 2


def pack_weight_panels(w: np.ndarray, use_ref: bool = False) -> np.ndarray:
    """kernels::PackWeightPanels: w [n, k] (float32, or uint16 bit patterns of
    bf16 / fp16) -> [ceil(n/16), k, 16] of the same dtype, 0 past n."""
    n, k = w.shape
    panels = (n + 15) // 16
    if w.dtype == np.float32:
        out = np.empty((panels, k, 16), np.float32)
        fn = (ref().ref_pack_weight_panels_f32 if use_ref else lib().orc_pack_weight_panels_f32)
    else:
        w = w.astype(np.uint16, copy=False)
        out = np.empty((panels, k, 16), np.uint16)
        fn = (ref().ref_pack_weight_panels_u16 if use_ref else lib().orc_pack_weight_panels_u16)
    fn(np.ascontiguousarray(w).reshape(-1), n, k, out.reshape(-1))
    return out


def fp16_bits_to_f32(b: int) -> float:
    return float(lib().orc_fp16_bits_to_fp32(int(b)))


def packed_gemm(x: np.ndarray, wp: np.ndarray, dtype: int, n: int, bias=None, isa: int = 0,
                use_ref: bool = False) -> np.ndarray:
    """kernels::PackedGemm: y [m, n] = x [m, k] W^T (+ bias) over the packed
    weight; the restatement of the scalar tile, or (use_ref) the reference's
    own tile of `isa` (0 scalar, 1 AVX2, -1 the public threaded entry)."""
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    y = np.empty((m, n), np.float32)
    wpc = np.ascontiguousarray(wp)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    bp = None if b is None else b.ctypes.data
    if use_ref:
        ref().ref_packed_gemm(isa, dtype, x.reshape(-1), m, k, wpc.ctypes.data, n, bp,
                              y.reshape(-1))
    else:
        rc = lib().orc_packed_gemm(x.reshape(-1), m, k, wpc.ctypes.data, dtype, n, bp,
                                   y.reshape(-1))
        if rc != 0:
            raise ValueError(f"orc_packed_gemm rejected the call ({rc})")
    return y
