"""The contiguous-cache entry points (ehip_decode_attention_f32,
ehip_prefill_attention_f32, ehip_prefill_attention_varlen_f32 = the
reference's DecodeAttentionF32, PrefillAttentionF32 and
PrefillAttentionVarlenF32, src/kernels/attention.h:40-73, :221-227) against
the oracle's restatements of the same functions: fp32, within 1e-4 relative
per output vector and the reference allclose (rtol 1e-4, atol 1e-5)."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import rel_norm
from paged_util import allclose_ref, scale_for

pytestmark = pytest.mark.gpu


def _dev(gctx, *arrs):
    return [gctx.to_device(np.ascontiguousarray(a, np.float32)) for a in arrs]


def _check(got, ref):
    assert rel_norm(got, ref) <= 1e-4, rel_norm(got, ref)
    assert allclose_ref(got, ref, 1e-4, 1e-5)


@pytest.mark.parametrize("H,Hkv,d,L", [(14, 2, 64, 513), (32, 8, 128, 2048), (8, 8, 128, 1),
                                       (28, 4, 64, 1000), (6, 3, 18, 77), (64, 8, 128, 20000)])
def test_decode_attention_contiguous(gctx, ehip_mod, orc, H, Hkv, d, L):
    rng = np.random.default_rng(H * L + d)
    q = rng.standard_normal((H, d)).astype(np.float32)
    k = rng.standard_normal((Hkv, L, d)).astype(np.float32)
    v = rng.standard_normal((Hkv, L, d)).astype(np.float32)
    dq, dk, dv = _dev(gctx, q, k, v)
    out = gctx.alloc(q.nbytes)
    rc = ehip_mod.lib().ehip_decode_attention_f32(gctx.h, dq.ptr, dk.ptr, dv.ptr, out.ptr, H, Hkv,
                                                  d, L, C.c_float(scale_for(d)))
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    _check(got, orc.decode_contig(q, k, v, H, Hkv, d, scale_for(d)))
    if L == 1:  # one key: every head of group hk returns v[hk, 0]
        assert np.array_equal(got, np.repeat(v[:, 0, :], H // Hkv, axis=0))


@pytest.mark.parametrize("H,Hkv,d", [(32, 8, 128), (14, 2, 64)])
@pytest.mark.parametrize("T,L", [(1, 1), (16, 16), (37, 100), (128, 128), (5, 300), (300, 301)])
def test_prefill_attention_contiguous(gctx, ehip_mod, orc, H, Hkv, d, T, L):
    rng = np.random.default_rng(T * 1000 + L + H)
    q = rng.standard_normal((T, H, d)).astype(np.float32)
    k = rng.standard_normal((Hkv, L, d)).astype(np.float32)
    v = rng.standard_normal((Hkv, L, d)).astype(np.float32)
    dq, dk, dv = _dev(gctx, q, k, v)
    out = gctx.alloc(q.nbytes)
    rc = ehip_mod.lib().ehip_prefill_attention_f32(gctx.h, dq.ptr, dk.ptr, dv.ptr, out.ptr, T, H,
                                                   Hkv, d, L, C.c_float(scale_for(d)))
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    _check(got, orc.prefill(q, k, v, H, Hkv, d, scale_for(d)))


VARLEN_CASES = {
    # (T_b, L_b) per sequence: ragged chunks continuing a cache (P > 0),
    # fresh chunks (P = 0), and decode-shaped members (T = 1).
    "mixed": [(37, 137), (1, 900), (16, 16), (1, 1), (130, 645), (5, 300)],
    "decode_only": [(1, 513), (1, 2049), (1, 17)],
    "one_long": [(300, 4300)],
}


@pytest.mark.parametrize("H,Hkv,d", [(32, 8, 128), (14, 2, 64), (6, 3, 18)])
@pytest.mark.parametrize("case", sorted(VARLEN_CASES))
def test_prefill_attention_varlen(gctx, ehip_mod, orc, H, Hkv, d, case):
    """Per-sequence contiguous K/V at separate device addresses, ragged query
    counts packed by cu_seqlens: against the oracle's varlen restatement (the
    reference's PrefillUnitsImpl order), which is bit-identical to the
    reference build."""
    seqs = VARLEN_CASES[case]
    rng = np.random.default_rng(H + d + len(seqs))
    cu = np.concatenate([[0], np.cumsum([t for t, _ in seqs])]).astype(np.int32)
    q = rng.standard_normal((int(cu[-1]), H, d)).astype(np.float32)
    ks = [rng.standard_normal((Hkv, L, d)).astype(np.float32) for _, L in seqs]
    vs = [rng.standard_normal((Hkv, L, d)).astype(np.float32) for _, L in seqs]
    dq = gctx.to_device(q)
    dks, dvs = _dev(gctx, *ks), _dev(gctx, *vs)
    out = gctx.alloc(q.nbytes)
    rc = gctx.prefill_attention_varlen(dq, cu, dks, dvs, [L for _, L in seqs], out, H, Hkv, d,
                                       scale_for(d))
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref = orc.prefill_varlen(q, cu, ks, vs, H, Hkv, d, scale_for(d), isa=orc.ISA_AVX2)
    _check(got, ref)
    for b in [dq, out] + dks + dvs:
        b.free()


def test_varlen_validates_before_launching(gctx, ehip_mod):
    """A bad member anywhere is refused before any sequence runs (out keeps
    its poison), and B == 0 is a no-op."""
    H, Hkv, d = 8, 2, 16
    q = np.ones((6, H, d), np.float32)
    k = np.ones((Hkv, 8, d), np.float32)
    dq, dk = gctx.to_device(q), gctx.to_device(k)
    poison = np.full(q.shape, np.nan, np.float32)
    out = gctx.to_device(poison)
    # T_1 = 4 > L_1 = 3.
    rc = gctx.prefill_attention_varlen(dq, [0, 2, 6], [dk, dk], [dk, dk], [8, 3], out, H, Hkv, d,
                                       0.25)
    assert rc == ehip_mod.INVALID_ARGUMENT and "sequence 1" in gctx.last_error()
    assert np.isnan(out.download(np.float32, q.shape)).all()
    assert gctx.prefill_attention_varlen(None, [0], [], [], [], None, H, Hkv, d, 0.25) == 0
    for b in (dq, dk, out):
        b.free()


def test_contiguous_entry_points_validate(gctx, ehip_mod):
    buf = gctx.alloc(4096)
    L_ = ehip_mod.lib()
    s = C.c_float(0.125)
    assert L_.ehip_prefill_attention_f32(gctx.h, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 5, 8, 8, 16,
                                         4, s) == ehip_mod.INVALID_ARGUMENT  # T > L
    assert L_.ehip_decode_attention_f32(gctx.h, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 6, 4, 16, 4,
                                        s) == ehip_mod.INVALID_ARGUMENT  # H % Hkv
    assert L_.ehip_decode_attention_f32(gctx.h, None, buf.ptr, buf.ptr, buf.ptr, 8, 8, 16, 4,
                                        s) == ehip_mod.INVALID_ARGUMENT
    buf.free()
