"""The allocation-free single-sequence decode (ehip_paged_decode_attention_f32_noalloc):
called through the C ABI, its output must equal the allocating entry point's
(ehip_paged_decode_attention_f32) on the same inputs, to the fp32 parity bar,
over consecutive calls that reuse the device's static scratch (a long row cut
into key splits, then a smaller one, then the long one again), and match the
oracle."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import rel_norm
from paged_util import allclose_ref, paged_layout, scale_for

FP32_REL = 1e-4

pytestmark = pytest.mark.gpu


def _case(orc, seed, L, H, Hkv, d, bs):
    kc = orc.fill_normal(Hkv * L * d, 0.0, 1.0, seed).reshape(Hkv, L, d)
    vc = orc.fill_normal(Hkv * L * d, 0.0, 1.0, seed + 1).reshape(Hkv, L, d)
    q = orc.fill_normal(H * d, 0.0, 1.0, seed + 2).reshape(H, d)
    ks, vs, table = paged_layout(kc, vc, bs, extra_blocks=3, rng=np.random.default_rng(seed))
    return q, ks, vs, table


def _call(gctx, ehip_mod, fn, q, ks, vs, table, L, H, Hkv, d, bs):
    dq, dk, dv, dt = (gctx.to_device(x) for x in (q, ks, vs, table))
    out = gctx.alloc(q.nbytes)
    rc = fn(gctx.h, dq.ptr, dk.ptr, dv.ptr, dt.ptr, len(table), L, H, Hkv, d, bs, Hkv * bs * d,
            ks.shape[0], C.c_float(scale_for(d)), out.ptr)
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    for b in (dq, dk, dv, dt, out):
        b.free()
    return got


# (L, H, Hkv, d, bs): a long row split into many key splits (merge kernel),
# then a smaller one (one workgroup per kv head, no partials), then the long
# one again after the scratch held the small call's plan.
CALLS = [(20000, 32, 8, 128, 16), (513, 14, 2, 64, 16), (20000, 32, 8, 128, 16),
         (3000, 8, 1, 128, 32)]


def test_noalloc_decode_matches_allocating_entry_point(gctx, ehip_mod, orc, monkeypatch):
    L_ = ehip_mod.lib()
    for i, (L, H, Hkv, d, bs) in enumerate(CALLS):
        q, ks, vs, table = _case(orc, 700 + 10 * i, L, H, Hkv, d, bs)
        print(f"[noalloc] call {i}: L={L} H={H} Hkv={Hkv} d={d} bs={bs}", flush=True)
        got = _call(gctx, ehip_mod, L_.ehip_paged_decode_attention_f32_noalloc, q, ks, vs, table,
                    L, H, Hkv, d, bs)
        want = _call(gctx, ehip_mod, L_.ehip_paged_decode_attention_f32, q, ks, vs, table, L, H,
                     Hkv, d, bs)
        assert rel_norm(got, want) <= FP32_REL
        assert allclose_ref(got, want, 1e-4, 1e-5)
        ref = orc.paged_decode(q, ks, vs, table, L, H, Hkv, d, bs, scale_for(d))
        assert rel_norm(got, ref) <= FP32_REL
        assert allclose_ref(got, ref, 1e-4, 1e-5)


def test_noalloc_decode_rejects_rows_beyond_its_scratch(gctx, ehip_mod):
    # 64 key splits x 128 query heads x (128 + 2) floats of partials exceed
    # the 4 MiB scratch: refused before anything is launched.
    L, H, Hkv, d, bs = 65536, 128, 8, 128, 16
    nblk = L // bs
    dq, dk, dv, out = (gctx.alloc(256) for _ in range(4))
    dt = gctx.to_device(np.arange(nblk, dtype=np.int32))
    rc = ehip_mod.lib().ehip_paged_decode_attention_f32_noalloc(
        gctx.h, dq.ptr, dk.ptr, dv.ptr, dt.ptr, nblk, L, H, Hkv, d, bs, Hkv * bs * d, nblk,
        C.c_float(0.088), out.ptr)
    assert rc == ehip_mod.RESOURCE_EXHAUSTED
    assert "scratch" in gctx.last_error()
    for b in (dq, dk, dv, out, dt):
        b.free()


def test_noalloc_two_contexts_share_the_scratch_in_call_order(gctx, ehip_mod, orc):
    """Two contexts on one device (two streams) issue _noalloc calls of
    different lengths in turn, with no synchronisation between the calls: the
    device's one scratch array serves them all, and each call waits for the
    previous call's end whichever context made it. Every output equals the
    allocating entry point's on the same inputs. Every table holds valid ids
    for the longest row, so each call reads in bounds whatever its plan."""
    L_ = ehip_mod.lib()
    H, Hkv, d, bs = 32, 8, 128, 16
    lengths = [20000, 3000, 20000, 700]
    nblk = (max(lengths) + bs - 1) // bs
    other = ehip_mod.Context(0)
    try:
        cases, want = [], []
        for i, L in enumerate(lengths):
            q, ks, vs, table = _case(orc, 900 + 10 * i, L, H, Hkv, d, bs)
            table = np.concatenate([table, np.zeros(nblk - len(table), np.int32)])
            want.append(_call(gctx, ehip_mod, L_.ehip_paged_decode_attention_f32, q, ks, vs,
                              table, L, H, Hkv, d, bs))
            bufs = [gctx.to_device(x) for x in (q, ks, vs, table)]
            cases.append((L, ks.shape[0], bufs, gctx.alloc(q.nbytes), q.shape))
        for i, (L, slab_blocks, (dq, dk, dv, dt), out, _) in enumerate(cases):
            ctx = gctx if i % 2 == 0 else other
            print(f"[noalloc] context {i % 2}: L={L}", flush=True)
            rc = L_.ehip_paged_decode_attention_f32_noalloc(
                ctx.h, dq.ptr, dk.ptr, dv.ptr, dt.ptr, nblk, L, H, Hkv, d, bs, Hkv * bs * d,
                slab_blocks, C.c_float(scale_for(d)), out.ptr)
            assert rc == 0, ctx.last_error()
        gctx.sync()
        other.sync()
        for (L, _, bufs, out, shape), ref in zip(cases, want):
            got = out.download(np.float32, shape)
            assert rel_norm(got, ref) <= FP32_REL, L
            assert allclose_ref(got, ref, 1e-4, 1e-5)
            for b in bufs + [out]:
                b.free()
    finally:
        other.close()
