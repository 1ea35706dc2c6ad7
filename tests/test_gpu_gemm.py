"""The attention output's consumer, o_proj: ehip_packed_gemm and
ehip_pack_weight_panels (kernels::PackedGemm / PackWeightPanels,
src/kernels/gemm.h:61-78) against the oracle's restatement of the reference's
scalar tile, which is bit-identical to the reference build.

Bars: the device pack is bit-exact; the GEMM meets the reference's own GEMM
tolerance (allclose rtol 1e-4, atol 1e-5 * sqrt(k), packed_gemm_test.cpp:180-184)
over its shape list and the benchmark configurations' o_proj shapes; repeated
calls are bit-identical (split-k partials added in split order)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# The reference's PackedGemm shapes (tests/unit/packed_gemm_test.cpp:132-145)
# and the configs' o_proj: C4 decode (256 rows, 4096 -> 4096), C2 decode
# (32 rows, 896 -> 896), a C3-sized chunk slice (600 rows).
SHAPES = [(16, 64, 64), (16, 64, 96), (16, 176, 64), (8, 64, 512), (1, 64, 64),
          (1, 2048, 512), (4, 2048, 8192), (33, 8192, 256), (130, 300, 70), (7, 1, 33),
          (65, 129, 1000), (5, 40, 17), (32, 896, 896)]
# The largest shapes run for the bf16 checkpoints the configs use (the CPU
# oracle's fp32 and fp16 passes at these sizes would dominate the suite).
CASES = ([(s, d) for s in SHAPES for d in ("bf16", "f16", "f32")] +
         [((256, 4096, 4096), "bf16"), ((600, 4096, 1024), "bf16")])


def _weights(orc, ehip_mod, n, k, dtype, seed):
    wf = orc.fill_normal(n * k, 0.0, 1.0, seed).reshape(n, k)
    if dtype == ehip_mod.WEIGHT_F32:
        return wf
    if dtype == ehip_mod.WEIGHT_BF16:
        return orc.to_bf16_bits(wf)
    return wf.astype(np.float16).view(np.uint16)


def _run(gctx, ehip_mod, x, w, dtype, bias):
    m, k = x.shape
    n = w.shape[0]
    dw = gctx.to_device(w)
    dwp = gctx.alloc(((n + 15) // 16) * k * 16 * w.itemsize)
    assert gctx.pack_weight_panels(dw, dtype, n, k, dwp) == 0, gctx.last_error()
    dx = gctx.to_device(x)
    db = gctx.to_device(bias) if bias is not None else None
    dy = gctx.alloc(m * n * 4)
    assert gctx.packed_gemm(dx, m, k, dwp, dtype, n, db, dy) == 0, gctx.last_error()
    gctx.sync()
    y = dy.download(np.float32, (m, n))
    wp = dwp.download(w.dtype, ((n + 15) // 16, k, 16))
    for b in (dw, dx, dy, db):
        if b is not None:
            b.free()
    return y, wp, dwp


@pytest.mark.parametrize("shape,dtype", CASES, ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
def test_packed_gemm_matches_reference_tile(gctx, ehip_mod, orc, shape, dtype):
    m, k, n = shape
    dt = {"bf16": ehip_mod.WEIGHT_BF16, "f16": ehip_mod.WEIGHT_F16, "f32": ehip_mod.WEIGHT_F32}[dtype]
    seed = 100 + m + k + n
    x = orc.fill_normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    w = _weights(orc, ehip_mod, n, k, dt, seed + 1)
    bias = orc.fill_normal(n, 0.0, 1.0, seed + 2) if (m + n) % 2 else None
    print(f"[gemm] m={m} k={k} n={n} {dtype} bias={bias is not None}", flush=True)
    y, wp, dwp = _run(gctx, ehip_mod, x, w, dt, bias)
    dwp.free()
    want_wp = orc.pack_weight_panels(w)
    assert np.array_equal(wp.view(np.uint8), want_wp.view(np.uint8)), "device pack differs"
    ref = orc.packed_gemm(x, want_wp, dt, n, bias)
    atol = 1e-5 * np.sqrt(k)
    err = np.abs(y.astype(np.float64) - ref)
    bad = err > atol + 1e-4 * np.abs(ref)
    assert not bad.any(), (int(bad.sum()), float(err.max()))


def test_packed_gemm_split_k_is_deterministic(gctx, ehip_mod, orc):
    """The decode-shaped o_proj (256 rows) splits k over workgroups: two calls
    give the same bits, and match the oracle."""
    m, k, n = 256, 4096, 4096
    x = orc.fill_normal(m * k, 0.0, 1.0, 5).reshape(m, k)
    w = _weights(orc, ehip_mod, n, k, ehip_mod.WEIGHT_BF16, 6)
    dw, dx = gctx.to_device(w), gctx.to_device(x)
    dwp = gctx.alloc(n * k * 2)
    assert gctx.pack_weight_panels(dw, ehip_mod.WEIGHT_BF16, n, k, dwp) == 0
    outs = []
    for _ in range(2):
        dy = gctx.alloc(m * n * 4)
        assert gctx.packed_gemm(dx, m, k, dwp, ehip_mod.WEIGHT_BF16, n, None, dy) == 0
        gctx.sync()
        outs.append(dy.download(np.float32, (m, n)))
        dy.free()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for b in (dw, dx, dwp):
        b.free()


def test_packed_gemm_validates(gctx, ehip_mod):
    buf = gctx.alloc(4096)
    L_ = ehip_mod.lib()
    assert L_.ehip_packed_gemm(gctx.h, buf.ptr, 0, 4, buf.ptr, 1, 4, None, buf.ptr) == \
        ehip_mod.INVALID_ARGUMENT
    assert L_.ehip_packed_gemm(gctx.h, buf.ptr, 2, 4, buf.ptr, 7, 4, None, buf.ptr) == \
        ehip_mod.INVALID_ARGUMENT
    assert L_.ehip_packed_gemm(gctx.h, buf.ptr, 2, 4, buf.ptr + 2, 1, 4, None, buf.ptr) == \
        ehip_mod.INVALID_ARGUMENT
    assert L_.ehip_pack_weight_panels(gctx.h, buf.ptr, 1, 0, 4, buf.ptr) == \
        ehip_mod.INVALID_ARGUMENT
    buf.free()
