"""GPU parity of the INT8 and FP8 (E4M3) KV paths (per-(block, kv head) scales).

The INT8 format is the one the reference reserves (docs/design/paged-kv-cache.md:
219-231) but does not implement; FP8 takes the same seam with E4M3 codes. The
semantics are the CPU restatements in oracle/oracle.h (orc_kv_append_int8,
orc_kv_append_fp8), pinned by closed forms and, for the E4M3 codes, against
torch.float8_e4m3fn in tests/test_oracle.py. Bars: the slabs and fp32 scales
bit-identical to that restatement after every step (fresh blocks, growing
blocks whose scale rises and older rows are requantised, stale state from an
earlier owner); attention within the fp32 bar (1e-4 relative, per output
vector) of the reference attention over the dequantised K/V.
"""
import numpy as np
import pytest

from gpu_util import rel_norm

pytestmark = pytest.mark.gpu

FORMATS = ["int8", "fp8"]


def make_tables(rng, lens, bs, pool):
    perm = rng.permutation(pool).astype(np.int32)
    tabs, off = [], 0
    for L in lens:
        n = (L + bs - 1) // bs
        tabs.append(perm[off:off + n].copy())
        off += n
    assert off <= pool
    return tabs


def slots_for(tabs, qlens, clens, bs):
    out = []
    for t, T, L in zip(tabs, qlens, clens):
        for pos in range(L - T, L):
            out.append(int(t[pos // bs]) * bs + pos % bs)
    return np.asarray(out, np.int64)


class ScaledRun:
    """Device slabs/scales and their oracle mirrors over a series of steps
    (fmt "int8" or "fp8")."""

    def __init__(self, gctx, ehip_mod, H, Hkv, d, bs, pool, seed, fmt="int8"):
        self.gctx, self.E, self.fmt = gctx, ehip_mod, fmt
        self.H, self.Hkv, self.d, self.bs, self.pool = H, Hkv, d, bs, pool
        self.kv_dtype = ehip_mod.KV_FP8 if fmt == "fp8" else ehip_mod.KV_INT8
        self.elem = np.uint8 if fmt == "fp8" else np.int8
        rng = np.random.default_rng(seed)
        shape = (pool, Hkv, bs, d)
        # Stale contents everywhere (an earlier owner's rows and scales). Rows
        # a test never appends are read as context, so FP8 takes every code
        # but the NaN ones (0x7F / 0xFF).
        if fmt == "fp8":
            codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
            self.k = rng.choice(codes, shape)
            self.v = rng.choice(codes, shape)
        else:
            self.k = rng.integers(-127, 128, shape).astype(np.int8)
            self.v = rng.integers(-127, 128, shape).astype(np.int8)
        self.ks = rng.uniform(1e3, 1e6, (pool, Hkv)).astype(np.float32)
        self.vs = rng.uniform(1e3, 1e6, (pool, Hkv)).astype(np.float32)
        self.dk, self.dv = gctx.to_device(self.k), gctx.to_device(self.v)
        self.dks, self.dvs = gctx.to_device(self.ks), gctx.to_device(self.vs)

    def step(self, orc, tabs, qlens, clens, rng, amp):
        E, g = self.E, self.gctx
        geo = E.geometry(self.H, self.Hkv, self.d, self.bs, self.kv_dtype, self.pool,
                         float(np.float32(1 / np.sqrt(self.d))))
        slots = slots_for(tabs, qlens, clens, self.bs)
        st = E.StepArrays(np.asarray(qlens, np.int32), np.asarray(clens, np.int64), tabs, slots)
        assert g.step_upload(geo, st) == 0, g.last_error()
        R = int(sum(qlens))
        kn = (rng.standard_normal((R, self.Hkv, self.d)) * amp).astype(np.float32)
        vn = (rng.standard_normal((R, self.Hkv, self.d)) * amp).astype(np.float32)
        q = rng.standard_normal((R, self.H, self.d)).astype(np.float32)
        dkn, dvn, dq = g.to_device(kn), g.to_device(vn), g.to_device(q)
        out = g.alloc(q.nbytes)
        append = getattr(g, f"step_kv_append_{self.fmt}")
        attention = getattr(g, f"step_attention_{self.fmt}")
        assert append(dkn, dvn, self.dk, self.dv, self.dks, self.dvs) == 0, g.last_error()
        assert attention(dq, self.dk, self.dv, self.dks, self.dvs, out) == 0, g.last_error()
        g.sync()
        getattr(orc, f"kv_append_{self.fmt}")(kn, vn, slots, self.Hkv, self.d, self.bs, self.k,
                                              self.v, self.ks, self.vs)
        got = out.download(np.float32, q.shape)
        for b in (dkn, dvn, dq, out):
            b.free()
        return q, got, geo

    def check_slabs(self):
        assert np.array_equal(self.dk.download(self.elem, self.k.shape), self.k)
        assert np.array_equal(self.dv.download(self.elem, self.v.shape), self.v)
        assert np.array_equal(self.dks.download(np.float32, self.ks.shape).view(np.uint32),
                              self.ks.view(np.uint32))
        assert np.array_equal(self.dvs.download(np.float32, self.vs.shape).view(np.uint32),
                              self.vs.view(np.uint32))

    def reference(self, orc, q, tabs, qlens, clens):
        dequant = getattr(orc, f"{self.fmt}_dequant")
        kd, vd = dequant(self.k, self.ks), dequant(self.v, self.vs)
        cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
        kseq = [orc.paged_to_contig(kd, t, int(L), self.Hkv, self.d, self.bs)
                for t, L in zip(tabs, clens)]
        vseq = [orc.paged_to_contig(vd, t, int(L), self.Hkv, self.d, self.bs)
                for t, L in zip(tabs, clens)]
        return orc.prefill_varlen(q, cu, kseq, vseq, self.H, self.Hkv, self.d,
                                  float(np.float32(1 / np.sqrt(self.d))), isa=1)

    def free(self):
        for b in (self.dk, self.dv, self.dks, self.dvs):
            b.free()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("H,Hkv,d", [(32, 8, 128), (8, 2, 64), (8, 8, 128), (16, 2, 64)])
def test_int8_steps_bit_exact_append_and_attention(gctx, ehip_mod, orc, H, Hkv, d, fmt):
    """Three steps over stale slabs: prompts (fresh blocks, chunks ending
    mid-block), decode rows whose amplitude grows (scale rises, older rows
    requantised), then a mixed step with a continuation chunk."""
    rng = np.random.default_rng(H + d)
    bs = 16
    final = [70, 33, 300, 17, 129, 64]
    pool = sum((L + 20 + bs - 1) // bs for L in final) + 9
    tabs = make_tables(rng, [L + 20 for L in final], bs, pool)
    run = ScaledRun(gctx, ehip_mod, H, Hkv, d, bs, pool, seed=H * d, fmt=fmt)
    steps = [
        ([60, 30, 250, 5, 100, 64], [60, 30, 250, 5, 100, 64], 1.0),
        ([1, 1, 1, 1, 1, 1], [61, 31, 251, 6, 101, 65], 4.0),
        ([9, 2, 49, 11, 28, 1], [70, 33, 300, 17, 129, 66], 0.5),
    ]
    for qlens, clens, amp in steps:
        q, got, _ = run.step(orc, tabs, qlens, clens, rng, amp)
        run.check_slabs()
        ref = run.reference(orc, q, tabs, qlens, clens)
        assert rel_norm(got, ref) <= 1e-4, rel_norm(got, ref)
    run.free()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("split", ["64", "128", "2048"])
def test_int8_long_rows_split_and_merged(ehip_mod, orc, tctx, split, fmt):
    """Decode rows long enough to be split into several key ranges (the split
    partials go through the shared merge); 2048-key ranges span 128 blocks, the
    longest an INT8 work item takes."""
    gctx = tctx(EHIP_SPLIT_TOKENS=split)
    rng = np.random.default_rng(7)
    H, Hkv, d, bs = 32, 8, 128, 16
    lens = [1500, 2049, 17, 640, 4100]
    pool = sum((L + bs - 1) // bs for L in lens) + 5
    tabs = make_tables(rng, lens, bs, pool)
    run = ScaledRun(gctx, ehip_mod, H, Hkv, d, bs, pool, seed=11, fmt=fmt)
    prompt = [L - 1 for L in lens]
    run.step(orc, tabs, prompt, prompt, rng, 1.0)
    q, got, _ = run.step(orc, tabs, [1] * len(lens), lens, rng, 1.0)
    run.check_slabs()
    assert gctx.step_info()[2] > len(lens) * Hkv  # split partials were used
    ref = run.reference(orc, q, tabs, [1] * len(lens), lens)
    assert rel_norm(got, ref) <= 1e-4, rel_norm(got, ref)
    run.free()


def shared_pair_tables(rng, pairs, bs, extra=7, groups=()):
    """Tables for row pairs that share leading blocks: pairs of (len_a, len_b,
    shared_blocks), then larger fork groups of (shared_blocks, [lengths]);
    each row's remaining blocks (its last included) are its own. Returns
    (tables, pool)."""
    all_groups = [(sb, [la, lb]) for la, lb, sb in pairs] + list(groups)
    need = sum(sb + sum((L + bs - 1) // bs - sb for L in ls) for sb, ls in all_groups)
    pool = need + extra
    perm = rng.permutation(pool).astype(np.int32)
    tabs, off = [], 0
    for sb, ls in all_groups:
        shared = perm[off:off + sb]
        off += sb
        for L in ls:
            own = (L + bs - 1) // bs - sb
            assert own >= 1
            tabs.append(np.concatenate([shared, perm[off:off + own]]).astype(np.int32))
            off += own
    return tabs, pool


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("H,Hkv,d", [(32, 8, 128), (64, 8, 128), (8, 2, 64), (8, 8, 128)])
def test_int8_shared_prefix_joint_items(ehip_mod, orc, tctx, H, Hkv, d, fmt):
    """Pair-shared prefix blocks (the C4 construction's sharing) and, for
    g <= 4, a fork of four rows through the INT8 kernel: with joint work items
    (one pass over the shared blocks, row r's g heads in MFMA rows
    r*g..r*g+g-1) and with the plain per-row partition, each against the
    reference attention over the dequantised K/V, and the two against each
    other."""
    bs = 16
    pairs = [(700, 530, 20), (1300, 2100, 33), (300, 900, 12), (260, 129, 8)]
    # g <= 4: forks of four rows share 20 blocks (joint items of four rows)
    quads = [(20, [500, 700, 330, 900])] if H // Hkv <= 4 else []
    outs = []
    for flag in ("0", "1"):
        gctx = tctx(EHIP_NO_JOINT=flag)
        rng = np.random.default_rng(H + d)
        tabs, pool = shared_pair_tables(rng, pairs, bs, groups=quads)
        lens = [L for la, lb, _ in pairs for L in (la, lb)] + [L for _, ls in quads for L in ls]
        geo = ehip_mod.geometry(H, Hkv, d, bs,
                                ehip_mod.KV_FP8 if fmt == "fp8" else ehip_mod.KV_INT8, pool,
                                float(np.float32(1 / np.sqrt(d))))
        st = ehip_mod.StepArrays(np.ones(len(lens), np.int32), np.asarray(lens, np.int64), tabs,
                                 slots_for(tabs, [1] * len(lens), lens, bs))
        rc, *_, joint_items, shared = ehip_mod.plan_counts(geo, st, joint=True)
        assert rc == 0
        assert (joint_items > 0) == (flag == "0"), joint_items
        run = ScaledRun(gctx, ehip_mod, H, Hkv, d, bs, pool, seed=H * d + 1, fmt=fmt)
        q, got, _ = run.step(orc, tabs, [1] * len(lens), lens, rng, 1.0)
        run.check_slabs()
        ref = run.reference(orc, q, tabs, [1] * len(lens), lens)
        assert rel_norm(got, ref) <= 1e-4, (flag, rel_norm(got, ref))
        outs.append(got)
        run.free()
    assert rel_norm(outs[0], outs[1]) <= 1e-5


def test_int8_entry_points_reject_other_geometries(gctx, ehip_mod):
    """The fp32/bf16 entry points refuse INT8 and FP8 geometry (their element
    size would overrun the byte slabs), the INT8 ones refuse the others, FP8
    included, and the FP8 ones likewise."""
    E = ehip_mod
    tabs = [np.arange(2, dtype=np.int32)]
    st = E.StepArrays(np.array([1], np.int32), np.array([20], np.int64), tabs,
                      np.array([19], np.int64))
    buf = gctx.alloc(1 << 16)
    g8 = E.geometry(8, 2, 64, 16, E.KV_INT8, 2, 0.125)
    assert gctx.step_upload(g8, st) == 0
    assert gctx.step_kv_append(buf, buf, buf, buf) == E.INVALID_ARGUMENT
    assert gctx.step_attention(buf, buf, buf, buf) == E.INVALID_ARGUMENT
    assert gctx.step_kv_append_fp8(buf, buf, buf, buf, buf, buf) == E.INVALID_ARGUMENT
    assert gctx.step_attention_fp8(buf, buf, buf, buf, buf, buf) == E.INVALID_ARGUMENT
    gf8 = E.geometry(8, 2, 64, 16, E.KV_FP8, 2, 0.125)
    assert gctx.step_upload(gf8, st) == 0
    assert gctx.step_kv_append(buf, buf, buf, buf) == E.INVALID_ARGUMENT
    assert gctx.step_attention(buf, buf, buf, buf) == E.INVALID_ARGUMENT
    assert gctx.step_kv_append_int8(buf, buf, buf, buf, buf, buf) == E.INVALID_ARGUMENT
    assert gctx.step_attention_int8(buf, buf, buf, buf, buf, buf) == E.INVALID_ARGUMENT
    g16 = E.geometry(8, 2, 64, 16, E.KV_BF16, 2, 0.125)
    assert gctx.step_upload(g16, st) == 0
    for fmt in FORMATS:
        assert getattr(gctx, f"step_kv_append_{fmt}")(buf, buf, buf, buf, buf, buf) == \
            E.INVALID_ARGUMENT
        assert getattr(gctx, f"step_attention_{fmt}")(buf, buf, buf, buf, buf, buf) == \
            E.INVALID_ARGUMENT
    buf.free()
