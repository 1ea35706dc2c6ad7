"""The seeded synthetic steps (ehip.workloads) and the product-side fills they
draw from (ehip_rng_u64, ehip_host_fill_normal, ehip_host_fp32_to_bf16),
pinned against the oracle's restatement of the reference's Rng/fill_normal
(itself pinned by the mt19937_64 known answer) and against closed forms."""
import math

import numpy as np
import pytest


def test_rng_stream_matches_mt19937_64(ehip_mod, orc):
    from ehip import workloads
    st = workloads.Stream(12345)
    got = np.concatenate([st.raw(5), st.raw(5000), st.raw(3)])
    g = orc.Mt64(12345)
    want = np.array([g.next() for _ in range(5008)], np.uint64)
    assert np.array_equal(got, want)
    # The standard's known answer through the product entry point.
    x = np.empty(1, np.uint64)
    assert ehip_mod.lib().ehip_rng_u64(5489, 9999, x.ctypes.data, 1) == 0
    assert int(x[0]) == 9981545732273789042


@pytest.mark.parametrize("n", [0, 1, 2, 3, 1001, 4 * 1024 * 1024 + 3, 9_000_001])
def test_host_fill_normal_is_the_reference_fill(ehip_mod, orc, n):
    from ehip import workloads
    got = workloads.fill_normal(n, 0.25, 0.5, 99 + n)
    want = orc.fill_normal(n, 0.25, 0.5, 99 + n) if n else np.empty(0, np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_host_fill_rejects_bad_arguments(ehip_mod):
    import ctypes as C
    a = np.empty(4, np.float32)
    L = ehip_mod.lib()
    assert L.ehip_host_fill_normal(a.ctypes.data, 4, C.c_double(0), C.c_double(-1.0),
                                   C.c_uint64(1)) == ehip_mod.INVALID_ARGUMENT
    assert L.ehip_host_fill_normal(None, 4, C.c_double(0), C.c_double(1.0),
                                   C.c_uint64(1)) == ehip_mod.INVALID_ARGUMENT
    assert L.ehip_rng_u64(1, 0, None, 3) == ehip_mod.INVALID_ARGUMENT


def test_host_bf16_narrowing_matches_oracle(ehip_mod, orc):
    from ehip import workloads
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, 5_000_000, dtype=np.uint64).astype(np.uint32)
    bits[:6] = [0x7F800001, 0xFF800001, 0x7FC00000, 0x3F808000, 0x3F818000, 0x7F7FFFFF]
    x = bits.view(np.float32)
    assert np.array_equal(workloads.to_bf16_bits(x), orc.to_bf16_bits(x))


def test_stream_draw_transforms_closed_forms(ehip_mod, orc):
    from ehip import workloads
    g = orc.Mt64(77)
    raw = [g.next() for _ in range(6)]
    u = [(x >> 11) * 2.0 ** -53 for x in raw]
    st = workloads.Stream(77)
    assert st.uniform_int(10, 20, 2).tolist() == [10 + math.floor(v * 11) for v in u[:2]]
    assert st.log_uniform_int(256, 8192, 2).tolist() == [
        round(math.exp(math.log(256) + v * (math.log(8192) - math.log(256)))) for v in u[2:4]]
    # Fisher-Yates on two items swaps iff floor(2u) == 0 for the one draw.
    p = st.permutation(2).tolist()
    assert p == ([1, 0] if math.floor(u[4] * 2) == 0 else [0, 1])
    perm = workloads.Stream(3).permutation(10_000)
    assert np.array_equal(np.sort(perm), np.arange(10_000))


def test_c4_draw_statistics_and_sharing():
    from ehip import workloads
    mean, sd = workloads.c4_sum_context_stats()
    # Analytic moments against the lengths of 60 seeds (the lengths are the
    # stream's first draws).
    sums = []
    for seed in range(100, 160):
        ctx = workloads.Stream(seed).log_uniform_int(256, 8192, 256)
        sums.append(int(ctx.sum()) + 256)
    sums = np.array(sums, np.float64)
    assert abs(sums.mean() - mean) < 4 * sd / math.sqrt(len(sums))
    assert 0.7 * sd < sums.std() < 1.3 * sd
    w = workloads.c4()
    assert abs(int(w.context_lens.sum()) - mean) <= sd  # the headline draw is typical
    in_use = int((w.refcount > 0).sum())
    assert 0.09 <= int((w.refcount == 2).sum()) / in_use <= 0.11
    assert w.refcount.max() == 2
    # Every shared block is a leading full block of exactly two tables, at
    # the same logical index in both.
    owners = {}
    for b, t in enumerate(w.tables):
        for i, blk in enumerate(t.tolist()):
            owners.setdefault(blk, []).append((b, i))
    for blk, who in owners.items():
        if len(who) == 2:
            (a, ia), (b, ib) = who
            assert ia == ib and (ia + 1) * 16 <= min(w.context_lens[a], w.context_lens[b]) - 1


def test_workload_values_follow_their_seeds(ehip_mod, orc):
    from ehip import workloads
    w = workloads.c1()
    q = w.q(0)
    assert np.array_equal(q.ravel(), orc.fill_normal(q.size, 0.0, w.qkv_std,
                                                     workloads.value_seed(1, 0, 4)))
    k, v = w.pool(0)
    assert k.shape == (64, 2, 16, 64)
    assert np.array_equal(v.ravel(), orc.fill_normal(v.size, 0.0, w.qkv_std,
                                                     workloads.value_seed(1, 0, 6)))
    kn, vn = w.new_kv(3)
    assert kn.shape == (1, 2, 64) and not np.array_equal(kn, w.new_kv(2)[0])
