"""Host-side checks of the C ABI (no GPU needed): the library loads, exports
every function include/ehip.h declares, and the step planner validates and
partitions ragged steps as specified."""
import ctypes as C
import math

import numpy as np
import pytest


def test_library_exports_every_declared_symbol(ehip_mod):
    L = ehip_mod.lib()
    names = ehip_mod.header_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n


def test_device_count_without_context(ehip_mod):
    assert ehip_mod.device_count() >= 0


def geom(ehip_mod, **kw):
    base = dict(heads=32, kv_heads=8, head_dim=128, block_size=16, kv_dtype=1, slab_blocks=1000,
                scale=0.088)
    base.update(kw)
    return ehip_mod.geometry(**base)


def simple_step(ehip_mod, lens, qlens=None, bs=16, slots=None, start=0):
    tabs, off = [], start
    for L in lens:
        n = (L + bs - 1) // bs
        tabs.append(np.arange(off, off + n, dtype=np.int32))
        off += n
    q = np.ones(len(lens), np.int32) if qlens is None else qlens
    return ehip_mod.StepArrays(q, lens, tabs, slots)


def cut_tail(ranges, hkv, tail, frac=0.08, target=2048):
    """Range count per row after the planner's tail pieces. ranges: list of
    (rows, length) in the planner's order (joint ranges first, then rows in
    order, each in key order). When the ranges exceed the target item count,
    the smallest single-row ranges longer than the piece length, up to frac of
    the keys (times rows), are cut into pieces (a row keeps <= 64 ranges)."""
    count = {}
    for rows, _ in ranges:
        for r in rows:
            count[r] = count.get(r, 0) + 1
    tail = -(-tail // 64) * 64 if tail else 0
    if not tail or frac <= 0 or len(ranges) * hkv <= target:
        return count
    total = sum(n * len(rows) for rows, n in ranges)
    cand = sorted((i for i, (rows, n) in enumerate(ranges) if len(rows) == 1 and n > tail),
                  key=lambda i: ranges[i][1])
    acc = 0
    for i in cand:
        rows, n = ranges[i]
        if acc + n > frac * total:
            break
        extra = -(-n // tail) - 1
        if count[rows[0]] + extra > 64:
            continue
        count[rows[0]] += extra
        acc += n
    return count


def expected_items(lens, hkv, split, bs=16, tail=0):
    """Items of a plan without joint groups: each row in ranges of its split
    length (grown to keep at most 64 per row), then the tail pieces."""
    ranges = []
    for r, L in enumerate(lens):
        s = split
        if math.ceil(L / s) > 64:
            s = min(128 * bs, math.ceil(math.ceil(L / 64) / 64) * 64)
        ranges += [((r,), min(s, int(L) - t)) for t in range(0, int(L), s)]
    return sum(cut_tail(ranges, hkv, tail).values()) * hkv


@pytest.mark.parametrize("tail", [None, 0, 128, 512])
def test_plan_partitions_c4_shape(ehip_mod, monkeypatch, tail):
    monkeypatch.setenv("EHIP_NO_JOINT", "1")  # plain per-row partition
    if tail is not None:
        monkeypatch.setenv("EHIP_TAIL_SPLIT", str(tail))
    from ehip import workloads
    w = workloads.c4()
    g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                          w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    rc, rows, items, partials, split = ehip_mod.plan_counts(g, st)
    assert rc == 0
    assert rows == 256
    assert split % 64 == 0 and 128 <= split <= 128 * w.block_size
    assert items == expected_items(w.context_lens, w.kv_heads, split, tail=tail or 0)
    assert partials == items  # one partial slot per (row, kv head, split)
    if tail and tail < split:
        # C4 is past the item target: the tail pieces add items.
        assert items > expected_items(w.context_lens, w.kv_heads, split, tail=0)


def test_plan_split_override_and_long_rows(ehip_mod, monkeypatch):
    monkeypatch.setenv("EHIP_SPLIT_TOKENS", "100")  # rounds up to 128
    lens = [32768, 5, 128, 129]
    rc, rows, items, partials, split = ehip_mod.plan_counts(
        geom(ehip_mod, slab_blocks=4000), simple_step(ehip_mod, lens))
    assert rc == 0 and split == 128
    # (distinct tables: no joint items) 32768 keys would need 256 splits of 128: the row's split grows to keep
    # at most 64 splits (512 keys each).
    assert items == 8 * (64 + 1 + 1 + 2)


@pytest.mark.parametrize("even", [None, "0", "1"])
def test_plan_even_ranges_when_every_item_has_a_wavefront(ehip_mod, monkeypatch, even):
    """A step with no more items than the decode target (2048) cuts each row
    into the same number of ranges as fixed-length cuts, but of near-equal
    length: every range but the last has RoundUp(ceil(L / n), 64) keys and the
    last is no longer. EHIP_SPLIT_EVEN=0 keeps fixed cuts (sl, sl, ..., rest);
    =1 forces even cuts."""
    monkeypatch.setenv("EHIP_SPLIT_TOKENS", "1024")
    monkeypatch.setenv("EHIP_NO_JOINT", "1")
    if even is not None:
        monkeypatch.setenv("EHIP_SPLIT_EVEN", even)
    lens = [1100, 3000, 1024, 4097, 300, 2049]
    rc, items = ehip_mod.plan_items(geom(ehip_mod, slab_blocks=1000), simple_step(ehip_mod, lens))
    assert rc == 0
    sl = 1024
    for r, L in enumerate(lens):
        mine = items[(items[:, 0] == r) & (items[:, 6] == 0)]
        spans = sorted((int(kb), int(ke)) for kb, ke in mine[:, 4:6])
        n = -(-L // sl)
        assert len(spans) == n, (L, spans)  # the same count either way
        assert spans[0][0] == 0 and spans[-1][1] == L
        assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
        step = sl if even == "0" else min(sl, -(-(-(-L // n)) // 64) * 64)
        assert all(ke - kb == step for kb, ke in spans[:-1]), (L, spans)
        assert spans[-1][1] - spans[-1][0] <= step
    if even != "0":
        # 1100 keys: two ranges of 576 and 524 instead of 1024 and 76.
        mine = items[(items[:, 0] == 0) & (items[:, 6] == 0)]
        assert sorted(int(ke - kb) for kb, ke in mine[:, 4:6]) == [524, 576]


def test_plan_large_steps_take_1024_to_1536_key_ranges(ehip_mod):
    """Steps whose one-item-per-wavefront length (kv-head-keys / 2048) is 512
    keys or more take ranges clamped to [1024, 1536] keys (the measured best
    of C3's decode rows, C4 and C5); smaller steps keep the target length, and
    INT8 plans their own rule."""
    from ehip import workloads
    for name, want in (("c4", 1536), ("c5", 1408), ("c2", 128)):
        w = getattr(workloads, name)()
        g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                              w.pool_blocks, w.scale)
        st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
        rc, rows, items, partials, split = ehip_mod.plan_counts(g, st)
        assert rc == 0 and split == want, (name, split)
    # C3's decode rows alone (what its mixed step leaves to the decode kernel):
    # 1.06M kv-head-keys give a 515-key target, raised to 1024.
    w = workloads.c3()
    idx = [i for i, t in enumerate(w.query_lens) if t == 1]
    st = ehip_mod.StepArrays([1] * len(idx), [w.context_lens[i] for i in idx],
                             [w.tables[i] for i in idx])
    g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                          w.pool_blocks, w.scale)
    assert ehip_mod.plan_counts(g, st)[4] == 1024
    # The boundary (256 rows x 8 kv heads = 2048 units): rows of 511 keys give
    # a 511-key target (rounded to 512-key ranges), rows of 512 keys reach the
    # large-step clamp and take 1024.
    for L, want in ((511, 512), (512, 1024)):
        lens = [L] * 256
        rc, rows, items, partials, split = ehip_mod.plan_counts(
            geom(ehip_mod, slab_blocks=256 * ((L + 15) // 16)), simple_step(ehip_mod, lens))
        assert rc == 0 and split == want, (L, split)
    # INT8 keeps its own rule (half the item target, 128-block ranges).
    w = workloads.c4()
    g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, ehip_mod.KV_INT8,
                          w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert ehip_mod.plan_counts(g, st)[4] == 128 * w.block_size


def test_plan_small_steps_split_into_64_key_units(ehip_mod):
    """A step with fewer than 128 items of 128 keys (128 * 128 kv-head-keys)
    is split into 64-key ranges; C2 and larger keep at least 128 keys."""
    from ehip import workloads
    for w, want in ((workloads.c1(), 64), (workloads.c2(), 128)):
        g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                              w.pool_blocks, w.scale)
        st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
        rc, rows, items, partials, split = ehip_mod.plan_counts(g, st)
        assert rc == 0 and split == want
        assert items == expected_items(w.context_lens, w.kv_heads, split)
    # the boundary: 8 kv heads x 2047 keys is below 16384 units, 8 x 2048 is not
    for L, want in ((2047, 64), (2048, 128)):
        rc, rows, items, partials, split = ehip_mod.plan_counts(
            geom(ehip_mod, slab_blocks=200), simple_step(ehip_mod, [L]))
        assert rc == 0 and split == want


def test_plan_prefill_rows_are_causal(ehip_mod, monkeypatch):
    monkeypatch.setenv("EHIP_SPLIT_TOKENS", "128")
    monkeypatch.setenv("EHIP_NO_JOINT", "1")
    # One chunk of T=300 on top of P=100 cached tokens: rows attend 101..400 keys.
    st = simple_step(ehip_mod, [400], qlens=np.array([300], np.int32))
    rc, rows, items, partials, split = ehip_mod.plan_counts(geom(ehip_mod), st)
    assert rc == 0 and rows == 300
    assert items == 8 * sum(math.ceil(n / 128) for n in range(101, 401))


def test_plan_empty_step(ehip_mod):
    st = ehip_mod.StepArrays([], [], [])
    assert ehip_mod.plan_counts(geom(ehip_mod), st)[:4] == (0, 0, 0, 0)


@pytest.mark.parametrize("kw", [dict(block_size=12), dict(block_size=128), dict(heads=30),
                                dict(kv_dtype=4), dict(kv_dtype=-1), dict(head_dim=0),
                                dict(slab_blocks=0), dict(head_dim=512)])
def test_plan_rejects_bad_geometry(ehip_mod, kw):
    rc = ehip_mod.plan_counts(geom(ehip_mod, **kw), simple_step(ehip_mod, [40]))[0]
    assert rc in (ehip_mod.INVALID_ARGUMENT, ehip_mod.UNIMPLEMENTED)


def test_plan_rejects_bad_steps(ehip_mod):
    g = geom(ehip_mod, slab_blocks=10)
    # table shorter than ceil(L/bs)
    st = ehip_mod.StepArrays([1], [40], [np.array([0, 1], np.int32)])
    assert ehip_mod.plan_counts(g, st)[0] == ehip_mod.INVALID_ARGUMENT
    # id outside the slab
    st = ehip_mod.StepArrays([1], [20], [np.array([0, 10], np.int32)])
    assert ehip_mod.plan_counts(g, st)[0] == ehip_mod.INVALID_ARGUMENT
    st = ehip_mod.StepArrays([1], [20], [np.array([-1, 3], np.int32)])
    assert ehip_mod.plan_counts(g, st)[0] == ehip_mod.INVALID_ARGUMENT
    # slot outside the slab, and a negative slot
    for bad in (10 * 16, -1):
        st = ehip_mod.StepArrays([1], [20], [np.array([0, 1], np.int32)], [bad])
        assert ehip_mod.plan_counts(g, st)[0] == ehip_mod.INVALID_ARGUMENT
    # T > L, T < 1
    st = ehip_mod.StepArrays([5], [3], [np.array([0], np.int32)])
    assert ehip_mod.plan_counts(g, st)[0] == ehip_mod.INVALID_ARGUMENT
    st = ehip_mod.StepArrays([0], [3], [np.array([0], np.int32)])
    assert ehip_mod.plan_counts(g, st)[0] == ehip_mod.INVALID_ARGUMENT
    # a table longer than needed is fine (tables are a bound, like num_blocks)
    st = ehip_mod.StepArrays([1], [20], [np.array([0, 1, 9, 9], np.int32)])
    assert ehip_mod.plan_counts(g, st)[0] == 0


def test_workload_slots_follow_block_table_closed_form(ehip_mod):
    from ehip import workloads
    for w in (workloads.c1(), workloads.c2(), workloads.c3()):
        r = 0
        for t, T, L in zip(w.tables, w.query_lens, w.context_lens):
            for pos in range(int(L) - int(T), int(L)):
                # slot(pos) = blocks[pos / bs] * bs + pos % bs (block_table.cpp:97-103)
                assert w.slot_mapping[r] == t[pos // w.block_size] * w.block_size + pos % w.block_size
                r += 1
        assert r == len(w.slot_mapping)
        used = np.concatenate(w.tables)
        assert len(np.unique(used)) == len(used)  # C1-C3 tables never share
        assert used.max() < w.pool_blocks


def test_c4_sharing_and_byte_accounting():
    from ehip import workloads
    w = workloads.c4()
    rc = w.refcount
    in_use = int((rc > 0).sum())
    frac = int((rc == 2).sum()) / in_use
    assert 0.09 <= frac <= 0.11, frac
    b = w.bytes_per_layer(with_append=False)
    row = 8 * 128 * 2 * 2
    assert b["logical_kv"] == row * int(w.context_lens.sum())
    assert b["logical_kv"] - b["unique_kv"] == row * 16 * int((rc == 2).sum())
    # Shared blocks are full prefix blocks of both sharers: the appended token
    # never lands in one.
    blocks = w.slot_mapping // w.block_size
    assert (rc[blocks] == 1).all()


def joint_expectation(w, split, bs=16, min_joint=128):
    """Mirror of the planner's pairing for tables that share only as forked
    prefixes: rows ordered by (first block id, table, index), adjacent rows
    sharing >= min_joint keys of full leading blocks, short of either row's
    last key, are paired."""
    n = len(w.context_lens)
    first = [int(t[0]) for t in w.tables]
    order = sorted(range(n), key=lambda r: (first[r], r))
    joint_len = [0] * n
    pairs = []
    i = 0
    while i + 1 < n:
        a, b = order[i], order[i + 1]
        L = (min(int(w.context_lens[a]), int(w.context_lens[b])) - 1) // bs
        c = 0
        while c < L and w.tables[a][c] == w.tables[b][c]:
            c += 1
        if c * bs >= min_joint:
            joint_len[a] = joint_len[b] = c * bs
            pairs.append((a, b))
            i += 2
        else:
            i += 1
    return joint_len, pairs


@pytest.mark.parametrize("tail", [None, 256])
def test_plan_joint_items_for_shared_prefixes(ehip_mod, monkeypatch, tail):
    if tail is not None:
        monkeypatch.setenv("EHIP_TAIL_SPLIT", str(tail))
    tail = tail or 0  # off by default; C4 is past the item target, so 256 applies
    from ehip import workloads
    w = workloads.c4()
    g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                          w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    rc, rows, items, partials, split, joint, shared = ehip_mod.plan_counts(g, st, joint=True)
    assert rc == 0
    joint_len, pairs = joint_expectation(w, split)
    assert len(pairs) > 0
    assert shared == sum(joint_len[a] for a, _ in pairs)
    # every pair shares exactly the blocks the workload forked (>= 8 blocks)
    assert shared <= 16 * w.notes["shared_blocks"]
    exp_joint = sum(math.ceil(joint_len[a] / split) for a, _ in pairs) * w.kv_heads
    ranges = []
    for a, b in pairs:
        P = joint_len[a]
        ranges += [((a, b), min(split, P - t)) for t in range(0, P, split)]
    for r, L in enumerate(w.context_lens):
        P = joint_len[r]
        ranges += [((r,), min(split, int(L) - t)) for t in range(P, int(L), split)]
    nsplit = cut_tail(ranges, w.kv_heads, tail)
    n_ranges = len(ranges) + sum(nsplit.values()) - sum(len(rw) for rw, _ in ranges)
    assert joint == exp_joint
    assert items == n_ranges * w.kv_heads
    assert partials == sum(nsplit.values()) * w.kv_heads


def greedy_groups(order, shared_blocks, cap, bs=16, min_joint=128):
    """The planner's grouping rule, restated: from each row in order, take
    the following rows while the common prefix C' = min(C, shared with the
    first row) keeps at least min_joint keys and saves more re-reads than
    before (m * C' > (m - 1) * C), up to cap rows."""
    groups, i = [], 0
    while i + 1 < len(order):
        common, j = None, i + 1
        while j < len(order) and j - i < cap:
            c = shared_blocks(order[i], order[j])
            c = c if common is None else min(common, c)
            m = j - i
            if c * bs < min_joint or (common is not None and m * c <= (m - 1) * common):
                break
            common, j = c, j + 1
        if j - i < 2:
            i += 1
            continue
        groups.append((order[i:j], common))
        i = j
    return groups


def test_plan_chunk_rows_group_up(ehip_mod, monkeypatch):
    monkeypatch.setenv("EHIP_SPLIT_TOKENS", "128")
    # A chunk of 300 rows over 100 cached keys: row t attends 101 + t keys;
    # consecutive rows of one sequence read the same table, so they form
    # joint groups of four (g = 4: 16 / 4 virtual-head rows). A joint prefix
    # is whole blocks short of every member's last key.
    st = simple_step(ehip_mod, [400], qlens=np.array([300], np.int32))
    rc, rows, items, partials, split, joint, shared = ehip_mod.plan_counts(geom(ehip_mod), st,
                                                                           joint=True)
    assert rc == 0 and rows == 300
    lens = [101 + t for t in range(300)]
    groups = greedy_groups(list(range(300)), lambda a, b: (min(lens[a], lens[b]) - 1) // 16,
                           cap=4)
    assert max(len(m) for m, _ in groups) == 4
    joint_len = [0] * 300
    exp_joint = exp_shared = 0
    for members, c in groups:
        for r in members:
            joint_len[r] = 16 * c
        exp_shared += 16 * c * (len(members) - 1)
        exp_joint += math.ceil(16 * c / 128)
    exp_private = sum(math.ceil((L - P) / 128) for L, P in zip(lens, joint_len))
    assert shared == exp_shared
    assert joint == 8 * exp_joint
    assert items == 8 * (exp_joint + exp_private)


def check_partition(items, lens, hkv):
    """Every (row, kv head) has key ranges (its own and the joint ones it is a
    member of) that tile [0, L) exactly, numbered 0..n-1 in key order."""
    per = {}
    for r0, r1, r2, r3, tb, te, hk, sp in items.tolist():
        assert 0 <= tb < te
        for r in (r0, r1, r2, r3):
            if r >= 0:
                per.setdefault((r, hk), []).append((tb, te, sp))
    for r, L in enumerate(lens):
        ns = None
        for hk in range(hkv):
            rs = sorted(per[(r, hk)])
            assert rs[0][0] == 0 and rs[-1][1] == L
            assert all(a[1] == b[0] for a, b in zip(rs, rs[1:]))
            assert [sp for _, _, sp in rs] == list(range(len(rs)))
            assert ns is None or ns == len(rs)  # the same splits for every head
            ns = len(rs)


def test_plan_items_partition_c4(ehip_mod):
    """The work list of the C4 step (pair-shared prefixes, log-uniform
    lengths) tiles every row exactly, with split indices in key order and
    the same splits for every kv head; items are ordered costliest first
    (keys times rows served)."""
    from ehip import workloads
    w = workloads.c4()
    g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                          w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    rc, items = ehip_mod.plan_items(g, st)
    assert rc == 0
    check_partition(items, w.context_lens, w.kv_heads)
    # costliest first: keys times the rows an item serves
    cost = (items[:, 5] - items[:, 4]) * (items[:, :4] >= 0).sum(axis=1)
    assert (np.diff(cost) <= 0).all()
    rc, rows, n, partials, split, joint, shared = ehip_mod.plan_counts(g, st, joint=True)
    assert n == len(items) and joint == int((items[:, 1] >= 0).sum()) > 0


def group_step(ehip_mod, groups, bs=16, seed=5):
    """Rows forked from shared prefixes: groups of (shared_blocks, [lengths]);
    every member's blocks after the shared ones are its own."""
    rng = np.random.default_rng(seed)
    need = sum(sb + sum((L + bs - 1) // bs - sb for L in lens) for sb, lens in groups)
    perm = rng.permutation(need + 5).astype(np.int32)
    tabs, off = [], 0
    for sb, lens in groups:
        shared = perm[off:off + sb]
        off += sb
        for L in lens:
            own = (L + bs - 1) // bs - sb
            tabs.append(np.concatenate([shared, perm[off:off + own]]).astype(np.int32))
            off += own
    lens = [L for _, ls in groups for L in ls]
    st = ehip_mod.StepArrays(np.ones(len(lens), np.int32), np.asarray(lens, np.int64), tabs)
    return st, lens, need + 5


@pytest.mark.parametrize("H,Hkv,cap", [(32, 8, 4), (64, 8, 2), (8, 8, 4), (14, 2, 2)])
def test_plan_joint_groups_beyond_pairs(ehip_mod, H, Hkv, cap):
    """Rows forked from one prefix form joint groups of up to min(4, 16 / g)
    rows: a group of five sharers of 20 blocks is cut into groups of the cap;
    a member whose common prefix with the group is short joins only while it
    saves more re-read keys (m * C' > (m - 1) * C). Every row's key ranges
    still tile [0, L) with split indices in key order."""
    groups = [(20, [700, 530, 900, 400, 655]),   # five sharers of 320 keys
              (12, [300, 900, 260]),             # three sharers of 192 keys
              (30, [600, 610]),                  # a pair
              (0, [129, 77])]                    # no sharing
    st, lens, pool = group_step(ehip_mod, groups)
    g = ehip_mod.geometry(H, Hkv, 64, 16, ehip_mod.KV_BF16 if H % Hkv == 0 and (H // Hkv) in (1, 2, 4, 8) else ehip_mod.KV_F32, pool, 0.125)
    rc, items = ehip_mod.plan_items(g, st)
    assert rc == 0
    check_partition(items, lens, Hkv)
    sizes = (items[:, :4] >= 0).sum(axis=1)
    assert sizes.max() == cap
    # every joint item's rows are members of one fork group, over its shared prefix
    first = np.cumsum([0] + [len(ls) for _, ls in groups])
    group_of = {r: k for k in range(len(groups)) for r in range(first[k], first[k + 1])}
    for it in items[sizes > 1]:
        rows = [r for r in it[:4] if r >= 0]
        assert len({group_of[r] for r in rows}) == 1
        assert it[5] <= 16 * groups[group_of[rows[0]]][0]
    rc, rows, n, partials, split, joint, shared = ehip_mod.plan_counts(g, st, joint=True)
    # saved re-reads: the five sharers give groups of the cap (and a remainder
    # pair when cap = 2: 2 + 2 + 1), the three give cap-limited groups, the pair one
    exp = 0
    for sb, ls in groups:
        m = len(ls)
        while m >= 2 and sb * 16 >= 128:
            take = min(cap, m)
            exp += 16 * sb * (take - 1)
            m -= take
    assert shared == exp


def test_plan_joint_group_member_rule(ehip_mod):
    """A third sharer whose common prefix is much shorter stays out of the
    group (2 * 8 <= 1 * 30); one whose common prefix is close joins
    (2 * 25 > 1 * 30)."""
    bs = 16
    # rows 0, 1 share 30 blocks; row 2 shares the first 8 of them
    base = np.arange(40, dtype=np.int32)
    t0 = base[:40]
    t1 = np.concatenate([base[:30], np.arange(100, 110, dtype=np.int32)])
    t2 = np.concatenate([base[:8], np.arange(200, 232, dtype=np.int32)])
    g = ehip_mod.geometry(32, 8, 128, bs, ehip_mod.KV_BF16, 256, 0.088)
    st = ehip_mod.StepArrays(np.ones(3, np.int32), np.array([640, 640, 640], np.int64),
                             [t0, t1, t2])
    rc, *_, joint, shared = ehip_mod.plan_counts(g, st, joint=True)
    assert rc == 0 and shared == 30 * 16
    t2 = np.concatenate([base[:25], np.arange(200, 215, dtype=np.int32)])
    st = ehip_mod.StepArrays(np.ones(3, np.int32), np.array([640, 640, 640], np.int64),
                             [t0, t1, t2])
    rc, *_, joint, shared = ehip_mod.plan_counts(g, st, joint=True)
    assert rc == 0 and shared == 2 * 25 * 16


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_plan_int8_shapes_and_append_groups(ehip_mod, fmt, monkeypatch):
    """INT8 and FP8 KV: shapes outside the kernels' coverage are
    Unimplemented (9); rows landing in one block must take consecutive slots
    (2 otherwise); rows sharing leading blocks get joint items, as for bf16."""
    E = ehip_mod
    kv = E.KV_FP8 if fmt == "fp8" else E.KV_INT8
    tabs = [np.arange(4, dtype=np.int32), np.arange(4, 8, dtype=np.int32)]
    st = E.StepArrays(np.array([3, 1], np.int32), np.array([40, 20], np.int64), tabs,
                      np.array([37, 38, 39, 4 * 16 + 19], np.int64))
    ok = E.geometry(32, 8, 128, 16, kv, 16, 0.088)
    assert E.plan_counts(ok, st, joint=True)[0] == 0
    for bad in (E.geometry(14, 2, 64, 16, kv, 8, 0.125),   # g = 7
                E.geometry(32, 8, 96, 16, kv, 8, 0.1),     # d = 96
                E.geometry(32, 8, 128, 8, kv, 16, 0.088)):  # bs = 8
        assert E.plan_counts(bad, st)[0] == 9
    gap = E.StepArrays(np.array([3, 1], np.int32), np.array([40, 20], np.int64), tabs,
                       np.array([36, 38, 39, 4 * 16 + 19], np.int64))
    assert E.plan_counts(ok, gap)[0] == 2
    # two sequences forked from one prefix share 8 leading blocks (128 keys):
    # one joint range per kv head at 128-key splits, for INT8/FP8 as for bf16
    monkeypatch.setenv("EHIP_SPLIT_TOKENS", "128")
    shared = [np.arange(10, dtype=np.int32), np.array(list(range(8)) + [10, 11], np.int32)]
    st2 = E.StepArrays(np.array([1, 1], np.int32), np.array([150, 150], np.int64), shared,
                       np.array([9 * 16 + 5, 11 * 16 + 5], np.int64))
    rc, rows, items, partials, split, joint, sh = E.plan_counts(ok, st2, joint=True)
    assert rc == 0 and joint == 8 and sh == 128
    g16 = E.geometry(32, 8, 128, 16, E.KV_BF16, 16, 0.088)
    assert E.plan_counts(g16, st2, joint=True)[5:] == (joint, sh)


def prefill_items(ehip_mod, g, st):
    n = C.c_int64()
    L = ehip_mod.lib()
    assert L.ehip_plan_prefill_items(C.byref(g), C.byref(st.desc), None, 0, C.byref(n)) == 0
    out = np.zeros((max(n.value, 1), 9), np.int32)
    assert L.ehip_plan_prefill_items(C.byref(g), C.byref(st.desc), out.ctypes.data, n.value,
                                     C.byref(n)) == 0
    return out[:n.value]


@pytest.mark.parametrize("H,Hkv,T,P", [(8, 2, 16, 20000), (8, 2, 16, 40000), (32, 8, 4096, 0),
                                       (64, 8, 37, 60000), (16, 2, 300, 9000)])
def test_plan_prefill_split_ids_cover_recorded_splits(ehip_mod, H, Hkv, T, P):
    """Every MFMA prefill block cut into key splits writes exactly the split
    slots its rows record (ids 0 .. nsplit-1, once per kv head), and its
    pieces tile the block's keys [0, P + last row + 1) without gaps. A count
    above the pieces cut would make the merge read slots nothing wrote (the
    split cap of 64 per row forces fewer, longer pieces on long contexts)."""
    bs = 16
    L = P + T
    st = simple_step(ehip_mod, [L], qlens=np.array([T], np.int32))
    g = geom(ehip_mod, heads=H, kv_heads=Hkv, slab_blocks=(L + bs - 1) // bs + 8)
    items = prefill_items(ehip_mod, g, st)
    assert len(items) > 0
    blocks = {}
    for row_base, chunk, past, q0, hk, split, kb, ke, nsplit in items:
        assert (chunk, past) == (T, P)
        blocks.setdefault((q0, hk), []).append((split, kb, ke, nsplit))
    m = min(q0 for q0, _ in blocks if q0 > 0) if len({q0 for q0, _ in blocks}) > 1 else T
    for (q0, hk), pieces in blocks.items():
        keys = P + min(T, q0 + m)
        ns = {p[3] for p in pieces}
        assert len(ns) == 1, pieces
        nsplit = ns.pop()
        ids = sorted(p[0] for p in pieces)
        if nsplit == 0:
            assert ids == [0] and pieces[0][1:3] == (0, keys)
        else:
            assert ids == list(range(nsplit)), (q0, hk, nsplit, ids)
            spans = sorted((kb, ke) for _, kb, ke, _ in pieces)
            assert spans[0][0] == 0 and spans[-1][1] == keys
            assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
    # The first case is the one that exposed the cap: 626 key tiles cut in 64
    # requested pieces of 10 tiles make 63 pieces.
    if (H, Hkv, T, P) == (8, 2, 16, 20000):
        assert {p[3] for v in blocks.values() for p in v} == {63}


@pytest.mark.parametrize("L", [256, 257, 512])
def test_plan_every_row_keeps_a_range_ending_at_its_last_key(ehip_mod, L):
    """Rows whose tables agree on every block (a length that is a multiple of
    the block size included) still get a range of their own that ends at
    their last key: the item that appends the row's new token in the fused
    append + attention launch. The joint prefix stops a block short of it."""
    bs = 16
    n = (L + bs - 1) // bs
    shared = np.arange(n, dtype=np.int32)
    # Two decode rows over one table (as a fork that has not diverged yet),
    # and an unrelated third row.
    other = np.arange(n, 2 * n, dtype=np.int32)
    st = ehip_mod.StepArrays(np.ones(3, np.int32), np.array([L, L, L], np.int64),
                             [shared, shared, other], np.arange(3, dtype=np.int64))
    g = geom(ehip_mod, slab_blocks=2 * n + 4)
    rc, items = ehip_mod.plan_items(g, st)
    assert rc == 0
    assert (items[:, 1] >= 0).any(), "the shared prefix should make joint items"
    check_partition(items, [L, L, L], 8)
    for r in range(3):
        own = items[(items[:, 0] == r) & (items[:, 1] < 0)]
        assert (own[:, 5] == L).sum() == 8, f"row {r}: no range of its own ending at {L}"
    joint = items[items[:, 1] >= 0]
    assert joint[:, 5].max() <= (L - 1) // bs * bs
