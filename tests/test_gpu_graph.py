"""Captured-graph replay of the per-layer step launches.

A caller hands its stream to the context (ehip_set_stream) and captures the
per-layer append + attention launches of an uploaded step into a HIP graph
(stream capture through the HIP runtime the library uses). Each replay, with the slabs restored and the outputs
poisoned by eager copies in between, must reproduce the eager run bit for bit
(slabs and outputs): the launches record kernels only, and the persistent
decode kernel leaves its queue counters as it found them.
"""
import numpy as np
import pytest

from gpu_util import new_rows, seeded_pool

pytestmark = pytest.mark.gpu


def run_case(gctx, ehip_mod, orc, w, layers, int8=False):
    from ehip import hipgraph
    E = ehip_mod
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    g = E.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale)
    st = E.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    bufs = []
    for layer in range(layers):
        kp, vp = seeded_pool(orc, w, 100 + layer, poison=False)
        if int8:
            k8 = np.clip(np.rint(kp * 40), -127, 127).astype(np.int8)
            v8 = np.clip(np.rint(vp * 40), -127, 127).astype(np.int8)
            sc = np.full((w.pool_blocks, Hkv), 1 / 40, np.float32)
            slab_k, slab_v = k8, v8
            extra = (gctx.to_device(sc), gctx.to_device(sc.copy()))
        else:
            slab_k = orc.to_bf16_bits(kp) if w.kv_dtype == E.KV_BF16 else kp
            slab_v = orc.to_bf16_bits(vp) if w.kv_dtype == E.KV_BF16 else vp
            extra = None
        kn, vn, q = new_rows(orc, w, 300 + layer)
        bufs.append(dict(k0=slab_k, v0=slab_v, dk=gctx.to_device(slab_k),
                         dv=gctx.to_device(slab_v), dkn=gctx.to_device(kn),
                         dvn=gctx.to_device(vn), dq=gctx.to_device(q),
                         out=gctx.alloc(q.nbytes), shape=q.shape, scales=extra))

    def launches():
        for b in bufs:
            if int8:
                ks, vs = b["scales"]
                assert gctx.step_kv_append_int8(b["dkn"], b["dvn"], b["dk"], b["dv"], ks, vs) == 0
                assert gctx.step_attention_int8(b["dq"], b["dk"], b["dv"], ks, vs, b["out"]) == 0
            else:
                assert gctx.step_kv_append(b["dkn"], b["dvn"], b["dk"], b["dv"]) == 0
                assert gctx.step_attention(b["dq"], b["dk"], b["dv"], b["out"]) == 0

    def restore():
        for b in bufs:
            b["dk"].upload(b["k0"])
            b["dv"].upload(b["v0"])
            b["out"].upload(np.full(b["shape"], -7.0, np.float32))
            if int8:
                sc = np.full((w.pool_blocks, Hkv), 1 / 40, np.float32)
                b["scales"][0].upload(sc)
                b["scales"][1].upload(sc)

    def snapshot():
        return [(b["out"].download(np.float32, b["shape"]).copy(),
                 b["dk"].download(b["k0"].dtype, b["k0"].shape).copy(),
                 b["dv"].download(b["v0"].dtype, b["v0"].shape).copy()) for b in bufs]

    s = hipgraph.Stream()
    graph = hipgraph.Graph()
    assert ehip_mod.lib().ehip_set_stream(gctx.h, s.h) == 0
    try:
        assert gctx.step_upload(g, st) == 0, gctx.last_error()
        restore()
        launches()
        gctx.sync()
        eager = snapshot()
        graph.capture(s, launches)
        for _ in range(3):
            restore()
            graph.replay(s)
            gctx.sync()
            for (o, k, v), (eo, ek, ev) in zip(snapshot(), eager):
                assert np.array_equal(o.view(np.uint32), eo.view(np.uint32))
                assert np.array_equal(k.view(np.uint8), ek.view(np.uint8))
                assert np.array_equal(v.view(np.uint8), ev.view(np.uint8))
    finally:
        assert ehip_mod.lib().ehip_set_stream(gctx.h, None) == 0
        graph.close()
        s.close()
    for b in bufs:
        for key in ("dk", "dv", "dkn", "dvn", "dq", "out"):
            b[key].free()
        if b["scales"]:
            for x in b["scales"]:
                x.free()


def test_graph_replay_bf16_persistent_decode(ehip_mod, orc, tctx):
    """bf16 C4 shape at 24 sequences (joint items), the persistent decode
    kernel on 5 wavefronts so each drains the queue, three layers."""
    gctx = tctx(EHIP_DECODE_SLOTS="5")
    from ehip import workloads
    run_case(gctx, ehip_mod, orc, workloads.c4(num_seqs=24, share_frac=0.3), layers=3)


def test_graph_replay_fp32_small_step(gctx, ehip_mod, orc):
    """The C1 shape: the workgroup-per-row kernel (no merge launch)."""
    from ehip import workloads
    run_case(gctx, ehip_mod, orc, workloads.c1(), layers=2)


def test_graph_replay_fp32_split_kv(gctx, ehip_mod, orc):
    """C2: split-KV decode plus the merge kernel per layer."""
    from ehip import workloads
    run_case(gctx, ehip_mod, orc, workloads.c2(layers=2), layers=2)


def test_graph_replay_int8(gctx, ehip_mod, orc):
    """INT8 append (requantising growing blocks) and INT8 decode."""
    from ehip import workloads
    w = workloads.c4(num_seqs=16, share_frac=0.0)
    w.kv_dtype = ehip_mod.KV_INT8
    run_case(gctx, ehip_mod, orc, w, layers=2, int8=True)


def test_graph_replay_mixed_prefill_and_decode(gctx, ehip_mod, orc):
    """A step with causal prefill chunks (one from position 0, one after a
    cached prefix) and decode rows: the prefill kernel, the persistent decode
    kernel and the split merge (which also reduces the chunks' key splits)
    are all captured and replayed."""
    from ehip import workloads
    rng = np.random.default_rng(11)
    qlens = np.array([64, 96] + [1] * 8, np.int32)
    ctx_lens = np.concatenate([[64, 296], rng.integers(100, 700, 8) + 1]).astype(np.int64)
    need = (ctx_lens + 15) // 16
    pool = int(np.ceil(1.25 * need.sum()))
    tables, _ = workloads._tables_from_pool(need, pool, rng)
    w = workloads._finish("mixed", 32, 8, 128, 16, ehip_mod.KV_BF16, 2, qlens, ctx_lens, tables,
                          pool, 0.5)
    run_case(gctx, ehip_mod, orc, w, layers=2)


# ------------------------------------------------------- replay vs the oracle
def _oracle_step(orc, w, kb, vb, kn, vn, q, slots, lens, tables):
    """The oracle's append into the host bf16 slabs, then the reference
    attention on the widened post-append cache (and on nothing else: the
    caller compares)."""
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    orc.kv_scatter(kn, vn, slots, Hkv, d, bs, kb, vb)
    kr, vr = orc.bf16_bits_to_f32(kb), orc.bf16_bits_to_f32(vb)
    return orc.paged_decode_batched(q, kr, vr, tables, [int(x) for x in lens], H, Hkv, d, bs,
                                    w.scale, isa=orc.ISA_AVX2)


def _decode_steps(w, n_steps):
    """The workload advanced one token per sequence per step: each step's
    post-append lengths, tables (grown by a free block when a boundary is
    crossed) and append slots."""
    bs = w.block_size
    used = set(int(b) for t in w.tables for b in t)
    free = [b for b in range(w.pool_blocks) if b not in used]
    tables = [list(map(int, t)) for t in w.tables]
    steps = []
    for s in range(n_steps):
        lens = w.context_lens.astype(np.int64) + s
        slots = []
        for b, L in enumerate(lens):
            while len(tables[b]) * bs < L:
                tables[b].append(free.pop())
            pos = int(L) - 1
            slots.append(tables[b][pos // bs] * bs + pos % bs)
        steps.append((lens.copy(), [np.array(t, np.int32) for t in tables],
                      np.array(slots, np.int64)))
    return steps


def test_graph_replay_follows_a_changing_decode_plan(gctx, ehip_mod, orc):
    """A decode loop under one instantiated graph: every step each sequence
    grows by a token (new lengths, new slots, tables growing across block
    boundaries), the step's plan is uploaded eagerly, the layer launches are
    re-captured and written into the graph with hipGraphExecUpdate, and the
    replay is checked against the oracle (append bit-exact, outputs within
    1e-4 relative per vector on the same bf16 cache) and against an eager run
    of the same plan (bit-identical)."""
    from ehip import hipgraph, workloads
    from gpu_util import rel_norm
    E = ehip_mod
    w = workloads.c4(num_seqs=16, share_frac=0.0)
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    g = E.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale)
    layers, n_steps = 2, 4
    steps = _decode_steps(w, n_steps)
    host, dev = [], []
    for layer in range(layers):
        kp, vp = seeded_pool(orc, w, 500 + layer, poison=False)
        kb, vb = orc.to_bf16_bits(kp), orc.to_bf16_bits(vp)
        host.append([kb, vb])
        dev.append([gctx.to_device(kb), gctx.to_device(vb)])
    R = w.num_seqs
    rows = [[new_rows(orc, w, 700 + 10 * s + layer) for layer in range(layers)]
            for s in range(n_steps)]
    drows = [[[gctx.to_device(x) for x in rows[s][layer]] for layer in range(layers)]
             for s in range(n_steps)]
    outs = [gctx.alloc(R * H * d * 4) for _ in range(layers)]

    def launches(s):
        def fn():
            for layer in range(layers):
                dkn, dvn, dq = drows[s][layer]
                dk, dv = dev[layer]
                assert gctx.step_kv_append(dkn, dvn, dk, dv) == 0, gctx.last_error()
                assert gctx.step_attention(dq, dk, dv, outs[layer]) == 0, gctx.last_error()
        return fn

    gs = hipgraph.Stream()
    graph = hipgraph.Graph()
    assert E.lib().ehip_set_stream(gctx.h, gs.h) == 0
    try:
        for s, (lens, tables, slots) in enumerate(steps):
            st = E.StepArrays(np.ones(R, np.int32), lens, tables, slots)
            assert gctx.step_upload(g, st) == 0, gctx.last_error()
            if s == 0:
                graph.capture(gs, launches(0))
            else:
                graph.update(gs, launches(s))
            graph.replay(gs)
            gctx.sync()
            got = [o.download(np.float32, (R, H, d)).copy() for o in outs]
            for layer in range(layers):
                kn, vn, q = rows[s][layer]
                kb, vb = host[layer]
                ref = _oracle_step(orc, w, kb, vb, kn, vn, q, slots, lens, tables)
                dk, dv = dev[layer]
                assert np.array_equal(dk.download(np.uint16, kb.shape), kb), (s, layer)
                assert np.array_equal(dv.download(np.uint16, vb.shape), vb), (s, layer)
                assert rel_norm(got[layer], ref) <= 1e-4, (s, layer, rel_norm(got[layer], ref))
            launches(s)()  # eager, same plan: the append is idempotent
            gctx.sync()
            for layer in range(layers):
                eager = outs[layer].download(np.float32, (R, H, d))
                assert np.array_equal(eager.view(np.uint32), got[layer].view(np.uint32)), (s, layer)
    finally:
        assert E.lib().ehip_set_stream(gctx.h, None) == 0
        graph.close()
        gs.close()
    for x in [b for pair in dev for b in pair] + [b for s in drows for l in s for b in l] + outs:
        x.free()
