#!/usr/bin/env python3
"""Benchmark of the ragged paged-attention decode step on one MI355X.

One step = one scheduler step of the configured workload (default C4: the
Llama-3-8B-shape 256-sequence ragged bf16-KV decode, 32 layers): one step
descriptor upload (host packing + one async copy), then per layer the
KV-append of the step's new token rows and one attention call over every
sequence. All K/V pools, queries and new rows are resident in HBM before the
timed region.

Data: the step's structure (lengths, block tables, shared prefixes) is the
config's seeded mt19937_64 draw (ehip.workloads). Layer 0's queries, K/V
pools and new rows are the reference's fill_normal streams of their seeds,
generated on the host (they are what the parity check re-computes); the other
layers' pools come from a device-side generator of the same distribution.

Prints ONE JSON line (metric/value/unit as BASELINE.json names them):
  value        = algorithmic HBM bytes of the step (unique K/V + Q + O +
                 tables + append) / the median step time, in GB/s (each timed
                 step is bracketed by its own pair of HIP events);
  roofline     = the attention call alone (decode kernel + split merge): its
                 algorithmic bytes per launch / its average duration (HIP
                 events on the launch stream around every layer's attention
                 call of every EVENT_SAMPLE-th timed step);
  cpu_baseline = the oracle's AVX2 restatement of the reference's batched
                 paged decode, timed on this host on the benched step's layer
                 0 (fp32 K/V); its outputs are also the parity checker;
  parity       = the benched step's layer 0 against that oracle: the append
                 (bit-exact slabs), the outputs against the reference run on
                 the bf16-rounded K/V (per-vector max_rel, allclose) and on
                 the original fp32 K/V (max_abs); "pass" is those bars. The
                 elementwise max_rel <= 1e-4 gate is reported beside them
                 ("elementwise_max_rel_gate", with whether the reference's own
                 scalar and AVX2 backends meet it against each other).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
EVENT_SAMPLE = 4  # per-launch events on one timed step in four
sys.path.insert(0, str(ROOT / "llm-inference-engine_amd" / "python"))
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
KV_NAMES = {0: "f32", 1: "bf16", 2: "int8", 3: "fp8"}
CPU_SHARE_PER_GPU = 16  # host threads one GPU's job may use on a shared node


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C4", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--seed", type=int, default=0, help="structure seed (0: the config's own)")
    ap.add_argument("--layers", type=int, default=0, help="override the config's layer count")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU baseline and the parity check it carries")
    ap.add_argument("--no-ceiling-probe", action="store_true",
                    help="skip the read-bandwidth probes that price the practical ceiling")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the prefill, fused RoPE, o_proj and re-prefill side measurements")
    ap.add_argument("--kv", default="auto", choices=["auto", "int8", "fp8"],
                    help="KV element type: the config's own (auto), or INT8 or FP8 (E4M3) "
                         "with per-(block, kv head) scales")
    ap.add_argument("--graph", action="store_true",
                    help="time the step as one eager descriptor upload plus one replay of a "
                         "captured HIP graph of the per-layer launches (stream capture on a "
                         "stream handed to the context with ehip_set_stream)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run one device-to-device copy of this size first (a known-size "
                         "dispatch that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def host_cpu():
    """(physical cores, model name) from lscpu, or (None, None)."""
    try:
        rows = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True,
                              timeout=10).stdout
        cores = len({ln for ln in rows.splitlines() if ln and not ln.startswith("#")})
        info = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in info.splitlines()
                      if ln.startswith("Model name")), None)
        return cores or None, model
    except (OSError, subprocess.SubprocessError):
        return None, None


def traffic_from_profiles(config: str, kv: str = ""):
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE / WRITE_SIZE per dispatch, each scaled by the same counter's
    reading on a copy kernel of known size), or None when no summary exists
    for this workload draw. kv: "" for the config's own KV type, "int8", "fp8"."""
    suffix = f"_{kv}" if kv else ""
    p = ROOT / "profiles" / f"decode_{config.lower()}{suffix}_traffic.json"
    if not p.exists():
        return None
    t = json.loads(p.read_text())
    return (t["fetch_kib_per_dispatch"] * t["fetch_scale"]
            + t["write_kib_per_dispatch"] * t["write_scale"]) * 1024.0, t.get("sum_context")


def parity_metrics(got, ref) -> dict:
    """max_abs; max_rel = max over elements of |a-b| / max(|b|, 1e-6 max|b|)
    (the elementwise form); max_rel_vector = max over (row, head) vectors of
    max|a-b| / max|b|; the reference's allclose criterion
    |a-b| <= 1e-5 + 1e-4 |b| (src/tensor/ops.h:207)."""
    a = np.asarray(got, np.float64)
    b = np.asarray(ref, np.float64)
    diff = np.abs(a - b)
    floor = 1e-6 * float(np.abs(b).max())
    den = np.maximum(np.abs(b), floor)
    den[den == 0] = 1.0
    fails = int(np.count_nonzero(~(diff <= 1e-5 + 1e-4 * np.abs(b))))
    vec_den = np.maximum(np.abs(b).reshape(-1, b.shape[-1]).max(axis=1), 1e-30)
    return {"max_abs": float(diff.max()), "max_rel": float((diff / den).max()),
            "max_rel_vector": float((diff.reshape(-1, b.shape[-1]).max(axis=1) / vec_den).max()),
            "allclose_rtol1e-4_atol1e-5": fails == 0, "allclose_failures": fails,
            "elements": int(a.size)}


def cpu_baseline_and_parity(w, layer0, seconds: float):
    """The CPU leg: the oracle's AVX2 restatement of the reference's
    PagedDecodeAttentionBatchedF32 timed on this host over the benched step's
    layer 0 (all sequences, fp32 K/V), and the same oracle as the parity
    checker of the GPU's layer-0 results."""
    from oracle import oracle as orc
    phys, model = host_cpu()
    allowed = len(os.sched_getaffinity(0))
    threads = max(1, min(phys or allowed, allowed, CPU_SHARE_PER_GPU))
    orc.set_threads(threads)
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    lens = [int(x) for x in w.context_lens]
    k32, v32 = layer0["k32"], layer0["v32"]
    q, kn, vn = layer0["q"], layer0["kn"], layer0["vn"]
    par = {"layer": 0}
    bf16 = w.kv_dtype == 1
    if bf16:
        # The append, bit for bit: the oracle narrows the pre-append fp32
        # pool and scatters the new rows (RNE), the GPU slabs must equal it.
        kb, vb = orc.to_bf16_bits(k32), orc.to_bf16_bits(v32)
        orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kb, vb)
        par["append_slabs_bit_exact"] = bool(np.array_equal(kb, layer0["k_dev"]) and
                                             np.array_equal(vb, layer0["v_dev"]))
        del kb, vb
        kr = orc.bf16_bits_to_f32(layer0["k_dev"])
        vr = orc.bf16_bits_to_f32(layer0["v_dev"])
        ref_r = orc.paged_decode_batched(q, kr, vr, w.tables, lens, H, Hkv, d, bs, w.scale,
                                         isa=orc.ISA_AVX2)
        del kr, vr
        par["vs_reference_on_bf16_kv"] = parity_metrics(layer0["out"], ref_r)
    # The fp32 reference cache after the step's append, timed as the baseline.
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, k32, v32)
    if not bf16:
        par["append_slabs_bit_exact"] = bool(
            np.array_equal(k32.view(np.uint32), layer0["k_dev"].view(np.uint32)) and
            np.array_equal(v32.view(np.uint32), layer0["v_dev"].view(np.uint32)))
    times = []
    t_end = time.perf_counter() + seconds
    ref32 = None
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        ref32 = orc.paged_decode_batched(q, k32, v32, w.tables, lens, H, Hkv, d, bs, w.scale,
                                         isa=orc.ISA_AVX2)
        times.append(time.perf_counter() - t0)
        if len(times) >= 500:
            break
    t = float(np.median(times))
    kv_bytes = Hkv * d * 4 * 2 * sum(lens)
    nblk = sum((L + bs - 1) // bs for L in lens)
    bytes_ = kv_bytes + 4 * w.rows * H * d * 2 + 4 * nblk + 8 * w.num_seqs
    base = {"value": round(bytes_ / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"oracle AVX2 PagedDecodeAttentionBatchedF32 restatement on {threads} "
                       f"threads, fp32 K/V, layer 0 of the benched {w.name} step (all "
                       f"{w.num_seqs} sequences, sum L={sum(lens)}), median of {len(times)} "
                       f"calls"),
            "host_physical_cores": phys, "host_cpus_allowed": allowed, "cpu_model": model,
            "attended_kv_tok_per_s": round(sum(lens) / t, 1), "ms_per_call": round(t * 1e3, 3)}
    # How far the reference's own two backends (scalar and AVX2, both
    # bit-identical to the reference build) are apart on the same fp32 cache:
    # the elementwise max_rel of near-zero outputs (sums that cancel) is set
    # by summation order, not by correctness.
    ref_scalar = orc.paged_decode_batched(q, k32, v32, w.tables, lens, H, Hkv, d, bs, w.scale,
                                          isa=orc.ISA_SCALAR)
    par["reference_scalar_vs_avx2"] = parity_metrics(ref_scalar, ref32)
    del ref_scalar
    gate = "vs_reference_on_bf16_kv" if bf16 else "vs_reference"
    if bf16:
        par["vs_reference_on_fp32_kv"] = parity_metrics(layer0["out"], ref32)
    else:
        par["vs_reference"] = parity_metrics(layer0["out"], ref32)
    par["bars"] = {"append": "bit-exact",
                   gate: "max_rel_vector <= 1e-4 and the reference allclose (rtol 1e-4, atol 1e-5)"}
    ok = (par["append_slabs_bit_exact"] and par[gate]["max_rel_vector"] <= 1e-4 and
          par[gate]["allclose_rtol1e-4_atol1e-5"])
    if bf16:
        par["bars"]["vs_reference_on_fp32_kv"] = "max_abs <= 2e-2"
        ok = ok and par["vs_reference_on_fp32_kv"]["max_abs"] <= 2e-2
    par["pass"] = bool(ok)
    # The north star's literal fp32 gate is the elementwise max_rel <= 1e-4.
    # It is reported as its own gate, not folded into "pass": the reference's
    # own scalar and AVX2 backends miss it against each other on this cache
    # (near-zero outputs of cancelling sums keep only rounding noise), which
    # is why the bar above is per output vector plus the reference allclose.
    elem = par[gate]["max_rel"]
    ref_elem = par["reference_scalar_vs_avx2"]["max_rel"]
    par["elementwise_max_rel_gate"] = {
        "bar": "max_rel <= 1e-4 (elementwise)", "value": elem, "met": bool(elem <= 1e-4),
        "reference_scalar_vs_avx2": ref_elem,
        "reference_meets_it": bool(ref_elem <= 1e-4)}
    return base, par


def ceiling_probe(w, slab_pair, slab_bytes):
    """Practical read ceilings on this device (lib/libehip_probe.so, no
    arithmetic): a streaming read of one K slab, and the decode access pattern
    (random (block, kv head) tiles of K and V, 36 per wavefront) with the
    default and the non-temporal load policy."""
    from ehip import probe
    ks, vs = slab_pair
    tile = w.block_size * w.head_dim * w.kv_bytes
    rng = np.random.default_rng(5)
    blocks = rng.permutation(w.pool_blocks).astype(np.int32)
    tiles = 36
    blocks = blocks[: blocks.size // tiles * tiles]
    out = {"stream_read_gbps": round(probe.stream_read(ks, min(slab_bytes, (1 << 32) - 16),
                                                       nt=False), 1)}
    for nt in (False, True):
        g = probe.tile_gather(ks, vs, w.pool_blocks, blocks, tiles, w.kv_heads,
                              w.kv_heads * tile, tile, nt=nt)
        out["tile_gather_nt_gbps" if nt else "tile_gather_gbps"] = round(g, 1)
    out["note"] = ("best of 3; tile gather = the decode kernels' access pattern alone, "
                   f"{tile}-byte (block, head) tiles of both slabs")
    return out


def time_calls(ctx, layers, reps, call):
    """Mean seconds of call(layer) over reps passes of every layer (HIP
    events around each call, after one untimed pass)."""
    ev = [(ctx.event(), ctx.event()) for _ in range(reps * layers)]
    for r in range(reps + 1):
        for layer in range(layers):
            if r:
                ctx.record(ev[(r - 1) * layers + layer][0])
            call(layer)
            if r:
                ctx.record(ev[(r - 1) * layers + layer][1])
    ctx.sync()
    return float(np.mean([ctx.elapsed_ms(a, b) for a, b in ev])) / 1e3


def time_chunks(ctx, ehip, w, slabs, qs, outs, layers, reps=5):
    """Attention time per layer of the workload's prefill chunks alone (a
    step holding only the chunk sequences; their K/V are already in the
    pools), so the MFMA prefill kernel can be priced against its roofline."""
    idx = [i for i, T in enumerate(w.query_lens) if T > 1]
    if not idx:
        return None
    qlens = w.query_lens[idx]
    st = ehip.StepArrays(qlens, w.context_lens[idx], [w.tables[i] for i in idx])
    g = ehip.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                      w.pool_blocks, w.scale)
    ctx._check(ctx.step_upload(g, st))
    t = time_calls(ctx, layers, reps, lambda layer: ctx._check(
        ctx.step_attention(qs[layer], slabs[layer][0], slabs[layer][1], outs[layer])))
    flops = 0
    for T, L in zip(qlens, w.context_lens[idx]):
        P = int(L) - int(T)
        flops += 4 * w.heads * w.head_dim * (int(T) * P + int(T) * (int(T) + 1) // 2)
    return {"chunks": len(idx), "rows": int(qlens.sum()), "flops_per_layer": flops,
            "us_per_layer": round(t * 1e6, 2), "tflops": round(flops / t / 1e12, 2),
            "roofline": {"bound": "mfma", "achieved": round(flops / t / 1e12, 2),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(flops / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                         "kernel": "causal prefill chunks (bf16 MFMA)"}}


def time_rope_append(ctx, ehip, w, slabs, qs, kns, vns, layers, reps=5):
    """The fused RoPE + KV append (ehip_step_rope_kv_append) against the plain
    append, one launch per layer each, on the workload's own step. Bytes of
    the fused kernel per launch: q read and written, new K/V rows read (fp32),
    one cos and one sin row per query row, K/V written to the slab."""
    H, Hkv, d, R = w.heads, w.kv_heads, w.head_dim, w.rows
    n_pos = int(w.context_lens.max())
    half = d // 2
    pos = np.arange(n_pos, dtype=np.float32)[:, None]
    inv = (1.0 / np.power(10000.0, np.arange(half, dtype=np.float64) * 2.0 / d)).astype(np.float32)
    ang = pos * inv[None, :]
    cos = ctx.to_device(np.cos(ang).astype(np.float32))
    sin = ctx.to_device(np.sin(ang).astype(np.float32))
    g = ehip.geometry(H, Hkv, d, w.block_size, w.kv_dtype, w.pool_blocks, w.scale)
    ctx._check(ctx.step_upload(g, ehip.StepArrays(w.query_lens, w.context_lens, w.tables,
                                                  w.slot_mapping)))
    t_plain = time_calls(ctx, layers, reps, lambda layer: ctx._check(
        ctx.step_kv_append(kns[layer], vns[layer], slabs[layer][0], slabs[layer][1])))
    t_rope = time_calls(ctx, layers, reps, lambda layer: ctx._check(
        ctx.step_rope_kv_append(qs[layer], kns[layer], vns[layer], cos, sin, n_pos,
                                slabs[layer][0], slabs[layer][1])))
    cos.free()
    sin.free()
    nbytes = R * (2 * H * d * 4 + 2 * Hkv * d * 4 + d * 4 + 2 * Hkv * d * w.kv_bytes)
    return {"rows": R, "bytes_per_launch": nbytes, "us_per_launch": round(t_rope * 1e6, 2),
            "gbps": round(nbytes / t_rope / 1e9, 1),
            "plain_append_us_per_launch": round(t_plain * 1e6, 2)}


def time_o_proj(ctx, ehip, w, outs, layers, reps=5):
    """The attention output's consumer, o_proj (ehip_packed_gemm): per layer
    y [rows, hidden] = ctx [rows, H*d] W^T with a bf16 checkpoint weight per
    layer (hidden = H*d for the configs' models), packed once into the
    reference's panel layout. Algorithmic flops 2*rows*H*d*hidden; weight
    bytes hidden*H*d*2 per launch."""
    m, k = w.rows, w.heads * w.head_dim
    n = k
    wts = []
    for layer in range(layers):
        raw = ctx.alloc(n * k * 2)
        ctx.fill_normal(raw, n * k, ehip.KV_BF16, 0.0, float(1.0 / np.sqrt(k)), 7000 + layer)
        wp = ctx.alloc(((n + 15) // 16) * k * 16 * 2)
        ctx._check(ctx.pack_weight_panels(raw, ehip.WEIGHT_BF16, n, k, wp))
        raw.free()
        wts.append(wp)
    y = ctx.alloc(m * n * 4)
    t = time_calls(ctx, layers, reps, lambda layer: ctx._check(
        ctx.packed_gemm(outs[layer], m, k, wts[layer], ehip.WEIGHT_BF16, n, None, y)))
    for b in wts + [y]:
        b.free()
    flops = 2 * m * k * n
    tf = flops / t / 1e12
    return {"m": m, "k": k, "n": n, "weight_dtype": "bf16", "us_per_launch": round(t * 1e6, 2),
            "tflops": round(tf, 2), "weight_gbps": round(n * k * 2 / t / 1e9, 1),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                         "kernel": "o_proj packed GEMM (x in three bf16 planes: 3x the "
                                   "algorithmic flops issued)"}}


def c5_reprefill(ctx, ehip, w, slabs, layers, reps=3):
    """C5's preempt-and-recompute event: one evicted sequence re-prefilled as
    a 4096-token causal chunk (P = 0), per layer, on the C5 pools."""
    T = 4096
    table = np.asarray(w.tables[0][:T // w.block_size], np.int32)  # 256 blocks of the pool
    st = ehip.StepArrays([T], [T], [table])
    g = ehip.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                      w.pool_blocks, w.scale)
    q = ctx.alloc(T * w.heads * w.head_dim * 4)
    out = ctx.alloc(T * w.heads * w.head_dim * 4)
    ctx.fill_normal(q, T * w.heads * w.head_dim, ehip.KV_F32, 0.0, w.qkv_std, 77)
    ctx._check(ctx.step_upload(g, st))
    t = time_calls(ctx, layers, reps, lambda layer: ctx._check(
        ctx.step_attention(q, slabs[layer][0], slabs[layer][1], out)))
    flops = 4 * w.heads * w.head_dim * (T * (T + 1) // 2)
    q.free()
    out.free()
    return {"tokens": T, "flops_per_layer": flops, "us_per_layer": round(t * 1e6, 2),
            "tflops": round(flops / t / 1e12, 2), "event_ms": round(t * layers * 1e3, 3),
            "roofline": {"bound": "mfma", "achieved": round(flops / t / 1e12, 2),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(flops / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                         "kernel": "causal prefill chunk (bf16 MFMA)"}}


class Bench:
    """Device state of one workload draw: pools, queries, new rows, outputs
    for every layer, and the step loop."""

    def __init__(self, ctx, ehip, w, layers, q8, host_layer0):
        # q8: "" for the config's own KV type, else "int8" or "fp8" (scaled slabs)
        self.ctx, self.ehip, self.w, self.layers, self.q8 = ctx, ehip, w, layers, q8
        H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
        R = w.rows
        self.slab_bytes = w.pool_blocks * Hkv * bs * d * w.kv_bytes
        self.slabs, self.scales, self.qs, self.kns, self.vns, self.outs = [], [], [], [], [], []
        self.layer0 = None
        for layer in range(layers):
            ks, vs = ctx.alloc(self.slab_bytes), ctx.alloc(self.slab_bytes)
            q, kn, vn = ctx.alloc(R * H * d * 4), ctx.alloc(R * Hkv * d * 4), ctx.alloc(R * Hkv * d * 4)
            if q8 == "fp8":
                # E4M3 slabs: N(0, 64) codes; scales: fp32 normals per (block, kv head)
                ctx.fill_normal(ks, self.slab_bytes, ehip.KV_FP8, 0.0, 64.0, 10 + layer)
                ctx.fill_normal(vs, self.slab_bytes, ehip.KV_FP8, 0.0, 64.0, 1000 + layer)
            if q8 == "int8":
                # int8 slabs: random bytes (bf16 normals over the same memory);
                # scales: fp32 normals, one per (block, kv head)
                n16 = self.slab_bytes // 2
                ctx.fill_normal(ks, n16, ehip.KV_BF16, 0.0, 1.0, 10 + layer)
                ctx.fill_normal(vs, n16, ehip.KV_BF16, 0.0, 1.0, 1000 + layer)
            if q8:
                kss, vss = ctx.alloc(w.pool_blocks * Hkv * 4), ctx.alloc(w.pool_blocks * Hkv * 4)
                ctx.fill_normal(kss, w.pool_blocks * Hkv, ehip.KV_F32, 0.0, 0.01, 5000 + layer)
                ctx.fill_normal(vss, w.pool_blocks * Hkv, ehip.KV_F32, 0.0, 0.01, 6000 + layer)
                self.scales.append((kss, vss))
            elif layer == 0 and host_layer0:
                self.layer0 = self._host_layer0(ks, vs, q, kn, vn)
            else:
                n = w.pool_blocks * Hkv * bs * d
                ctx.fill_normal(ks, n, w.kv_dtype, 0.0, w.qkv_std, 10 + layer)
                ctx.fill_normal(vs, n, w.kv_dtype, 0.0, w.qkv_std, 1000 + layer)
            if not (layer == 0 and self.layer0 is not None):
                ctx.fill_normal(q, R * H * d, ehip.KV_F32, 0.0, w.qkv_std, 2000 + layer)
                ctx.fill_normal(kn, R * Hkv * d, ehip.KV_F32, 0.0, w.qkv_std, 3000 + layer)
                ctx.fill_normal(vn, R * Hkv * d, ehip.KV_F32, 0.0, w.qkv_std, 4000 + layer)
            self.slabs.append((ks, vs))
            self.qs.append(q)
            self.kns.append(kn)
            self.vns.append(vn)
            self.outs.append(ctx.alloc(R * H * d * 4))
        ctx.sync()
        self.geom = ehip.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale)
        self.st = ehip.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)

    def _host_layer0(self, ks, vs, q, kn, vn):
        """Layer 0 from the workload's seeded fill_normal streams (host)."""
        from ehip import workloads
        w = self.w
        t0 = time.perf_counter()
        k32, v32 = w.pool(0)
        qh = w.q(0)
        knh, vnh = w.new_kv(0)
        if w.kv_dtype == self.ehip.KV_BF16:
            ks.upload(workloads.to_bf16_bits(k32))
            vs.upload(workloads.to_bf16_bits(v32))
        else:
            ks.upload(k32)
            vs.upload(v32)
        q.upload(qh)
        kn.upload(knh)
        vn.upload(vnh)
        log(f"[bench] layer 0 from the seeded host streams in {time.perf_counter() - t0:.1f} s")
        return {"k32": k32, "v32": v32, "q": qh, "kn": knh, "vn": vnh}

    def step(self, evs=None):
        ctx = self.ctx
        ctx._check(ctx.step_upload(self.geom, self.st))
        for layer in range(self.layers):
            ks, vs = self.slabs[layer]
            # The layer's append + attention: one call (one launch, plus the
            # split merge, for an all-decode bf16 step). The sampled events
            # bracket the whole call.
            if evs is not None:
                ctx.record(evs[layer][0])
            if self.q8:
                kss, vss = self.scales[layer]
                append = getattr(ctx, f"step_kv_append_{self.q8}")
                attention = getattr(ctx, f"step_attention_{self.q8}")
                ctx._check(append(self.kns[layer], self.vns[layer], ks, vs, kss, vss))
                ctx._check(attention(self.qs[layer], ks, vs, kss, vss, self.outs[layer]))
            else:
                ctx._check(ctx.step_append_attention(self.kns[layer], self.vns[layer],
                                                     self.qs[layer], ks, vs, self.outs[layer]))
            if evs is not None:
                ctx.record(evs[layer][1])

    def time_steps(self, steps, warmup):
        """Per-step seconds (HIP events at every step boundary), per-launch
        attention seconds of the sampled steps, and the wall time."""
        ctx = self.ctx
        for _ in range(warmup):
            self.step()
        ctx.sync()
        sampled = [s for s in range(steps) if s % EVENT_SAMPLE == EVENT_SAMPLE // 2] or [0]
        evs = {s: [(ctx.event(), ctx.event()) for _ in range(self.layers)] for s in sampled}
        marks = [ctx.event() for _ in range(steps + 1)]
        ctx.sync()
        t0 = time.perf_counter()
        ctx.record(marks[0])
        for s in range(steps):
            self.step(evs.get(s))
            ctx.record(marks[s + 1])
        ctx.sync()
        wall = time.perf_counter() - t0
        per_step = np.array([ctx.elapsed_ms(marks[s], marks[s + 1]) for s in range(steps)]) / 1e3
        attn = np.array([ctx.elapsed_ms(a, b) for s in sampled for (a, b) in evs[s]]) / 1e3
        return per_step, attn.reshape(len(sampled), self.layers), wall

    def capture_layer0(self):
        """Layer 0's post-step slabs and outputs, downloaded (before any side
        measurement reuses the buffers)."""
        w = self.w
        shape = (w.pool_blocks, w.kv_heads, w.block_size, w.head_dim)
        dt = np.uint16 if w.kv_dtype == self.ehip.KV_BF16 else np.float32
        ks, vs = self.slabs[0]
        self.layer0["k_dev"] = ks.download(dt, shape)
        self.layer0["v_dev"] = vs.download(dt, shape)
        self.layer0["out"] = self.outs[0].download(np.float32, (w.rows, w.heads, w.head_dim))

    def free(self):
        for b in [x for pair in self.slabs for x in pair] + self.qs + self.kns + self.vns + \
                self.outs + [x for pair in self.scales for x in pair]:
            b.free()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the per-GPU throughput at N=1 is the figure it reports", file=sys.stderr)
        sys.exit(2)
    import ehip
    from ehip import workloads

    make = workloads.CONFIGS[args.config]
    w = make(seed=args.seed) if args.seed else make()
    q8 = args.kv if args.kv in ("int8", "fp8") else ""
    if q8:
        w.kv_dtype = ehip.KV_FP8 if q8 == "fp8" else ehip.KV_INT8
    layers = args.layers or w.layers
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    tok = int(w.context_lens.sum())
    draw = {"seed": w.seed, "sum_context": tok}
    seeds = [w.seed]
    if w.name == "C4":
        mean, sd = workloads.c4_sum_context_stats(w.num_seqs)
        draw.update(expected_sum_context=round(mean), sd=round(sd), z=round((tok - mean) / sd, 3))
        if abs(tok - mean) > sd:  # an atypical draw: report the median of three seeds
            seeds = [w.seed, w.seed + 1, w.seed + 2]
    log(f"[bench] {w.name}: B={w.num_seqs} rows={w.rows} sumL={tok} pool={w.pool_blocks} blocks, "
        f"{layers} layers, draw {draw}")

    ctx = ehip.Context(0)
    if args.copy_probe_mib:
        nbytes = args.copy_probe_mib << 20
        a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
        ctx._check(ehip.lib().ehip_copy_device(ctx.h, b.ptr, a.ptr, nbytes))
        ctx.sync()
        a.free()
        b.free()
        log(f"[bench] copy probe: {nbytes} bytes device-to-device")
    want_cpu = not args.no_cpu_baseline and not q8
    bench = Bench(ctx, ehip, w, layers, q8, host_layer0=want_cpu)
    log(f"[bench] pools resident ({2 * layers * bench.slab_bytes / 2**30:.1f} GiB of slabs)")

    per_step, attn, wall = bench.time_steps(args.steps, args.warmup)
    rows, items, partials = ctx.step_info()
    log(f"[bench] timed {args.steps} steps: wall {wall * 1e3:.2f} ms, step median "
        f"{np.median(per_step) * 1e3:.3f} ms, mean {per_step.mean() * 1e3:.3f} ms")
    qs = np.percentile(attn * 1e6, [0, 10, 50, 90, 100])
    log("[bench] attention us per launch: min %.1f p10 %.1f p50 %.1f p90 %.1f max %.1f" % tuple(qs))
    per_layer = w.bytes_per_layer(with_append=True)
    step_bytes = per_layer["total"] * layers
    runs = [{"seed": w.seed, "sum_context": tok, "ms_per_step": float(np.median(per_step)) * 1e3,
             "gbps": step_bytes / float(np.median(per_step)) / 1e9}]
    if bench.layer0 is not None:
        bench.capture_layer0()

    graph_info = None
    if args.graph:
        # The per-layer launches of the uploaded step, captured once and
        # replayed per step (the step's plan is the same every step here); the
        # descriptor upload stays eager.
        from ehip import hipgraph
        gs = hipgraph.Stream()
        ctx._check(ehip.lib().ehip_set_stream(ctx.h, gs.h))
        ctx._check(ctx.step_upload(bench.geom, bench.st))
        ctx.sync()
        graph = hipgraph.Graph()

        def layer_launches():
            for layer in range(layers):
                ks, vs = bench.slabs[layer]
                ctx._check(ctx.step_append_attention(bench.kns[layer], bench.vns[layer],
                                                     bench.qs[layer], ks, vs, bench.outs[layer]))

        graph.capture(gs, layer_launches)
        for _ in range(args.warmup):
            ctx._check(ctx.step_upload(bench.geom, bench.st))
            graph.replay(gs)
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            ctx._check(ctx.step_upload(bench.geom, bench.st))
            graph.replay(gs)
        ctx.sync()
        t_graph = (time.perf_counter() - t0) / args.steps
        log(f"[bench] graph replay: {t_graph * 1e3:.3f} ms/step")
        graph_info = {"eager_ms_per_step_median": round(runs[0]["ms_per_step"], 4),
                      "graph_ms_per_step": round(t_graph * 1e3, 4)}
        ctx._check(ehip.lib().ehip_set_stream(ctx.h, None))
        graph.close()
        gs.close()

    result_extra = {}
    if not args.no_ceiling_probe:
        result_extra["ceiling"] = ceiling_probe(w, bench.slabs[0], bench.slab_bytes)
        log(f"[bench] read ceiling: {result_extra['ceiling']}")
    # The chunk, fused-RoPE and re-prefill measurements run the fp32/bf16
    # entry points; an INT8 run reports the decode step alone.
    if not q8 and not args.no_extras:
        pre = time_chunks(ctx, ehip, w, bench.slabs, bench.qs, bench.outs, layers)
        if pre is not None:
            result_extra["prefill"] = pre
            log(f"[bench] prefill chunks: {pre['us_per_layer']} us/layer, {pre['tflops']} TFLOP/s")
        ra = time_rope_append(ctx, ehip, w, bench.slabs, bench.qs, bench.kns, bench.vns, layers)
        result_extra["rope_append"] = ra
        log(f"[bench] fused RoPE + append: {ra}")
        op = time_o_proj(ctx, ehip, w, bench.outs, layers)
        result_extra["o_proj"] = op
        log(f"[bench] o_proj: {op['us_per_launch']} us/launch, {op['tflops']} TFLOP/s, "
            f"weights {op['weight_gbps']} GB/s")
        if w.name == "C5":
            ev = c5_reprefill(ctx, ehip, w, bench.slabs, layers)
            result_extra["reprefill_event"] = ev
            # One 4096-token re-prefill every 50 decode steps, amortised per step.
            result_extra["ms_per_step_with_reprefill"] = round(runs[0]["ms_per_step"] +
                                                               ev["event_ms"] / 50, 4)
            log(f"[bench] C5 re-prefill: {ev['us_per_layer']} us/layer, {ev['tflops']} TFLOP/s")
    layer0 = bench.layer0
    bench.free()

    # Further seeds of an atypical draw (timing only).
    for seed in seeds[1:]:
        wx = make(seed=seed)
        bx = Bench(ctx, ehip, wx, layers, q8, host_layer0=False)
        ps, _, _ = bx.time_steps(args.steps, args.warmup)
        bx.free()
        bx_bytes = wx.bytes_per_layer(with_append=True)["total"] * layers
        runs.append({"seed": seed, "sum_context": int(wx.context_lens.sum()),
                     "ms_per_step": float(np.median(ps)) * 1e3,
                     "gbps": bx_bytes / float(np.median(ps)) / 1e9})
        log(f"[bench] seed {seed}: {runs[-1]}")
    headline = sorted(runs, key=lambda r: r["gbps"])[len(runs) // 2]

    t_step = float(np.median(per_step))
    # The timed call is the layer's append + attention: its algorithmic bytes
    # include the append's (fp32 rows read, slab rows written).
    attn_bytes = per_layer["total"]
    attn_avg = float(attn.mean())
    achieved = attn_bytes / attn_avg / 1e9
    tr = traffic_from_profiles(w.name, q8)
    traffic = tr[0] if tr is not None and tr[1] == tok else None  # measured on this draw

    result = {
        "metric": "ragged paged-attn decode: HBM GB/s (% of 8 TB/s) + attended KV tok/s per step",
        "value": round(headline["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(headline["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic: structure from the config's seeded mt19937_64 draw; layer 0 "
                 "values from the reference fill_normal streams, other layers from a device "
                 "generator of the same N(0, std)"),
        "config": {
            "workload": (f"{w.name}: {w.num_seqs} sequences, {layers} layers, H={H} Hkv={Hkv} "
                         f"d={d} bs={bs}, kv {KV_NAMES[w.kv_dtype]}, sum L={tok}, "
                         f"rows={w.rows}"),
            "kv_dtype": KV_NAMES[w.kv_dtype],
            "num_seqs": w.num_seqs, "layers": layers, "sum_context": tok,
            "draw": draw, "work_items": items, "split_partials": partials,
            "parallelism": "single GPU",
        },
        "step_time": {"median_ms": round(t_step * 1e3, 4),
                      "mean_ms": round(float(per_step.mean()) * 1e3, 4),
                      "min_ms": round(float(per_step.min()) * 1e3, 4),
                      "max_ms": round(float(per_step.max()) * 1e3, 4),
                      "wall_ms_per_step": round(wall / args.steps * 1e3, 4)},
        "hbm_frac": round(headline["gbps"] / HBM_PEAK_GBS, 4),
        "attended_kv_tok_per_s": round(headline["sum_context"] * layers /
                                       (headline["ms_per_step"] / 1e3), 1),
        "bytes_per_step": step_bytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "the layer's append + paged decode attention call (decode kernel with "
                      "the append fused for all-decode steps on the matrix-core kernel, + split merge)",
            "algorithmic_bytes_per_launch": attn_bytes,
            "avg_launch_us": round(attn_avg * 1e6, 3),
            "launches_timed": int(attn.size),
            "timed_steps_sampled": int(attn.shape[0]),
        },
    }
    if len(runs) > 1:
        result["seeds"] = runs
    if graph_info is not None:
        result["launch"] = dict(graph_info, mode="captured graph of the per-layer launches")
    result.update(result_extra)
    if want_cpu and layer0 is not None:
        log("[bench] cpu baseline + parity ...")
        base, par = cpu_baseline_and_parity(w, layer0, args.cpu_seconds)
        result["cpu_baseline"] = base
        result["parity"] = par
        log(f"[bench] parity: {par}")
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
