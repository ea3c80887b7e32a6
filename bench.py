"""Benchmark of the MI355X prefill->decode cache handoff (one JSON line on stdout).

Headline (`value`): device-side fused carve -> scatter of config 3 - a 48-layer hybrid at 131072 tokens (12 QSA
layers of K/V [131072][2][256] f16, 36 GDN layers of (128, 32, 128) f32 recurrence + [8192][3] f32 history,
P = 3 300 261 888 bytes) - from the prefill layout into one decode slot, inputs resident in HBM.  One step = one
handoff = one launch of the move kernel.  value = P / step time (GB/s).

Also reported: the roofline of that kernel (2P algorithmic HBM bytes per launch over its event-timed duration,
against MI355X's 8 TB/s), the p50 latency of the 32K handoff (config 2, first enqueue to completion event, over
>= 20 repetitions) and of the 32K park + resume through pinned host memory (host wall clock and device events), the
two-pass gather -> scatter rate, park (D2H) and resume (H2D) of the 128K slot (p50 of 20) against a probe of the host
link at the same transfer size, the device payload codec, the hand-off arena (payload published from HBM into a
tmpfs slot and read back, against the host link), the same-GPU hand-off between processes (exported device segments),
the quantizing carve, configs 4 and 5, and the CPU baselines: the oracle's single-core carve of a bounded sample of
the same workload, plus the reference-style host pipeline (16 MiB segment save, FNV-1a encode, decode + re-hash,
restore); for the codec and arena rows the reference's own codec and arena, compiled from its sources.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "strata-concurrent_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "handoff GB/s (HBM + host park/resume) and p50 handoff latency at 32K ctx"
PMC_SUMMARY = ROOT / "profiles" / "sc_move_kernel_fused_carve_128k_pmc.md"


def measured_traffic() -> int | None:
    """HBM bytes per launch of the fused 128K carve from the committed FETCH_SIZE / WRITE_SIZE counter runs (each
    scaled by what the counter reads for a plain copy of known size), or None when no summary is committed."""
    try:
        for line in PMC_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None
HBM_PEAK_GBPS = 8000.0
# BASELINE.json's model geometry (the headline's slot) and the 18 geometry fields its wire payloads carry
HEADLINE_GEO = dict(n_layers=48, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=128,
                    ssm_k_heads=16, ssm_v_heads=32, ssm_d_conv=4, ssm_conv_channels=8192, idx_key_dim=128)
WIRE_GEOKEY = [2560, 48, 4, 128, 16, 32, 4, 8192, 4096, 24, 2, 256, 128, 4, 4, 3, 1, 0]


def synth():
    """The seeded synthetic workloads (imported once the device library is known to load)."""
    import sc_synthetic
    return sc_synthetic
# PCIe Gen5 x16, one direction: 32 GT/s x 16 lanes x 128/130 line coding / 8 bits (before packet overheads)
PCIE5_X16_GBPS = 32.0 * 16 * 128 / 130 / 8
REF_BIN = ROOT / "oracle" / "_ref"


def spread(ms: list[float]) -> dict:
    """p50 / p90 / min of a list of timings in ms, with the repetition count."""
    xs = sorted(ms)
    return {"p50_ms": round(xs[len(xs) // 2], 4), "p90_ms": round(xs[min(len(xs) - 1, int(len(xs) * 0.9))], 4),
            "min_ms": round(xs[0], 4), "reps": len(xs)}


def link_at(sc, dev_ptr: int, host_ptr: int, n: int, reps: int = 3) -> tuple[float, float]:
    """The host link at one transfer size: p50 GB/s of `reps` plain pinned copies of n bytes each way (one
    hipMemcpyAsync each, event-timed on a side stream), so a row's fraction of the link compares transfers of the
    same size."""
    st = sc.Stream()
    e0, e1 = sc.Event(), sc.Event()
    out = []
    for dst, src in ((dev_ptr, host_ptr), (host_ptr, dev_ptr)):
        sc.check(sc.lib.sc_copy_async(dst, src, n, st.handle), "link probe")   # warm-up
        ms = []
        for _ in range(reps):
            e0.record(st)
            sc.check(sc.lib.sc_copy_async(dst, src, n, st.handle), "link probe")
            e1.record(st)
            e1.sync()
            ms.append(e0.elapsed_ms(e1))
        out.append(n / (sorted(ms)[len(ms) // 2] * 1e-3) / 1e9)
    return out[0], out[1]


def link_fracs(gbps: float, probe: float, small_probe: float | None = None) -> dict:
    """A host-link rate against the same-size probe, the 256 MiB probe (when given) and the PCIe Gen5 x16 line rate."""
    out = {"frac_of_probe": round(gbps / probe, 3)}
    if small_probe:
        out["frac_of_small_probe"] = round(gbps / small_probe, 3)
    out["frac_of_pcie5_x16"] = round(gbps / PCIE5_X16_GBPS, 3)
    return out


def settle_link(sc, floor_gbps: float, limit_s: float = 3.0) -> float:
    """Waits until a 64 MiB pinned D2H copy runs at >= 97% of `floor_gbps` again and returns the wait in ms.

    Device memory this process frees is wiped by the driver on the same copy engines that carry the host link: right
    after a row frees a few GB, parks and resumes run at about half the link rate for up to half a second (measured:
    30 GB/s right after freeing 3.3 GB of pools, 57 GB/s again after ~0.5 s).  A serving process keeps its pools,
    so each host-link row starts once the link is back to its rate; the wait is reported beside the row."""
    n = 64 << 20
    host, dev = sc.PinnedBuffer(n), sc.DeviceBuffer(n, "uint8")
    st = sc.Stream()
    e0, e1 = sc.Event(), sc.Event()
    t0 = time.perf_counter()
    while True:
        e0.record(st)
        sc.check(sc.lib.sc_copy_async(host.ptr, dev.ptr, n, st.handle), "settle copy")
        e1.record(st)
        e1.sync()
        if n / (e0.elapsed_ms(e1) * 1e-3) / 1e9 >= 0.97 * floor_gbps or time.perf_counter() - t0 > limit_s:
            break
    host.free()
    dev.free()
    return round((time.perf_counter() - t0) * 1e3, 1)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_launches(plan, stream, steps: int, warmup: int, sc) -> tuple[float, list[float]]:
    """Warm up, then time exactly `steps` launches: total wall (ms) bracketed by synchronizes, and per-launch
    durations from event pairs recorded on the launch stream."""
    for _ in range(warmup):
        plan.launch(stream)
    sc.device_sync()
    starts = [sc.Event() for _ in range(steps)]
    ends = [sc.Event() for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        plan.launch(stream)
        ends[i].record(stream)
    sc.device_sync()
    wall_ms = (time.perf_counter() - t0) * 1e3
    per = [s.elapsed_ms(e) for s, e in zip(starts, ends)]
    return wall_ms, per


def trace_summary(path: str, kernel: str, warmup: int, steps: int, payload_bytes: int) -> dict:
    """The headline launches in a rocprofv3 kernel trace (its *_kernel_trace.csv) of `bench.py --kernel-only`: the
    first warmup + steps dispatches of `kernel` in start order are the bench's warm-up and timed launches; each part's
    mean / p50 / min / max duration and the roofline fraction 2P / mean of the timed ones, the statistic the line's
    roofline reports from HIP events."""
    import csv
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    ds = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-6 for r in rows if kernel in r["Kernel_Name"]]
    if len(ds) < warmup + steps:
        raise SystemExit(f"{path}: {len(ds)} dispatches of {kernel}, fewer than {warmup} + {steps}")

    def stats(xs):
        ys = sorted(xs)
        mean = sum(xs) / len(xs)
        return {"n": len(xs), "mean_ms": round(mean, 4), "p50_ms": round(ys[len(ys) // 2], 4),
                "min_ms": round(ys[0], 4), "max_ms": round(ys[-1], 4)}
    timed = stats(ds[warmup:warmup + steps])
    return {"kernel": kernel, "dispatches": len(ds), "warmup": stats(ds[:warmup]) if warmup else None, "timed": timed,
            "all": stats(ds),
            "frac_timed_mean": round(2 * payload_bytes / (timed["mean_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}


def retarget_latency(sc, geo, tokens: int, case, slot, plan, stream, reps: int) -> dict:
    """A serving engine's hand-off at 32K with one plan per decode slot: the plan re-pointed at the next prefill
    sequence (sc_plan_retarget) and launched, host wall clock from before the retarget to the completion event's sync,
    alternating between two sequences; beside the bare launch of an already-targeted plan and a plan built per hand-off
    (sc_plan_carve + launch + destroy), timed the same way.  Every wall time includes the host's enqueue and wait."""
    import ctypes as C
    other = synth().SyntheticCase(geo, tokens=tokens, seed=0x5EED + 7)
    views = [case.prefill.view(0, True), other.prefill.view(0, True)]   # built once: the library call is timed
    done = sc.Event()
    for k in range(4):   # warm-up of every path
        sc.check(sc.lib.sc_plan_retarget(plan.handle, C.byref(views[k % 2][0]), stream.handle), "retarget")
        plan.launch(stream)
    stream.sync()

    def timed(body) -> list[float]:
        out = []
        for k in range(reps):
            t0 = time.perf_counter()
            body(k)
            done.record(stream)
            done.sync()
            out.append((time.perf_counter() - t0) * 1e3)
        return out

    def retarget_launch(k):
        sc.check(sc.lib.sc_plan_retarget(plan.handle, C.byref(views[k % 2][0]), stream.handle), "retarget")
        plan.launch(stream)

    def build_launch(k):
        cs = slot.c_struct()
        h = C.c_void_p()
        sc.check(sc.lib.sc_plan_carve(C.byref(geo), C.byref(views[k % 2][0]), C.byref(cs), C.byref(h)), "build")
        sc.check(sc.lib.sc_plan_launch(h.value, stream.handle), "launch")
        done.record(stream)
        done.sync()
        sc.check(sc.lib.sc_plan_destroy(h.value), "destroy")

    ra = timed(retarget_launch)
    # the bare launch of the plan as last targeted, and a plan built for every hand-off
    bare = timed(lambda k: plan.launch(stream))
    build = timed(build_launch)
    plan.retarget(other.prefill, stream=stream)
    plan.launch(stream)
    stream.sync()
    ref = sc.new_slot(geo, tokens, fill=0)
    other_plan = sc.plan_carve(geo, other.prefill, ref)
    other_plan.launch(stream)
    stream.sync()
    exact = all(sc.fnv1a64_device(x.ptr, x.nbytes) == sc.fnv1a64_device(y.ptr, y.nbytes)
                for x, y in zip(slot.buffers(), ref.buffers()))
    other_plan.destroy()
    for b in ref.buffers():
        b.free()
    r, b, c = spread(ra), spread(bare), spread(build)
    return {"tokens": tokens, "retarget_launch": r, "bare_launch": b, "build_launch": c,
            "retarget_overhead_p50_ms": round(r["p50_ms"] - b["p50_ms"], 4),
            "retargeted_equals_fresh_plan": bool(exact),
            "method": "host wall clock from before the call to the completion event's sync, p50 over the reps; "
                      "retarget_launch alternates between two 32K prefill sequences; build_launch builds, launches "
                      "and destroys a plan per hand-off (device allocations and blocking uploads included)"}


def cpu_baseline(geo_kw: dict, tokens: int, budget_s: float) -> dict:
    """The oracle's carve on one core over a bounded sample of config 3: 1 QSA layer + 3 GDN layers (the 1:3 mix of
    the full model) at the full 131072 tokens, repeated until `budget_s` of CPU time; then the reference-style host
    pipeline over the same sample's image."""
    import numpy as np
    from oracle import sc_oracle as oracle

    sample_kw = dict(geo_kw, n_layers=4)
    g = oracle.Geometry(**sample_kw)
    H, D, S, HV, Cc = g.n_head_kv, g.head_dim, g.ssm_state_size, g.ssm_v_heads, g.ssm_conv_channels
    seed = 0x5EED
    k = oracle.fill_uniform_f16(tokens * H * D, -4.0, 4.0, seed, 1000).reshape(tokens, H, D)
    v = oracle.fill_uniform_f16(tokens * H * D, -4.0, 4.0, seed, 1001).reshape(tokens, H, D)
    recs = [oracle.fill_normal_f32(HV * S * S, seed, 5000 + i).reshape(HV, S, S) for i in range(3)]
    convs = [oracle.fill_normal_f32(3 * Cc, seed, 9000 + i).reshape(3, Cc) for i in range(3)]
    inputs = {"tokens": tokens, "k": [k], "v": [v], "rec": recs, "conv": convs, "conv_rows": 3}
    _, sample_bytes = oracle.image_layout(g, tokens)
    n_pages = tokens // g.page_size
    state = oracle.new_state(g, n_pages)
    oracle.carve_into(g, inputs, state, n_pages)    # touch every destination page before timing
    reps, t_carve = 0, 0.0
    while t_carve < budget_s * 0.5 or reps < 1:
        t0 = time.perf_counter()
        oracle.carve_into(g, inputs, state, n_pages)
        t_carve += time.perf_counter() - t0
        reps += 1
    image = oracle.park(g, tokens, state)
    dst = np.zeros_like(image)
    scratch = np.zeros(3 * image.size, dtype=np.uint8)
    oracle.cpu_handoff(image, dst, scratch)          # touch every page of the buffers before timing
    preps, t_pipe = 0, 0.0
    while t_pipe < budget_s * 0.5 or preps < 1:
        t0 = time.perf_counter()
        oracle.cpu_handoff(image, dst, scratch)
        t_pipe += time.perf_counter() - t0
        preps += 1
    # labelled, not the reference: the same image copied by N host threads (the box's CPU share), the host's plain
    # copy ceiling that any CPU implementation of the path sits under
    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.memcpy_threads(image, dst, threads)
    mreps, t_mem = 0, 0.0
    while t_mem < 0.5 or mreps < 3:
        t0 = time.perf_counter()
        oracle.memcpy_threads(image, dst, threads)
        t_mem += time.perf_counter() - t0
        mreps += 1
    carve_gbps = sample_bytes * reps / t_carve / 1e9
    return {
        "value": round(carve_gbps, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": (f"oracle carve (sco_handoff_carve, 1 thread) of 1 QSA + 3 GDN layers of config 3 at {tokens} tokens "
                   f"({sample_bytes} B) x {reps} reps in {t_carve:.2f} s"),
        "pipeline_gbps": round(sample_bytes * preps / t_pipe / 1e9, 3),
        "pipeline": ("reference-style host handoff of the same image: 16 MiB segment save, FNV-1a encode, decode + "
                     f"re-hash, restore; {preps} reps in {t_pipe:.2f} s, 1 thread"),
        "memcpy_ncore_gbps": round(sample_bytes * mreps / t_mem / 1e9, 2),
        "memcpy_ncore": (f"NOT the reference: memcpy of the same image by {threads} threads, one share each, "
                         f"{mreps} reps in {t_mem:.2f} s (the host's copy ceiling)"),
        "cpu": cpu_model(), "nproc": os.cpu_count(),
    }


def config4(sc, geo, seed: int, link_gbps: float, streams=None) -> dict:
    """Config 3 slots: contexts 8K / 32K / 96K assigned to roles from `seed`.  One slot keeps decoding (a synthetic
    decode step reads all of its K/V) on its own stream; the other two park to pinned host memory on a park stream;
    the first parked one is resumed into a fresh slot on a resume stream as soon as its park lands, overlapping the
    second park (the link is full duplex).  Checks the round trip bit for bit and reports rates against the link."""
    import numpy as np
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.permutation([8192, 32768, 98304])]
    decode_len, park_a, park_b = lens
    cases = {L: synth().SyntheticCase(geo, L, seed + L) for L in lens}
    slots = {L: cases[L].new_slot(max_cells=L) for L in lens}
    for L in lens:
        cases[L].carve_into(slots[L])
    del cases
    images = {L: sc.PinnedBuffer(sc.image_layout(geo, L)[1]) for L in (park_a, park_b)}
    for L in (park_a, park_b):   # touch the pinned pages once
        sc.park_async(geo, slots[L], L, images[L].ptr, images[L].nbytes)
    restored = sc.new_slot(geo, park_a, fill=0)
    sink = sc.DeviceBuffer(4096, "uint32")
    sc.device_sync()
    # the warm-up left correct bytes in the images: poison them, so a resume that read an image before the timed
    # park had landed would restore the poison and fail the round-trip check below
    for im in images.values():
        im.numpy()[:] = 0xEE
    decode, park, resume = streams if streams is not None else (sc.Stream(), sc.Stream(), sc.Stream())
    pools = slots[decode_len].k_pool + slots[decode_len].v_pool

    def decode_step():
        for b in pools:
            sc.check(sc.lib.sc_decode_probe(b.ptr, b.nbytes, sink.ptr, 4096, decode.handle), "decode probe")

    # decode alone
    e0, e1 = sc.Event(), sc.Event()
    for _ in range(3):
        decode_step()
    decode.sync()
    e0.record(decode)
    for _ in range(20):
        decode_step()
    e1.record(decode)
    e1.sync()
    alone_ms = e0.elapsed_ms(e1) / 20
    # enough decode steps to outlast the two parks at the link rate measured in this run
    est_ms = (images[park_a].nbytes + images[park_b].nbytes) / (link_gbps * 1e9) * 1e3
    decode_steps = max(20, int(1.5 * est_ms / alone_ms))
    # the overlapped window: decode keeps running while two parks and one resume move over the link
    d0, d1 = sc.Event(), sc.Event()
    p0, pa, pb, r0, r1 = sc.Event(), sc.Event(), sc.Event(), sc.Event(), sc.Event()
    d0.record(decode)
    for _ in range(decode_steps):
        decode_step()
    d1.record(decode)
    p0.record(park)
    sc.park_async(geo, slots[park_a], park_a, images[park_a].ptr, images[park_a].nbytes, stream=park, done=pa.handle)
    sc.park_async(geo, slots[park_b], park_b, images[park_b].ptr, images[park_b].nbytes, stream=park, done=pb.handle)
    resume.wait(pa)
    r0.record(resume)
    sc.resume_async(geo, images[park_a].ptr, images[park_a].nbytes, park_a, restored, stream=resume, done=r1.handle)
    d1.sync()
    pb.sync()
    r1.sync()
    window_ms = p0.elapsed_ms(pb) if p0.elapsed_ms(pb) > p0.elapsed_ms(r1) else p0.elapsed_ms(r1)
    decode_ms = d0.elapsed_ms(d1) / decode_steps
    bytes_a, bytes_b = images[park_a].nbytes, images[park_b].nbytes
    park_ms = p0.elapsed_ms(pb)
    resume_ms = r0.elapsed_ms(r1)
    # bit-exact round trip: the restored slot equals the parked one, the images equal the slots
    ok = True
    for a, b in zip(slots[park_a].buffers(), restored.buffers()):
        ok &= bool(np.array_equal(a.numpy().view(np.uint8), b.numpy().view(np.uint8)))
    for L in (park_a, park_b):
        _, total = sc.image_layout(geo, L)
        dev = sc.DeviceBuffer(total, "uint8")
        cap = sc.plan_capture(geo, slots[L], L, dev.ptr, total)
        cap.launch()
        sc.device_sync()
        ok &= bool(np.array_equal(dev.numpy(total), images[L].numpy()))
        dev.free()
    for im in images.values():
        im.free()
    return {"lens": {"decode": decode_len, "park": [park_a, park_b], "resume": park_a},
            "park_bytes": bytes_a + bytes_b, "resume_bytes": bytes_a,
            "park_ms": round(park_ms, 3), "park_gbps": round((bytes_a + bytes_b) / (park_ms * 1e-3) / 1e9, 2),
            "resume_ms": round(resume_ms, 3), "resume_gbps": round(bytes_a / (resume_ms * 1e-3) / 1e9, 2),
            "window_ms": round(window_ms, 3),
            "decode_steps": decode_steps,
            "decode_step_alone_ms": round(alone_ms, 4), "decode_step_during_ms": round(decode_ms, 4),
            "decode_slowdown": round(decode_ms / alone_ms, 3), "round_trip_bit_exact": ok,
            "streams": "decode, park and resume on three non-blocking streams at the default priority"}


def config5(sc, geo, seed: int, fragmented: bool = True) -> dict:
    """Config 5: 8 slots, L_i ~ U[1K, 128K] from `seed`: batched resume of the parked prefixes (one H2D per slot into
    a staging buffer) plus a fresh 2K-token chunk per slot, all scattered into the shared-arena decode layout by one
    launch whose ragged offsets come from a device-side scan."""
    import numpy as np
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(1024, 131072 + 1, size=8)]
    chunk = 2048
    case = synth().BatchCase(geo, lens, chunk, seed=seed, fragmented=fragmented)
    plan = case.plan()
    side = sc.Stream()
    case.stage(side)   # warm-up of the link and of the pinned pages
    plan.launch(side)
    side.sync()
    s0, s1, k1 = sc.Event(), sc.Event(), sc.Event()
    stage_ms, launch_ms = [], []
    for _ in range(5):
        s0.record(side)
        case.stage(side)
        s1.record(side)
        plan.launch(side)
        k1.record(side)
        k1.sync()
        stage_ms.append(s0.elapsed_ms(s1))
        launch_ms.append(s1.elapsed_ms(k1))
    parked = case.parked_bytes
    kv_chunk = len(lens) * chunk * geo.n_head_kv * geo.head_dim * 2 * 2 * geo.n_qsa
    moved = parked + kv_chunk
    st, ln = sorted(stage_ms)[2], sorted(launch_ms)[2]
    ok = list(case.lens_out.numpy()) == [L + chunk for L in lens]
    case.free()
    return {"lens": lens, "chunk_tokens": chunk, "parked_bytes": parked, "chunk_kv_bytes": kv_chunk,
            "resume_h2d_ms": round(st, 3), "resume_h2d_gbps": round(parked / (st * 1e-3) / 1e9, 2),
            "scatter_launch_ms": round(ln, 4), "scatter_hbm_gbps": round(2 * moved / (ln * 1e-3) / 1e9, 1),
            "scatter_frac": round(2 * moved / (ln * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "total_ms": round(st + ln, 3), "lens_out_ok": ok,
            "method": "p50 of 5; the launch (events around it) is the pre-pass (slot scan, inverse arena table, "
                      "count, compaction: four small kernels) and the move; the arena is one random permutation of "
                      "its pages over all slots (a fragmented allocator)"}


def paged_carve(sc, geo, case, tokens: int, stream) -> dict:
    """The config-3 carve into a slot whose pages go through a shuffled page table per QSA layer, in destination order
    (the library default) and in source order."""
    import numpy as np
    P = sc.payload_bytes(geo, tokens)
    n_pages = (tokens + geo.page_size - 1) // geo.page_size
    tables = sc.device_tables([np.random.default_rng(j).permutation(n_pages).astype(np.int32)
                               for j in range(geo.n_qsa)])
    paged_slot = case.new_slot(max_cells=tokens, tables=tables)
    paged = sc.plan_carve(geo, case.prefill, paged_slot)
    _, per_paged = time_launches(paged, stream, 10, 2, sc)
    paged_ms = sorted(per_paged)[len(per_paged) // 2]
    prev = sc.set_order_min_pages(0)
    source_order = sc.plan_carve(geo, case.prefill, paged_slot)
    sc.set_order_min_pages(prev)
    _, per_src = time_launches(source_order, stream, 10, 2, sc)
    src_ms = sorted(per_src)[len(per_src) // 2]
    out = {"ms": round(paged_ms, 4), "hbm_gbps": round(2 * P / (paged_ms * 1e-3) / 1e9, 1),
           "frac": round(2 * P / (paged_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
           "ordered_tables": paged.order_groups,
           "source_order_ms": round(src_ms, 4),
           "source_order_frac": round(2 * P / (src_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
           "table": "a random permutation of the pool's pages per QSA layer",
           "method": "p50 of 10 launches, events around each, which includes the destination-order pre-pass (three "
                     "small kernels) before the move kernel"}
    source_order.destroy()
    paged.destroy()
    # park and resume of the paged slot itself: its pages go through the tables straight to and from pinned memory
    _, total = sc.image_layout(geo, tokens)
    host = sc.PinnedBuffer(total)
    dev = sc.DeviceBuffer(total, "uint8")
    side = sc.Stream()
    sc.park_async(geo, paged_slot, tokens, host.ptr, total, stream=side)   # warm-up: touch the pinned pages
    side.sync()
    probe_h2d, probe_d2h = link_at(sc, dev.ptr, host.ptr, total)
    dev.free()
    e0, e1 = sc.Event(), sc.Event()
    pk, rs = [], []
    for _ in range(5):
        e0.record(side)
        sc.park_async(geo, paged_slot, tokens, host.ptr, total, stream=side)
        e1.record(side)
        e1.sync()
        pk.append(e0.elapsed_ms(e1))
        e0.record(side)
        sc.resume_async(geo, host.ptr, total, tokens, paged_slot, stream=side)
        e1.record(side)
        e1.sync()
        rs.append(e0.elapsed_ms(e1))
    host.free()
    pk_ms, rs_ms = sorted(pk)[2], sorted(rs)[2]
    out["park_resume"] = {
        "bytes": total, "park_ms": round(pk_ms, 3), "resume_ms": round(rs_ms, 3),
        "park_gbps": round(total / (pk_ms * 1e-3) / 1e9, 2), "resume_gbps": round(total / (rs_ms * 1e-3) / 1e9, 2),
        "park_vs_link": link_fracs(total / (pk_ms * 1e-3) / 1e9, probe_d2h),
        "resume_vs_link": link_fracs(total / (rs_ms * 1e-3) / 1e9, probe_h2d),
        "method": "p50 of 5; sc_park_async / sc_resume_async of the paged slot: one kernel per 32 layers moves every "
                  "K/V page through its table straight between the pool and the pinned image, then one copy of the "
                  "GDN rows; the probe is a plain pinned copy of the same byte count"}
    for b in paged_slot.buffers():
        b.free()
    for t in tables:
        t.free()
    return out


def wire_payload(sc, geo, tokens: int, slot, link_h2d: float, link_d2h: float, reps: int = 5) -> dict:
    """The codec row: the slot written straight into a wire payload on the device (one launch gathering the slot and the
    staged head and hashing the whole payload with the parallel FNV-1a), mounted back (device hash check, one scatter launch), and the checked
    park / resume through pinned host memory.  Compared with the reference's host codec, whose byte-serial FNV-1a
    runs twice per handoff (encode, then the reader's check)."""
    import numpy as np
    import sc_wire
    ids = (np.arange(tokens, dtype=np.int64) % 151_000).astype(np.int32)
    live, keep = sc_wire.make_live(WIRE_GEOKEY, ids, layer_hi=48, idx_dim=128)
    enc = sc_wire.Encoder(geo, slot, tokens, live, 0x1122334455667788, 0x0AABBCCDDEEFF001)
    n = enc.bytes
    payload = sc.DeviceBuffer(n, "uint8")
    stream = sc.Stream()
    hp = sc.HashPlan(n)
    for _ in range(2):
        enc.encode(payload.ptr, n, stream)
    h = enc.hash()
    # a cold encode, as for a conversation's first hand-off: the encoder made (host) and its first encode until done
    # (the capture plan and hash map built on that call, then the launches)
    create_ms, first_ms = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        cold = sc_wire.Encoder(geo, slot, tokens, live, 0x1122334455667788, 0x0AABBCCDDEEFF001)
        t1 = time.perf_counter()
        cold.encode(payload.ptr, n, stream)
        assert cold.hash() == h
        t2 = time.perf_counter()
        create_ms.append((t1 - t0) * 1e3)
        first_ms.append((t2 - t1) * 1e3)
        cold.destroy()
    e0, e1 = sc.Event(), sc.Event()
    enc_ms, hash_ms = [], []
    for _ in range(2 * reps):
        e0.record(stream)
        enc.encode(payload.ptr, n, stream)
        e1.record(stream)
        e1.sync()
        enc_ms.append(e0.elapsed_ms(e1))
        e0.record(stream)
        hp.launch(payload.ptr, n, stream=stream)
        e1.record(stream)
        e1.sync()
        hash_ms.append(e0.elapsed_ms(e1))
    assert hp.result() == h
    dst = sc.new_slot(geo, tokens, fill=0)
    mount_ms, mount_dev_ms, open_ms, reopen_ms, scatter_ms = [], [], [], [], []
    dec = None
    for _ in range(2 * reps):
        # the first mount opens a decoder, later ones open it again for the next payload (its buffers and scatter
        # plan kept, as an engine holding one decoder per slot does)
        t0 = time.perf_counter()
        if dec is None:
            dec = sc_wire.Decoder(payload.ptr, n, geo, dst, payload_hash=h, check_hash=True)
        else:
            dec.reopen(payload.ptr, n, h)
        t1 = time.perf_counter()
        e0.record(stream)
        dec.restore(stream)
        e1.record(stream)
        mount_ms.append((time.perf_counter() - t1) * 1e3)
        e1.sync()
        mount_dev_ms.append(e0.elapsed_ms(e1))
        (reopen_ms if open_ms else open_ms).append((t1 - t0) * 1e3)
    dec.destroy()
    same = all(sc.fnv1a64_device(a.ptr, a.nbytes) == sc.fnv1a64_device(b.ptr, b.nbytes)
               for a, b in zip(slot.buffers(), dst.buffers()))
    # the same mount given the payload's carries (written by the encode beside the payload): the hash check starts
    # every 64 KiB from its carry instead of looking back across the payload
    carry = sc.DeviceBuffer(max(sc.carry_bytes(n), 1), "uint8")
    enc.set_carry(carry.ptr)
    enc.encode(payload.ptr, n, stream)
    assert enc.hash() == h
    enc.set_carry(None)
    mount_c_ms, mount_c_dev_ms = [], []
    dec = sc_wire.Decoder(payload.ptr, n, geo, dst, payload_hash=h, check_hash=True, carry=carry.ptr)
    for i in range(2 * reps):
        if i:
            dec.reopen(payload.ptr, n, h, carry=carry.ptr)
        t1 = time.perf_counter()
        e0.record(stream)
        dec.restore(stream)
        e1.record(stream)
        mount_c_ms.append((time.perf_counter() - t1) * 1e3)
        e1.sync()
        mount_c_dev_ms.append(e0.elapsed_ms(e1))
    dec.destroy()
    same = same and all(sc.fnv1a64_device(a.ptr, a.nbytes) == sc.fnv1a64_device(b.ptr, b.nbytes)
                        for a, b in zip(slot.buffers(), dst.buffers()))
    carry.free()
    # the bare scatter of the same blobs (no hash): the device mount is this plus the hash, with no round trip between
    # (from an unset transfer image into the mount's slot, which the checked resume below mounts again)
    _, total = sc.image_layout(geo, tokens)
    image = sc.DeviceBuffer(total, "uint8")
    plain = sc.plan_scatter(geo, image.ptr, total, tokens, dst)
    for _ in range(reps + 1):
        e0.record(stream)
        plain.launch(stream)
        e1.record(stream)
        e1.sync()
        scatter_ms.append(e0.elapsed_ms(e1))
    plain.destroy()
    image.free()
    # checked park: encode on the device, then one D2H of the payload on a second stream that starts as soon as the
    # payload bytes are in place, overlapping the hash; checked resume: the H2D in 64 MiB pieces, each piece hashed on
    # a second stream as soon as it lands (the running hash chained on the device), the hash compared, then the mount
    # (decoder open + one scatter launch, no second hash)
    host = sc.PinnedBuffer(n)
    sc.check(sc.lib.sc_copy_async(host.ptr, payload.ptr, n, stream.handle), "touch")   # touch the pinned pages once
    stream.sync()
    probe_h2d, probe_d2h = link_at(sc, payload.ptr, host.ptr, n)
    side, copy = sc.Stream(), sc.Stream()
    gathered, e2, landed = sc.Event(), sc.Event(), sc.Event()
    piece = 64 << 20
    park_ms, resume_ms = [], []
    for _ in range(reps):
        e0.record(side)
        enc.encode(payload.ptr, n, side, gathered=gathered)
        copy.wait(gathered)
        sc.check(sc.lib.sc_copy_async(host.ptr, payload.ptr, n, copy.handle), "park copy")
        e1.record(copy)
        e2.record(side)
        e1.sync()
        e2.sync()
        park_ms.append(max(e0.elapsed_ms(e1), e0.elapsed_ms(e2)))
        assert enc.hash() == h
        t0 = time.perf_counter()
        hp.start()
        for at in range(0, n, piece):
            k = min(piece, n - at)
            sc.check(sc.lib.sc_copy_async(payload.ptr + at, host.ptr + at, k, side.handle), "resume copy")
            landed.record(side)
            copy.wait(landed)
            hp.chain(payload.ptr + at, k, stream=copy)
        copy.sync()
        if hp.result() != h:
            raise RuntimeError("checked resume: the payload hash differs")
        dec = sc_wire.Decoder(payload.ptr, n, geo, dst, payload_hash=h, check_hash=False)
        dec.restore(side)
        resume_ms.append((time.perf_counter() - t0) * 1e3)
        dec.destroy()
    same = same and all(sc.fnv1a64_device(a.ptr, a.nbytes) == sc.fnv1a64_device(b.ptr, b.nbytes)
                        for a, b in zip(slot.buffers(), dst.buffers()))
    host.free()
    payload.free()
    hp.free()
    def p50(xs):
        return sorted(xs)[len(xs) // 2]
    enc_t, hash_t, mount_t = p50(enc_ms), p50(hash_ms), p50(mount_ms)
    pk, rs = p50(park_ms), p50(resume_ms)
    pk_gbps, rs_gbps = n / (pk * 1e-3) / 1e9, n / (rs * 1e-3) / 1e9
    return {"tokens": tokens, "payload_bytes": n, "pool_offset": enc.pool_offset,
            "encode_ms": round(enc_t, 3), "encode_gbps": round(n / (enc_t * 1e-3) / 1e9, 1),
            "encoder_create_ms": round(sorted(create_ms)[1], 3), "first_encode_ms": round(sorted(first_ms)[1], 3),
            "hash_ms": round(hash_t, 3), "hash_gbps": round(n / (hash_t * 1e-3) / 1e9, 1),
            "mount_ms": round(mount_t, 3), "mount_gbps": round(n / (mount_t * 1e-3) / 1e9, 1),
            "open_ms": round(p50(open_ms), 3), "reopen_ms": round(p50(reopen_ms), 3),
            "mount_carried_ms": round(p50(mount_c_ms), 3), "mount_carried_device_ms": round(p50(mount_c_dev_ms), 3),
            "mount_carried_gbps": round(n / (p50(mount_c_ms) * 1e-3) / 1e9, 1),
            "checked_park_ms": round(pk, 2), "checked_park_gbps": round(pk_gbps, 2),
            "checked_park_vs_link": link_fracs(pk_gbps, probe_d2h, link_d2h),
            "checked_resume_ms": round(rs, 2), "checked_resume_gbps": round(rs_gbps, 2),
            "checked_resume_vs_link": link_fracs(rs_gbps, probe_h2d, link_h2d),
            "link_probe_d2h_gbps": round(probe_d2h, 2), "link_probe_h2d_gbps": round(probe_h2d, 2),
            "round_trip_bit_exact": bool(same),
            "mount_device_ms": round(p50(mount_dev_ms), 3), "scatter_ms": round(p50(scatter_ms[1:]), 3),
            "timing": (f"p50 of {2 * reps} encodes, hashes and mounts and of {reps} checked parks and resumes; the "
                       "link probe is one plain pinned copy of the payload's size each way between the same buffers"),
            "method": "payload in the reference's wire format; encode = one launch that gathers the slot into the payload and hashes it from the same registers (FNV-1a), its copy rows writing the head from device staging (a warm encoder: plans and map built); "
                      "encoder_create_ms = sc_wire_encoder_create (host), first_encode_ms = a new encoder's first encode "
                      "until done (its capture plan and hash map built on that call), median of 3; "
                      "mount = device FNV-1a whose last kernel compares with the expected hash and leaves a verdict "
                      "word, then one scatter launch gated by it (all or nothing, no host round trip); mount_ms is the "
                      "host's wall time of the call, mount_device_ms the events around it; open_ms = the first "
                      "decoder open, reopen_ms = the same decoder opened again for the next payload "
                      "(sc_wire_decoder_reopen); park = encode with the "
                      "pinned D2H of the payload on a second stream overlapping the hash; resume = pinned H2D in 64 MiB "
                      "pieces, each hashed on a second stream as it lands (chained device FNV-1a), then the mount "
                      "without a second hash; mount_carried = the mount given the payload's carries (the low byte of "
                      "the running hash after every 64 KiB, written by the encode beside the payload): the same "
                      "verdict, every 64 KiB of the hash starting from its carry instead of looking back"}


def arena_dir(need: int) -> str:
    """/dev/shm when it has room for `need` bytes (the reference's default hand-off directory is a tmpfs), else the
    temp directory."""
    import os
    st = os.statvfs("/dev/shm") if os.path.isdir("/dev/shm") else None
    if st and st.f_bavail * st.f_frsize > need + (1 << 30):
        return "/dev/shm"
    return os.environ.get("TMPDIR", "/tmp")


def arena_handoff(sc, geo, tokens: int, slot, link_h2d: float, link_d2h: float, chunk_mib: int = 32, depth: int = 4,
                  threads: int = 8, reps: int = 5) -> dict:
    """The cross-process row: the 128K slot's payload written on the device, handed through a hand-off arena slot
    (the reference's HandoffArena file, same format) and mounted into a fresh slot.  Writer = device encode, then the
    mover (pinned DMA chunks copied into the slot's mapped window by host threads, device FNV-1a beside it) and publish;
    reader = the mover (slot -> pinned chunks -> HBM) and the device mount with its hash check.  Both directions are
    bounded by the host link; the reference moves the same payload with one pwrite and checks it with a byte-serial
    FNV-1a on the CPU."""
    import os
    import shutil
    import numpy as np
    import sc_arena
    import sc_wire
    geokey = [2560, 48, 4, 128, 16, 32, 4, 8192, 4096, 24, 2, 256, 128, 4, 4, 3, 1, 0]
    pack, geom = 0x0AABBCCDDEEFF001, 0x1122334455667788
    ids = (np.arange(tokens, dtype=np.int64) % 151_000).astype(np.int32)
    live, keep = sc_wire.make_live(geokey, ids, layer_hi=48, idx_dim=128)
    enc = sc_wire.Encoder(geo, slot, tokens, live, geom, pack)
    n = enc.bytes
    payload = sc.DeviceBuffer(n, "uint8")
    arrived = sc.DeviceBuffer(n, "uint8")
    stream = sc.Stream()
    enc.encode(payload.ptr, n, stream)
    h = enc.hash()
    # the link at the payload's size: plain pinned copies of n bytes each way
    probe_host = sc.PinnedBuffer(n)
    sc.check(sc.lib.sc_copy_async(probe_host.ptr, payload.ptr, n, stream.handle), "touch")
    stream.sync()
    probe_h2d, probe_d2h = link_at(sc, arrived.ptr, probe_host.ptr, n)
    probe_host.free()
    base = arena_dir(n + (64 << 20))
    d = os.path.join(base, f"sc-bench-arena-{os.getpid()}")
    path = os.path.join(d, "arena")
    out = {"tokens": tokens, "payload_bytes": n, "arena_dir": base, "chunk_mib": chunk_mib, "depth": depth,
           "threads": threads}
    try:
        mover = sc_arena.Mover(chunk_mib << 20, depth, threads)
        t0 = time.perf_counter()
        w = sc_arena.Arena.writer(path, [(tokens, 1)], [n], pack, geom, reserve=False)
        c = w.claim(0, 7, 1)
        mover.publish(w, c, payload.ptr, n, tokens, stream.handle)        # first hand-off: the slot's pages are new
        out["cold_publish_ms"] = round(mover.last()[1], 2)
        w.release(c.index, c.nonce)
        t0 = time.perf_counter()
        w.close()
        w = sc_arena.Arena.writer(path, [(tokens, 1)], [n], pack, geom, reserve=True)   # re-open: pages committed, mapped
        out["reserve_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
        r = sc_arena.Arena.reader(path, pack, geom)
        t0 = time.perf_counter()
        r.reserve()                                       # the reader's one mapping of the arena, populated
        out["reader_reserve_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
        dst = sc.new_slot(geo, tokens, fill=0)
        side, gathered = sc.Stream(), sc.Event()
        pub, mpub, rd, rdv, mnt, opn, rim, rim_mover = [], [], [], [], [], [], [], []
        for rep in range(reps):
            c = w.claim(0, 7, 2 + rep)
            t0 = time.perf_counter()
            # the mover's D2H starts once the gather has placed every payload byte; the encoder's FNV-1a (which is
            # the arena's payload hash: the same function and seed over the same bytes) runs beside it, so the
            # mover does not hash again and the arena publishes the encoder's hash
            enc.encode(payload.ptr, n, stream, gathered=gathered)
            side.wait(gathered)
            mover.write(w, c, payload.ptr, n, side.handle, want_hash=False)
            w.publish(c, tokens, n, enc.hash())
            pub.append((time.perf_counter() - t0) * 1e3)
            w.release(c.index, c.nonce)
            c = w.claim(0, 7, 2 + rep)
            stream.sync()                                   # the payload is in place: the mover alone
            t0 = time.perf_counter()
            mover.publish(w, c, payload.ptr, n, tokens, stream.handle)
            mpub.append((time.perf_counter() - t0) * 1e3)
            t0 = time.perf_counter()
            s = mover.read(r, c.index, c.nonce, 7, arrived.ptr, n, stream.handle, verify=True)
            t1 = time.perf_counter()
            rim_mover.append(mover.last()[1:])
            # the mover checked the bytes against the slot's payload hash as they landed: the mount does not hash again
            dec = sc_wire.Decoder(arrived.ptr, s.payload_bytes, geo, dst, payload_hash=s.payload_hash, check_hash=False)
            t2 = time.perf_counter()
            dec.restore(stream)
            mnt.append((time.perf_counter() - t0) * 1e3)
            opn.append((t2 - t1) * 1e3)
            rim.append((t1 - t0) * 1e3)
            dec.destroy()
            t0 = time.perf_counter()
            mover.read(r, c.index, c.nonce, 7, arrived.ptr, n, stream.handle, verify=False)
            rd.append((time.perf_counter() - t0) * 1e3)
            t0 = time.perf_counter()
            mover.read(r, c.index, c.nonce, 7, arrived.ptr, n, stream.handle, verify=True)
            rdv.append((time.perf_counter() - t0) * 1e3)
            w.release(c.index, c.nonce)
        same = all(sc.fnv1a64_device(a.ptr, a.nbytes) == sc.fnv1a64_device(b.ptr, b.nbytes)
                   for a, b in zip(slot.buffers(), dst.buffers()))
        assert s.payload_hash == h
        r.close()
        w.close()
        mover.destroy()
        for b in dst.buffers():
            b.free()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    payload.free()
    arrived.free()
    def p50(xs):
        return sorted(xs)[len(xs) // 2]
    p, q, qv, m, mp = p50(pub), p50(rd), p50(rdv), p50(mnt), p50(mpub)
    gb = lambda ms: round(n / (ms * 1e-3) / 1e9, 2)   # noqa: E731
    out.update({
        "publish_ms": round(p, 2), "publish_gbps": gb(p), "publish_vs_link": link_fracs(gb(p), probe_d2h, link_d2h),
        "mover_publish_ms": round(mp, 2), "mover_publish_gbps": gb(mp),
        "mover_publish_vs_link": link_fracs(gb(mp), probe_d2h, link_d2h),
        "read_ms": round(q, 2), "read_gbps": gb(q), "read_vs_link": link_fracs(gb(q), probe_h2d, link_h2d),
        "read_verified_ms": round(qv, 2), "read_verified_gbps": gb(qv),
        "read_verified_vs_link": link_fracs(gb(qv), probe_h2d, link_h2d),
        "read_and_mount_ms": round(m, 2), "read_and_mount_gbps": gb(m), "decoder_open_ms": round(p50(opn), 2),
        "read_before_mount_ms": round(p50(rim), 2),
        "link_probe_d2h_gbps": round(probe_d2h, 2), "link_probe_h2d_gbps": round(probe_h2d, 2),
        "read_before_mount_mover": [[round(x, 2) for x in t] for t in rim_mover],
        "round_trip_bit_exact": bool(same),
        "method": "publish = device encode, with the mover's D2H (pinned chunks, host threads copying each chunk "
                  "into the slot's mapped window while later chunks are in flight) starting once the gather has "
                  "placed the payload and the encoder's FNV-1a beside it, then the arena's publish with that hash; "
                  "mover_publish = the mover alone on an encoded payload (its own device FNV-1a on a side stream) + "
                  "the publish; read = mover (host threads copy slot chunks into pinned buffers, H2D of each "
                  "while the next is copied); read_verified adds the device FNV-1a check, each chunk hashed as it "
                  "lands with the running hash chained on the device; read_and_mount = verified read + decoder open + "
                  "one scatter launch; host wall clock around each call, p50 of the reps; the writer's "
                  "arena reserved (posix_fallocate + populated mapping) and the reader's mapping populated before the "
                  "timed reps"})
    return out


def wire_spec(geo, tokens: int) -> str:
    """The wire spec (the grammar of oracle/ref_wire_driver.cpp) of a slot's image at `tokens`: one f16 K/V record per
    QSA layer, the empty draft record, and the live checkpoint with the ids and the slot's GDN rows."""
    import sc_handoff as sc
    cells = geo.cells(tokens)
    kvb = cells * geo.n_head_kv * geo.head_dim * 2
    gdn = sc.payload_bytes(geo, tokens) - 2 * kvb * geo.n_qsa
    geokey = [2560, geo.n_layers, 4, 128, 16, 32, 4, 8192, 4096, 24, 2, 256, 128, 4, 4, 3, 1, 0]
    words = [0x1122334455667788, 0x0AABBCCDDEEFF001, *geokey, 0, geo.n_layers, 1, geo.n_qsa + 1]
    for _ in range(geo.n_qsa):
        words += [0, cells, geo.n_head_kv, geo.head_dim, geo.page_size, 0, 128, kvb, kvb, 0, 0, 0]
    words += [0] * 12
    words += [tokens, 0, gdn, 0, 0, 0, 0, tokens * 3, 0]   # live checkpoint
    words += [0, 0]                                          # no retained checkpoints, no stage parts
    return " ".join(str(w) for w in words)


def wire_cpu_baseline(geo_kw: dict, tokens: int, reps: int = 3) -> dict:
    """The reference's own codec on one core (src/core/conversation_wire.cpp, compiled from its sources into
    oracle/_ref/ref_wire): encode into memory with the payload's FNV-1a, then decode with the hash checked, over a
    bounded sample - the 48-layer slot's image at `tokens` tokens."""
    import subprocess
    import tempfile
    import sc_handoff as sc
    exe = REF_BIN / "ref_wire"
    if not exe.exists():
        return {"kind": "reference", "skipped": f"{exe} is not built"}
    geo = sc.geometry(**geo_kw)
    with tempfile.NamedTemporaryFile("w", suffix=".spec", delete=False) as f:
        f.write(wire_spec(geo, tokens))
        spec = f.name
    try:
        out = subprocess.run([str(exe), "time", spec, str(reps)], capture_output=True, text=True, timeout=600,
                             check=True).stdout.split()
    finally:
        os.unlink(spec)
    kv = dict(w.split("=", 1) for w in out)
    n, te, td = int(kv["bytes"]), float(kv["encode_s"]), float(kv["decode_s"])
    return {"value": round(n / (te + td) / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "reference",
            "encode_gbps": round(n / te / 1e9, 3), "decode_checked_gbps": round(n / td / 1e9, 3),
            "sample": (f"the reference codec (oracle/_ref/ref_wire, built from src/core/conversation_wire.cpp) on the "
                       f"48-layer slot's image at {tokens} tokens ({n} payload bytes): encode into memory with the "
                       f"payload hash, then decode with the hash checked; best of {reps}, 1 thread"),
            "cpu": cpu_model()}


def arena_cpu_baseline(sc, budget_bytes: int = 1 << 30) -> dict:
    """The reference's hand-off path on the host for a bounded sample: write_payload (one pwrite) + the byte-serial
    FNV-1a of the writer + publish, then read_slot + payload_hash_of (src/core/handoff.cpp:821-901, 1053-1136), timed
    on the reference's own arena (oracle/_ref/ref_arena, built from its sources) when it is built, else on this
    library's arena (same file format and algorithm) with the oracle's FNV-1a."""
    import subprocess
    exe = REF_BIN / "ref_arena"
    if exe.exists():
        n = budget_bytes
        base = arena_dir(n + (64 << 20))
        d = os.path.join(base, f"sc-bench-arena-ref-{os.getpid()}")
        os.makedirs(d, exist_ok=True)
        try:
            out = subprocess.run([str(exe), "time", os.path.join(d, "arena"), "0aabbccddeeff001", "1122334455667788",
                                  "131072:1", str(n), str(n), "3"], capture_output=True, text=True, timeout=600,
                                 check=True).stdout.split()
        finally:
            import shutil
            shutil.rmtree(d, ignore_errors=True)
        kv = dict(w.split("=", 1) for w in out if "=" in w)
        if kv.get("ok") == "1":
            tw, tr = float(kv["write_s"]), float(kv["read_s"])
            return {"sample_bytes": n, "write_gbps": round(n / tw / 1e9, 2), "read_gbps": round(n / tr / 1e9, 2),
                    "handoff_gbps": round(n / (tw + tr) / 1e9, 2), "cores": 1, "kind": "reference",
                    "sample": (f"the reference arena (oracle/_ref/ref_arena, built from src/core/handoff.cpp): "
                               f"{n} payload bytes, claim + write_payload + fnv1a64 + publish, then read_slot + "
                               "payload_hash_of; best of 3, 1 thread")}
    import shutil
    import numpy as np
    import sc_arena
    from oracle import sc_oracle
    n = budget_bytes
    data = np.random.default_rng(1).integers(0, 256, n, dtype=np.uint8)
    base = arena_dir(n + (64 << 20))
    d = os.path.join(base, f"sc-bench-arena-cpu-{os.getpid()}")
    try:
        w = sc_arena.Arena.writer(os.path.join(d, "arena"), [(131072, 1)], [n], 7, 9)
        r = sc_arena.Arena.reader(os.path.join(d, "arena"), 7, 9)
        best_w = best_r = None
        for rep in range(2):
            c = w.claim(0, 1, rep)
            t0 = time.perf_counter()
            w.write(c, 0, data)
            hh = sc_oracle.fnv1a64(data)
            w.publish(c, 1, n, hh)
            tw = time.perf_counter() - t0
            t0 = time.perf_counter()
            got, s = r.read_host(c.index, c.nonce, 1, n, check_hash=True)
            tr = time.perf_counter() - t0
            w.release(c.index, c.nonce)
            best_w = tw if best_w is None else min(best_w, tw)
            best_r = tr if best_r is None else min(best_r, tr)
        r.close()
        w.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return {"sample_bytes": n, "write_gbps": round(n / best_w / 1e9, 2), "read_gbps": round(n / best_r / 1e9, 2),
            "handoff_gbps": round(n / (best_w + best_r) / 1e9, 2), "cores": 1, "kind": "port"}


def ipc_export_role(tokens: int) -> int:
    """The exporting process of the same-GPU row (started by ipc_handoff): a decode slot of the headline geometry
    holding `tokens` tokens (seeded values), segments of 1 GiB exported, and on every "encode" line the slot's wire
    payload encoded straight into the exported segments (no payload buffer, no staging copy), answered with the
    encode's device time and the payload hash."""
    import numpy as np
    import sc_handoff as sc
    import sc_wire
    geo = sc.geometry(**HEADLINE_GEO)
    stream = sc.Stream()
    slot = sc.new_slot(geo, tokens, fill=0)
    for i, b in enumerate(slot.buffers()):
        sc.check(sc.lib.sc_fill_uniform_f16(b.ptr, b.nbytes // 2, -1.0, 1.0, 5, i, stream.handle), "fill")
    stream.sync()
    ids = (np.arange(tokens, dtype=np.int64) % 151_000).astype(np.int32)
    live, keep = sc_wire.make_live(WIRE_GEOKEY, ids, layer_hi=48, idx_dim=128)
    enc = sc_wire.Encoder(geo, slot, tokens, live, 0x1122334455667788, 0x0AABBCCDDEEFF001)
    n = enc.bytes
    nc = max(sc.carry_bytes(n), 1)
    # the payload's carries ride in the exported segments after the payload, inside one segment
    at = (n + 255) // 256 * 256
    if at % sc.IPC_MAX_SEGMENT + nc > sc.IPC_MAX_SEGMENT:
        at = (at + sc.IPC_MAX_SEGMENT - 1) // sc.IPC_MAX_SEGMENT * sc.IPC_MAX_SEGMENT
    ex = sc.IpcExport(at + nc, sc.IPC_MAX_SEGMENT)
    ptrs, seg = ex.layout()
    enc.set_carry(ptrs[at // seg] + at % seg)
    print(json.dumps({"segments": [[h.hex(), k] for h, k in ex.segments()], "bytes": n, "carry_at": at,
                      "buffers": [sc.fnv1a64_device(b.ptr, b.nbytes) for b in slot.buffers()]}), flush=True)
    e0, e1 = sc.Event(), sc.Event()
    for line in sys.stdin:
        if line.strip() != "encode":
            break
        e0.record(stream)
        enc.encode_segments(ptrs, seg, stream)
        e1.record(stream)
        e1.sync()
        print(json.dumps({"encode_ms": e0.elapsed_ms(e1), "hash": enc.hash()}), flush=True)
    enc.destroy()
    ex.destroy()
    return 0


def ipc_handoff(sc, geo, tokens: int, reps: int = 5) -> dict:
    """The same-GPU row, zero-copy: another process on this GPU encodes its slot's wire payload straight into device
    segments it exports, and this process mounts the payload where it lies in the imported segments (the hash checked
    over the segments on the device, then one gated scatter launch straight from them).  No payload buffer, staging copy
    or fetch copy exists on either side; the hand-off is the encode plus the mount."""
    import subprocess
    import sc_wire
    proc = subprocess.Popen([sys.executable, "-u", __file__, "--ipc-export", str(tokens)], stdin=subprocess.PIPE,
                            stdout=subprocess.PIPE, text=True)
    imp = None
    try:
        first = json.loads(proc.stdout.readline())
        n = first["bytes"]
        imp = sc.IpcImport([(bytes.fromhex(h), k) for h, k in first["segments"]])
        ptrs, seg = imp.layout()
        at = first["carry_at"]
        carry = ptrs[at // seg] + at % seg   # the exporter's carries of each payload, in its exported segments
        dst = sc.new_slot(geo, tokens, fill=0)
        stream = sc.Stream()
        e0, e1 = sc.Event(), sc.Event()
        enc_ms, open_ms, mount_ms, mount_dev_ms = [], [], [], []
        dec = None
        for _ in range(reps + 1):
            proc.stdin.write("encode\n")
            proc.stdin.flush()
            r = json.loads(proc.stdout.readline())
            enc_ms.append(r["encode_ms"])
            # one decoder for the slot, opened again for each payload in the same segments
            t0 = time.perf_counter()
            if dec is None:
                dec = sc_wire.Decoder(0, n, geo, dst, payload_hash=r["hash"], check_hash=True, segments=(ptrs, seg),
                                      carry=carry)
            else:
                dec.reopen(None, n, r["hash"], carry=carry)
            t1 = time.perf_counter()
            e0.record(stream)
            dec.restore(stream)
            e1.record(stream)
            mount_ms.append((time.perf_counter() - t1) * 1e3)
            e1.sync()
            mount_dev_ms.append(e0.elapsed_ms(e1))
            open_ms.append((t1 - t0) * 1e3)
        dec.destroy()
        same = [sc.fnv1a64_device(b.ptr, b.nbytes) for b in dst.buffers()] == first["buffers"]
        for b in dst.buffers():
            b.free()
    finally:
        if imp:
            imp.close()
        try:
            proc.stdin.write("done\n")
            proc.stdin.flush()
        except BrokenPipeError:
            pass
        proc.wait(timeout=120)

    def p50(xs):
        return sorted(xs[1:])[len(xs[1:]) // 2]
    en, mo, ro = p50(enc_ms), p50(mount_ms), p50(open_ms)
    return {"tokens": tokens, "payload_bytes": n, "segments": len(ptrs), "segment_bytes": seg,
            "encode_ms": round(en, 3), "mount_ms": round(mo, 3), "mount_device_ms": round(p50(mount_dev_ms), 3),
            "open_ms": round(open_ms[0], 3), "reopen_ms": round(ro, 3), "handoff_ms": round(en + mo, 3),
            "handoff_with_reopen_ms": round(en + ro + mo, 3),
            "handoff_gbps": round(n / ((en + mo) * 1e-3) / 1e9, 1), "copies": 0, "bit_exact": bool(same),
            "timing": f"p50 of {reps} hand-offs after one warm-up",
            "method": "exporter process: the slot's payload encoded into 1 GiB hipMalloc segments exported with "
                      "hipIpcGetMemHandle (head copies + the fused gather and FNV-1a, cut at segment ends; HIP events); "
                      "importer (this process): segments opened once with hipIpcOpenMemHandle, the payload mounted "
                      "from them (device FNV-1a over the segments leaving a verdict, one scatter launch gated by it, "
                      "reading the segments; host wall time of the synchronous restore; one decoder opened once and "
                      "opened again for each payload, reopen_ms), the hash check given the "
                      "payload's carries (the low byte of the running hash after every 64 KiB, written by the "
                      "exporter's encode after the payload in its segments); handoff_ms = encode + mount; "
                      "bit_exact = every destination slot buffer's device hash equals the exporter's source buffer's"}


def copy_ceiling(sc, nbytes: int, stream, reps: int = 5) -> dict:
    """What a plain device-to-device copy of the headline's bytes achieves on this part: the library's tile copy
    (sc_copy_device_async, one 16 KiB tile per workgroup) and the runtime's hipMemcpyAsync, HIP events, best of reps.
    The fused carve moves the same 2P bytes with layout changes on top."""
    src, dst = sc.DeviceBuffer(nbytes, "uint8"), sc.DeviceBuffer(nbytes, "uint8")
    src.fill(1, stream)
    dst.fill(2, stream)
    e0, e1 = sc.Event(), sc.Event()
    out = {}
    for name, fn in (("tile_copy", sc.lib.sc_copy_device_async), ("hip_memcpy", sc.lib.sc_copy_async)):
        best = None
        for _ in range(reps + 1):
            e0.record(stream)
            sc.check(fn(dst.ptr, src.ptr, nbytes, stream.handle), name)
            e1.record(stream)
            e1.sync()
            ms = e0.elapsed_ms(e1)
            best = ms if best is None else min(best, ms)
        gbps = 2 * nbytes / (best * 1e-3) / 1e9
        out[name] = {"ms": round(best, 4), "hbm_gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4)}
    src.free()
    dst.free()
    return out


def quant_carve(sc, geo, tokens: int, stream, reps: int = 10) -> dict:
    """The quantizing carve of the config-3 geometry: f32 K/V rows into int8 / q4_0 / K8V4 pools plus the GDN state,
    one launch each (and int8 once more through a shuffled page table).  HBM bytes = the f32 rows read + the codes and
    scales written + the GDN rows read and written."""
    import numpy as np
    case = synth().SyntheticCase(geo, tokens, seed=0x5EED, kv_dtype=sc.SC_DTYPE_F32)
    out = {"tokens": tokens}
    n_pages = (tokens + geo.page_size - 1) // geo.page_size
    shuffled = sc.device_tables([np.random.default_rng(j).permutation(n_pages).astype(np.int32)
                                 for j in range(geo.n_qsa)])
    for name, fmt, tables in (("int8", sc.SC_KV_INT8, None), ("q4_0", sc.SC_KV_Q4, None),
                              ("k8v4", sc.SC_KV_K8V4, None), ("int8_paged", sc.SC_KV_INT8, shuffled)):
        slot = sc.new_quant_slot(geo, fmt, tokens, tables=tables)
        plan = sc.plan_carve_quant(geo, case.prefill, slot)
        # 20 untimed launches (~30 ms) first: the GPU raises its clocks over the first tens of milliseconds of load
        # (measured: the first 12 launches after an idle second average 1.56 ms, the next 1.43 ms for int8)
        _, per = time_launches(plan, stream, reps, 20, sc)
        ms = sum(per) / len(per)
        moved = plan.payload_bytes
        out[name] = {"ms": round(ms, 4), "hbm_bytes": moved, "hbm_gbps": round(moved / (ms * 1e-3) / 1e9, 1),
                     "frac": round(moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        plan.destroy()
        for b in slot.buffers():
            b.free()
    # the per-layer writers with the reference's arguments (sc_kv_append_async: one launch per QSA layer, nothing
    # allocated), K and V of every QSA layer in turn, f16 and int8 pools; HBM bytes = the f32 rows read + what is written
    T, H, D = tokens, geo.n_head_kv, geo.head_dim
    ev0, ev1 = sc.Event(), sc.Event()
    per_layer = {}
    for name, f16 in (("f16", True), ("int8", False)):
        slot = sc.new_slot(geo, max_cells=tokens) if f16 else sc.new_quant_slot(geo, sc.SC_KV_INT8, tokens)

        def appends():
            for j in range(geo.n_qsa):
                K, V = case.prefill.k[j].data_ptr(), case.prefill.v[j].data_ptr()
                if f16:
                    rc = sc.lib.sc_kv_append_async(K, V, T, 0, None, geo.page_size, slot.k_pool[j].data_ptr(),
                                                   slot.v_pool[j].data_ptr(), None, None, None, None, stream.handle,
                                                   None, None)
                else:
                    rc = sc.lib.sc_kv_append_async(K, V, T, 0, None, geo.page_size, None, None, slot.k_codes[j].ptr,
                                                   slot.v_codes[j].ptr, slot.k_scale[j].ptr, slot.v_scale[j].ptr,
                                                   stream.handle, None, None)
                sc.check(rc, "sc_kv_append_async")
        for _ in range(20):
            appends()
        times = []
        for _ in range(reps):
            ev0.record(stream)
            appends()
            ev1.record(stream)
            ev1.sync()
            times.append(ev0.elapsed_ms(ev1))
        ms = sum(times) / len(times)
        moved = geo.n_qsa * 2 * T * H * (D * 4 + (D * 2 if f16 else D + 8))
        per_layer[name] = {"ms_all_layers": round(ms, 4), "launches": geo.n_qsa, "hbm_bytes": moved,
                           "hbm_gbps": round(moved / (ms * 1e-3) / 1e9, 1),
                           "frac": round(moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        for b in slot.buffers():
            b.free()
    out["kv_append_per_layer"] = per_layer
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tokens", type=int, default=131072)
    ap.add_argument("--latency-tokens", type=int, default=32768)
    ap.add_argument("--latency-reps", type=int, default=30)
    ap.add_argument("--cpu-budget", type=float, default=16.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--grid", type=int, default=0, help="workgroups of the move kernel (0 = library default)")
    ap.add_argument("--kernel-only", action="store_true", help="only the timed handoff (for profiler runs)")
    ap.add_argument("--wire-only", action="store_true",
                    help="only the wire payload row of the same slot (for profiler runs); prints its JSON")
    ap.add_argument("--quant-only", action="store_true",
                    help="only the quantizing carve row of the same geometry (for profiler runs); prints its JSON")
    ap.add_argument("--paged-only", action="store_true",
                    help="only the paged carve row of the same slot (for profiler runs); prints its JSON")
    ap.add_argument("--config5-only", action="store_true",
                    help="only the config-5 batched resume + append row (for profiler runs); prints its JSON")
    ap.add_argument("--arena-only", action="store_true",
                    help="only the hand-off arena row of the same geometry; prints its JSON")
    ap.add_argument("--mover", default="64,4,8", help="arena mover chunk MiB, depth, threads")
    ap.add_argument("--ipc-only", action="store_true", help="only the same-GPU inter-process row; prints its JSON")
    ap.add_argument("--ipc-export", type=int, default=0, metavar="TOKENS", help=argparse.SUPPRESS)
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarize the headline launches of a kernel trace of --kernel-only (same --steps/--warmup)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run 5 device-to-device copies of BYTES (the counter calibration of profiler runs)")
    args = ap.parse_args()
    if args.ipc_export:
        return ipc_export_role(args.ipc_export)
    if args.trace_summary:
        import sc_handoff as sc
        P = sc.payload_bytes(sc.geometry(**HEADLINE_GEO), args.tokens)
        print(json.dumps(trace_summary(args.trace_summary, "sc_move_kernel", args.warmup, args.steps, P)), flush=True)
        return 0

    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the handoff's sharding across GPUs is a design note, not a measured path", file=sys.stderr)
        return 2

    import sc_handoff as sc

    if sc.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    stream = sc.Stream()   # every timed launch and its events go on this one non-blocking stream
    if args.copy_calibration:
        n = args.copy_calibration
        src, dst = sc.DeviceBuffer(n, "uint8"), sc.DeviceBuffer(n, "uint8")
        src.fill(1)
        dst.fill(2)
        sc.device_sync()
        for _ in range(5):
            sc.check(sc.lib.sc_copy_async(dst.ptr, src.ptr, n, stream.handle), "copy")
        sc.device_sync()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)
        return 0
    # the host link, measured before anything large is allocated (the reference's probe method, both directions)
    h2d, d2h = sc.probe_link(256 << 20, 4)
    geo_kw = HEADLINE_GEO
    geo = sc.geometry(**geo_kw)
    T = args.tokens
    P = sc.payload_bytes(geo, T)

    if args.quant_only:
        print(json.dumps({"quant_carve": quant_carve(sc, geo, T, stream)}), flush=True)
        return 0
    if args.ipc_only:
        print(json.dumps({"ipc_handoff": ipc_handoff(sc, geo, T)}), flush=True)
        return 0
    if args.config5_only:
        print(json.dumps({"config5": config5(sc, geo, 0x5EED)}), flush=True)
        return 0
    log(f"config 3: {T} tokens, payload {P} B; generating inputs on the device")
    case = synth().SyntheticCase(geo, tokens=T, seed=0x5EED)
    slot = case.new_slot(max_cells=T)
    sc.device_sync()
    plan = sc.plan_carve(geo, case.prefill, slot)
    if args.grid:
        plan.set_grid(args.grid)
    log(f"timing {args.steps} fused carve -> scatter launches after {args.warmup} warm-up")
    wall_ms, per = time_launches(plan, stream, args.steps, args.warmup, sc)
    ms_per_step = wall_ms / args.steps
    # the statistic of the roofline: the mean of the timed launches only (no warm-up), as the committed kernel-trace
    # summary states it for the same dispatches
    kernel_ms = sum(per) / len(per)
    per_sorted = sorted(per)
    value = P / (ms_per_step * 1e-3) / 1e9
    achieved = 2 * P / (kernel_ms * 1e-3) / 1e9
    log(f"fused: {ms_per_step:.3f} ms/step wall, {kernel_ms:.3f} ms/launch (events) -> {value:.1f} GB/s payload, "
        f"{achieved:.1f} GB/s HBM")
    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8", "data": "synthetic",
        "config": {"workload": ("config 3: fused carve -> scatter of one 131072-token sequence, 48-layer hybrid "
                                "(12 QSA K/V [T][2][256] f16 -> paged [page][2][4][256]; 36 GDN recurrence "
                                "[32][128][128] f32 -> (128,32,128) and conv [3][8192] f32 -> [8192][3]) into one "
                                "decode slot, inputs resident in HBM"),
                   "tokens": T, "layers": 48, "payload_bytes": P},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic() if T == 131072 else None,
                     "kernel": "sc_move_kernel", "kernel_ms": round(kernel_ms, 4),
                     "kernel_ms_p50": round(per_sorted[len(per_sorted) // 2], 4),
                     "kernel_ms_min": round(per_sorted[0], 4),
                     "timing": f"mean of the {args.steps} timed launches (event pairs on the launch stream), warm-up "
                               "launches excluded",
                     "algorithmic_bytes_per_launch": 2 * P},
    }
    if args.wire_only:
        print(json.dumps({"wire_payload": wire_payload(sc, geo, T, slot, h2d, d2h)}), flush=True)
        return 0
    if args.paged_only:
        print(json.dumps({"paged_carve": paged_carve(sc, geo, case, T, stream)}), flush=True)
        return 0
    mv = [int(x) for x in args.mover.split(",")]
    if args.arena_only:
        rows = {"link_h2d_gbps": round(h2d, 2), "link_d2h_gbps": round(d2h, 2)}
        for cfg in ([mv] if len(mv) == 3 else [mv[i:i + 3] for i in range(0, len(mv), 3)]):
            settle_link(sc, d2h)
            key = "arena_%d_%d_%d" % tuple(cfg)
            rows[key] = arena_handoff(sc, geo, T, slot, h2d, d2h, *cfg)
            log(f"{key}: " + json.dumps(rows[key]))
        rows["arena_cpu_baseline"] = arena_cpu_baseline(sc)
        print(json.dumps(rows), flush=True)
        return 0
    result["roofline"]["copy_ceiling"] = copy_ceiling(sc, P, stream)
    if args.kernel_only:
        print(json.dumps(result), flush=True)
        return 0

    # the same carve into a slot whose pages are placed through a shuffled page table (a decode slot's pages are
    # wherever the pool had them free)
    result["paged_carve"] = pc = paged_carve(sc, geo, case, T, stream)
    log(f"paged carve (shuffled page table): {pc['ms']:.3f} ms in destination order, {pc['source_order_ms']:.3f} ms "
        "in source order")

    # two-pass gather -> scatter through a transfer buffer (the cross-instance path)
    _, total = sc.image_layout(geo, T)
    image = sc.DeviceBuffer(total, "uint8")
    gather = sc.plan_gather(geo, case.prefill, image.ptr, total)
    scatter = sc.plan_scatter(geo, image.ptr, total, T, slot)
    for _ in range(2):
        gather.launch(stream)
        scatter.launch(stream)
    sc.device_sync()
    e = [sc.Event() for _ in range(3)]
    reps = 5
    g_ms = s_ms = 0.0
    for _ in range(reps):
        e[0].record(stream)
        gather.launch(stream)
        e[1].record(stream)
        scatter.launch(stream)
        e[2].record(stream)
        e[2].sync()
        g_ms += e[0].elapsed_ms(e[1]) / reps
        s_ms += e[1].elapsed_ms(e[2]) / reps
    result["two_pass"] = {"gather_ms": round(g_ms, 4), "scatter_ms": round(s_ms, 4),
                          "handoff_gbps": round(P / ((g_ms + s_ms) * 1e-3) / 1e9, 1),
                          "gather_hbm_gbps": round(2 * P / (g_ms * 1e-3) / 1e9, 1),
                          "scatter_hbm_gbps": round(2 * P / (s_ms * 1e-3) / 1e9, 1)}
    log(f"two-pass: gather {g_ms:.3f} ms, scatter {s_ms:.3f} ms")

    # park / resume of the 128K slot against the host link measured at the start of the run
    settle_pr = settle_link(sc, d2h)
    host = sc.PinnedBuffer(total)
    side = sc.Stream()
    t0, t1 = sc.Event(), sc.Event()
    sc.park_async(geo, slot, T, host.ptr, total, stream=side)   # warm-up: touch the pinned pages once
    side.sync()
    # the link at the payload's own size: plain copies of `total` bytes between the same two buffers
    big_h2d, big_d2h = link_at(sc, image.ptr, host.ptr, total)
    park_ms, resume_ms = [], []
    for _ in range(20):
        t0.record(side)
        sc.park_async(geo, slot, T, host.ptr, total, stream=side)
        t1.record(side)
        t1.sync()
        park_ms.append(t0.elapsed_ms(t1))
        t0.record(side)
        sc.resume_async(geo, host.ptr, total, T, slot, stream=side)
        t1.record(side)
        t1.sync()
        resume_ms.append(t0.elapsed_ms(t1))
    pk, rs = spread(park_ms), spread(resume_ms)
    pk_gbps = total / (pk["p50_ms"] * 1e-3) / 1e9
    rs_gbps = total / (rs["p50_ms"] * 1e-3) / 1e9
    result["park_resume"] = {
        "bytes": total, "park": pk, "resume": rs,
        "park_gbps": round(pk_gbps, 2), "resume_gbps": round(rs_gbps, 2),
        "link_probe_d2h_gbps": round(big_d2h, 2), "link_probe_h2d_gbps": round(big_h2d, 2),
        "link_small_probe_d2h_gbps": round(d2h, 2), "link_small_probe_h2d_gbps": round(h2d, 2),
        "pcie5_x16_gbps": round(PCIE5_X16_GBPS, 2),
        "park_vs_link": link_fracs(pk_gbps, big_d2h, d2h), "resume_vs_link": link_fracs(rs_gbps, big_h2d, h2d),
        "method": "p50 of 20 reps, device events around the enqueue; hipMemcpyAsync per blob on a non-blocking side "
                  "stream, pinned hipHostMalloc image; the probe is one plain pinned copy of the same byte count "
                  "between the same buffers (p50 of 3), the small probe 256 MiB x 4 at the start of the run",
        "link_settle_ms": settle_pr}
    log(f"park p50 {pk['p50_ms']:.1f} ms, resume p50 {rs['p50_ms']:.1f} ms; same-size link d2h {big_d2h:.1f} GB/s, "
        f"h2d {big_h2d:.1f} GB/s")
    host.free()
    image.free()

    # p50 latency of the 32K handoff (config 2): first enqueue to completion event
    TL = args.latency_tokens
    PL = sc.payload_bytes(geo, TL)
    case_l = synth().SyntheticCase(geo, tokens=TL, seed=0x5EED + 1)
    slot_l = case_l.new_slot(max_cells=TL)
    plan_l = sc.plan_carve(geo, case_l.prefill, slot_l)
    sc.device_sync()
    for _ in range(3):
        plan_l.launch(stream)
    sc.device_sync()
    lat = []
    a, b = sc.Event(), sc.Event()
    for _ in range(args.latency_reps):
        a.record(stream)
        plan_l.launch(stream)
        b.record(stream)
        b.sync()
        lat.append(a.elapsed_ms(b))
    lat.sort()
    p50 = lat[len(lat) // 2]
    result["latency_32k"] = {"tokens": TL, "payload_bytes": PL, "p50_ms": round(p50, 4),
                             "p90_ms": round(lat[int(len(lat) * 0.9)], 4), "reps": len(lat),
                             "p50_gbps": round(PL / (p50 * 1e-3) / 1e9, 1)}
    log(f"32K handoff p50 {p50:.4f} ms over {len(lat)} reps")
    result["retarget_32k"] = retarget_latency(sc, geo, TL, case_l, slot_l, plan_l, stream, args.latency_reps)
    rl = result["retarget_32k"]
    log(f"32K retarget + launch p50 {rl['retarget_launch']['p50_ms']} ms (bare launch "
        f"{rl['bare_launch']['p50_ms']} ms, plan build + launch {rl['build_launch']['p50_ms']} ms)")
    # the 32K hand-off through host memory: park to a pinned image, resume into a second slot; wall clock from the
    # first enqueue to the host seeing completion, beside the device events around the same work
    settle_32 = settle_link(sc, d2h)
    _, total_l = sc.image_layout(geo, TL)
    host_l = sc.PinnedBuffer(total_l)
    dev_l = sc.DeviceBuffer(total_l, "uint8")
    back_l = sc.new_slot(geo, TL, fill=0)
    side = sc.Stream()
    sc.park_async(geo, slot_l, TL, host_l.ptr, total_l, stream=side)   # warm-up: touch the pinned pages once
    sc.resume_async(geo, host_l.ptr, total_l, TL, back_l, stream=side)
    side.sync()
    l_h2d, l_d2h = link_at(sc, dev_l.ptr, host_l.ptr, total_l)
    dev_l.free()
    wall, dev = [], []
    for _ in range(max(20, args.latency_reps)):
        t0 = time.perf_counter()
        a.record(side)
        sc.park_async(geo, slot_l, TL, host_l.ptr, total_l, stream=side)
        sc.resume_async(geo, host_l.ptr, total_l, TL, back_l, stream=side)
        b.record(side)
        b.sync()
        wall.append((time.perf_counter() - t0) * 1e3)
        dev.append(a.elapsed_ms(b))
    same = all(sc.fnv1a64_device(x.ptr, x.nbytes) == sc.fnv1a64_device(y.ptr, y.nbytes)
               for x, y in zip(slot_l.buffers(), back_l.buffers()))
    w, d = spread(wall), spread(dev)
    both = total_l / (d["p50_ms"] * 1e-3) / 1e9
    ideal_ms = total_l / (l_d2h * 1e9) * 1e3 + total_l / (l_h2d * 1e9) * 1e3
    result["park_resume_32k"] = {
        "tokens": TL, "bytes": total_l, "wall": w, "device": d, "round_trip_bit_exact": bool(same),
        "link_probe_d2h_gbps": round(l_d2h, 2), "link_probe_h2d_gbps": round(l_h2d, 2),
        "probe_round_trip_ms": round(ideal_ms, 3), "device_p50_vs_probe": round(ideal_ms / d["p50_ms"], 3),
        "bytes_each_way_gbps_p50": round(both, 2),
        "method": "park (D2H of every blob) then resume (H2D) of the 32K slot on one non-blocking stream, pinned "
                  "image; wall = host clock from before the first enqueue to the completion event's sync; device = "
                  "events around the same work; probe = one plain pinned copy of the image's size each way",
        "link_settle_ms": settle_32}
    log(f"32K park+resume p50: wall {w['p50_ms']:.3f} ms, device {d['p50_ms']:.3f} ms (probe round trip "
        f"{ideal_ms:.3f} ms)")
    host_l.free()
    for x in back_l.buffers():
        x.free()

    log("wire payload: device encode / hash / mount of the 128K slot, checked park and resume")
    settle_wire = settle_link(sc, d2h)
    result["wire_payload"] = wire_payload(sc, geo, T, slot, h2d, d2h)
    result["wire_payload"]["link_settle_ms"] = settle_wire
    wp = result["wire_payload"]
    log(f"wire: encode {wp['encode_ms']} ms ({wp['encode_gbps']} GB/s), hash {wp['hash_ms']} ms, mount "
        f"{wp['mount_ms']} ms (given the carries {wp['mount_carried_ms']} ms); checked park "
        f"{wp['checked_park_gbps']} GB/s, resume {wp['checked_resume_gbps']} GB/s")

    log("hand-off arena: the 128K slot's payload through a tmpfs arena slot and back into a fresh slot")
    settle_ar = settle_link(sc, d2h)
    result["arena_handoff"] = arena_handoff(sc, geo, T, slot, h2d, d2h, *mv[:3])
    result["arena_handoff"]["link_settle_ms"] = settle_ar
    ah = result["arena_handoff"]
    log(f"arena: publish {ah['mover_publish_gbps']} GB/s ({ah['mover_publish_vs_link']['frac_of_probe']} of the "
        f"probe), read {ah['read_gbps']} GB/s ({ah['read_vs_link']['frac_of_probe']}), read+mount "
        f"{ah['read_and_mount_ms']} ms")
    if not args.no_cpu:
        result["arena_handoff"]["cpu_baseline"] = arena_cpu_baseline(sc, 512 << 20)
        result["wire_payload"]["cpu_baseline"] = wire_cpu_baseline(geo_kw, 8192)
    log("same-GPU hand-off between processes: exported device segments")
    result["ipc_handoff"] = ipc_handoff(sc, geo, T)
    ih = result["ipc_handoff"]
    log(f"ipc: encode {ih['encode_ms']} ms + mount {ih['mount_ms']} ms = {ih['handoff_ms']} ms "
        f"({ih['handoff_gbps']} GB/s), no copies, bit-exact {ih['bit_exact']}")

    log("quantizing carve: int8 / q4_0 / K8V4 pools from f32 rows, 128K")
    result["quant_carve"] = quant_carve(sc, geo, T, stream)
    qc = result["quant_carve"]
    log("quant carve: " + ", ".join(f"{k} {v['ms']} ms ({v['hbm_gbps']} GB/s)" for k, v in qc.items()
                                    if isinstance(v, dict) and "ms" in v))
    log("kv_append per layer: " + ", ".join(f"{k} {v['ms_all_layers']} ms for {v['launches']} launches "
                                            f"({v['hbm_gbps']} GB/s)" for k, v in qc["kv_append_per_layer"].items()))

    log("config 4: three slots, two parks and one resume overlapped with decode")
    settle_c4 = settle_link(sc, d2h)
    result["config4"] = config4(sc, geo, 0x5EED, d2h)
    result["config4"]["link_settle_ms"] = settle_c4
    c4 = result["config4"]
    log(f"config 4: park {c4['park_gbps']} GB/s, resume {c4['resume_gbps']} GB/s, decode slowdown "
        f"{c4['decode_slowdown']}x, bit-exact {c4['round_trip_bit_exact']}")
    # against the 128K payload-size probe (config 4 moves 0.2-2.4 GB per transfer) and the small probe
    result["config4"]["park_vs_link"] = link_fracs(c4["park_gbps"], big_d2h, d2h)
    result["config4"]["resume_vs_link"] = link_fracs(c4["resume_gbps"], big_h2d, h2d)
    log("config 5: eight ragged slots, batched resume + append in one launch")
    settle_c5 = settle_link(sc, d2h)
    result["config5"] = config5(sc, geo, 0x5EED)
    result["config5"]["link_settle_ms"] = settle_c5
    c5 = result["config5"]
    result["config5"]["resume_h2d_vs_link"] = link_fracs(c5["resume_h2d_gbps"], big_h2d, h2d)
    log(f"config 5: resume {c5['resume_h2d_gbps']} GB/s, one-launch scatter {c5['scatter_launch_ms']} ms "
        f"({c5['scatter_hbm_gbps']} GB/s HBM)")

    if not args.no_cpu:
        log(f"CPU baseline (~{args.cpu_budget:.0f} s on one core)")
        result["cpu_baseline"] = cpu_baseline(geo_kw, T, args.cpu_budget)
        log(f"CPU carve {result['cpu_baseline']['value']} GB/s, pipeline {result['cpu_baseline']['pipeline_gbps']} GB/s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
