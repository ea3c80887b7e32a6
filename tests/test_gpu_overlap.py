"""Config 4: three slots (8K / 32K / 96K tokens, roles from the seed) - two parked to pinned host memory and one
resumed while the third keeps decoding, on three non-blocking streams ordered only by events.

The reference orders these moves by synchronizing the device before a save and after a restore
(include/strata/core/conversation_snapshot.hpp:11; src/core/conversation_state.cpp:381,478).  This build replaces the
synchronizations with events, so the test proves the two orderings that must survive the change:
  (i)  a resume reads a parked image only after that park's D2H copy has landed, and whatever reads the resumed slot
       (the decode) runs only after the resume's event;
  (ii) a parked slot's device memory is overwritten (by the next conversation's carve) only after its D2H copy has
       landed.
A delay kernel (long work that always ends) sits ahead of the parks on the park stream, so a resume or an overwrite
that did not wait would run during it; the pinned images start poisoned (0xEE) and the resume target filled with 0x5A,
so an early read would resume poison and an early decode would read 0x5A.  Every parked, resumed and overwritten blob
is compared with the CPU oracle's hash of the bytes it must hold (sco_synth_*_hash).
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

MAX_BLOB = 98304 * 2 * 256 * 2
DELAY_US = 100_000


def _host_image_hashes(sc, oracle, geo, image, tokens):
    blobs, _ = sc.image_layout(geo, tokens)
    host = image.numpy()
    with ThreadPoolExecutor(max_workers=16) as pool:
        return list(pool.map(lambda b: oracle.fnv1a64(host[b.offset:b.offset + b.bytes]), blobs))


def _slot_hashes(sc, hp, geo, slot, tokens):
    kv = geo.cells(tokens) * geo.n_head_kv * geo.head_dim * 2
    spans = []
    for j in range(geo.n_qsa):
        spans += [(slot.k_pool[j].ptr, kv), (slot.v_pool[j].ptr, kv)]
    spans.append((slot.gdn.ptr, geo.n_gdn * geo.gdn_row_floats * 4))
    out = []
    for ptr, n in spans:
        hp.launch(ptr, n)
        out.append(hp.result())
    return out


def test_config4_park_resume_overlap_event_ordering(sc, oracle, cuda):
    geo = sc.geometry()
    rng = np.random.default_rng(0x5EED)
    decode_len, park_a, park_b = (int(x) for x in rng.permutation([8192, 32768, 98304]))
    cap = 98304   # every slot has the capacity of the longest context, as a serving system's slots do
    seeds = {L: 0xC4000 + L for L in (decode_len, park_a, park_b)}
    new_tokens, new_seed = 4096, 0xC4E
    print(f"config 4: decode {decode_len}, park {park_a} and {park_b}, resume {park_a}", flush=True)
    want = {L: oracle.synthetic_image_hashes(geo, L, seeds[L]) for L in (park_a, park_b)}
    want_new = oracle.synthetic_image_hashes(geo, new_tokens, new_seed)

    slots = {}
    for L in (decode_len, park_a, park_b):
        case = synth.SyntheticCase(geo, L, seeds[L])
        slots[L] = case.new_slot(max_cells=cap)
        case.carve_into(slots[L])
        del case
    newcomer = synth.SyntheticCase(geo, new_tokens, new_seed)
    carve_new = sc.plan_carve(geo, newcomer.prefill, slots[park_a])
    images = {L: sc.PinnedBuffer(sc.image_layout(geo, L)[1]) for L in (park_a, park_b)}
    for im in images.values():
        im.numpy()[:] = 0xEE
    target = sc.new_slot(geo, cap, fill=0x5A)
    sink = sc.DeviceBuffer(4096, "uint32")
    hp = sc.HashPlan(MAX_BLOB)
    sc.device_sync()

    decode, park, resume = sc.Stream(), sc.Stream(), sc.Stream()
    t0, delay_done, pa, pb, c0, r1, n1, dec_done = (sc.Event() for _ in range(8))
    t0.record(park)
    sc.delay_async(DELAY_US, park)
    delay_done.record(park)
    sc.park_async(geo, slots[park_a], park_a, images[park_a].ptr, images[park_a].nbytes, stream=park, done=pa.handle)
    sc.park_async(geo, slots[park_b], park_b, images[park_b].ptr, images[park_b].nbytes, stream=park, done=pb.handle)
    # the first parked conversation resumes into a free slot once its own park has landed (overlapping the second
    # park: the link is full duplex), then its old slot memory takes the next conversation's carve
    resume.wait(pa)
    c0.record(resume)
    sc.resume_async(geo, images[park_a].ptr, images[park_a].nbytes, park_a, target, stream=resume, done=r1.handle)
    carve_new.launch(resume)
    n1.record(resume)
    # decode keeps reading the third slot meanwhile, and reads the resumed slot once the resume's event has fired
    pools = slots[decode_len].k_pool + slots[decode_len].v_pool
    for _ in range(50):
        for b in pools:
            sc.check(sc.lib.sc_decode_probe(b.ptr, b.nbytes, sink.ptr, 4096, decode.handle), "decode probe")
    dec_done.record(decode)
    decode.wait(r1)
    hp.launch(target.k_pool[0].ptr, geo.cells(park_a) * geo.n_head_kv * geo.head_dim * 2, stream=decode)
    sc.device_sync()
    decode_read = hp.result()

    delay_ms = t0.elapsed_ms(delay_done)
    print(f"delay {delay_ms:.1f} ms; park a done {t0.elapsed_ms(pa):.1f} ms, park b {t0.elapsed_ms(pb):.1f} ms, "
          f"resume start {t0.elapsed_ms(c0):.1f} ms, done {t0.elapsed_ms(r1):.1f} ms, decode {t0.elapsed_ms(dec_done):.1f} ms",
          flush=True)
    assert delay_ms >= 0.9 * DELAY_US / 1000
    # the gated stream started only after the delayed park had landed
    assert t0.elapsed_ms(c0) >= t0.elapsed_ms(pa) - 0.05 >= delay_ms
    # decode was not held behind the parks
    assert t0.elapsed_ms(dec_done) < t0.elapsed_ms(pa)

    # (ii) the images hold the slots as they were before the next conversation's carve overwrote the first one
    for L in (park_a, park_b):
        got = _host_image_hashes(sc, oracle, geo, images[L], L)
        assert got == want[L], f"image of the {L}-token slot differs from the oracle"
    # (i) the resumed slot holds the parked conversation, not the poison, and the decode read it after the resume
    assert _slot_hashes(sc, hp, geo, target, park_a) == want[park_a]
    assert decode_read == want[park_a][0]
    # the next conversation's carve landed in full in the parked slot's memory
    assert _slot_hashes(sc, hp, geo, slots[park_a], new_tokens) == want_new
    hp.free()
    for im in images.values():
        im.free()
