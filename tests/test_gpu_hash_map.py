"""The capture fused with the payload hash (sc_hash_map_*) against the capture plans launched on their own followed by
the plain device hash, and against the oracle's byte loop.

A hash map gathers the rows of capture plans (page gathers through page tables, copies, zero fills) into the payload
and hashes the whole payload in one kernel; the bytes no row writes (a head copied in first, a page the table does not
place) are hashed as the payload holds them.  Each case fills the payload with a pattern, runs the plans and the plain
hash, fills it again, runs the map, and requires the same payload bytes and the same hash, which must also be the byte
loop's (sco_fnv1a64, pinned to the published FNV-1a vectors).  Sizes cover a payload under one lane segment, tails
that are not whole lane segments, several blobs inside one lane segment (the small scale and indexer blobs of
quantized slots), pages that cross lane segments, and a table with holes.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
TINY = dict(SMALL, n_layers=4, head_dim=8, page_size=1, ssm_state_size=4, ssm_v_heads=1, ssm_conv_channels=4)


def _compare(sc, oracle, plans, payload, nbytes, pattern, head=None):
    def reset():
        payload.fill(pattern)
        if head is not None:
            payload.upload(head)
        sc.device_sync()

    hp = sc.HashPlan(nbytes)
    reset()
    for p in plans:
        p.launch()
    hp.launch(payload.ptr, nbytes)
    sc.device_sync()
    want_bytes, want = payload.numpy(nbytes).copy(), hp.result()
    assert want == oracle.fnv1a64(want_bytes)
    hmap = sc.HashMap(plans, payload.ptr, nbytes)
    reset()
    hp.fault.fill(0xAB)
    hmap.launch(hp)
    sc.device_sync()
    got_bytes = payload.numpy(nbytes)
    assert np.array_equal(got_bytes, want_bytes), np.flatnonzero(got_bytes != want_bytes)[:8]
    assert hp.result() == want
    hmap.destroy()
    hp.free()


@pytest.mark.parametrize("geo_kw,tokens", [(SMALL, 77), (SMALL, 1), (SMALL, 0), (TINY, 5), (TINY, 0)])
@pytest.mark.parametrize("table", ["identity", "shuffled", "holes"])
def test_fused_capture_equals_capture_then_hash(sc, oracle, cuda, geo_kw, tokens, table):
    geo = sc.geometry(**geo_kw)
    print(f"case hash map {geo.n_layers}x{geo.head_dim} {tokens} tokens {table}", flush=True)
    case = synth.SyntheticCase(geo, tokens, seed=0x4A5 + tokens)
    max_cells = 128
    n_pages = max_cells // geo.page_size + 3
    tables = None
    if table != "identity":
        tabs = []
        for j in range(geo.n_qsa):
            t = np.random.default_rng(j + tokens).permutation(n_pages)[:max_cells // geo.page_size].astype(np.int32)
            if table == "holes":
                t[1::3] = -1
            tabs.append(t)
        tables = sc.device_tables(tabs)
    slot = case.new_slot(max_cells=max_cells, n_pages=n_pages if tables else None, tables=tables, fill=0x33)
    case.carve_into(slot)
    _, total = sc.image_layout(geo, tokens)
    if total == 0:
        pytest.skip("an empty geometry has no payload")
    payload = sc.DeviceBuffer(total + 16, "uint8")
    plan = sc.plan_capture(geo, slot, tokens, payload.ptr, total)
    _compare(sc, oracle, [plan], payload, total, 0x5A)
    plan.destroy()


def test_fused_map_with_head_and_offsets(sc, oracle, cuda):
    """Blobs placed at caller offsets after a head of host bytes (the wire payload's shape): two capture plans into one
    payload (a main slot and a second slot, as a layer split's stage part), the head copied in before the launch, every
    gap zero-filled by the rows; a total that is not a whole lane segment."""
    geo = sc.geometry(**SMALL)
    tokens = 53
    a = synth.SyntheticCase(geo, tokens, seed=11)
    b = synth.SyntheticCase(geo, tokens, seed=12)
    sa, sb = a.new_slot(max_cells=64), b.new_slot(max_cells=64)
    a.carve_into(sa)
    b.carve_into(sb)
    blobs, image = sc.image_layout(geo, tokens)
    head = 4096 + 48
    total = head + 2 * image + 80
    payload = sc.DeviceBuffer(total, "uint8")
    plans = []
    for k, slot in enumerate((sa, sb)):
        base = head + k * image
        plans.append(sc.plan_capture(geo, slot, tokens, payload.ptr + base, image))
    head_bytes = np.random.default_rng(5).integers(0, 256, size=head, dtype=np.uint8)
    _compare(sc, oracle, plans, payload, total, 0x11, head=head_bytes)
    for p in plans:
        p.destroy()


def test_copy_plan_alone_and_as_rows_of_a_map(sc, oracle, cuda):
    """A plan of plain device copies (sc_plan_copies): launched on its own it writes exactly its copies (and nothing
    between them); as rows of a map beside a capture plan (a head staged in device memory and two small blobs, the
    wire encoder's use) the map writes the same payload as launching both plans, with the byte loop's hash - here with
    no head copied in before the launch: the map's copy rows write it."""
    geo = sc.geometry(**SMALL)
    tokens = 53
    case = synth.SyntheticCase(geo, tokens, seed=21)
    slot = case.new_slot(max_cells=64)
    case.carve_into(slot)
    _, image = sc.image_layout(geo, tokens)
    head, blob1, blob2 = 4096 + 48, 96, 64 * 1024 + 16
    at1 = head + image
    at2 = at1 + blob1 + 32          # a gap left as the payload holds it
    total = at2 + blob2 + 48       # and a tail past the last row
    rng = np.random.default_rng(9)
    staged_host = rng.integers(0, 256, size=head + blob1 + blob2, dtype=np.uint8)
    staged = sc.DeviceBuffer(staged_host.size, "uint8")
    staged.upload(staged_host)
    payload = sc.DeviceBuffer(total, "uint8")
    copies = [(payload.ptr, staged.ptr, head), (payload.ptr + at1, staged.ptr + head, blob1),
              (payload.ptr + at2, staged.ptr + head + blob1, blob2)]
    cp = sc.plan_copies(copies)
    assert cp.payload_bytes == head + blob1 + blob2
    payload.fill(0x5D)
    cp.launch()
    sc.device_sync()
    got = payload.numpy(total)
    want = np.full(total, 0x5D, np.uint8)
    want[:head] = staged_host[:head]
    want[at1:at1 + blob1] = staged_host[head:head + blob1]
    want[at2:at2 + blob2] = staged_host[head + blob1:]
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]
    cap = sc.plan_capture(geo, slot, tokens, payload.ptr + head, image)
    _compare(sc, oracle, [cap, cp], payload, total, 0x33)
    # the same map over a payload whose length is not a whole lane segment, a head inside the first workgroup only
    _compare(sc, oracle, [cp, cap], payload, at2 + blob2, 0x44)
    cap.destroy()
    cp.destroy()
    # refusals: overlapping destinations, unaligned or partial chunks
    for bad in ([(payload.ptr, staged.ptr, 64), (payload.ptr + 48, staged.ptr, 64)],
                [(payload.ptr + 8, staged.ptr, 64)], [(payload.ptr, staged.ptr, 40)]):
        with pytest.raises(sc.ScError):
            sc.plan_copies(bad)
    for b in (staged, payload):
        b.free()


def test_map_extent_boundaries_at_wave_and_workgroup_edges(sc, oracle, cuda):
    """Copy rows whose boundaries fall exactly on a wave's edge (16 KiB), on a workgroup's edge (64 KiB), 16 bytes
    past either, inside a lane segment, and three extents inside one workgroup, with gaps left as the payload holds
    them: every wave that lies inside one of its workgroup's first two extents takes the uniform gather, the others
    walk the extent table, and all give the payload the rows write and the byte loop's hash."""
    W, G = 16 << 10, 64 << 10
    cuts = [0, W, 2 * W + 16, G, G + 48, G + 64, 2 * G - 16, 2 * G + W, 3 * G, 3 * G + 4096, 5 * G + 256]
    total = 5 * G + 256 + 3 * W + 80     # then a gap, and a tail that is not a whole lane segment
    src = sc.DeviceBuffer(total, "uint8")
    data = np.random.default_rng(17).integers(0, 256, size=total, dtype=np.uint8)
    src.upload(data)
    payload = sc.DeviceBuffer(total, "uint8")
    copies = []
    for k in range(len(cuts) - 1):
        lo, hi = cuts[k], cuts[k + 1]
        if k % 4 == 3:
            continue                     # a gap: self bytes
        # every other row reads its bytes from a shifted place of the source, so a row boundary is also a source jump
        shift = 4096 * (k % 3)
        copies.append((payload.ptr + lo, src.ptr + (lo + shift) % (total - (hi - lo)) // 16 * 16, hi - lo))
    cp = sc.plan_copies(copies)
    _compare(sc, oracle, [cp], payload, total - 80 + 64, 0x6B)
    _compare(sc, oracle, [cp], payload, total, 0x6C)
    cp.destroy()
    src.free()
    payload.free()


def test_fused_map_with_large_zero_ranges(sc, oracle, cuda):
    """Zero ranges of a capture plan large enough to hold whole waves and workgroups (the uniform gather's zero
    extents, which write zeros without a load), one starting mid-workgroup and one across a workgroup's end, between a
    slot's blobs and after them: the map writes the zeros and the blobs the plan writes, with the byte loop's hash."""
    geo = sc.geometry(**SMALL)
    fmt, index, tokens = 1, True, 77
    pools = sc.LayerPools(geo, fmt, 96, index)
    pools.randomize(0x5E)
    sizes = sc.layer_blob_bytes(geo, fmt, index, tokens)
    G = 64 << 10
    at, offsets, zero = 896, [], []
    for j in range(geo.n_qsa):
        for b in range(5):
            offsets.append(at if sizes[b] else None)
            at += (sizes[b] + 63) // 64 * 64
        if j == 0:   # a zero range from inside a workgroup across its end and the whole next one
            zero += [at, 2 * G + 4096]
            at += 2 * G + 4096
    offsets.append(at)
    at += (geo.n_gdn * geo.gdn_row_floats * 4 + 63) // 64 * 64
    zero += [at, 3 * G + 48 * 16]   # after the blobs: three whole workgroups and a ragged end
    total = at + 3 * G + 48 * 16 + 64
    payload = sc.DeviceBuffer(total, "uint8")
    plan = sc.plan_capture_layers(geo, pools, tokens, payload.ptr, total, offsets=offsets, zero=zero)
    head = np.random.default_rng(3).integers(0, 256, size=896, dtype=np.uint8)
    _compare(sc, oracle, [plan], payload, total, 0xD7, head=head)
    plan.destroy()
    payload.free()


@pytest.mark.parametrize("fmt", [1, 2, 3])
@pytest.mark.parametrize("index", [False, True])
@pytest.mark.parametrize("tokens", [1, 77])
def test_fused_map_small_blobs_of_every_format(sc, oracle, cuda, fmt, index, tokens):
    """Blobs of a quantized slot packed as a wire payload's pool (64-byte aligned, in record order, after a head):
    with one token the scales and indexer rows are 32-512 bytes, so one lane segment holds the end of a code blob and
    two or three whole small blobs (a segment over three runs and more, the first ending at its extent's end)."""
    geo = sc.geometry(**SMALL)
    print(f"case hash map format {fmt} index {index} tokens {tokens}", flush=True)
    pools = sc.LayerPools(geo, fmt, 96, index)
    pools.randomize(0x3B + fmt)
    sizes = sc.layer_blob_bytes(geo, fmt, index, tokens)
    at, offsets = 896, []
    for _ in range(geo.n_qsa):
        for b in range(5):
            offsets.append(at if sizes[b] else None)
            at += (sizes[b] + 63) // 64 * 64
    offsets.append(at)
    total = at + geo.n_gdn * geo.gdn_row_floats * 4 + 48
    payload = sc.DeviceBuffer(total, "uint8")
    plan = sc.plan_capture_layers(geo, pools, tokens, payload.ptr, total, offsets=offsets)
    head = np.random.default_rng(fmt).integers(0, 256, size=896, dtype=np.uint8)
    _compare(sc, oracle, [plan], payload, total, 0xC4, head=head)
    plan.destroy()


def test_fused_map_at_full_size(sc, oracle, cuda):
    """Config 2's slot (48 layers, 32K tokens) captured into its image: the fused hash equals the plain hash of the
    captured image, and the image equals the capture's."""
    geo = sc.geometry()
    tokens = 32768
    case = synth.SyntheticCase(geo, tokens, seed=0x32)
    slot = case.new_slot(max_cells=tokens)
    case.carve_into(slot)
    _, total = sc.image_layout(geo, tokens)
    payload = sc.DeviceBuffer(total, "uint8")
    plan = sc.plan_capture(geo, slot, tokens, payload.ptr, total)
    hp = sc.HashPlan(total)
    payload.fill(0x77)
    plan.launch()
    hp.launch(payload.ptr, total)
    sc.device_sync()
    want = hp.result()
    want_bytes = sc.fnv1a64_device(payload.ptr, total)
    hmap = sc.HashMap([plan], payload.ptr, total)
    payload.fill(0x77)
    hmap.launch(hp)
    sc.device_sync()
    assert hp.result() == want == want_bytes
    assert sc.fnv1a64_device(payload.ptr, total) == want
    hmap.destroy()
    hp.free()


def test_hash_map_refusals(sc, cuda):
    geo = sc.geometry(**SMALL)
    case = synth.SyntheticCase(geo, 9, seed=3)
    slot = case.new_slot(max_cells=16)
    _, total = sc.image_layout(geo, 9)
    payload = sc.DeviceBuffer(total + 64, "uint8")
    carve = sc.plan_carve(geo, case.prefill, slot)
    with pytest.raises(sc.ScError) as e:
        sc.HashMap([carve], payload.ptr, total)
    assert e.value.code == sc.SC_EINVAL and "capture plans" in sc.last_error()
    capture = sc.plan_capture(geo, slot, 9, payload.ptr, total)
    with pytest.raises(sc.ScError):
        sc.HashMap([capture], payload.ptr, total - 64)        # a row past the payload
    with pytest.raises(sc.ScError):
        sc.HashMap([capture], payload.ptr + 8, total)         # misaligned
    with pytest.raises(sc.ScError):
        sc.HashMap([capture, capture], payload.ptr, total)    # two rows on the same bytes
