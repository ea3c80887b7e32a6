"""Full-size parity: every byte of the 32K and 128K handoffs (configs 2 and 3) and of every slot of config 5, compared
with the CPU oracle through per-blob FNV-1a hashes.

The oracle computes each blob's hash straight from the counter-based generators (sco_synth_kv_blob_hash,
sco_synth_gdn_hash; pinned on the CPU against fill -> carve -> park in tests/test_oracle.py), without materialising the
expected bytes.  The device hashes the same blob with the library's parallel FNV-1a (pinned against the byte loop in
tests/test_gpu_hash.py).  A wrong byte anywhere in a 3.3 GB slot changes its blob's hash, so a plan-builder offset error
past a layer index or past 2^31 bytes fails here.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

MAX_BLOB = 131072 * 2 * 256 * 2   # the largest blob at the configs: one 128K-token K or V pool prefix


def _hashes(hp, spans):
    out = []
    for ptr, n in spans:
        hp.launch(ptr, n)
        out.append(hp.result())
    return out


def _slot_spans(geo, slot, tokens):
    """The image blobs of an identity slot, in place: K and V pool prefixes per QSA layer, then every GDN row."""
    kv = geo.cells(tokens) * geo.n_head_kv * geo.head_dim * 2
    spans = []
    for j in range(geo.n_qsa):
        spans += [(slot.k_pool[j].ptr, kv), (slot.v_pool[j].ptr, kv)]
    spans.append((slot.gdn.ptr, geo.n_gdn * geo.gdn_row_floats * 4))
    return spans


def _image_spans(sc, geo, ptr, tokens):
    blobs, _ = sc.image_layout(geo, tokens)
    return [(ptr + b.offset, b.bytes) for b in blobs]


def _mismatch(got, want):
    bad = [i for i, (a, b) in enumerate(zip(got, want)) if a != b]
    return f"{len(bad)} of {len(want)} blobs differ, first blob {bad[0] if bad else None}"


@pytest.mark.parametrize("tokens", [32768, 131072, 131069])
def test_full_depth_oracle_hash(sc, oracle, cuda, tokens):
    """Configs 2 and 3 (and a 128K sequence ending mid-page): the fused carve into an identity slot, the two-pass
    transfer buffer, and the carve through a shuffled page table captured back out, each equal to the oracle in every
    blob.  The slot starts filled with 0x5A, so the cells of a partial last page that the carve does not write are
    checked too (the transfer buffer zeroes them)."""
    geo = sc.geometry()
    seed = 0x5EED + tokens
    print(f"oracle hashes for {tokens} tokens", flush=True)
    want_slot = oracle.synthetic_image_hashes(geo, tokens, seed, tail=0x5A)
    want_image = oracle.synthetic_image_hashes(geo, tokens, seed, tail=0) if tokens % geo.page_size else want_slot
    hp = sc.HashPlan(MAX_BLOB)
    case = synth.SyntheticCase(geo, tokens=tokens, seed=seed)
    slot = case.new_slot(max_cells=geo.cells(tokens), fill=0x5A)
    case.carve_into(slot)
    got = _hashes(hp, _slot_spans(geo, slot, tokens))
    assert got == want_slot, "fused carve: " + _mismatch(got, want_slot)
    del slot
    _, total = sc.image_layout(geo, tokens)
    image = sc.DeviceBuffer(total, "uint8")
    image.fill(0x77)
    gather = sc.plan_gather(geo, case.prefill, image.ptr, total)
    gather.launch()
    sc.device_sync()
    got = _hashes(hp, _image_spans(sc, geo, image.ptr, tokens))
    assert got == want_image, "gather: " + _mismatch(got, want_image)
    n_pages = geo.cells(tokens) // geo.page_size
    perm = np.random.default_rng(tokens).permutation(n_pages).astype(np.int32)
    paged = case.new_slot(max_cells=geo.cells(tokens), tables=sc.device_tables([perm] * geo.n_qsa), fill=0x5A)
    sc.device_sync()
    carve = sc.plan_carve(geo, case.prefill, paged)
    carve.launch()
    image.fill(0x77)
    capture = sc.plan_capture(geo, paged, tokens, image.ptr, total)
    capture.launch()
    sc.device_sync()
    got = _hashes(hp, _image_spans(sc, geo, image.ptr, tokens))
    assert got == want_slot, "paged carve: " + _mismatch(got, want_slot)
    hp.free()


def test_full_depth_oracle_hash_f32_rows(sc, oracle, cuda):
    """Config 2 from f32 K/V rows (rounded to f16 by the carve): the same bytes as the f16 sequence of the same seed,
    as RNE rounding of the generator's f32 values is the f16 generator."""
    geo = sc.geometry()
    tokens = 32768
    want = oracle.synthetic_image_hashes(geo, tokens, 0xF32)
    case = synth.SyntheticCase(geo, tokens=tokens, seed=0xF32, kv_dtype=sc.SC_DTYPE_F32)
    slot = case.new_slot(max_cells=tokens)
    case.carve_into(slot)
    hp = sc.HashPlan(MAX_BLOB)
    got = _hashes(hp, _slot_spans(geo, slot, tokens))
    assert got == want, _mismatch(got, want)
    hp.free()


def test_config5_every_slot_matches_oracle_hash(sc, oracle, cuda):
    """Config 5: 8 slots, L_i ~ U[1K, 128K] from the seed, a 2K-token chunk each, one launch.  Every slot read through
    its fragmented page table equals, blob for blob, the oracle's image of its parked prefix with the chunk appended
    at cell L_i (two sources per K/V blob), and its GDN rows equal the oracle's."""
    geo = sc.geometry()
    rng = np.random.default_rng(0x5EED)
    lens = [int(x) for x in rng.integers(1024, 131072 + 1, size=8)]
    chunk, seed = 2048, 5
    case = synth.BatchCase(geo, lens, chunk, seed=seed)
    case.stage()
    plan = case.plan()
    plan.launch()
    sc.device_sync()
    assert list(case.lens_out.numpy()) == [L + chunk for L in lens]
    hp = sc.HashPlan(MAX_BLOB + (chunk + 4) * 2 * 256 * 2)
    image = sc.DeviceBuffer(sc.image_layout(geo, max(lens) + chunk)[1], "uint8")
    for i, L in enumerate(lens):
        print(f"slot {i}: {L} + {chunk} tokens", flush=True)
        want = oracle.synthetic_image_hashes(geo, L, seed * 1000 + i, chunk=(seed * 1000 + 500 + i, chunk))
        _, total = sc.image_layout(geo, L + chunk)
        capture = sc.plan_capture(geo, case.slot_view(i), L + chunk, image.ptr, total)
        capture.launch()
        sc.device_sync()
        got = _hashes(hp, _image_spans(sc, geo, image.ptr, L + chunk))
        assert got == want, f"slot {i} (L={L}): " + _mismatch(got, want)
        capture.destroy()
    hp.free()
    case.free()


@pytest.mark.parametrize("fmt", ["int8", "q4_0", "k8v4"])
def test_quant_carve_128k_every_blob(sc, oracle, cuda, fmt):
    """Config 3's quantizing carves (the bench's quant_carve rows): f32 K/V rows of 131072 tokens into int8, q4_0 and
    K8V4 pools plus the GDN rows, in one launch; every pool blob (codes, and scales where the format has them) and the
    GDN rows equal the oracle's streamed hashes (sco_synth_quant_blob_hash over sco_q8_row / sco_q4_row, pinned on the
    CPU against the materialised quantizers), so every byte of the 128K carve is compared."""
    geo = sc.geometry()
    tokens = 131072
    code = {"int8": sc.SC_KV_INT8, "q4_0": sc.SC_KV_Q4, "k8v4": sc.SC_KV_K8V4}[fmt]
    seed = 0x5EED + 0x8
    print(f"oracle hashes for the {fmt} carve of {tokens} tokens", flush=True)
    want = oracle.synthetic_quant_hashes(geo, tokens, seed, code, tail=0x5A)
    case = synth.SyntheticCase(geo, tokens=tokens, seed=seed, kv_dtype=sc.SC_DTYPE_F32)
    slot = sc.new_quant_slot(geo, code, tokens, fill=0x5A)
    plan = sc.plan_carve_quant(geo, case.prefill, slot)
    plan.launch()
    sc.device_sync()
    plan.destroy()
    del case
    spans = []
    for j in range(geo.n_qsa):
        spans += [(slot.k_codes[j].ptr, slot.k_codes[j].nbytes), (slot.v_codes[j].ptr, slot.v_codes[j].nbytes)]
        if slot.k_scale:
            spans.append((slot.k_scale[j].ptr, slot.k_scale[j].nbytes))
        if slot.v_scale:
            spans.append((slot.v_scale[j].ptr, slot.v_scale[j].nbytes))
    spans.append((slot.gdn.ptr, slot.gdn.nbytes))
    hp = sc.HashPlan(MAX_BLOB)
    got = _hashes(hp, spans)
    assert got == want, f"{fmt}: " + _mismatch(got, want)
    hp.free()
