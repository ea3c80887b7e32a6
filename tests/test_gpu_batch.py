"""Batched ragged resume + append (configs 5): many slots, one launch, offsets computed on the device.

Parity rule (no reference counterpart for the multi-slot layout): each slot, read through its own page table,
equals the single-slot handoff of that slot's sequence - its parked prefix resumed and its chunk appended at cell
L_i.  Small cases compare every byte with the oracle; config 5 at full size compares every slot with the
single-slot HIP path (resume into an identity slot, then the fused carve of the chunk at pos0 = L_i).
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)


def _captured(sc, geo, slot, tokens):
    """The slot's first `tokens` tokens read through its page tables into an image (on the device, then host)."""
    _, total = sc.image_layout(geo, tokens)
    img = sc.DeviceBuffer(total, "uint8")
    plan = sc.plan_capture(geo, slot, tokens, img.ptr, total)
    plan.launch()
    sc.device_sync()
    out = img.numpy(total)
    plan.destroy()
    img.free()
    return out


def test_staging_layout_is_the_padded_prefix_sum(sc):
    geo = sc.geometry(**SMALL)
    lens = [0, 1, 7, 64, 130]
    offs, total = sc.staging_layout(geo, lens)
    at = 0
    for L, off in zip(lens, offs):
        assert off == at
        at += -(-sc.image_layout(geo, L)[1] // 256) * 256
    assert total == at


@pytest.mark.parametrize("lens,chunk", [([0, 1, 7, 64, 130], 9), ([5, 3, 2, 1], 1), ([33] * 7 + [100], 16),
                                        ([4096, 1001, 2], 2048)])
def test_batch_matches_oracle(sc, oracle, cuda, lens, chunk):
    geo = sc.geometry(**SMALL)
    case = synth.BatchCase(geo, lens, chunk, seed=len(lens) * 7 + chunk)
    case.stage()
    plan = case.plan()
    plan.launch()
    sc.device_sync()
    assert list(case.lens_out.numpy()) == [L + chunk for L in lens]
    for i, L in enumerate(lens):
        # oracle: the parked image resumed into an identity slot, then the chunk appended at cell L
        n_pages = case.table_pages
        state = oracle.new_state(geo, n_pages)
        oracle.resume(geo, L, case.images[i].numpy(), state)
        inputs = case.chunks[i].host()
        inputs["rec"], inputs["conv"] = [], []
        oracle.carve_into(geo, inputs, state, n_pages, pos0=L, with_gdn=False)
        want = oracle.park(geo, L + chunk, state)
        got = _captured(sc, geo, case.slot_view(i), L + chunk)
        assert np.array_equal(got, want), f"slot {i} (L={L})"
    case.free()


def test_batch_is_all_or_nothing(sc, cuda):
    """One length beyond max_tokens refuses the whole batch on the device: nothing is written, lens_out is -1."""
    geo = sc.geometry(**SMALL)
    lens = [12, 40, 7]
    case = synth.BatchCase(geo, lens, 5, seed=3)
    case.stage()
    plan = case.plan()
    case.lens_dev.upload(np.array([12, max(lens) + 1, 7], dtype=np.int64))
    for b in case.arena_k + case.arena_v + case.gdn:
        b.fill(0x5C)
    sc.device_sync()
    plan.launch()
    sc.device_sync()
    assert list(case.lens_out.numpy()) == [-1, -1, -1]
    for b in case.arena_k + case.arena_v + case.gdn:
        assert np.all(b.numpy().view(np.uint8) == 0x5C)
    # the same plan with valid lengths then runs normally (lengths are read at launch time)
    case.lens_dev.upload(np.array(lens, dtype=np.int64))
    plan.launch()
    sc.device_sync()
    assert list(case.lens_out.numpy()) == [L + 5 for L in lens]
    case.free()


def test_config5_full_size_equals_single_slot_path(sc, cuda):
    """Config 5: 8 slots, L_i ~ U[1K, 128K] from a seed, 2K-token chunks, 48-layer geometry; every slot read through
    its table equals the single-slot path (resume into an identity slot + fused carve of the chunk at L_i)."""
    geo = sc.geometry()
    rng = np.random.default_rng(0x5EED)
    lens = [int(x) for x in rng.integers(1024, 131072 + 1, size=8)]
    chunk = 2048
    case = synth.BatchCase(geo, lens, chunk, seed=5)
    case.stage()
    plan = case.plan()
    plan.launch()
    sc.device_sync()
    assert list(case.lens_out.numpy()) == [L + chunk for L in lens]
    for i, L in enumerate(lens):
        single = sc.new_slot(geo, L + chunk)
        sc.device_sync()
        sc.resume_async(geo, case.images[i].ptr, case.image_bytes[i], L, single)
        carve = sc.plan_carve(geo, case.chunks[i], single, pos0=L, with_gdn=False)
        carve.launch()
        sc.device_sync()
        want = _captured(sc, geo, single, L + chunk)
        got = _captured(sc, geo, case.slot_view(i), L + chunk)
        assert np.array_equal(got, want), f"slot {i} (L={L})"
        carve.destroy()
        del single
    case.free()
