"""Slot images in every K/V format: blob sizes, the image layout, and the C-ABI's refusals (CPU only).

The oracle's sizes (layer_blob_bytes) restate layout() of src/core/conversation_snapshot.cpp:27-66; they are pinned by
the reference's own per-cell figures (generate.cpp's --kv help: int8 1,056 B/cell, K8V4 816 B/cell for the model's two
KV heads of 256) and by the f16 layout the published payload totals fix.  The image layout (image_layout_layers) is the
wire pool order; it is pinned by the oracle codec, which reproduces the reference codec's bytes (including records with
int8 scales and indexer rows): an image whose buffers have these sizes is encoded and every buffer is found by its
content at the offset the layout gives.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import sc_wire

FORMATS = [0, 1, 2, 3]
TOKENS = [0, 1, 3, 4, 5, 77, 4096]


def _small(sc):
    return sc.geometry(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
                       ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)


@pytest.mark.parametrize("fmt,per_cell", [(0, 2048), (1, 1056), (2, 576), (3, 816)])
def test_bytes_per_cell_match_the_reference(oracle, sc, fmt, per_cell):
    """K + V + scales per cell and layer for 2 KV heads of 256: fp16 2048, int8 1056 and K8V4 816 (the reference's
    --kv help text), q4_0 2 x 8 blocks of 18 bytes."""
    geo = sc.geometry()
    for T in (4, 64, 131072):
        b = oracle.layer_blob_bytes(geo, fmt, False, T)
        assert sum(b[:4]) == per_cell * T
        assert b[4] == 0


def test_pooled_rows_are_completed_blocks_plus_the_spare(oracle, sc):
    geo = sc.geometry()
    assert oracle.layer_blob_bytes(geo, 0, True, 0)[4] == 0
    for T, rows in ((1, 1), (3, 1), (4, 2), (5, 2), (131072, 32769)):
        assert oracle.layer_blob_bytes(geo, 1, True, T)[4] == rows * 128 * 4


def test_f16_without_index_is_the_image_layout(oracle, sc):
    for geo in (sc.geometry(), _small(sc)):
        for T in TOKENS:
            offs, total = oracle.image_layout_layers(geo, 0, False, T)
            blobs, total_f16 = oracle.image_layout(geo, T)
            assert total == total_f16
            want = [b[2] for b in blobs if b[3]]   # the f16 layout also lists zero-byte K/V blobs at 0 tokens
            assert [o for o in offs if o is not None] == want


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("index", [False, True])
def test_layout_is_where_the_codec_puts_the_blobs(oracle, sc, fmt, index):
    """The slot image equals the pool of the wire payload of the same image: encode the image with distinct contents
    in every buffer and find each buffer where the layout says it is."""
    geo = _small(sc)
    n_qsa = geo.n_layers // geo.qsa_interval
    for T in (1, 5, 77):
        sizes = oracle.layer_blob_bytes(geo, fmt, index, T)
        offs, total = oracle.image_layout_layers(geo, fmt, index, T)
        cells = (T + 3) // 4 * 4
        salt = 1
        kv = []
        for _ in range(n_qsa):
            k = {"format": fmt, "cells": cells, "heads": 2, "head_dim": 256, "page_size": 4,
                 "pooled_rows": sizes[4] // 512, "idx_dim": 128}
            for name, n in zip(sc_wire.KV_BUFFERS, sizes):
                k[name] = sc_wire._pattern(salt, n)
                salt += 1
            kv.append(k)
        gdn_bytes = (geo.n_layers - n_qsa) * int(sc.lib.sc_gdn_row_floats(C.byref(geo))) * 4
        live = {"ids": np.arange(T, dtype=np.int32), "imgs": [], "gdn": sc_wire._pattern(999, gdn_bytes), "ple": b"",
                "tails": b"", "dead": b"", "block_pos": b"", "used": 0, "stage_parts": []}
        image = {"geometry": [0] * 18, "layer_lo": 0, "layer_hi": geo.n_layers, "cvec": False, "kv": kv, "live": live,
                 "checkpoints": [], "stage_parts": []}
        payload = sc_wire.encode(image)
        sc_wire.decode(payload)   # the codec accepts its own payload
        # blob_pool_off: the header word after magic/version/flags, the 18 geometry words and 6 count words
        pool_off = int(np.frombuffer(payload[8 + 18 * 8 + 6 * 8: 8 + 18 * 8 + 7 * 8], dtype="<u8")[0])
        assert len(payload) - pool_off == total   # the pool is exactly the slot image
        for j in range(n_qsa):
            for b, name in enumerate(sc_wire.KV_BUFFERS):
                o = offs[j * 5 + b]
                if sizes[b]:
                    assert o is not None and payload[pool_off + o: pool_off + o + sizes[b]] == kv[j][name], (j, name)
                else:
                    assert o is None
        assert payload[pool_off + offs[-1]: pool_off + offs[-1] + gdn_bytes] == live["gdn"]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("index", [False, True])
def test_c_abi_layout_equals_the_oracle(oracle, sc, fmt, index):
    for geo in (sc.geometry(), _small(sc)):
        for T in TOKENS + [131072]:
            assert sc.layer_blob_bytes(geo, fmt, index, T) == oracle.layer_blob_bytes(geo, fmt, index, T)
            assert sc.image_layout_layers(geo, fmt, index, T) == oracle.image_layout_layers(geo, fmt, index, T)


def test_refusals_before_any_device_work(sc):
    geo = sc.geometry(head_dim=32)
    with pytest.raises(sc.ScError):            # int8 groups of 64 do not divide head_dim 32
        sc.layer_blob_bytes(geo, sc.SC_KV_INT8, False, 8)
    assert sc.layer_blob_bytes(geo, sc.SC_KV_Q4, False, 8)[0] == 8 * 2 * 18
    with pytest.raises(sc.ScError):
        sc.layer_blob_bytes(sc.geometry(), 7, False, 8)   # unknown format
    with pytest.raises(sc.ScError):
        sc.layer_blob_bytes(sc.geometry(), 0, False, -1)
    with pytest.raises(sc.ScError):            # a GDN row that is not whole 16-byte chunks
        sc.layer_blob_bytes(sc.geometry(ssm_conv_channels=10), 0, False, 8)
    # a capture of a slot with a missing buffer is refused on the host (SC_EINVAL, nothing enqueued)
    geo = _small(sc)
    st = sc.SlotLayers(format=sc.SC_KV_INT8, with_index=0, max_cells=16, pooled_capacity=0, gdn_state=None)
    h = C.c_void_p()
    rc = sc.lib.sc_plan_capture_layers(C.byref(geo), C.byref(st), 8, C.c_void_p(16), 1 << 20, None, C.byref(h))
    assert rc == sc.SC_EINVAL and "missing" in sc.last_error()
