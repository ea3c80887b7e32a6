"""Seeded synthetic workloads for the tests, smoke() and the bench: prefill sequences generated on the device by the
library's counter-based generators (sc_fill_uniform_f16 / _f32, sc_fill_normal_f32), and the multi-slot batch of the
batched resume + append.  Not part of the hand-off interface (sc_handoff.py is); the CPU oracle regenerates the same
values from the same seeds and stream ids (oracle/sc_oracle.c)."""
from __future__ import annotations

import ctypes as C

import sc_handoff as sc


# Stream ids of the synthetic inputs (one counter stream per buffer).
def sid_k(j: int) -> int: return 1000 + 2 * j
def sid_v(j: int) -> int: return 1001 + 2 * j
def sid_rec(i: int) -> int: return 5000 + i
def sid_conv(i: int) -> int: return 9000 + i


def synthetic_prefill(geo: sc.Geometry, tokens: int, seed: int, kv_dtype: int = sc.SC_DTYPE_F16,
                      conv_rows: int | None = None, stream=None) -> sc.PrefillBuffers:
    """K/V ~ U[-4, 4] (f16, or f32 when kv_dtype is F32), recurrence and conv rows ~ N(0, 1) (Irwin-Hall 12),
    generated on the device by the library's counter-based generators."""
    H, D = geo.n_head_kv, geo.head_dim
    S, HV, Cc = geo.ssm_state_size, geo.ssm_v_heads, geo.ssm_conv_channels
    conv_rows = min(tokens, geo.ssm_d_conv - 1) if conv_rows is None else conv_rows
    s = sc._stream(stream)
    ks, vs, recs, convs = [], [], [], []
    for j in range(geo.n_qsa):
        for lst, sid in ((ks, sid_k(j)), (vs, sid_v(j))):
            n = tokens * H * D
            if kv_dtype == sc.SC_DTYPE_F16:
                t = sc.DeviceBuffer((max(tokens, 1), H, D), "uint16")
                sc.check(sc.lib.sc_fill_uniform_f16(t.ptr, n, -4.0, 4.0, seed, sid, s), "fill")
            else:
                t = sc.DeviceBuffer((max(tokens, 1), H, D), "float32")
                sc.check(sc.lib.sc_fill_uniform_f32(t.ptr, n, -4.0, 4.0, seed, sid, s), "fill")
            lst.append(t)
    for i in range(geo.n_gdn):
        r = sc.DeviceBuffer((HV, S, S), "float32")
        sc.check(sc.lib.sc_fill_normal_f32(r.ptr, r.numel(), seed, sid_rec(i), s), "fill")
        recs.append(r)
        c = sc.DeviceBuffer((max(conv_rows, 1), Cc), "float32")
        sc.check(sc.lib.sc_fill_normal_f32(c.ptr, conv_rows * Cc, seed, sid_conv(i), s), "fill")
        convs.append(c)
    return sc.PrefillBuffers(geo, tokens, ks, vs, recs, convs, conv_rows, kv_dtype)


class SyntheticCase:
    """A seeded prefill sequence on the device plus the helpers smoke() and the tests use."""

    def __init__(self, geo: sc.Geometry, tokens: int, seed: int, kv_dtype: int = sc.SC_DTYPE_F16):
        self.geo, self.tokens, self.seed = geo, tokens, seed
        self.prefill = synthetic_prefill(geo, tokens, seed, kv_dtype)

    def new_slot(self, max_cells: int, **kw) -> sc.Slot:
        return sc.new_slot(self.geo, max_cells, **kw)

    def carve_into(self, slot: sc.Slot, pos0: int = 0, stream=None) -> None:
        plan = sc.plan_carve(self.geo, self.prefill, slot, pos0)
        plan.launch(stream)
        sc.device_sync()
        plan.destroy()

    def host_inputs(self) -> dict:
        return self.prefill.host()


class BatchCase:
    """`n` slots with parked prefixes of lens[i] tokens (seeded images in pinned host memory) plus a fresh chunk of
    `chunk` tokens each, resumed and appended into shared per-layer page arenas through fragmented per-slot page
    tables.  Holds everything the batched plan reads and writes."""

    def __init__(self, geo: sc.Geometry, lens, chunk: int, seed: int, stream=None, fragmented: bool = True):
        import numpy as np
        self.geo, self.lens, self.chunk, self.seed = geo, list(lens), chunk, seed
        n = len(self.lens)
        ps = geo.page_size
        # parked images: gather each slot's seeded prefill into a device image, park it in pinned host memory
        self.images, self.image_bytes = [], []
        for i, L in enumerate(self.lens):
            case = SyntheticCase(geo, L, seed * 1000 + i)
            _, total = sc.image_layout(geo, L)
            dev = sc.DeviceBuffer(total, "uint8")
            plan = sc.plan_gather(geo, case.prefill, dev.ptr, total)
            plan.launch()
            host = sc.PinnedBuffer(total)
            sc.check(sc.lib.sc_copy_async(host.ptr, dev.ptr, total, None), "park copy")
            sc.device_sync()
            plan.destroy()
            dev.free()
            del case
            self.images.append(host)
            self.image_bytes.append(total)
        self.offsets, self.staging_bytes = sc.staging_layout(geo, self.lens)
        self.staging = sc.DeviceBuffer(max(self.staging_bytes, 16), "uint8")
        # fresh chunks, K/V only
        self.chunks = [synthetic_prefill(geo, chunk, seed * 1000 + 500 + i, conv_rows=0) for i in range(n)]
        # page tables: every slot's pages drawn from one shuffled arena (a fragmented allocator)
        self.table_pages = (max(self.lens) + chunk + ps - 1) // ps
        need = [(L + chunk + ps - 1) // ps for L in self.lens]
        self.arena_pages = sum(need) + 3
        rng = np.random.default_rng(seed)
        # fragmented: every page drawn from a shuffled arena; otherwise each slot gets one contiguous run
        order = (rng.permutation(self.arena_pages) if fragmented else np.arange(self.arena_pages)).astype(np.int32)
        self.host_tables, at = [], 0
        for k in need:
            t = np.full(self.table_pages, -1, dtype=np.int32)
            t[:k] = order[at:at + k]
            at += k
            self.host_tables.append(t)
        self.tables = sc.device_tables(self.host_tables)
        shape = (self.arena_pages, geo.n_head_kv, ps, geo.head_dim)
        self.arena_k = [sc.DeviceBuffer(shape, "uint16") for _ in range(geo.n_qsa)]
        self.arena_v = [sc.DeviceBuffer(shape, "uint16") for _ in range(geo.n_qsa)]
        for b in self.arena_k + self.arena_v:
            b.fill(0)
        self.gdn = [sc.DeviceBuffer((geo.n_gdn, geo.gdn_row_floats), "float32") for _ in range(n)] if geo.n_gdn else []
        self.lens_dev = sc.DeviceBuffer(n, "int64")
        self.lens_dev.upload(np.array(self.lens, dtype=np.int64))
        self.lens_out = sc.DeviceBuffer(n, "int64")
        self.lens_out.fill(0)
        sc.device_sync()

    @property
    def parked_bytes(self) -> int:
        return sum(self.image_bytes)

    def stage(self, stream=None) -> None:
        """The batched resume: one H2D copy per slot into the staging buffer at its offset."""
        for host, off, nbytes in zip(self.images, self.offsets, self.image_bytes):
            sc.check(sc.lib.sc_copy_async(self.staging.ptr + off, host.ptr, nbytes, sc._stream(stream)), "stage copy")

    def plan(self) -> sc.Plan:
        geo, n = self.geo, len(self.lens)
        ck = sc._ptrs([self.chunks[i].k[j].ptr for i in range(n) for j in range(geo.n_qsa)])
        cv = sc._ptrs([self.chunks[i].v[j].ptr for i in range(n) for j in range(geo.n_qsa)])
        ak = sc._ptrs([b.ptr for b in self.arena_k])
        av = sc._ptrs([b.ptr for b in self.arena_v])
        ts = sc._ptrs([t.ptr for t in self.tables])
        gs = sc._ptrs([g.ptr for g in self.gdn])
        P = C.POINTER(C.c_void_p)
        desc = sc.BatchDesc(n_slots=n, lens=self.lens_dev.ptr, max_tokens=max(self.lens), staging=self.staging.ptr,
                         staging_bytes=self.staging_bytes, chunk_tokens=self.chunk, chunk_k=C.cast(ck, P),
                         chunk_v=C.cast(cv, P), arena_k=C.cast(ak, P), arena_v=C.cast(av, P),
                         arena_pages=self.arena_pages, tables=C.cast(ts, P), table_pages=self.table_pages,
                         gdn=C.cast(gs, P), lens_out=self.lens_out.ptr)
        h = C.c_void_p()
        sc.check(sc.lib.sc_plan_resume_append(C.byref(self.geo), C.byref(desc), C.byref(h)), "sc_plan_resume_append")
        return sc.Plan(h.value, (ck, cv, ak, av, ts, gs))

    def slot_view(self, i: int) -> sc.Slot:
        """sc.Slot i as a decode slot: the shared arenas read through its page table."""
        return sc.Slot(self.geo, self.arena_pages, self.table_pages * self.geo.page_size, self.arena_k, self.arena_v,
                    self.gdn[i] if self.gdn else None, [self.tables[i]] * self.geo.n_qsa)

    def free(self) -> None:
        for h in self.images:
            h.free()
        self.images = []
