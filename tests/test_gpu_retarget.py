"""A carve plan re-pointed at other prefill sequences (sc_plan_retarget) carves each one exactly as a plan built for it
would: the decode slot after every retarget + launch equals the oracle's carve of that sequence on top of what the slot
held (oracle.expected_slot with `initial`, the restatement of kv_append's row map, src/prefill/kernels.cu:560-601, and
of the GDN carve), through identity and shuffled page tables (the latter in destination order), for fewer tokens,
a mid-page pos0 without the GDN rows, f32 rows on a plan built from f16 ones, and several retargets queued back to back
on one stream without a wait.  A view the plan cannot hold is refused and the plan keeps carving its last target."""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

GEO = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
           ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520)
CAP = 300   # the slot's cells, and the view the plan is built with


def _assert_state(got: dict, want: dict, what: str):
    for name in want:
        if not np.array_equal(got[name].view(np.uint8), want[name].view(np.uint8)):
            raise AssertionError(f"{what}: {name} differs from the oracle")


@pytest.mark.parametrize("paged", [False, True])
def test_retargets_equal_fresh_carves(sc, oracle, cuda, paged):
    geo = sc.geometry(**GEO)
    print(f"case retarget paged={paged}", flush=True)
    n_pages = CAP // geo.page_size + 5
    tables = host_tables = None
    previous = sc.lib.sc_set_order_min_pages(1) if paged else None   # small tables in destination order too
    try:
        if paged:
            host_tables = [np.random.default_rng(40 + j).permutation(n_pages)[:CAP // geo.page_size].astype(np.int32)
                           for j in range(geo.n_qsa)]
            tables = sc.device_tables(host_tables)
        slot = sc.new_slot(geo, CAP, n_pages=n_pages if paged else None, tables=tables)
        first = synth.SyntheticCase(geo, CAP, seed=0xA0)
        plan = sc.plan_carve(geo, first.prefill, slot)
        assert plan.order_groups == (geo.n_qsa if paged else 0)
        stream = sc.Stream()
        plan.launch(stream)
        stream.sync()
        state = oracle.expected_slot(geo, first.host_inputs(), CAP, tables=host_tables,
                                     n_pages=n_pages if paged else None)
        _assert_state(slot.host_state(), state, "the build's own carve")
        targets = [   # (tokens, pos0, with_gdn, dtype)
            (77, 0, True, sc.SC_DTYPE_F16),
            (29, 61, False, sc.SC_DTYPE_F16),     # an appended chunk: mid-page, K/V only
            (CAP, 0, True, sc.SC_DTYPE_F32),      # f32 rows rounded to f16 on a plan built from f16 rows
            (0, 0, True, sc.SC_DTYPE_F16),        # no K/V: the GDN rows alone
            (150, 150, False, sc.SC_DTYPE_F16),
        ]
        for k, (tokens, pos0, with_gdn, dtype) in enumerate(targets):
            case = synth.SyntheticCase(geo, tokens, seed=0xB0 + k, kv_dtype=dtype)
            plan.retarget(case.prefill, pos0=pos0, with_gdn=with_gdn, stream=stream)
            plan.launch(stream)
            stream.sync()
            state = oracle.expected_slot(geo, case.host_inputs(), CAP, pos0=pos0, tables=host_tables,
                                         n_pages=n_pages if paged else None, initial=state, with_gdn=with_gdn)
            _assert_state(slot.host_state(), state, f"retarget {k} ({tokens} tokens at {pos0})")
        # back to back on one stream, no wait in between: each launch carves its own target
        cases = [synth.SyntheticCase(geo, t, seed=0xC0 + t) for t in (120, 40, 200, 300, 8)]
        for case in cases:
            plan.retarget(case.prefill, stream=stream)
            plan.launch(stream)
        stream.sync()
        for case in cases:
            state = oracle.expected_slot(geo, case.host_inputs(), CAP, tables=host_tables,
                                         n_pages=n_pages if paged else None, initial=state)
        _assert_state(slot.host_state(), state, "queued retargets")
        # refusals leave the plan as it was: the next launch carves the last target again
        over = synth.SyntheticCase(geo, CAP + 4, seed=0xD0)
        with pytest.raises(sc.ScError) as e:
            plan.retarget(over.prefill, stream=stream)
        assert e.value.code == sc.SC_EINVAL
        with pytest.raises(sc.ScError) as e:
            plan.retarget(cases[0].prefill, pos0=CAP - 100, stream=stream)
        assert e.value.code == sc.SC_EINVAL
        slot.fill(0x3C)
        sc.device_sync()
        plan.launch(stream)
        stream.sync()
        base = oracle.new_state(geo, n_pages if paged else CAP // geo.page_size)
        for key in base:
            base[key].view(np.uint8)[...] = 0x3C
        want = oracle.expected_slot(geo, cases[-1].host_inputs(), CAP, tables=host_tables,
                                    n_pages=n_pages if paged else None, initial=base)
        _assert_state(slot.host_state(), want, "the last target after refusals")
        plan.destroy()
    finally:
        if previous is not None:
            sc.lib.sc_set_order_min_pages(previous)


def test_retarget_capacity_and_kind(sc, cuda):
    """A plan built for fewer tokens, or without the GDN rows, refuses a view that needs more (SC_ERANGE); only carve
    plans can be retargeted."""
    geo = sc.geometry(**GEO)
    slot = sc.new_slot(geo, CAP)
    small = synth.SyntheticCase(geo, 40, seed=1)
    plan = sc.plan_carve(geo, small.prefill, slot, with_gdn=False)
    big = synth.SyntheticCase(geo, 200, seed=2)
    with pytest.raises(sc.ScError) as e:
        plan.retarget(big.prefill, with_gdn=False)
    assert e.value.code == sc.SC_ERANGE and "larger handoff table" in sc.last_error()
    with pytest.raises(sc.ScError) as e:
        plan.retarget(small.prefill, with_gdn=True)
    assert e.value.code == sc.SC_ERANGE and "GDN" in sc.last_error()
    plan.retarget(synth.SyntheticCase(geo, 33, seed=3).prefill, with_gdn=False)   # fewer tokens fit
    plan.destroy()
    _, total = sc.image_layout(geo, 40)
    image = sc.DeviceBuffer(total, "uint8")
    gather = sc.plan_gather(geo, small.prefill, image.ptr, total)
    with pytest.raises(sc.ScError) as e:
        gather.retarget(small.prefill)
    assert e.value.code == sc.SC_EINVAL and "only a carve plan" in sc.last_error()
    gather.destroy()
