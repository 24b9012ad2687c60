"""GPU parity of the prefill path: qg_moe_forward above 17 tokens (grouped
GEMMs over device-built per-expert row lists).

Bars as for the decode path: routing ids, weights, coverage flags, pruning
counters and the CSR dispatch are bit-exact against the oracle; fp32 layer
outputs within max-abs 1e-3 and rel-L2 1e-4.  Full 2048-token outputs would
take the scalar oracle minutes, so outputs are checked on every token of the
small batches and on a seeded sample of the large ones (tokens are
independent in this layer, so a sample row equals the oracle's layer applied
to that row alone).  Expert bytes for the oracle are copied from the device
(the device generator is checked equal to the oracle's in
test_gpu_parity.py).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
from nebula_amd import qg, synth
from nebula_amd.qg import Device, call

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 1e-3, 1e-4

CFG3 = synth.LayerSpec(seed=300, gate_type=12, up_type=12, down_type=20, bias_seed=33)
CFG1 = synth.LayerSpec(seed=200, gate_type=12, up_type=12, down_type=20, shared=True, sh_types=(12, 12, 12))
CFG0 = synth.LayerSpec(seed=100, gate_type=12, up_type=12, down_type=12)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def assert_close(got, want, what=""):
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    diff = g - w
    maxabs = float(np.abs(diff).max()) if diff.size else 0.0
    rel = float(np.linalg.norm(diff) / max(np.linalg.norm(w), 1e-30))
    assert maxabs <= MAX_ABS and rel <= REL_L2, f"{what}: max-abs {maxabs:.3g} rel-L2 {rel:.3g}"
    return maxabs, rel


def host_layer(spec):
    return O.HostLayer(spec.seed, width=spec.width, ff=spec.ff, gt=spec.gate_type, ut=spec.up_type, dt=spec.down_type,
                       shared=spec.shared, sh_types=spec.sh_types,
                       router_bias=None if spec.bias_seed is None else synth.zipf_bias(spec.bias_seed))


def fetcher(L):
    return lambda name, e: synth.read_expert(L, name, e)


@pytest.fixture(scope="module")
def layer3(qgl):
    say("building config-3 layer on device")
    return synth.build_layer(CFG3), host_layer(CFG3)


@pytest.fixture(scope="module")
def layer1(qgl):
    say("building config-1 layer on device")
    return synth.build_layer(CFG1), host_layer(CFG1)


@pytest.fixture(scope="module")
def layer0(qgl):
    say("building config-0 layer on device")
    return synth.build_layer(CFG0), host_layer(CFG0)


def forward(L, x):
    nt = x.shape[0]
    fw = synth.Forward(L.spec.width, L.spec.ff, nt)
    fw.x.set(x)
    say(f"prefill forward nt={nt}")
    fw.run(L, nt)
    qg.call("sync")
    return fw


def check_routing(fw, H, x, resident=None):
    """ids/weights/flags of every token bit-exact; returns the oracle's (ids, w, flags)."""
    nt = x.shape[0]
    ids, w = O.route(H.logits(x))
    flags = np.zeros(nt, np.uint8)
    if resident is not None:
        flags, _ = O.coverage(ids, w, resident)
        ids, w, _ = O.prune(ids, w, resident)
    np.testing.assert_array_equal(fw.ids.get()[:nt], ids, err_msg="routing ids")
    np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), w.view('u4'), err_msg="routing weights")
    np.testing.assert_array_equal(fw.flags.get()[:nt], flags, err_msg="flags")
    return ids, w, flags


def check_outputs(fw, L, H, x, rows, what, resident=None):
    out, oids, ow, _, oflags, _ = H.forward(x[rows], resident, fetch=fetcher(L))
    got = fw.out.get()[rows]
    keep = oflags < 2
    maxabs, rel = assert_close(got[keep], out[keep], what)
    from test_gpu_parity import check_flagged_rows
    check_flagged_rows(got, H, x[rows], oflags, what)
    say(f"  {what}: {len(rows)} rows, max-abs {maxabs:.2e}, rel-L2 {rel:.2e}")


def sample_rows(nt, k, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([np.arange(min(4, nt)), np.arange(nt - 4, nt), rng.choice(nt, k, replace=False)]))


def test_prefill_config3_routing_dispatch_outputs(layer3):
    """Config 3: 2048 tokens, Zipf(1.1)-biased router, Q4_K gate/up, IQ4_NL down."""
    L, H = layer3
    x = synth.inputs(3003, 2048, 2048)
    fw = forward(L, x)
    ids, w, _ = check_routing(fw, H, x)
    n = np.bincount(ids.ravel(), minlength=512)
    say(f"  per-expert rows: max {n.max()}, >=256: {(n >= 256).sum()} experts / {n[n >= 256].sum()} rows, "
        f"empty {(n == 0).sum()}")
    assert n.max() >= 256, "the Zipf bias should make a dense pass"
    # the CSR dispatch entry point (same histogram/scan/fill kernels) on these ids
    off, tok, slot, status = (Device(shape=(513,), dtype=np.int32), Device(shape=(20480,), dtype=np.int32),
                              Device(shape=(20480,), dtype=np.int32), Device(shape=(1,), dtype=np.int32))
    call("moe_dispatch", off.p, tok.p, slot.p, status.p, fw.ids.p, 2048)
    ooff, otok, oslot = O.dispatch(ids)
    assert status.get()[0] == 0
    np.testing.assert_array_equal(off.get(), ooff)
    np.testing.assert_array_equal(tok.get(), otok)
    np.testing.assert_array_equal(slot.get(), oslot)
    # outputs on a sample that covers the dense experts' rows
    dense = np.flatnonzero(n >= 256)
    rows_dense = np.flatnonzero(np.isin(ids, dense).any(axis=1))
    rows = np.union1d(sample_rows(2048, 40, 7), rows_dense[:: max(1, len(rows_dense) // 16)])
    check_outputs(fw, L, H, x, rows, "config3 B=2048")


def test_prefill_wide_hidden_item_ring_refill(qgl):
    """D = 8192 (the widest accepted width) at 8192 tokens: each persistent
    workgroup of the down pass runs about 250 items, so its ring of decoded
    items (128 entries, refilled 64 at a time) is refilled and reread several
    times.  Routing of sampled rows bit-exact, their outputs within the bars."""
    spec = synth.LayerSpec(seed=8192, width=8192, ff=512, gate_type=12, up_type=12, down_type=20)
    say("building a 8192/512 layer on device")
    L, H = synth.build_layer(spec), host_layer(spec)
    nt = 8192
    x = synth.inputs(8193, nt, 8192)
    fw = forward(L, x)
    rows = sample_rows(nt, 12, 13)
    ids, w = O.route(H.logits(x[rows]))
    np.testing.assert_array_equal(fw.ids.get()[rows], ids, err_msg="routing ids")
    np.testing.assert_array_equal(fw.w.get()[rows].view('u4'), w.view('u4'), err_msg="routing weights")
    all_ids = fw.ids.get()[:nt]
    n = np.bincount(all_ids.ravel(), minlength=512)
    tiles = int(np.sum((n + 63) // 64))
    say(f"  tiles {tiles}: about {tiles * 32 // 256} down items per workgroup on 256 CUs")
    assert tiles * 32 > 128 * 256, "the item ring must be refilled and reread"
    check_outputs(fw, L, H, x, rows, "8192/512 B=8192")


@pytest.mark.parametrize("mode", [1, 2])
def test_prefill_dense_split_launches(layer3, layer1, mode):
    """The dense experts' gate/up in a launch of their own
    (qg_prefill_int8_dense: mode 1 on int8 matrix cores, mode 2 on fp16):
    config 3's dense experts, and a 300-token config-1 batch with correlated
    routing (dense experts next to the shared expert), against the oracle at
    the same bars."""
    prev = qg.lib().qg_prefill_int8_dense(mode)
    try:
        L, H = layer3
        x = synth.inputs(3003, 2048, 2048)
        fw = forward(L, x)
        ids, _, _ = check_routing(fw, H, x)
        n = np.bincount(ids.ravel(), minlength=512)
        dense = np.flatnonzero(n >= 256)
        rows_dense = np.flatnonzero(np.isin(ids, dense).any(axis=1))
        check_outputs(fw, L, H, x, rows_dense[:: max(1, len(rows_dense) // 24)], f"config3 dense launch, mode {mode}")
        L1, H1 = layer1
        x1 = synth.inputs(3101, 300, L1.spec.width, correlated=True)
        fw1 = forward(L1, x1)
        check_routing(fw1, H1, x1)
        check_outputs(fw1, L1, H1, x1, sample_rows(300, 24, 5), f"300 correlated tokens, mode {mode}")
    finally:
        qg.lib().qg_prefill_int8_dense(prev)


def test_prefill_concentrated_routing(qgl):
    """A router bias that sends nearly every token to the same few experts:
    six experts take over 2000 of the 2048 tokens (32 tiles each, the same
    row-count bucket, so their pass order falls back to expert id), ten more
    share most of the remaining selections and the tail reaches the other
    experts; the shared expert sits after the dense ones, and the XCD shares
    are cut inside such groups.  Routing bit-exact, sampled rows against the
    oracle."""
    spec = synth.LayerSpec(seed=207, gate_type=12, up_type=12, down_type=20, shared=True, sh_types=(12, 12, 12))
    bias = np.zeros(512, np.float32)
    rng = np.random.default_rng(207)
    hot = rng.choice(512, 16, replace=False)
    bias[hot[:6]] = 6.0
    bias[hot[6:]] = 3.0
    L = synth.build_layer(spec)
    L.bufs["router_bias"] = Device(bias)
    L.desc.router_bias = L.bufs["router_bias"].p
    H = O.HostLayer(spec.seed, width=spec.width, ff=spec.ff, gt=spec.gate_type, ut=spec.up_type, dt=spec.down_type,
                    shared=spec.shared, sh_types=spec.sh_types, router_bias=bias)
    x = synth.inputs(3207, 2048, spec.width)
    fw = forward(L, x)
    ids, _, _ = check_routing(fw, H, x)
    n = np.bincount(ids.ravel(), minlength=512)
    say(f"  per-expert rows: top {np.sort(n)[::-1][:8].tolist()}, >=256: {(n >= 256).sum()}, touched {(n > 0).sum()}")
    assert (n >= 2000).sum() == 6 and (n >= 256).sum() >= 16, "six hot experts, ten warm ones"
    check_outputs(fw, L, H, x, sample_rows(2048, 32, 11), "concentrated routing, B=2048")


@pytest.mark.parametrize("nt", [18, 33, 100])
def test_prefill_q4k_down_every_token(layer0, nt):
    """Config-0 formats (Q4_K down, min terms in both products), every row checked;
    partial 64-row tiles and row tiles skipped past the group's end."""
    L, H = layer0
    x = synth.inputs(400 + nt, nt, 2048, correlated=(nt == 100))
    fw = forward(L, x)
    check_routing(fw, H, x)
    check_outputs(fw, L, H, x, np.arange(nt), f"config0 B={nt}")


@pytest.mark.parametrize("ff,shared", [(128, False), (256, True)])
def test_prefill_narrow_ff_step_counts(ff, shared):
    """F = 128 and 256 at D = 1024: the down items have one or two K steps, so
    the weight copies two steps ahead belong to the next item or the one after
    (F = 128), and the Q4_K shared down (F = 256) has a single superblock step;
    every row checked."""
    spec = synth.LayerSpec(seed=430 + ff, width=1024, ff=ff, gate_type=12, up_type=12, down_type=20, shared=shared,
                           sh_types=(12, 12, 12))
    say(f"building a 1024/{ff} layer on device")
    L, H = synth.build_layer(spec), host_layer(spec)
    nt = 150
    x = synth.inputs(440 + ff, nt, 1024, correlated=True)
    fw = forward(L, x)
    check_routing(fw, H, x)
    check_outputs(fw, L, H, x, np.arange(nt), f"1024/{ff} B={nt}")


def test_prefill_shared_expert_mixed_formats(layer1):
    """Config-1 formats: IQ4_NL routed down, Q4_K shared down (its own down
    launch), sigmoid-gated shared expert on every token; correlated rows give
    dense experts (>= 256 rows)."""
    L, H = layer1
    nt = 600
    x = synth.inputs(601, nt, 2048, correlated=True)
    fw = forward(L, x)
    ids, _, _ = check_routing(fw, H, x)
    n = np.bincount(ids.ravel(), minlength=512)
    say(f"  unique experts {np.count_nonzero(n)}, dense {(n >= 256).sum()}")
    check_outputs(fw, L, H, x, sample_rows(nt, 24, 11), "config1-formats B=600")


def test_prefill_partial_residency(layer1):
    """Config-4 semantics at a prefill size: coverage flags and pruning
    bit-exact, counters equal, handoff rows holding the shared part alone."""
    L, H = layer1
    nt = 200
    # correlated rows, ranked on their own routing, so that the batch mixes
    # fully covered (0), pruned (1) and handoff (2) tokens
    x = synth.inputs(77, nt, 2048, correlated=True)
    ids_all, w_all = O.route(H.logits(x))
    score = np.zeros(512)
    np.add.at(score, ids_all.ravel(), w_all.ravel().astype(np.float64))
    resident = np.zeros(512, np.uint8)
    resident[np.lexsort((np.arange(512), -score))[:20]] = 1
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    rdev = Device(resident)
    desc.resident, desc.threshold = rdev.p, 0.10
    saved = L.desc
    L.desc = desc
    try:
        fw = synth.Forward(2048, 512, nt)
        fw.x.set(x)
        call("zero", fw.stats.p, fw.stats.nbytes)
        say(f"prefill forward with residency nt={nt}")
        fw.run(L, nt)
        qg.call("sync")
        _, _, flags = check_routing(fw, H, x, resident)
        counts = np.bincount(flags, minlength=4)
        say(f"  flags: {counts}")
        assert counts[0] > 0 and counts[1] > 0 and counts[2] > 0, counts
        # counters from the oracle's prune over the same routing
        ids, w = O.route(H.logits(x))
        _, _, ost = O.prune(ids, w, resident)
        gst = qg.PruneStats.from_buffer_copy(fw.stats.get())
        assert (gst.token_layers, gst.missing_selections, gst.skipped_selections, gst.avoided_token_handoffs) == \
               (ost.token_layers, ost.missing_selections, ost.skipped_selections, ost.avoided_token_handoffs)
        assert abs(gst.skipped_mass - ost.skipped_mass) <= 1e-12 * max(1.0, abs(ost.skipped_mass))
        check_outputs(fw, L, H, x, sample_rows(nt, 20, 5), "residency B=200", resident=resident)
    finally:
        L.desc = saved


def test_prefill_handoff_round_trip(layer1):
    """The CPU handoff at a prefill size (200 tokens, 20 resident experts):
    nm_moe_handoff packs the flag-2 tokens (count and rows checked against the
    oracle's flags), the oracle computes their routed part, and after the
    merge sampled rows of every flag match the oracle's full layer."""
    from test_gpu_parity import _cpu_moe_callback
    L, H = layer1
    nt = 200
    x = synth.inputs(77, nt, 2048, correlated=True)
    ids_all, w_all = O.route(H.logits(x))
    score = np.zeros(512)
    np.add.at(score, ids_all.ravel(), w_all.ravel().astype(np.float64))
    resident = np.zeros(512, np.uint8)
    resident[np.lexsort((np.arange(512), -score))[:20]] = 1
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    rdev = Device(resident)
    desc.resident, desc.threshold = rdev.p, 0.10
    saved = L.desc
    L.desc = desc
    try:
        fw = synth.Forward(2048, 512, nt)
        fw.x.set(x)
        say(f"prefill forward with residency nt={nt}")
        fw.run(L, nt)
        qg.call("sync")
    finally:
        L.desc = saved
    flags, _ = O.coverage(ids_all, w_all, resident)
    np.testing.assert_array_equal(fw.flags.get()[:nt], flags)
    want = np.nonzero(flags == 2)[0]
    assert 0 < len(want) < nt
    h = qg.host()
    sb = h.nm_handoff_scratch_bytes(2048, nt)
    scratch = Device(nbytes=sb)
    calls = []
    cb = _cpu_moe_callback(H, calls, fetch=fetcher(L))
    handed = C.c_int(-1)
    say(f"prefill handoff round trip: {len(want)} of {nt} tokens to the host")
    assert h.nm_moe_handoff(fw.out.p, None, fw.flags.p, fw.x.p, fw.ids.p, fw.w.p, nt, 2048, scratch.p, sb, cb, None,
                            C.byref(handed)) == 0, h.nm_last_error()
    assert handed.value == len(want) and len(calls) == 1
    np.testing.assert_array_equal(calls[0][0].view('u4'), x[want].view('u4'))
    rows = np.unique(np.concatenate([sample_rows(nt, 16, 3), want[:8]]))
    out, _, _, _, oflags, _ = H.forward(x[rows], resident, fetch=fetcher(L))
    ok = oflags < 3
    maxabs, rel = assert_close(fw.out.get()[rows][ok], out[ok], "prefill handoff round trip")
    say(f"  {len(rows)} sampled rows, max-abs {maxabs:.2e}, rel-L2 {rel:.2e}")


def test_prefill_residual_matches_forward(layer1):
    """qg_moe_forward_residual at a prefill size: h + MoE(RMSNorm(h))."""
    L, H = layer1
    nt = 40
    h0 = (synth.inputs(940, nt, 2048, correlated=True) * 3.0).astype(np.float32)
    fw = synth.Forward(2048, 512, nt)
    hd = Device(h0)
    xn = Device(shape=(nt, 2048), dtype=np.float32)
    out = Device(shape=(nt, 2048), dtype=np.float32)
    say(f"prefill forward_residual nt={nt}")
    call("moe_forward_residual", hd.p, fw.ids.p, fw.w.p, fw.flags.p, None, xn.p, out.p, nt, C.byref(L.desc), fw.ws.p,
         fw.ws_bytes)
    qg.call("sync")
    xs = xn.get()
    np.testing.assert_allclose(xs, synth.rmsnorm(h0), rtol=2e-6, atol=2e-6)
    want, ids, w, *_ = H.forward(xs, fetch=fetcher(L))
    np.testing.assert_array_equal(fw.ids.get()[:nt], ids)
    np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), w.view('u4'))
    assert_close(out.get(), want, "residual B=40")
    np.testing.assert_array_equal(hd.get(), (h0 + out.get()).astype(np.float32))


def test_prefill_graph_replay(layer3):
    """The prefill layer captured into a graph and replayed, with eager work
    in between, equals the eager result every time."""
    L, _ = layer3
    nt = 96
    fw = synth.Forward(2048, 512, nt)
    fw.x.set(synth.inputs(5, nt, 2048))
    fw.run(L, nt)
    qg.call("sync")
    eager = fw.out.get()
    g = C.c_void_p()
    say("graph capture of the prefill layer")
    call("graph_begin", C.byref(g))
    fw.run(L, nt)
    call("graph_end", g)
    for rep in range(3):
        call("zero", fw.out.p, fw.out.nbytes)
        call("sync")
        call("graph_launch", g)
        call("sync")
        np.testing.assert_array_equal(fw.out.get().view('u4'), eager.view('u4'), err_msg=f"replay {rep}")
    qg.lib().qg_graph_destroy(g)


def test_prefill_rejects_unsupported(layer1, qgl):
    """Prefill needs Q4_K gate/up: another format above 17 tokens is an error
    (below, the decode kernels take it)."""
    L, _ = layer1
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    desc.gate_type = 20
    fw = synth.Forward(2048, 512, 18)
    assert qgl.qg_moe_forward(fw.out.p, fw.ids.p, fw.w.p, None, None, fw.x.p, 18, C.byref(desc), fw.ws.p, fw.ws_bytes) != 0
    assert qgl.qg_moe_workspace_bytes(2048, 512, 8193) == 0
