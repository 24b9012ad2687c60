"""GPU parity tests through libqwen_gpu.so's C ABI against the CPU oracle.

Bars: routing ids, weights, coverage flags, dispatch permutations and the
drop-in qg_matmul are bit-exact; fp32 layer outputs are within max-abs 1e-3
and rel-L2 1e-4 of the oracle (the tolerance stated for this path).
Inputs are seeded; weights are generated on the device and, independently,
on the host by the oracle's generator (their bytes are checked equal).
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


def check_flagged_rows(got, H, x, flags, what):
    """Handoff rows (flag 2) hold the sigmoid-gated shared expert alone (its
    routed part is the host's, qwen.c:658-678; the shared expert stays on the
    device, qwen.c:661-663), or 0 without one; invalid rows (flag 3) are 0."""
    h = flags == 2
    if h.any():
        if H.shared:
            assert_close(got[h], H.shared_part(x[h]), f"{what}: handoff rows (shared part)")
        else:
            assert np.all(got[h] == 0), f"{what}: handoff rows"
    assert np.all(got[flags == 3] == 0), f"{what}: invalid rows"


def legal_blocks(rng, typ, rows, cols):
    from test_oracle_cpu import legal_blocks as lb
    return np.ascontiguousarray(lb(rng, typ, rows, cols))


# ---------------- generator ----------------

@pytest.mark.parametrize("typ,rows,cols", [(0, 3, 2048), (12, 5, 2048), (20, 7, 512), (12, 4, 512)])
def test_device_generator_matches_host(qgl, typ, rows, cols):
    say(f"synth type={typ} {rows}x{cols}")
    strm = synth.stream(synth.GATE, 37)
    dev = Device(nbytes=rows * qg.row_bytes(typ, cols))
    qg.call("synth_matrix", dev.p, typ, 1234, strm, rows, cols, qg.F(0.02))
    np.testing.assert_array_equal(dev.get(), O.fill_matrix(typ, 1234, strm, rows, cols))
    # several experts of one tensor in one launch: expert e from stream (tensor << 32 | e)
    per = rows * qg.row_bytes(typ, cols)
    many = Device(nbytes=3 * per)
    qg.call("synth_experts", many.p, typ, 1234, synth.UP, 3, rows, cols, qg.F(0.02))
    got = many.get()
    for e in range(3):
        np.testing.assert_array_equal(got[e * per:(e + 1) * per], O.fill_matrix(typ, 1234, synth.stream(synth.UP, e), rows, cols))


# ---------------- drop-in operators ----------------

def test_matmul_bitexact_all_formats(qgl):
    """qg_matmul == the oracle (== cpu.c qc_matmul) bit for bit, every format,
    the batch tails of qwen/test_gpu.py:157."""
    rng = np.random.default_rng(812603)
    for typ in (0, 1, 30, 2, 6, 7, 8, 12, 13, 14, 20):
        for cols in ((512, 2048) if typ in (12, 13, 14) else (320, 640)):
            rows = 13
            w = legal_blocks(rng, typ, rows, cols)
            dw = Device(w)
            for nt in (1, 4, 16, 17, 33, 512):
                say(f"matmul type={typ} cols={cols} nt={nt}")
                x = rng.normal(0, .2, (nt, cols)).astype(np.float32)
                dx, out = Device(x), Device(shape=(nt, rows), dtype=np.float32)
                call("matmul", out.p, dw.p, typ, rows, cols, dx.p, nt)
                np.testing.assert_array_equal(out.get().view('u4'), O.matmul(w, typ, rows, cols, x).view('u4'),
                                              err_msg=f"type {typ} cols {cols} nt {nt}")


def test_matmul_tiled_shapes_bitexact(qgl):
    """The tiled Q4_K / IQ4_NL path of qg_matmul (widths a multiple of 256)
    at dense-projection widths: several K chunks per block, every token-tile
    size (1, 4, 8, 16, 20 and tails past them), rows not a multiple of 8, and a
    matrix tall enough for two rows per lane;
    bit for bit against the oracle."""
    rng = np.random.default_rng(91011)
    for typ in (12, 20):
        for rows, cols in ((37, 2560), (9, 6144), (8, 256), (8203, 256)):
            w = legal_blocks(rng, typ, rows, cols)
            dw = Device(w)
            for nt in (1, 2, 5, 8, 9, 17, 20, 21):
                say(f"matmul tiled type={typ} {rows}x{cols} nt={nt}")
                x = rng.normal(0, .5, (nt, cols)).astype(np.float32)
                dx, out = Device(x), Device(shape=(nt, rows), dtype=np.float32)
                call("matmul", out.p, dw.p, typ, rows, cols, dx.p, nt)
                np.testing.assert_array_equal(out.get().view('u4'), O.matmul(w, typ, rows, cols, x).view('u4'),
                                              err_msg=f"type {typ} {rows}x{cols} nt {nt}")


def test_matmul_unaligned_operands_bitexact(qgl):
    """Q4_K rows and x at addresses that are only 4-byte aligned take the
    byte-granular kernel; results stay bit for bit the oracle's."""
    rng = np.random.default_rng(27)
    rows, cols, nt = 11, 512, 5
    w = legal_blocks(rng, 12, rows, cols)
    x = rng.normal(0, .5, (nt, cols)).astype(np.float32)
    dw = Device(nbytes=w.nbytes + 16)
    dx = Device(nbytes=x.nbytes + 16)
    call("write", dw.p + 4, w.ctypes.data, w.nbytes)
    call("write", dx.p + 4, x.ctypes.data, x.nbytes)
    out = Device(shape=(nt, rows), dtype=np.float32)
    say("matmul unaligned Q4_K")
    call("matmul", out.p, dw.p + 4, 12, rows, cols, dx.p + 4, nt)
    np.testing.assert_array_equal(out.get().view('u4'), O.matmul(w, 12, rows, cols, x).view('u4'))


def test_forward_rejects_unaligned_pointers(layer1):
    """qg_moe_forward / _residual with a misaligned activation, output or
    expert pointer return an invalid-value error (nothing is launched)."""
    L, _ = layer1
    nt = 4
    fw = synth.Forward(2048, 512, nt)
    bad_desc = qg.MoeLayer.from_buffer_copy(L.desc)
    bad_desc.gate = bad_desc.gate + 4
    cases = [("x", fw.out.p, fw.x.p + 4, L.desc), ("out", fw.out.p + 4, fw.x.p, L.desc), ("gate", fw.out.p, fw.x.p, bad_desc)]
    for what, out, x, desc in cases:
        say(f"forward with misaligned {what}")
        rc = qg.lib().qg_moe_forward(out, fw.ids.p, fw.w.p, fw.flags.p, None, x, nt, C.byref(desc), fw.ws.p, fw.ws_bytes)
        assert rc != 0, what
    rc = qg.lib().qg_moe_forward_residual(fw.x.p + 4, fw.ids.p, fw.w.p, fw.flags.p, None, None, None, nt, C.byref(L.desc),
                                          fw.ws.p, fw.ws_bytes)
    assert rc != 0
    qg.call("sync")


def test_matmul_router_shape_and_errors(qgl):
    rng = np.random.default_rng(1)
    w = rng.normal(0, .02, (512, 2048)).astype(np.float32)
    x = rng.normal(0, 1, (2048, 2048)).astype(np.float32)
    dw, dx, out = Device(w), Device(x), Device(shape=(2048, 512), dtype=np.float32)
    say("matmul router 512x2048 nt=2048")
    call("matmul", out.p, dw.p, 0, 512, 2048, dx.p, 2048)
    got = out.get()
    for t in (0, 1, 777, 2047):
        np.testing.assert_array_equal(got[t].view('u4'), O.matmul(w, 0, 512, 2048, x[t:t + 1])[0].view('u4'))
    # odd F32 width (partial last lane step), as the reference's k<cols loop allows
    w2 = rng.normal(0, .1, (5, 100)).astype(np.float32)
    x2 = rng.normal(0, 1, (3, 100)).astype(np.float32)
    o2, dw2, dx2 = Device(shape=(3, 5), dtype=np.float32), Device(w2), Device(x2)
    call("matmul", o2.p, dw2.p, 0, 5, 100, dx2.p, 3)
    np.testing.assert_allclose(o2.get(), x2.astype(np.float64) @ w2.T.astype(np.float64), rtol=1e-5, atol=1e-5)
    assert qgl.qg_matmul(out.p, dw.p, 12, 512, 100, dx.p, 1) != 0  # Q4_K needs 256-multiples
    assert qgl.qg_matmul(out.p, dw.p, 0, 512, 2048, dx.p, 8193) != 0


def test_route_matches_oracle_and_kat(qgl):
    rng = np.random.default_rng(812603)
    logits = (rng.normal(size=(300, 512))).astype(np.float32)
    logits[0] = 0
    logits[1, 100:120] = logits[1, 5]  # ties
    # heavy ties (more candidates than a 32-lane half ranks) in either half of a token pair
    logits[2, 3:200:3] = logits[2].max() + 1.0
    logits[9, 40:90] = logits[9].max() + 0.5
    logits[10, :] = 0.25
    dl = Device(logits)
    ids, w = Device(shape=(300, 10), dtype=np.int32), Device(shape=(300, 10), dtype=np.float32)
    oi, ow = O.route(logits)
    for nt in (300, 299, 1):
        say(f"route {nt} tokens")
        call("route", ids.p, w.p, dl.p, nt)
        np.testing.assert_array_equal(ids.get()[:nt], oi[:nt])
        np.testing.assert_array_equal(w.get()[:nt].view('u4'), ow[:nt].view('u4'))
    np.testing.assert_array_equal(ids.get()[:, :10], np.argsort(-logits, axis=1, kind='stable')[:, :10])
    logits[5, 7] = np.nan
    logits[6, 511] = -np.inf
    dl.set(logits)
    call("route", ids.p, w.p, dl.p, 300)
    np.testing.assert_array_equal(ids.get()[[5, 6]], -1)
    np.testing.assert_array_equal(w.get()[[5, 6]], 0)


def test_prune_known_answer_gpu(qgl):
    """qwen/test_gpu.py:84-95 on the device."""
    ids = np.tile(np.arange(10, dtype=np.int32), (5, 1))
    weights = np.full((5, 10), .1, np.float32)
    resident = np.zeros(512, np.uint8)
    resident[:8] = 1
    weights[0, 8:] = .04; weights[1, 8:] = .05; weights[2, 8:] = .06; weights[3, 8:] = 0; weights[4, 8:] = [.01, .10]
    di, dw, dr, dc = Device(ids), Device(weights), Device(resident), Device(nbytes=C.sizeof(qg.PruneStats))
    say("prune KAT")
    call("prune_routes", di.p, dw.p, dr.p, 5, .10, dc.p)
    actual = di.get()
    assert np.all(actual[[0, 3], 8:] <= -2)
    np.testing.assert_array_equal(actual[[1, 2, 4]], ids[[1, 2, 4]])
    np.testing.assert_array_equal(dw.get()[:, :8], weights[:, :8])
    st = qg.PruneStats.from_buffer_copy(dc.get())
    assert (st.token_layers, st.missing_selections, st.skipped_selections, st.avoided_token_handoffs) == (5, 10, 4, 2)
    oi, ow, ost = O.prune(ids, weights, resident)
    np.testing.assert_array_equal(actual, oi)
    np.testing.assert_array_equal(dw.get(), ow)
    assert st.skipped_mass == ost.skipped_mass
    assert qgl.qg_prune_routes(di.p, dw.p, dr.p, 5, .2, dc.p) != 0


def test_moe_map_and_dispatch(qgl):
    """qwen/test_gpu.py:352-359 at nt 511/513/1025/2048 and the CSR dispatch."""
    rng = np.random.default_rng(812603)
    for nt in (1, 17, 511, 513, 1025, 2048):
        say(f"map/dispatch nt={nt}")
        ids = np.stack([rng.choice(512, 10, replace=False) for _ in range(nt)]).astype(np.int32)
        dids = Device(ids)
        mapping = Device(shape=(512, nt), dtype=np.int32)
        call("moe_map", mapping.p, dids.p, nt)
        om, counts = O.moe_map(ids)
        got = mapping.get()
        for e in range(512):
            np.testing.assert_array_equal(got[e, :counts[e]], om[e, :counts[e]])
        off, tok, slot, status = (Device(shape=(513,), dtype=np.int32), Device(shape=(nt * 10,), dtype=np.int32),
                                  Device(shape=(nt * 10,), dtype=np.int32), Device(shape=(1,), dtype=np.int32))
        call("moe_dispatch", off.p, tok.p, slot.p, status.p, dids.p, nt)
        ooff, otok, oslot = O.dispatch(ids)
        assert status.get()[0] == 0
        np.testing.assert_array_equal(off.get(), ooff)
        np.testing.assert_array_equal(tok.get()[:len(otok)], otok)
        np.testing.assert_array_equal(slot.get()[:len(oslot)], oslot)
    # pruned encodings (-e-2) are skipped
    pruned = ids.copy()
    pruned[::7, 9] = -pruned[::7, 9] - 2
    dids = Device(pruned)
    call("moe_dispatch", off.p, tok.p, slot.p, status.p, dids.p, nt)
    ooff, otok, oslot = O.dispatch(pruned)
    assert status.get()[0] == 0
    np.testing.assert_array_equal(off.get(), ooff)
    np.testing.assert_array_equal(tok.get()[:len(otok)], otok)
    np.testing.assert_array_equal(slot.get()[:len(oslot)], oslot)
    # invalid ids and duplicates set the status
    for r, k, v in ((3, 4, 700), (5, 2, -1), (9, 1, -600), (11, 8, None)):
        bad = ids.copy()
        bad[r, k] = bad[r, 0] if v is None else v
        dids = Device(bad)
        call("moe_dispatch", off.p, tok.p, slot.p, status.p, dids.p, nt)
        assert status.get()[0] != 0, (r, k, v)


def test_gather_scatter_reduce_order_independent(qgl):
    """qwen/test_gpu.py:361-384: warm/cold expert order must not change the
    router-rank summation."""
    rng = np.random.default_rng(812603)
    call("moe_configure", 2560, 640)
    nt = 4
    ids = np.stack([rng.choice(27, 10, replace=False) for _ in range(nt)]).astype(np.int32)
    weights = np.exp((rng.normal(size=(nt, 10)) * .2).astype(np.float32))
    weights /= weights.sum(1, keepdims=True)
    values = (rng.normal(size=(27, nt, 2560)) * 6).astype(np.float32)
    dids, dw = Device(ids), Device(weights.astype(np.float32))
    mapping = Device(shape=(512, nt), dtype=np.int32)
    call("moe_map", mapping.p, dids.p, nt)
    slots = Device(shape=(nt, 10, 2560), dtype=np.float32)
    out = Device(shape=(nt, 2560), dtype=np.float32)
    expected = np.zeros((nt, 2560), np.float32)
    for k in range(10):
        expected += values[ids[:, k], np.arange(nt)] * weights[:, k, None]
    results = []
    for order in (np.unique(ids), rng.permutation(np.unique(ids))):
        call("zero", slots.p, slots.nbytes)
        for expert in order:
            selected = (ids == expert).any(1)
            dx = Device(values[expert])
            compact = Device(shape=values[expert].shape, dtype=np.float32)
            token_map = mapping.p + int(expert) * nt * 4
            call("moe_gather", compact.p, dx.p, token_map, int(selected.sum()))
            np.testing.assert_array_equal(compact.get()[:selected.sum()], values[expert, selected])
            call("moe_scatter", slots.p, compact.p, dw.p, dids.p, token_map, int(expert), int(selected.sum()))
        call("moe_reduce", out.p, slots.p, nt)
        results.append(out.get())
    np.testing.assert_array_equal(results[0], results[1])
    np.testing.assert_allclose(results[0], expected, atol=2e-5, rtol=2e-5)


def _mtp_oracle(x, ids, weights, gate, up, down, D, Fd, dt):
    """slots/mid of gpu.cu:528-543 from the oracle's fixed-order products."""
    nt = x.shape[0]
    gb, ub, db = Fd * O.row_bytes(12, D), Fd * O.row_bytes(12, D), D * O.row_bytes(dt, Fd)
    slots = np.full((nt, 10, D), np.nan, np.float32)
    mid = np.full((nt, 10, Fd), np.nan, np.float32)
    for t in range(nt):
        for k in range(10):
            e = int(ids[t, k])
            if not 0 <= e < 512:
                continue
            g = O.matmul(gate[e * gb:(e + 1) * gb], 12, Fd, D, x[t:t + 1])[0]
            u = O.matmul(up[e * ub:(e + 1) * ub], 12, Fd, D, x[t:t + 1])[0]
            ex = np.array([O.lib().nbo_expf(float(-v)) for v in g], np.float32)
            m = (g * (np.float32(1) / (np.float32(1) + ex))) * u
            mid[t, k] = m
            slots[t, k] = O.matmul(down[e * db:(e + 1) * db], dt, D, Fd, m[None])[0] * weights[t, k]
    return slots, mid


@pytest.mark.parametrize("D,Fd,nt", [(2560, 640, 4), (2560, 640, 17), (2048, 512, 4), (2048, 512, 17)])
def test_mtp_moe(qgl, D, Fd, nt):
    """qwen/test_gpu.py:164-187: up to seventeen rows, Q4_K gate/up, IQ4_NL
    down, repeated ids across tokens, 18 rows rejected.  Up to four rows at the
    2560/640 shape run the fixed-order kernels (bit-exact with cpu.c); the other
    cases run the fast GEMV (2048/512, <= 4 rows) or matrix-core kernels
    (> 4 rows) and are held to a tolerance."""
    rng = np.random.default_rng(812603)
    call("moe_configure", D, Fd)
    nexp = 3
    gate = legal_blocks(rng, 12, nexp * Fd, D).reshape(-1)
    up = legal_blocks(rng, 12, nexp * Fd, D).reshape(-1)
    down = legal_blocks(rng, 20, nexp * D, Fd).reshape(-1)
    for arr in (gate, up):
        v = arr.reshape(-1, 144)
        v[:, :2] = np.array([.0002], 'f2').view('u1')
        v[:, 2:4] = np.array([.0001], 'f2').view('u1')
    down.reshape(-1, 18)[:, :2] = np.array([.0002], 'f2').view('u1')
    x = (rng.normal(size=(nt, D)) * .2).astype(np.float32)
    ids = rng.integers(0, nexp, (nt, 10)).astype(np.int32)
    ids[2, 3] = -1
    scales = rng.uniform(.01, .2, (nt, 10)).astype(np.float32)
    dx, di, dw = Device(x), Device(ids), Device(scales)
    mid = Device(shape=(nt, 10, Fd), dtype=np.float32)
    slots = Device(shape=(nt, 10, D), dtype=np.float32)
    dg, du, dd = Device(gate), Device(up), Device(down)
    say(f"mtp_moe D={D} F={Fd} nt={nt}")
    call("mtp_moe", slots.p, mid.p, dx.p, di.p, dw.p, dg.p, 12, du.p, 12, dd.p, 20, nt)
    want_slots, want_mid = _mtp_oracle(x, ids, scales, gate, up, down, D, Fd, 20)
    got_slots, got_mid = slots.get(), mid.get()
    assert np.all(np.isnan(got_slots[2, 3])) and np.all(np.isnan(got_mid[2, 3]))
    ok = ~np.isnan(want_slots[..., 0])
    if D == 2560 and nt <= 4:
        np.testing.assert_array_equal(got_mid[ok].view('u4'), want_mid[ok].view('u4'))
        np.testing.assert_array_equal(got_slots[ok].view('u4'), want_slots[ok].view('u4'))
    else:
        for got, want in ((got_mid[ok], want_mid[ok]), (got_slots[ok], want_slots[ok])):
            np.testing.assert_allclose(got, want, atol=2e-5, rtol=5e-5)
            assert np.linalg.norm(got - want) <= 1e-5 * np.linalg.norm(want)
    assert qgl.qg_mtp_moe(slots.p, mid.p, dx.p, di.p, dw.p, dg.p, 12, du.p, 12, dd.p, 20, 18) != 0
    call("moe_configure", 2560, 640)


# ---------------- the fused device-driven layer ----------------

CFG0 = synth.LayerSpec(seed=100, gate_type=12, up_type=12, down_type=12)
CFG1 = synth.LayerSpec(seed=200, gate_type=12, up_type=12, down_type=20, shared=True, sh_types=(12, 12, 12))


@pytest.fixture(scope="module")
def layer0(qgl):
    say("building config-0 layer on device")
    L = synth.build_layer(CFG0)
    H = O.HostLayer(CFG0.seed, gt=12, ut=12, dt=12)
    return L, H


@pytest.fixture(scope="module")
def layer1(qgl):
    say("building config-1 layer on device")
    L = synth.build_layer(CFG1)
    H = O.HostLayer(CFG1.seed, gt=12, ut=12, dt=20, shared=True, sh_types=(12, 12, 12))
    return L, H


def _check_layer(L, H, x, what, resident=None, fw=None):
    nt = x.shape[0]
    fw = fw if fw is not None else synth.Forward(2048, 512, nt)
    fw.x.set(np.concatenate([x, np.zeros((fw.tokens - nt, 2048), np.float32)]) if nt < fw.tokens else x)
    say(f"forward {what} nt={nt}")
    fw.run(L, nt)
    qg.call("sync")
    out, ids, w, logits, flags, st = H.forward(x, resident)
    gi, gw = fw.ids.get()[:nt], fw.w.get()[:nt]
    np.testing.assert_array_equal(gi, ids, err_msg=f"{what}: routing ids")
    np.testing.assert_array_equal(gw.view('u4'), w.view('u4'), err_msg=f"{what}: routing weights")
    gf = fw.flags.get()[:nt]
    np.testing.assert_array_equal(gf, flags, err_msg=f"{what}: flags")
    keep = gf < 2
    maxabs, rel = assert_close(fw.out.get()[:nt][keep], out[keep], what)
    check_flagged_rows(fw.out.get()[:nt], H, x, gf, what)
    say(f"  {what}: unique experts {len(np.unique(ids[ids >= 0]))}, max-abs {maxabs:.2e}, rel-L2 {rel:.2e}")
    return fw, st


def test_layer_config0_batch1(layer0):
    L, H = layer0
    for seed in (1, 2, 3):
        _check_layer(L, H, synth.inputs(seed, 1, 2048), f"config0 seed{seed}")


@pytest.mark.parametrize("nt", list(range(1, 18)))
def test_layer_config1_verify_batches(layer1, nt):
    L, H = layer1
    _check_layer(L, H, synth.inputs(50 + nt, nt, 2048, correlated=True), f"config1 B={nt}")


def test_layer_workspace_reused_across_calls(layer1):
    """One workspace through consecutive verify batches of different sizes:
    every call's routing and output match the oracle, so nothing of an
    earlier call's plan (the per-expert token masks among it) leaks into the
    next one."""
    L, H = layer1
    fw = synth.Forward(2048, 512, 17)
    for i, nt in enumerate((17, 8, 17, 4, 17, 2, 17)):
        _check_layer(L, H, synth.inputs(70 + i, nt, 2048, correlated=(i % 2 == 0)), f"reused workspace call {i} B={nt}", fw=fw)


@pytest.mark.parametrize("nt", [5, 12, 17])
def test_layer_config0_multitoken_no_shared(layer0, nt):
    L, H = layer0
    _check_layer(L, H, synth.inputs(9, nt, 2048, correlated=nt > 5), f"config0 B={nt}")


@pytest.mark.parametrize("nt", [1, 4, 17])
def test_layer_partial_residency_flags(layer1, nt):
    """Config 4: 128 resident experts ranked by the reference's rule
    (activation count, routed weight, id; qwen/README.md:38) over 4096 tokens
    from 8 correlated contexts, one of them the batch's own.  The batch then
    mixes covered (flag 0), pruned (1) and handed-off (2) tokens: flags and
    pruning exact, every unflagged row (resident experts only, pruned weights
    0) within tolerance of the oracle; 1 and 4 tokens are routed inside the
    gate/up kernels, 17 by the routing kernel."""
    L, H = layer1
    xs = synth.ranking_inputs(77, 4242)
    dx = Device(xs)
    n = xs.shape[0]
    logits = Device(shape=(n, 512), dtype=np.float32)
    ids, w = Device(shape=(n, 10), dtype=np.int32), Device(shape=(n, 10), dtype=np.float32)
    call("matmul", logits.p, L.bufs["router"].p, 0, 512, 2048, dx.p, n)
    call("route", ids.p, w.p, logits.p, n)
    resident = synth.resident_ranking(ids.get(), w.get(), 128)
    assert int(resident.sum()) == 128
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    rdev = Device(resident)
    desc.resident, desc.threshold = rdev.p, 0.10
    saved = L.desc
    L.desc = desc
    try:
        x = synth.inputs(77, nt, 2048, correlated=True)
        fw, st = _check_layer(L, H, x, f"config4 B={nt}", resident=resident)
        flags = fw.flags.get()[:nt]
        say(f"  config4 B={nt}: flags {np.bincount(flags, minlength=4).tolist()}")
        if nt >= 4:
            # resident-only routed compute is exercised and compared
            assert np.count_nonzero(flags < 2) > 0
        if nt == 17:
            assert np.count_nonzero(flags == 0) > 0 and np.count_nonzero(flags == 1) > 0
        gst = qg.PruneStats.from_buffer_copy(fw.stats.get())
        assert (gst.token_layers, gst.missing_selections, gst.skipped_selections, gst.avoided_token_handoffs) == \
               (st.token_layers, st.missing_selections, st.skipped_selections, st.avoided_token_handoffs)
        assert gst.skipped_mass == st.skipped_mass
    finally:
        L.desc = saved


@pytest.mark.parametrize("nt", [4, 17])
def test_layer_partial_residency_mixed_flags(layer1, nt):
    """Residency with the 16 experts of largest routed mass over the batch
    itself: the batch mixes covered (0), pruned (1) and handoff (2) tokens, so
    the pruned computation is checked against the oracle row by row."""
    L, H = layer1
    x = synth.inputs(77, nt, 2048, correlated=True)
    ids, w = O.route(H.logits(x))
    score = np.zeros(512)
    np.add.at(score, ids.ravel(), w.ravel().astype(np.float64))
    resident = np.zeros(512, np.uint8)
    resident[np.lexsort((np.arange(512), -score))[:16]] = 1
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    rdev = Device(resident)
    desc.resident, desc.threshold = rdev.p, 0.10
    saved = L.desc
    L.desc = desc
    try:
        fw = synth.Forward(2048, 512, nt)
        call("zero", fw.stats.p, fw.stats.nbytes)
        fw.x.set(x)
        say(f"forward mixed residency nt={nt}")
        fw.run(L, nt)
        qg.call("sync")
        out, oids, ow, _, flags, st = H.forward(x, resident)
        counts = np.bincount(flags, minlength=4)
        assert counts[0] > 0 and counts[1] > 0 and counts[2] > 0, counts
        np.testing.assert_array_equal(fw.ids.get()[:nt], oids)
        np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), ow.view('u4'))
        np.testing.assert_array_equal(fw.flags.get()[:nt], flags)
        keep = flags < 2
        maxabs, rel = assert_close(fw.out.get()[:nt][keep], out[keep], f"mixed residency B={nt}")
        check_flagged_rows(fw.out.get()[:nt], H, x, flags, f"mixed residency B={nt}")
        gst = qg.PruneStats.from_buffer_copy(fw.stats.get())
        assert (gst.token_layers, gst.missing_selections, gst.skipped_selections, gst.avoided_token_handoffs) == \
               (st.token_layers, st.missing_selections, st.skipped_selections, st.avoided_token_handoffs)
        assert gst.skipped_mass == st.skipped_mass
        say(f"  flags {counts}, max-abs {maxabs:.2e}, rel-L2 {rel:.2e}")
    finally:
        L.desc = saved


def _mass_resident(H, x, top):
    """The `top` experts of largest routed mass over the batch itself."""
    ids, w = O.route(H.logits(x))
    score = np.zeros(512)
    np.add.at(score, ids.ravel(), w.ravel().astype(np.float64))
    resident = np.zeros(512, np.uint8)
    resident[np.lexsort((np.arange(512), -score))[:top]] = 1
    return resident


def _cpu_moe_callback(H, calls, D=2048, fetch=None):
    """nm_cpu_moe_fn running the oracle's routed part (the stand-in for the
    reference's qc_moe, cpu.c:235-261) on the packed rows (expert bytes from
    `fetch`, a copy of the device's, when given)."""
    def fn(ctx, out, xp, idp, wp, n):
        try:
            xs = np.ctypeslib.as_array((C.c_float * (n * D)).from_address(xp)).reshape(n, D).copy()
            ids = np.ctypeslib.as_array((C.c_int * (n * 10)).from_address(idp)).reshape(n, 10).copy()
            w = np.ctypeslib.as_array((C.c_float * (n * 10)).from_address(wp)).reshape(n, 10).copy()
            y = np.ascontiguousarray(H.routed(xs, ids, w, fetch), np.float32)
            C.memmove(out, y.ctypes.data, y.nbytes)
            calls.append((xs, ids, w, y))
            return 0
        except Exception as exc:  # noqa: BLE001 - reported through the return code
            say(f"  callback failed: {exc!r}")
            return 1
    return qg.CPU_MOE_FN(fn)


@pytest.mark.parametrize("nt", [1, 4, 17])
def test_handoff_round_trip(layer1, nt):
    """CPU handoff of the flag-2 tokens (qwen.c:658-678): the device packs
    exactly those tokens' input rows, ids and weights (bit-exact), the host
    computes their routed part (oracle) through nm_moe_handoff's callback, and
    after the merge every row matches the oracle's full layer (routed +
    shared) within tolerance; a second accumulator gets the host rows exactly."""
    L, H = layer1
    x = synth.inputs(77, nt, 2048, correlated=True)
    if nt == 1:
        # the token's three largest selections not resident: coverage below 90 %
        resident = np.ones(512, np.uint8)
        resident[O.route(H.logits(x))[0][0, :3]] = 0
    else:
        resident = _mass_resident(H, x, 16)
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    rdev = Device(resident)
    desc.resident, desc.threshold = rdev.p, 0.10
    saved = L.desc
    L.desc = desc
    try:
        fw = synth.Forward(2048, 512, nt)
        fw.x.set(np.concatenate([x, np.zeros((fw.tokens - nt, 2048), np.float32)]) if nt < fw.tokens else x)
        say(f"handoff forward nt={nt}")
        fw.run(L, nt)
        qg.call("sync")
    finally:
        L.desc = saved
    out, oids, ow, _, flags, _ = H.forward(x, resident)
    np.testing.assert_array_equal(fw.flags.get()[:nt], flags)
    want = np.nonzero(flags == 2)[0]
    assert len(want) > 0 and (nt == 1 or len(want) < nt), flags
    check_flagged_rows(fw.out.get()[:nt], H, x, flags, f"handoff B={nt}")
    # the pack alone
    cnt, rows = Device(shape=(1,), dtype=np.int32), Device(shape=(nt,), dtype=np.int32)
    xp, ip, wp = Device(shape=(nt, 2048), dtype=np.float32), Device(shape=(nt, 10), dtype=np.int32), Device(shape=(nt, 10), dtype=np.float32)
    say(f"handoff pack nt={nt}")
    call("moe_handoff_pack", cnt.p, rows.p, xp.p, ip.p, wp.p, fw.flags.p, fw.x.p, fw.ids.p, fw.w.p, nt, 2048)
    n = int(cnt.get()[0])
    assert n == len(want)
    np.testing.assert_array_equal(rows.get()[:n], want)
    np.testing.assert_array_equal(xp.get()[:n].view('u4'), x[want].view('u4'))
    np.testing.assert_array_equal(ip.get()[:n], oids[want])
    np.testing.assert_array_equal(wp.get()[:n].view('u4'), ow[want].view('u4'))
    # the round trip through the host driver
    h = qg.host()
    sb = h.nm_handoff_scratch_bytes(2048, nt)
    scratch, acc2 = Device(nbytes=sb), Device(np.zeros((nt, 2048), np.float32))
    calls = []
    cb = _cpu_moe_callback(H, calls)
    handed = C.c_int(-1)
    say(f"handoff round trip nt={nt}, {n} tokens to the host")
    assert h.nm_moe_handoff(fw.out.p, acc2.p, fw.flags.p, fw.x.p, fw.ids.p, fw.w.p, nt, 2048, scratch.p, sb, cb, None,
                            C.byref(handed)) == 0, h.nm_last_error()
    assert handed.value == n and len(calls) == 1
    _, cids, _, y = calls[0]
    np.testing.assert_array_equal(cids, oids[want])
    got = fw.out.get()[:nt]
    ok = flags < 3
    maxabs, rel = assert_close(got[ok], out[ok], f"handoff round trip B={nt}")
    a2 = acc2.get()
    np.testing.assert_array_equal(a2[want].view('u4'), y.view('u4'))
    assert np.all(np.delete(a2, want, axis=0) == 0)
    say(f"  {n} of {nt} tokens handed off, max-abs {maxabs:.2e}, rel-L2 {rel:.2e}")
    # no flagged token: nothing read, no callback
    zf = Device(np.zeros(nt, np.uint8))
    calls.clear()
    assert h.nm_moe_handoff(fw.out.p, None, zf.p, fw.x.p, fw.ids.p, fw.w.p, nt, 2048, scratch.p, sb, cb, None,
                            C.byref(handed)) == 0, h.nm_last_error()
    assert handed.value == 0 and not calls
    np.testing.assert_array_equal(fw.out.get()[:nt].view('u4'), got.view('u4'))


def test_handoff_pack_merge_large():
    """Pack and merge at 3000 tokens (three 1024-token scan chunks) with
    seeded flags 0..3: rows ascending, packed rows bit-exact, merge adds the
    host rows at exactly the flagged rows."""
    rng = np.random.default_rng(5)
    nt, D = 3000, 256
    flags = rng.integers(0, 4, nt).astype(np.uint8)
    x = rng.standard_normal((nt, D)).astype(np.float32)
    ids = rng.integers(0, 512, (nt, 10)).astype(np.int32)
    w = rng.random((nt, 10)).astype(np.float32)
    dflags, dx, dids, dw = Device(flags), Device(x), Device(ids), Device(w)
    cnt, rows = Device(shape=(1,), dtype=np.int32), Device(shape=(nt,), dtype=np.int32)
    xp, ip, wp = Device(shape=(nt, D), dtype=np.float32), Device(shape=(nt, 10), dtype=np.int32), Device(shape=(nt, 10), dtype=np.float32)
    say(f"handoff pack nt={nt}")
    call("moe_handoff_pack", cnt.p, rows.p, xp.p, ip.p, wp.p, dflags.p, dx.p, dids.p, dw.p, nt, D)
    want = np.nonzero(flags == 2)[0]
    n = int(cnt.get()[0])
    assert n == len(want)
    np.testing.assert_array_equal(rows.get()[:n], want)
    np.testing.assert_array_equal(xp.get()[:n].view('u4'), x[want].view('u4'))
    np.testing.assert_array_equal(ip.get()[:n], ids[want])
    np.testing.assert_array_equal(wp.get()[:n].view('u4'), w[want].view('u4'))
    base = rng.standard_normal((nt, D)).astype(np.float32)
    y = np.zeros((nt, D), np.float32)
    y[:n] = rng.standard_normal((n, D)).astype(np.float32)
    dout, dy = Device(base), Device(y)
    say(f"handoff merge nt={nt}")
    call("moe_handoff_merge", dout.p, dy.p, cnt.p, rows.p, nt, D)
    expect = base.copy()
    expect[want] += y[:n]
    np.testing.assert_array_equal(dout.get().view('u4'), expect.view('u4'))


@pytest.mark.parametrize("nt,ties", [(5, 40), (17, 40), (17, 70)])
def test_layer_router_heavy_ties(layer1, nt, ties):
    """`ties` identical router rows that beat every other logit of every
    token: more tied candidates than a 32-lane half ranks (40) or than a whole
    wave ranks (70), so the routing kernel's whole-wave paths run.  Ids,
    weights and flags stay exact; every token picks experts 0..9, so each
    expert carries the whole batch (several tiles)."""
    L, H = layer1
    x = synth.inputs(91, nt, 2048, correlated=True)
    u = x.mean(axis=0)
    u /= np.linalg.norm(u)
    proj = x @ u
    assert proj.min() > 1.0
    natural = (x @ H.router.reshape(512, 2048).T).max()
    router = H.router.copy()
    router.reshape(512, 2048)[:ties] = ((natural + 1.0) / proj.min() * u).astype(np.float32)
    rdev = Device(router)
    desc = qg.MoeLayer.from_buffer_copy(L.desc)
    desc.router = rdev.p
    saved_desc, saved_router = L.desc, H.router
    L.desc, H.router = desc, router
    try:
        _, oids, _, _, _, _ = H.forward(x)
        np.testing.assert_array_equal(oids, np.tile(np.arange(10), (nt, 1)))
        _check_layer(L, H, x, f"heavy ties {ties} B={nt}")
    finally:
        L.desc, H.router = saved_desc, saved_router


@pytest.mark.parametrize("nt", [2, 8])
def test_layer_graph_replay(layer1, nt):
    """The fused layer captured into a graph and replayed, with eager work in
    between, equals the eager result every time."""
    L, H = layer1
    fw = synth.Forward(2048, 512, nt)
    fw.x.set(synth.inputs(5, nt, 2048, correlated=True))
    fw.run(L, nt)
    eager = fw.out.get()
    g = C.c_void_p()
    say("graph capture of the fused layer")
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


def test_stack_per_layer_routing(qgl):
    """Config 2 in miniature: 3 seeded layers, h <- h + MoE(RMSNorm(h)),
    graph-captured; per layer, routing from the recorded input is bit-exact
    and the layer output is within tolerance."""
    specs = [synth.LayerSpec(seed=300 + l) for l in range(3)]
    layers = [synth.build_layer(s) for s in specs]
    hosts = [O.HostLayer(s.seed) for s in specs]
    arr = (qg.MoeLayer * 3)(*[l.desc for l in layers])
    h = qg.host()
    stack = h.nm_stack_create(arr, 3, 1, 1)
    assert stack, h.nm_last_error()
    try:
        x0 = synth.inputs(31, 1, 2048)
        call("write", h.nm_stack_hidden(stack), x0.ctypes.data, x0.nbytes)
        say("stack forward (graph)")
        assert h.nm_stack_forward(stack, 1, 1) == 0, h.nm_last_error()
        call("sync")
        hfin = np.empty((1, 2048), np.float32)
        call("read", hfin.ctypes.data, h.nm_stack_hidden(stack), hfin.nbytes)
        hcur = x0.copy()
        for l in range(3):
            px, pids, pw, pout = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
            assert h.nm_stack_record(stack, l, C.byref(px), C.byref(pids), C.byref(pw), C.byref(pout)) == 0
            xl = np.empty((1, 2048), np.float32); ol = np.empty((1, 2048), np.float32)
            il = np.empty((1, 10), np.int32); wl = np.empty((1, 10), np.float32)
            for arr_, p in ((xl, px), (ol, pout), (il, pids), (wl, pw)):
                call("read", arr_.ctypes.data, p.value, arr_.nbytes)
            out, ids, w, _, _, _ = hosts[l].forward(xl)
            np.testing.assert_array_equal(il, ids, err_msg=f"layer {l} ids")
            np.testing.assert_array_equal(wl.view('u4'), w.view('u4'), err_msg=f"layer {l} weights")
            assert_close(ol, out, f"stack layer {l}")
            hcur = (hcur + ol).astype(np.float32)
        np.testing.assert_array_equal(hfin, hcur)
    finally:
        h.nm_stack_destroy(stack)


def test_forward_rejects_bad_arguments(layer0):
    L, _ = layer0
    fw = synth.Forward(2048, 512, 17)
    lib = qg.lib()
    for nt in (0, 8193):  # token counts outside 1..8192 (18..8192 is the prefill path)
        assert lib.qg_moe_forward(fw.out.p, fw.ids.p, fw.w.p, None, None, fw.x.p, nt, C.byref(L.desc), fw.ws.p, fw.ws_bytes) != 0
    # a workspace sized for 17 tokens is too small for a 2048-token prefill
    assert lib.qg_moe_workspace_bytes(2048, 512, 2048) > fw.ws_bytes
    assert lib.qg_moe_forward(fw.out.p, fw.ids.p, fw.w.p, None, None, fw.x.p, 1, C.byref(L.desc), fw.ws.p, 16) != 0
    assert lib.qg_moe_workspace_bytes(2048, 512, 8193) == 0


def test_unrecorded_event_does_not_poison_next_call(layer0):
    """Timing a kernel that did not run reports an error, and the next layer
    call still succeeds (the runtime's sticky error is cleared)."""
    L, H = layer0
    b, e = qg.Event(), qg.Event()
    t = C.c_float()
    assert qg.lib().qg_event_elapsed(C.byref(t), b.p, e.p) != 0
    fw = synth.Forward(2048, 512, 1)
    x = synth.inputs(3, 1, 2048)
    fw.x.set(x)
    fw.run(L, 1)
    qg.call("sync")
    out, ids, *_ = H.forward(x)
    np.testing.assert_array_equal(fw.ids.get()[:1], ids)


def test_layer_generic_fallback_width(qgl):
    """A width the decode fast path does not take (D=1024, F=256) runs the
    generic kernels behind the same entry point; same bars."""
    spec = synth.LayerSpec(seed=404, width=1024, ff=256, down_type=20, shared=True)
    L = synth.build_layer(spec)
    H = O.HostLayer(spec.seed, width=1024, ff=256, gt=12, ut=12, dt=20, shared=True, sh_types=(12, 12, 12))
    for nt in (1, 6):
        x = synth.inputs(12 + nt, nt, 1024, correlated=True)
        fw = synth.Forward(1024, 256, nt)
        fw.x.set(x)
        say(f"forward generic D=1024 nt={nt}")
        fw.run(L, nt)
        qg.call("sync")
        out, ids, w, *_ = H.forward(x)
        np.testing.assert_array_equal(fw.ids.get()[:nt], ids)
        np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), w.view('u4'))
        assert_close(fw.out.get()[:nt], out, f"generic nt={nt}")


@pytest.mark.parametrize("nt", [3, 17])
def test_forward_residual_matches_forward(layer1, nt):
    """qg_moe_forward_residual(h) == h + qg_moe_forward(RMSNorm(h)) with the
    normalised rows it reports, and the routing of those rows is the oracle's."""
    L, H = layer1
    h0 = (synth.inputs(900 + nt, nt, 2048, correlated=True) * 3.0).astype(np.float32)
    fw = synth.Forward(2048, 512, nt)
    hd = Device(h0)
    xn = Device(shape=(nt, 2048), dtype=np.float32)
    out = Device(shape=(nt, 2048), dtype=np.float32)
    say(f"forward_residual nt={nt}")
    call("moe_forward_residual", hd.p, fw.ids.p, fw.w.p, fw.flags.p, None, xn.p, out.p, nt, C.byref(L.desc), fw.ws.p, fw.ws_bytes)
    qg.call("sync")
    xs = xn.get()
    ref = synth.rmsnorm(h0)
    np.testing.assert_allclose(xs, ref, rtol=2e-6, atol=2e-6)
    want, ids, w, *_ = H.forward(xs)
    np.testing.assert_array_equal(fw.ids.get()[:nt], ids)
    np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), w.view('u4'))
    assert_close(out.get(), want, f"residual out nt={nt}")
    np.testing.assert_array_equal(hd.get(), (h0 + out.get()).astype(np.float32))
