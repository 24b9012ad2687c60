"""GPU parity of the drop-in boundary at the reference's own shape.

1. qg_moe_forward at D=2560 / F=640 (the shape cpu.c:11 and gpu.cu:508-553
   hard-code): Q4_K gate/up, IQ4_NL down, a shared expert, at the decode
   batches 1/4/17 and the prefill sizes 40/600.
2. The exact qg_* call sequence of the reference's moe() / grouped_moe() /
   shared_direct() (qwen.c:633-735, no hotlist), replayed through the
   drop-in entry points at 2560/640 and 2048/512.
3. The remaining gpu.h entry points: qg_gather / qg_dequant against the
   oracle's per-element dequantisation, qg_norm, qg_unary / qg_binary /
   qg_shared_add against float64 closed forms, the pinned expert uploader's
   byte round trip.
4. Library scratch buffers outgrown after a graph captured them (qg_mtp_moe,
   qg_moe_dispatch): the graph still replays its own results.

Bars: ids, weights and dispatch bit-exact; fp32 outputs within max-abs 1e-3
and rel-L2 1e-4 of the oracle.
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
REF = synth.LayerSpec(seed=2560, width=2560, ff=640, gate_type=12, up_type=12, down_type=20, shared=True,
                      sh_types=(12, 12, 20))
CFG1 = synth.LayerSpec(seed=200, gate_type=12, up_type=12, down_type=20, shared=True, sh_types=(12, 12, 12))


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
                       shared=spec.shared, sh_types=spec.sh_types)


def fetcher(L):
    return lambda name, e: synth.read_expert(L, name, e)


@pytest.fixture(scope="module")
def ref_layer(qgl):
    say("building a 2560/640 layer on device")
    return synth.build_layer(REF), host_layer(REF)


@pytest.fixture(scope="module")
def cfg1_layer(qgl):
    say("building config-1 layer on device")
    return synth.build_layer(CFG1), host_layer(CFG1)


# ---------------- 1. the fused layer at the reference's shape ----------------

@pytest.mark.parametrize("nt", [1, 4, 17, 40, 600])
def test_forward_reference_shape(ref_layer, nt):
    L, H = ref_layer
    D, Fd = REF.width, REF.ff
    x = synth.inputs(7000 + nt, nt, D, correlated=True)
    fw = synth.Forward(D, Fd, nt)
    fw.x.set(x)
    say(f"forward 2560/640 nt={nt}")
    fw.run(L, nt)
    call("sync")
    ids, w = O.route(H.logits(x))
    np.testing.assert_array_equal(fw.ids.get()[:nt], ids, err_msg="routing ids")
    np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), w.view('u4'), err_msg="routing weights")
    assert not fw.flags.get()[:nt].any()
    rows = np.arange(nt) if nt <= 40 else np.unique(np.concatenate(
        [np.arange(4), np.arange(nt - 4, nt), np.random.default_rng(nt).choice(nt, 24, replace=False)]))
    out, *_ = H.forward(x[rows], fetch=fetcher(L))
    maxabs, rel = assert_close(fw.out.get()[rows], out, f"2560/640 nt={nt}")
    say(f"  2560/640 nt={nt}: {len(rows)} rows, unique experts {len(np.unique(ids))}, max-abs {maxabs:.2e} rel-L2 {rel:.2e}")


def test_forward_residual_reference_shape(ref_layer):
    L, H = ref_layer
    D, Fd, nt = REF.width, REF.ff, 5
    h0 = (synth.inputs(7100, nt, D, correlated=True) * 2.0).astype(np.float32)
    fw = synth.Forward(D, Fd, nt)
    hd, xn, out = Device(h0), Device(shape=(nt, D), dtype=np.float32), Device(shape=(nt, D), dtype=np.float32)
    say("forward_residual 2560/640 nt=5")
    call("moe_forward_residual", hd.p, fw.ids.p, fw.w.p, fw.flags.p, None, xn.p, out.p, nt, C.byref(L.desc), fw.ws.p,
         fw.ws_bytes)
    call("sync")
    xs = xn.get()
    np.testing.assert_allclose(xs, synth.rmsnorm(h0), rtol=2e-6, atol=2e-6)
    want, ids, *_ = H.forward(xs, fetch=fetcher(L))
    np.testing.assert_array_equal(fw.ids.get()[:nt], ids)
    assert_close(out.get(), want, "residual 2560/640")
    np.testing.assert_array_equal(hd.get(), (h0 + out.get()).astype(np.float32))


# ---------------- 2. moe() / grouped_moe() / shared_direct() replay ----------------

def replay_moe(L, x_dev, nt):
    """The qg_* sequence of qwen.c:714-735 for a target layer without a fixed
    hotlist and every expert resident: router qg_matmul, qg_route, host read
    of the ids (qwen.c:649), qg_moe_map for nt > 1 (:680), qg_zero of the
    slots (:684), per active expert in ascending id (:683-698) qg_moe_gather
    when it has fewer than nt tokens, gate/up qg_matmul, qg_unary op 0,
    qg_binary op 1, down qg_matmul, qg_moe_scatter; then qg_moe_reduce
    (:725) and shared_direct (:708-713).  Returns (out, ids, weights)."""
    s = L.spec
    D, Fd = s.width, s.ff
    call("moe_configure", D, Fd)
    logits = Device(shape=(nt, 512), dtype=np.float32)
    ids_d, w_d = Device(shape=(nt, 10), dtype=np.int32), Device(shape=(nt, 10), dtype=np.float32)
    route_map = Device(shape=(512, nt), dtype=np.int32)
    slots = Device(shape=(nt, 10, D), dtype=np.float32)
    ex = Device(shape=(nt, D), dtype=np.float32)
    ffg, ffu, ffmid = (Device(shape=(nt, Fd), dtype=np.float32) for _ in range(3))
    ffout, moeout, shared = (Device(shape=(nt, D), dtype=np.float32) for _ in range(3))
    shared_gate = Device(shape=(nt, 1), dtype=np.float32)
    call("matmul", logits.p, L.bufs["router"].p, 0, 512, D, x_dev.p, nt)
    call("route", ids_d.p, w_d.p, logits.p, nt)
    ids = ids_d.get()
    assert ids.min() >= 0, "non-finite router distribution"
    counts = np.bincount(ids.ravel(), minlength=512)
    if nt > 1:
        call("moe_map", route_map.p, ids_d.p, nt)
    call("zero", slots.p, slots.nbytes)
    gb = Fd * qg.row_bytes(s.gate_type, D)
    ub = Fd * qg.row_bytes(s.up_type, D)
    db = D * qg.row_bytes(s.down_type, Fd)
    for e in np.nonzero(counts)[0]:
        ne = int(counts[e])
        inp, tmap = x_dev.p, None
        if ne < nt:
            tmap = route_map.p + int(e) * nt * 4
            call("moe_gather", ex.p, x_dev.p, tmap, ne)
            inp = ex.p
        call("matmul", ffg.p, L.bufs["gate"].p + int(e) * gb, s.gate_type, Fd, D, inp, ne)
        call("matmul", ffu.p, L.bufs["up"].p + int(e) * ub, s.up_type, Fd, D, inp, ne)
        call("unary", ffmid.p, ffg.p, ne * Fd, 0, qg.F(1.0))
        call("binary", ffmid.p, ffmid.p, ffu.p, ne * Fd, 1)
        call("matmul", ffout.p, L.bufs["down"].p + int(e) * db, s.down_type, D, Fd, ffmid.p, ne)
        call("moe_scatter", slots.p, ffout.p, w_d.p, ids_d.p, tmap, int(e), ne)
    call("moe_reduce", moeout.p, slots.p, nt)
    if s.shared:
        sg, su, sd = s.sh_types
        call("matmul", ffg.p, L.bufs["sh_gate"].p, sg, Fd, D, x_dev.p, nt)
        call("matmul", ffu.p, L.bufs["sh_up"].p, su, Fd, D, x_dev.p, nt)
        call("unary", ffmid.p, ffg.p, nt * Fd, 0, qg.F(1.0))
        call("binary", ffmid.p, ffmid.p, ffu.p, nt * Fd, 1)
        call("matmul", shared.p, L.bufs["sh_down"].p, sd, D, Fd, ffmid.p, nt)
        call("matmul", shared_gate.p, L.bufs["sh_inp"].p, 0, 1, D, x_dev.p, nt)
        call("shared_add", moeout.p, shared.p, shared_gate.p, nt)
    call("sync")
    call("moe_configure", 2560, 640)
    return moeout.get(), ids, w_d.get()


@pytest.mark.parametrize("which,nt", [("ref", 1), ("ref", 17), ("ref", 40), ("cfg1", 4), ("cfg1", 17)])
def test_reference_call_sequence(ref_layer, cfg1_layer, which, nt):
    """The drop-in entry points driven exactly as qwen.c drives them give the
    oracle's layer, and the fused qg_moe_forward gives the same routing."""
    L, H = ref_layer if which == "ref" else cfg1_layer
    D = L.spec.width
    x = synth.inputs(7200 + nt, nt, D, correlated=True)
    xd = Device(x)
    say(f"moe() replay {which} D={D} nt={nt}")
    got, ids, w = replay_moe(L, xd, nt)
    want, oids, ow, *_ = H.forward(x, fetch=fetcher(L))
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(w.view('u4'), ow.view('u4'))
    maxabs, rel = assert_close(got, want, f"moe() replay {which} nt={nt}")
    bit = np.array_equal(got.view('u4'), want.view('u4'))
    say(f"  replay {which} nt={nt}: max-abs {maxabs:.2e} rel-L2 {rel:.2e} bit-exact={bit}")
    fw = synth.Forward(D, L.spec.ff, nt)
    fw.x.set(x)
    fw.run(L, nt)
    call("sync")
    np.testing.assert_array_equal(fw.ids.get()[:nt], ids)
    assert_close(fw.out.get()[:nt], got, f"fused vs replay {which} nt={nt}")


# ---------------- 3. remaining gpu.h entry points ----------------

def legal_blocks(rng, typ, rows, cols):
    from test_oracle_cpu import legal_blocks as lb
    return np.ascontiguousarray(lb(rng, typ, rows, cols))


def oracle_rows(w, typ, rows, cols):
    rb = O.row_bytes(typ, cols)
    out = np.empty((rows, cols), np.float32)
    lib = O.lib()
    for r in range(rows):
        p = w.ctypes.data + r * rb
        for c in range(cols):
            out[r, c] = lib.nbo_weight_at(p, typ, c)
    return out


@pytest.mark.parametrize("typ,cols", [(0, 320), (1, 320), (30, 320), (2, 320), (8, 320), (12, 512), (14, 512), (20, 640)])
def test_gather_dequant_bitexact(qgl, typ, cols):
    """qg_gather (one row, gpu.cu:190-196) and qg_dequant (all rows,
    gpu.cu:197-203) equal the per-element dequantisation of cpu.c:43-67."""
    rng = np.random.default_rng(91011 + typ)
    rows = 5
    w = legal_blocks(rng, typ, rows, cols)
    want = oracle_rows(w, typ, rows, cols)
    dw = Device(w)
    full = Device(shape=(rows, cols), dtype=np.float32)
    say(f"dequant type={typ} cols={cols}")
    call("dequant", full.p, dw.p, typ, rows, cols)
    np.testing.assert_array_equal(full.get().view('u4'), want.view('u4'))
    one = Device(shape=(cols,), dtype=np.float32)
    for r in (0, 3):
        call("gather", one.p, dw.p, typ, cols, r)
        np.testing.assert_array_equal(one.get().view('u4'), want[r].view('u4'))
    assert qgl.qg_gather(one.p, dw.p, typ, cols, -1) != 0
    assert qgl.qg_dequant(full.p, dw.p, 99, rows, cols) != 0


def test_norm_unary_binary_shared_add(qgl):
    """qg_norm (gpu.cu:204-214), qg_unary ops 0/1/2 (:215-220), qg_binary ops
    0/1 (:221-226) and qg_shared_add (:552-553) against float64 forms."""
    rng = np.random.default_rng(27)
    D, nt, groups = 2048, 3, 4
    x = rng.normal(0, 1.5, (nt, D)).astype(np.float32)
    dx = Device(x)
    out = Device(shape=(nt, D), dtype=np.float32)
    say("norm / unary / binary / shared_add")
    call("norm", out.p, dx.p, None, D, 1, nt, 0, 0, qg.F(1e-6))
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(out.get(), want, rtol=3e-6, atol=1e-6)
    # grouped, weighted, l2 form: rows of width 512, weight row per group
    W = 512
    wgt = rng.normal(1, .1, (groups, W)).astype(np.float32)
    dwg = Device(wgt)
    call("norm", out.p, dx.p, dwg.p, W, groups, nt, 1, 1, qg.F(1e-6))
    xg = x64.reshape(nt * groups, W)
    wantg = xg / np.sqrt((xg * xg).sum(-1, keepdims=True) + 1e-6) * np.tile(wgt, (nt, 1))
    np.testing.assert_allclose(out.get().reshape(nt * groups, W), wantg, rtol=3e-6, atol=1e-6)
    n = nt * D
    a = rng.normal(0, 3, n).astype(np.float32)
    b = rng.normal(0, 1, n).astype(np.float32)
    da, db, do = Device(a), Device(b), Device(shape=(n,), dtype=np.float32)
    a64 = a.astype(np.float64) * np.float64(np.float32(0.5))
    sig = 1 / (1 + np.exp(-a64))
    for op, want in ((0, a64 * sig), (1, sig), (2, a64)):
        call("unary", do.p, da.p, n, op, qg.F(0.5))
        np.testing.assert_allclose(do.get(), want, rtol=2e-6, atol=1e-7, err_msg=f"unary op {op}")
    call("binary", do.p, da.p, db.p, n, 0)
    np.testing.assert_array_equal(do.get(), a + b)
    call("binary", do.p, da.p, db.p, n, 1)
    np.testing.assert_array_equal(do.get(), a * b)
    call("moe_configure", D, 512)
    g = rng.normal(0, 2, nt).astype(np.float32)
    base = rng.normal(0, 1, (nt, D)).astype(np.float32)
    dbase, dg = Device(base), Device(g)
    call("shared_add", dbase.p, dx.p, dg.p, nt)
    want = base.astype(np.float64) + x64 / (1 + np.exp(-g.astype(np.float64)))[:, None]
    np.testing.assert_allclose(dbase.get(), want, rtol=2e-6, atol=2e-6)
    call("moe_configure", 2560, 640)
    call("sync")


def test_upload_expert_round_trip(qgl):
    """The pinned double-buffered uploader (gpu.cu:48-85): two experts in a
    row land byte for byte as gate|up|down; oversize uploads are refused."""
    rng = np.random.default_rng(5)
    ng, nu, nd = 921600, 921600, 921600
    u = qgl.qg_upload_create(ng + nu + nd)
    assert u
    try:
        dst = Device(nbytes=2 * (ng + nu + nd))
        parts = []
        for i in range(2):
            g, up, d = (rng.integers(0, 256, n, dtype=np.uint8) for n in (ng, nu, nd))
            parts.append(np.concatenate([g, up, d]))
            say(f"upload expert {i}")
            call("upload_expert", u, dst.p + i * (ng + nu + nd), g.ctypes.data, ng, up.ctypes.data, nu, d.ctypes.data, nd)
        call("sync")
        np.testing.assert_array_equal(dst.get(), np.concatenate(parts))
        assert qgl.qg_upload_seconds(u) > 0
        big = np.zeros(ng + nu + nd + 1, np.uint8)
        assert qgl.qg_upload_expert(u, dst.p, big.ctypes.data, big.nbytes, big.ctypes.data, 0, big.ctypes.data, 0) != 0
    finally:
        qgl.qg_upload_destroy(u)


# ---------------- 4. scratch buffers outgrown after a capture ----------------

def test_graph_survives_scratch_growth(qgl):
    """qg_mtp_moe and qg_moe_dispatch keep library scratch that grows with
    the widths / token count; a graph captured before a growth must replay
    the same results after it (the outgrown buffer stays allocated)."""
    rng = np.random.default_rng(3)
    D, Fd, nt = 1024, 256, 3
    call("moe_configure", D, Fd)
    x = rng.normal(0, 1, (nt, D)).astype(np.float32)
    ids = np.array([rng.choice(16, 10, replace=False) for _ in range(nt)], np.int32)
    w = np.full((nt, 10), 0.1, np.float32)
    gate = legal_blocks(rng, 12, 16 * Fd, D)
    up = legal_blocks(rng, 12, 16 * Fd, D)
    down = legal_blocks(rng, 20, 16 * D, Fd)
    dx, di, dw, dg, du, dd = (Device(a) for a in (x, ids, w, gate, up, down))
    slots = Device(shape=(nt, 10, D), dtype=np.float32)
    mid = Device(shape=(nt, 10, Fd), dtype=np.float32)
    say("mtp_moe capture at 1024/256")
    call("mtp_moe", slots.p, mid.p, dx.p, di.p, dw.p, dg.p, 12, du.p, 12, dd.p, 20, nt)
    call("sync")
    eager = slots.get()
    g = C.c_void_p()
    call("graph_begin", C.byref(g))
    call("mtp_moe", slots.p, mid.p, dx.p, di.p, dw.p, dg.p, 12, du.p, 12, dd.p, 20, nt)
    call("graph_end", g)
    # an eager call at wider shapes grows the scratch past the captured one
    call("moe_configure", 4096, 1024)
    D2, F2 = 4096, 1024
    x2 = Device(rng.normal(0, 1, (nt, D2)).astype(np.float32))
    g2, u2, d2 = Device(legal_blocks(rng, 12, 16 * F2, D2)), Device(legal_blocks(rng, 12, 16 * F2, D2)), Device(
        legal_blocks(rng, 20, 16 * D2, F2))
    s2, m2 = Device(shape=(nt, 10, D2), dtype=np.float32), Device(shape=(nt, 10, F2), dtype=np.float32)
    say("mtp_moe eager at 4096/1024")
    call("mtp_moe", s2.p, m2.p, x2.p, di.p, dw.p, g2.p, 12, u2.p, 12, d2.p, 20, nt)
    call("sync")
    for rep in range(2):
        call("zero", slots.p, slots.nbytes)
        call("sync")
        call("graph_launch", g)
        call("sync")
        np.testing.assert_array_equal(slots.get().view('u4'), eager.view('u4'), err_msg=f"mtp replay {rep}")
    qgl.qg_graph_destroy(g)
    call("moe_configure", 2560, 640)

    # qg_moe_dispatch: capture at 100 tokens, grow at 3000, replay
    def dispatch_bufs(n):
        r = np.array([np.random.default_rng(n).choice(512, 10, replace=False) for _ in range(n)], np.int32)
        return (Device(r), Device(shape=(513,), dtype=np.int32), Device(shape=(10 * n,), dtype=np.int32),
                Device(shape=(10 * n,), dtype=np.int32), Device(shape=(1,), dtype=np.int32), r)
    di1, off1, tok1, slot1, st1, r1 = dispatch_bufs(100)
    say("dispatch capture at 100 tokens")
    call("moe_dispatch", off1.p, tok1.p, slot1.p, st1.p, di1.p, 100)
    call("sync")
    want = O.dispatch(r1)
    g = C.c_void_p()
    call("graph_begin", C.byref(g))
    call("moe_dispatch", off1.p, tok1.p, slot1.p, st1.p, di1.p, 100)
    call("graph_end", g)
    di3, off3, tok3, slot3, st3, _ = dispatch_bufs(3000)
    say("dispatch eager at 3000 tokens")
    call("moe_dispatch", off3.p, tok3.p, slot3.p, st3.p, di3.p, 3000)
    call("sync")
    for rep in range(2):
        for b in (off1, tok1, slot1):
            call("zero", b.p, b.nbytes)
        call("sync")
        call("graph_launch", g)
        call("sync")
        np.testing.assert_array_equal(off1.get(), want[0])
        np.testing.assert_array_equal(tok1.get(), want[1])
        np.testing.assert_array_equal(slot1.get(), want[2])
    qgl.qg_graph_destroy(g)
