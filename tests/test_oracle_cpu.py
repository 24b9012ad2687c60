"""CPU tests: pin the oracle, then check host logic and the C-ABI exports.

The oracle (oracle/nb_oracle.c) is checked against
 - the reference's own cpu.c compiled in place (oracle/_ref), bit for bit;
 - the reference's known-answer tests (qwen/test_gpu.py:84-95, 338-359);
 - closed forms (vectorised GGML dequantisation, float64 products, libm exp).
No GPU is used here.
"""
import ctypes as C
import math
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle as O

ROOT = Path(__file__).resolve().parent.parent
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 20: (32, 18), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         12: (256, 144), 13: (256, 176), 14: (256, 210)}
ALL_TYPES = (0, 1, 30, 2, 20, 6, 7, 8, 12, 13, 14)
IQ4 = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float64)


def legal_blocks(rng, typ, rows, cols):
    """Random legal rows of a format: random payload bytes, fixed fp16 scales
    (the construction of qwen/test_cpu_dispatch.py:19-33)."""
    if typ == 0:
        return rng.normal(0, .05, (rows, cols)).astype('f4').view('u1')
    if typ == 1:
        return rng.normal(0, .05, (rows, cols)).astype('f2').view('u1')
    if typ == 30:
        return (rng.normal(0, .05, (rows, cols)).astype('f4').view('u4') >> 16).astype('u2').view('u1')
    block, size = BLOCK[typ]
    data = rng.integers(0, 256, (rows * cols // block, size), dtype='u1')
    off = 208 if typ == 14 else 0
    data[:, off:off + 2] = np.array([.0005], 'f2').view('u1')
    if typ in (7, 12, 13):
        data[:, 2:4] = np.array([.0002], 'f2').view('u1')
    return data.reshape(rows, -1)


def dequant_np(p, typ, rows, cols):
    """Vectorised float64 dequantisation of Q4_K / IQ4_NL from the GGML block
    layout (the layout stated in qwen/quant.py:44-54 and :26-36)."""
    if typ == 20:
        b = p.reshape(rows, cols // 32, 18)
        d = b[..., 0:2].copy().view('<f2').astype(np.float64)
        qs = b[..., 2:18]
        q = np.concatenate([qs & 15, qs >> 4], axis=-1)
        return (IQ4[q] * d).reshape(rows, cols)
    assert typ == 12
    b = p.reshape(rows, cols // 256, 144)
    d = b[..., 0:2].copy().view('<f2').astype(np.float64)
    dm = b[..., 2:4].copy().view('<f2').astype(np.float64)
    sc = b[..., 4:16].astype(np.int64)
    s = np.concatenate([sc[..., 0:4] & 63, (sc[..., 8:12] & 15) | ((sc[..., 0:4] >> 6) << 4)], axis=-1)
    m = np.concatenate([sc[..., 4:8] & 63, (sc[..., 8:12] >> 4) | ((sc[..., 4:8] >> 6) << 4)], axis=-1)
    qs = b[..., 16:144].reshape(rows, cols // 256, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=-2).reshape(rows, cols // 256, 8, 32).astype(np.float64)
    w = q * (d * s)[..., None] - (dm * m)[..., None]
    return w.reshape(rows, cols)


@pytest.fixture(scope="module")
def ref():
    r = O.ref_lib(2048)
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent and no prebuilt library)")
    return r


# ---------------- formats and the fixed summation order ----------------

def test_half_decodes_every_encoding():
    halves = np.arange(65536, dtype='<u2')
    got = np.array([O.lib().nbo_half(halves[i:i + 1].ctypes.data) for i in range(65536)], np.float32)
    with np.errstate(invalid='ignore'):
        want = halves.view('f2').astype('f4')
    fin = ~np.isnan(want)
    np.testing.assert_array_equal(got[fin].view('u4'), want[fin].view('u4'))
    assert np.all(np.isnan(got[~fin]))


@pytest.mark.parametrize("typ", (12, 20))
def test_dequant_matches_closed_form(typ):
    rng = np.random.default_rng(5)
    rows, cols = 7, 512
    p = np.ascontiguousarray(legal_blocks(rng, typ, rows, cols))
    want = dequant_np(p, typ, rows, cols)
    rb = O.row_bytes(typ, cols)
    got = np.array([[O.lib().nbo_weight_at(p.ctypes.data + r * rb, typ, i) for i in range(cols)] for r in range(rows)])
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-9)


def test_matmul_bitexact_vs_reference_cpu(ref):
    """All 11 formats, batch tails around the reference's 4-token tiles and its
    17-row boundary (qwen/test_cpu_dispatch.py:46-58), against qc_matmul."""
    rng = np.random.default_rng(91011)
    for typ in ALL_TYPES:
        w = np.ascontiguousarray(legal_blocks(rng, typ, 7, 512))
        for nt in (1, 3, 4, 5, 17, 18):
            x = rng.normal(0, .2, (nt, 512)).astype('f4')
            a = O.matmul(w, typ, 7, 512, x)
            b = np.empty((nt, 7), 'f4')
            assert ref.qc_matmul(b.ctypes.data, w.ctypes.data, typ, 7, 512, x.ctypes.data, nt, 2) == 0
            np.testing.assert_array_equal(a.view('u4'), b.view('u4'), err_msg=f"type {typ} nt {nt}")


def test_matmul_matches_float64(ref):
    rng = np.random.default_rng(3)
    for typ in (12, 20):
        w = np.ascontiguousarray(legal_blocks(rng, typ, 16, 2048))
        x = rng.normal(0, 1, (3, 2048)).astype('f4')
        got = O.matmul(w, typ, 16, 2048, x)
        want = x.astype(np.float64) @ dequant_np(w, typ, 16, 2048).T
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


def _moe_case(ref, width, ff, nt, rng):
    gate = np.ascontiguousarray(legal_blocks(rng, 12, 4 * ff, width))
    up = np.ascontiguousarray(legal_blocks(rng, 12, 4 * ff, width))
    dt = 20
    down = np.ascontiguousarray(legal_blocks(rng, dt, 4 * width, ff))
    x = rng.normal(0, .05, (nt, width)).astype('f4')
    ids = np.full((nt, 10), -2, np.int32)
    w = np.zeros((nt, 10), np.float32)
    for t in range(nt):
        k = rng.integers(1, 5)
        ids[t, :k] = rng.permutation(4)[:k]
        w[t, :k] = rng.uniform(.05, .6, k)
    ids[:, 9] = np.where(ids[:, 9] == -2, -5, ids[:, 9])  # a pruned encoding of expert 3 with weight 0
    return gate, up, down, dt, x, ids, w


@pytest.mark.parametrize("width,ff", [(2560, 640), (2048, 512)])
def test_moe_bitexact_vs_reference_cpu(width, ff):
    """nbo_moe == the reference's qc_moe on both sides of nt=17, with pruned ids
    skipped and a duplicate id rejected (qwen/test_cpu_dispatch.py:69-92)."""
    r = O.ref_lib(width)
    if r is None:
        pytest.skip("reference cpu.c not built")
    rng = np.random.default_rng(27)
    ws = r.qc_create(18, 4)
    try:
        for nt in (1, 5, 17, 18):
            gate, up, down, dt, x, ids, w = _moe_case(r, width, ff, nt, rng)
            a = np.empty((nt, width), 'f4')
            b = np.empty((nt, width), 'f4')
            assert O.lib().nbo_moe(a.ctypes.data, x.ctypes.data, ids.ctypes.data, w.ctypes.data, nt, width, ff,
                                   gate.ctypes.data, 12, up.ctypes.data, 12, down.ctypes.data, dt) == 0
            assert r.qc_moe(ws, b.ctypes.data, x.ctypes.data, ids.ctypes.data, w.ctypes.data, nt,
                            gate.ctypes.data, 12, up.ctypes.data, 12, down.ctypes.data, dt) == 0
            np.testing.assert_array_equal(a.view('u4'), b.view('u4'), err_msg=f"nt={nt}")
            bad = ids.copy()
            bad[0, 1] = bad[0, 0]
            assert O.lib().nbo_moe(a.ctypes.data, x.ctypes.data, bad.ctypes.data, w.ctypes.data, nt, width, ff,
                                   gate.ctypes.data, 12, up.ctypes.data, 12, down.ctypes.data, dt) == -1
            assert r.qc_moe(ws, b.ctypes.data, x.ctypes.data, bad.ctypes.data, w.ctypes.data, nt,
                            gate.ctypes.data, 12, up.ctypes.data, 12, down.ctypes.data, dt) == -1
    finally:
        r.qc_destroy(ws)


# ---------------- exp ----------------

def test_exp_double_accuracy():
    xs = np.concatenate([np.linspace(-700, 700, 20001), np.random.default_rng(1).uniform(-30, 30, 20000)])
    got = np.array([O.lib().nbo_exp_d(float(v)) for v in xs])
    rel = np.abs(got - np.exp(xs)) / np.exp(xs)
    assert rel.max() < 4e-16


def test_expf_is_correctly_rounded_on_samples():
    """(float)exp(double) is the correctly rounded float exp (checked against
    float64 np.exp rounded once), and within 1 ulp of libm's expf, which is
    itself a 0.502-ulp routine and so differs in a small fraction of cases."""
    libm = C.CDLL("libm.so.6")
    libm.expf.argtypes, libm.expf.restype = [C.c_float], C.c_float
    xs = np.random.default_rng(2).uniform(-87, 88, 200000).astype(np.float32)
    xs = np.concatenate([xs, np.float32([0, -0.0, 1, -1, 1e-8, -1e-8, 88.7, -103.0])])
    ours = np.array([O.lib().nbo_expf(float(v)) for v in xs], np.float32)
    rounded = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert int(np.sum(ours.view('u4') != rounded.view('u4'))) <= 1
    theirs = np.array([libm.expf(float(v)) for v in xs], np.float32)
    ulp = np.abs(ours.view('i4').astype(np.int64) - theirs.view('i4').astype(np.int64))
    assert ulp.max() <= 1 and ulp.mean() < 2e-3


# ---------------- routing, pruning, dispatch ----------------

def test_route_known_answers():
    """qwen/test_gpu.py:338-346: ids = stable argsort(-logits)[:10], weights =
    softmax over the winners, any NaN -> all -1."""
    rng = np.random.default_rng(812603)
    logits = (rng.normal(size=(3, 512)) * .2).astype(np.float32)
    logits[0] = 0
    ids, w = O.route(logits)
    sel = np.argsort(-logits, axis=1, kind='stable')[:, :10]
    np.testing.assert_array_equal(ids, sel)
    vals = np.take_along_axis(logits, sel, axis=1).astype(np.float64)
    p = np.exp(vals - vals.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(w, p, atol=2e-5, rtol=2e-5)
    logits[1, 7] = np.nan
    ids, w = O.route(logits)
    np.testing.assert_array_equal(ids[1], -1)
    np.testing.assert_array_equal(w[1], 0)
    logits[2, 3] = np.inf
    ids, _ = O.route(logits)
    np.testing.assert_array_equal(ids[2], -1)


def test_route_invariants():
    rng = np.random.default_rng(4)
    logits = rng.normal(0, 1, (64, 512)).astype(np.float32)
    ids, w = O.route(logits)
    assert np.all(np.diff(w, axis=1) <= 0)
    np.testing.assert_allclose(w.sum(1), 1, atol=1e-6)
    # rank-0 numerator is exp(0)=1 exactly, so w0 == 1/total with total the float sum of numerators
    tot = np.zeros(64, np.float32)
    for k in range(10):
        tot = (tot + np.array([O.lib().nbo_expf(float(logits[t, ids[t, k]] - logits[t].max())) for t in range(64)], np.float32)).astype(np.float32)
    np.testing.assert_array_equal(w[:, 0], (np.float32(1) / tot).astype(np.float32))
    # ties resolve to the lowest index
    ids, _ = O.route(np.zeros((1, 512), np.float32))
    np.testing.assert_array_equal(ids[0], np.arange(10))


def test_prune_known_answer():
    """qwen/test_gpu.py:84-95: strict threshold, counters (5,10,4,2)."""
    ids = np.tile(np.arange(10, dtype=np.int32), (5, 1))
    w = np.full((5, 10), .1, np.float32)
    resident = np.zeros(512, np.uint8)
    resident[:8] = 1
    w[0, 8:] = .04; w[1, 8:] = .05; w[2, 8:] = .06; w[3, 8:] = 0; w[4, 8:] = [.01, .10]
    out_ids, out_w, st = O.prune(ids, w, resident, .10)
    assert np.all(out_ids[[0, 3], 8:] <= -2)
    np.testing.assert_array_equal(out_ids[[0, 3], 8:], -ids[[0, 3], 8:] - 2)
    np.testing.assert_array_equal(out_ids[[1, 2, 4]], ids[[1, 2, 4]])
    np.testing.assert_array_equal(out_w[:, :8], w[:, :8])
    assert np.all(out_w[[0, 3], 8:] == 0)
    assert (st.token_layers, st.missing_selections, st.skipped_selections, st.avoided_token_handoffs) == (5, 10, 4, 2)
    assert st.skipped_mass == pytest.approx(2 * float(np.float32(.04)), abs=0)
    flags, mass = O.coverage(ids, w, resident)
    np.testing.assert_array_equal(flags, [1, 2, 2, 1, 2])
    assert mass[1] == 2 * float(np.float32(.05))  # float(.05)*2 > 0.10: handoff, not pruned
    # an invalid id makes the token uncounted
    ids2 = ids.copy(); ids2[2, 5] = 600
    _, _, st2 = O.prune(ids2, w, resident, .10)
    assert st2.token_layers == 4


def test_map_and_dispatch_brute_force():
    """qwen/test_gpu.py:352-359 at nt 511/513/1025/2048, plus the CSR form."""
    rng = np.random.default_rng(812603)
    for nt in (1, 17, 511, 513, 1025, 2048):
        ids = np.stack([rng.choice(512, 10, replace=False) for _ in range(nt)]).astype(np.int32)
        m, counts = O.moe_map(ids)
        off, tok, slot = O.dispatch(ids)
        for e in range(512):
            want = np.flatnonzero((ids == e).any(1))
            assert counts[e] == len(want)
            np.testing.assert_array_equal(m[e, :len(want)], want)
            np.testing.assert_array_equal(tok[off[e]:off[e + 1]], want)
            np.testing.assert_array_equal(ids.reshape(-1)[slot[off[e]:off[e + 1]]], e)
    ids = np.full((2, 10), -2, np.int32); ids[:, 0] = [3, 3]; ids[1, 1] = -40
    off, tok, slot = O.dispatch(ids)
    assert off[-1] == 2 and list(tok) == [0, 1]
    ids[0, 2] = 3
    assert O.dispatch(ids) is None
    ids[0, 2] = 512
    assert O.dispatch(ids) is None


# ---------------- config 3 inputs: router bias ----------------

def test_zipf_bias_closed_form():
    """bias = log p(pi(e)) / 3 with p(r) proportional to r**-1.1: exp(3*bias)
    is a probability vector whose sorted values are the Zipf law, and the
    permutation depends only on the seed."""
    from nebula_amd import synth
    b = synth.zipf_bias(33).astype(np.float64)
    p = np.exp(3.0 * b)
    assert abs(p.sum() - 1.0) < 1e-5
    r = np.arange(1, 513, dtype=np.float64)
    want = r ** -1.1 / (r ** -1.1).sum()
    np.testing.assert_allclose(np.sort(p)[::-1], want, rtol=2e-6)
    np.testing.assert_array_equal(synth.zipf_bias(33), b.astype(np.float32))
    assert not np.array_equal(synth.zipf_bias(34), synth.zipf_bias(33))


def test_resident_ranking_order():
    """Config 4's resident set: activation count first, then accumulated
    routed weight, then the lower id (qwen/README.md:38); ids outside 0..511
    (pruned encodings, invalid routing) are ignored."""
    from nebula_amd import synth
    ids = np.array([[5, 7, 9, -1], [7, 5, 3, -7], [9, 3, 600, 2]], np.int32)
    w = np.array([[0.1, 0.2, 0.3, 0.9], [0.3, 0.1, 0.05, 0.9], [0.1, 0.3, 0.9, 0.01]], np.float32)
    # counts: 5:2 7:2 9:2 3:2 2:1; weights: 5:.2 7:.5 9:.4 3:.35 2:.01
    m = synth.resident_ranking(ids, w, 3)
    assert sorted(np.flatnonzero(m).tolist()) == [3, 7, 9]
    assert synth.resident_ranking(ids, w, 4)[5] == 1 and synth.resident_ranking(ids, w, 4)[2] == 0
    # equal count and weight: the lower id
    m = synth.resident_ranking(np.array([[4, 8]], np.int32), np.array([[0.5, 0.5]], np.float32), 1)
    assert np.flatnonzero(m).tolist() == [4]


def test_ranking_inputs_share_the_batch_base():
    """Context 0 of the ranking set has the verify batch's base (the batch
    and the ranking rows differ only by their noise), the others do not."""
    from nebula_amd import synth
    batch = synth.inputs(77, 17, 256, correlated=True)
    rank = synth.ranking_inputs(77, 4242, tokens=64, width=256)
    c = lambda a, b: float(np.mean(a, 0) @ np.mean(b, 0) / np.linalg.norm(np.mean(a, 0)) / np.linalg.norm(np.mean(b, 0)))
    assert c(batch, rank[0::8]) > 0.95
    assert all(abs(c(batch, rank[k::8])) < 0.5 for k in range(1, 8))
    assert not np.any(np.all(np.isclose(rank[:, None, :], batch[None, :, :]), axis=2))


def test_layer_router_bias_changes_routing_as_logits_plus_bias():
    """nbo_layer with a router bias routes exactly as route(matmul(x) + bias)
    and returns those logits; a zero bias changes nothing."""
    from nebula_amd import synth
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (6, 256)).astype(np.float32)
    bias = synth.zipf_bias(7)
    H = O.HostLayer(11, width=256, ff=128, gt=12, ut=12, dt=20, router_bias=bias)
    out, ids, w, logits, flags, _ = H.forward(x)
    raw = O.matmul(H.router, 0, 512, 256, x)
    np.testing.assert_array_equal(logits, raw + bias)
    oi, ow = O.route(raw + bias)
    np.testing.assert_array_equal(ids, oi)
    np.testing.assert_array_equal(w.view('u4'), ow.view('u4'))
    assert not np.array_equal(ids, O.route(raw)[0])
    H0 = O.HostLayer(11, width=256, ff=128, gt=12, ut=12, dt=20, router_bias=np.zeros(512, np.float32))
    H1 = O.HostLayer(11, width=256, ff=128, gt=12, ut=12, dt=20)
    a, b = H0.forward(x), H1.forward(x)
    np.testing.assert_array_equal(a[0].view('u4'), b[0].view('u4'))
    np.testing.assert_array_equal(a[1], b[1])


# ---------------- shared expert and layer composition ----------------

def test_shared_expert_closed_form():
    rng = np.random.default_rng(8)
    D, Fd, nt = 512, 256, 3
    g = np.ascontiguousarray(legal_blocks(rng, 12, Fd, D)); u = np.ascontiguousarray(legal_blocks(rng, 12, Fd, D))
    dn = np.ascontiguousarray(legal_blocks(rng, 12, D, Fd))
    inp = rng.normal(0, .05, (1, D)).astype(np.float32)
    x = rng.normal(0, 1, (nt, D)).astype(np.float32)
    out = rng.normal(0, 1, (nt, D)).astype(np.float32)
    base = out.copy()
    assert O.lib().nbo_shared(out.ctypes.data, x.ctypes.data, nt, D, Fd, g.ctypes.data, 12, u.ctypes.data, 12,
                              dn.ctypes.data, 12, inp.ctypes.data) == 0
    x64 = x.astype(np.float64)
    gg = x64 @ dequant_np(g, 12, Fd, D).T
    uu = x64 @ dequant_np(u, 12, Fd, D).T
    mid = gg / (1 + np.exp(-gg)) * uu
    s = mid @ dequant_np(dn, 12, D, Fd).T
    lg = x64 @ inp[0].astype(np.float64)
    want = base + s / (1 + np.exp(-lg))[:, None]
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=2e-5)


# ---------------- generator ----------------

def test_gaussian_generator_moments():
    n = 400000
    z = np.array([O.lib().nbs_gauss(7, 3, i) for i in range(n)])
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert abs(((z - z.mean()) ** 4).mean() / z.var() ** 2 - 3) < 0.05
    assert abs((z > 1.96).mean() - 0.025) < 0.002


def test_encoders_are_legal_and_close():
    rng = np.random.default_rng(11)
    x = (rng.normal(0, .02, (64, 256))).astype(np.float32)
    blocks = np.zeros((64, 144), np.uint8)
    for r in range(64):
        O.lib().nbs_encode_q4k(blocks[r].ctypes.data, x[r].ctypes.data)
    deq = dequant_np(blocks, 12, 64, 256)
    # each value lies within half a quantisation step (plus the 6-bit scale error)
    assert np.abs(deq - x).max() < 0.02 * 5 / 15
    assert np.corrcoef(deq.ravel(), x.ravel())[0, 1] > 0.99
    xb = x.reshape(-1, 32)
    ib = np.zeros((xb.shape[0], 18), np.uint8)
    for r in range(xb.shape[0]):
        O.lib().nbs_encode_iq4nl(ib[r].ctypes.data, np.ascontiguousarray(xb[r]).ctypes.data)
    deq = dequant_np(ib.reshape(1, -1), 20, 1, xb.size).reshape(xb.shape)
    assert np.corrcoef(deq.ravel(), xb.ravel())[0, 1] > 0.99


def test_fill_matrix_deterministic():
    a = O.fill_matrix(12, 5, (2 << 32) | 7, 8, 512)
    b = O.fill_matrix(12, 5, (2 << 32) | 7, 8, 512)
    c = O.fill_matrix(12, 5, (2 << 32) | 8, 8, 512)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c)


# ---------------- C ABI exports (no GPU calls) ----------------

def _declared(header):
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b((?:qg|nm)_[a-z0-9_]+)\s*\(", text)))


def _exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_libraries_export_every_declared_symbol():
    gpu = ROOT / "nebula_amd" / "lib" / "libqwen_gpu.so"
    host = ROOT / "nebula_amd" / "lib" / "libnebula_moe.so"
    if not gpu.exists() or not host.exists():
        pytest.skip("native libraries not built")
    missing = [s for s in _declared("qwen_gpu.h") if s not in _exported(gpu)]
    assert not missing, missing
    missing = [s for s in _declared("nebula_moe.h") if s not in _exported(host)]
    assert not missing, missing
    C.CDLL(str(gpu))  # loads without a GPU; nothing is called
    C.CDLL(str(host))


def test_handoff_host_checks_without_gpu():
    """nm_moe_handoff's scratch size (count, rows, packed rows, ids, weights,
    host rows; 256-byte aligned pieces) and its argument checks, which reject
    before any device call."""
    gpu = ROOT / "nebula_amd" / "lib" / "libqwen_gpu.so"
    host = ROOT / "nebula_amd" / "lib" / "libnebula_moe.so"
    if not gpu.exists() or not host.exists():
        pytest.skip("native libraries not built")
    from nebula_amd import qg
    h = qg.host()
    a = lambda n: (n + 255) // 256 * 256
    for D, T in ((2048, 17), (2048, 1), (2560, 8192), (256, 3)):
        assert h.nm_handoff_scratch_bytes(D, T) == 256 + a(4 * T) + 2 * a(4 * T * D) + 2 * a(40 * T)
    assert h.nm_handoff_scratch_bytes(2048, 0) == 0 and h.nm_handoff_scratch_bytes(2048, 8193) == 0
    cb = qg.CPU_MOE_FN(lambda *args: 0)
    handed = C.c_int(7)
    assert h.nm_moe_handoff(None, None, None, None, None, None, 4, 2048, None, 0, cb, None, C.byref(handed)) != 0
    assert handed.value == 0 and b"invalid handoff arguments" in h.nm_last_error()
    buf = (C.c_char * 64)()
    p = C.addressof(buf)
    assert h.nm_moe_handoff(p, None, p, p, p, p, 4, 2048, p, 64, cb, None, None) != 0
    assert b"scratch" in h.nm_last_error()


def test_reference_signatures_bind():
    """Every qg_* name the reference's ctypes caller binds for the MoE path
    (qwen/test_gpu.py:14-33) exists with the same arity in the header."""
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "qwen_gpu.h").read_text(), flags=re.S)
    arity = {"alloc": 1, "free": 1, "write": 3, "read": 3, "copy": 3, "zero": 2, "sync": 0, "error": 1, "matmul": 7,
             "gather": 5, "norm": 9, "unary": 5, "binary": 5, "route": 4, "prune_routes": 6, "moe_map": 3,
             "moe_gather": 4, "moe_scatter": 7, "moe_reduce": 3, "mtp_moe": 12}
    for name, n in arity.items():
        m = re.search(r"\bqg_%s\(([^;]*)\);" % name, text)
        assert m, name
        args = [a for a in m.group(1).split(",") if a.strip() and a.strip() != "void"]
        assert len(args) == n, (name, args)


def test_tensor_bytes_host_logic():
    """qg_tensor_bytes (gpu.cu:114-120): row bytes of dims[0] columns times
    the other dims; columns must fill whole blocks; a zero dim or overflow is
    an error.  Pure host arithmetic, so it runs without a GPU."""
    gpu = ROOT / "nebula_amd" / "lib" / "libqwen_gpu.so"
    if not gpu.exists():
        pytest.skip("native libraries not built")
    from nebula_amd import qg
    lib = qg.lib()
    out = C.c_uint64()

    def tb(typ, dims):
        d = (C.c_uint64 * 4)(*dims)
        rc = lib.qg_tensor_bytes(typ, d, C.byref(out))
        return None if rc else out.value
    assert tb(0, (2560, 512, 1, 1)) == 2560 * 512 * 4
    assert tb(12, (2560, 640, 512, 1)) == 10 * 144 * 640 * 512
    assert tb(20, (640, 2560, 512, 1)) == 20 * 18 * 2560 * 512
    assert tb(12, (2048, 512, 512, 1)) == 8 * 144 * 512 * 512
    assert tb(1, (100, 3, 1, 1)) == 600
    assert tb(12, (2000, 1, 1, 1)) is None          # not a whole superblock
    assert tb(20, (48, 1, 1, 1)) is None
    assert tb(12, (2560, 0, 1, 1)) is None          # zero dim
    assert tb(0, (1 << 30, 1 << 30, 1 << 30, 1)) is None  # overflow
    assert tb(99, (256, 1, 1, 1)) is None           # unknown type


def test_prefill_launch_mode_switch_host_logic():
    """qg_prefill_int8_dense: a per-thread setting (0 one gate/up launch, 1
    the dense experts split off on int8, 2 split off on fp16; other values
    select 0) that returns the previous mode.  Host state only, so it runs
    without a GPU."""
    gpu = ROOT / "nebula_amd" / "lib" / "libqwen_gpu.so"
    if not gpu.exists():
        pytest.skip("native libraries not built")
    from nebula_amd import qg
    lib = qg.lib()
    prev = lib.qg_prefill_int8_dense(0)
    try:
        assert lib.qg_prefill_int8_dense(2) == 0
        assert lib.qg_prefill_int8_dense(1) == 2
        assert lib.qg_prefill_int8_dense(7) == 1
        assert lib.qg_prefill_int8_dense(-1) == 0
        assert lib.qg_prefill_int8_dense(0) == 0
    finally:
        lib.qg_prefill_int8_dense(prev)
