"""Randomised parity sweep through the C ABI against the CPU oracle.

Seeded random batch sizes and inputs (independent or correlated tokens) over
the decode path (1..17 tokens, configs 0 and 1), config-1 layers with a
ranked resident set (coverage flags, pruning, handoff rows), the prefill path
(18..3000 tokens, configs 0, 1 and the Zipf-routed config 3) and the
reference's own 2560/640 shape at both.  Each case holds the bars of the
fixed-case tests: routing ids, weights and flags bit for bit, outputs within
max-abs 1e-3 and rel-L2 1e-4.
"""
import numpy as np
import pytest

import oracle as O
from nebula_amd import qg, synth
from nebula_amd.qg import Device, call
from test_gpu_parity import CFG0, CFG1, _check_layer, say
import test_gpu_prefill as P

pytestmark = pytest.mark.gpu

SEED = 20261202


@pytest.fixture(scope="module")
def layers(qgl):
    say("building config-0, config-1 and config-3 layers on device")
    L1 = synth.build_layer(CFG1)
    H1 = O.HostLayer(CFG1.seed, gt=12, ut=12, dt=20, shared=True, sh_types=(12, 12, 12))
    L0 = synth.build_layer(CFG0)
    H0 = O.HostLayer(CFG0.seed, gt=12, ut=12, dt=12)
    L3 = synth.build_layer(P.CFG3)
    H3 = P.host_layer(P.CFG3)
    return (L0, H0), (L1, H1), (L3, H3)


def test_decode_random_batches(layers):
    (L0, H0), (L1, H1), _ = layers
    rng = np.random.default_rng(SEED)
    fw = synth.Forward(2048, 512, 17)
    for i in range(60):
        nt, corr, seed = int(rng.integers(1, 18)), bool(rng.integers(0, 2)), 5000 + i
        L, H, name = (L1, H1, "config1") if i % 3 else (L0, H0, "config0")
        _check_layer(L, H, synth.inputs(seed, nt, 2048, correlated=corr), f"{name} seed={seed} B={nt} corr={corr}", fw=fw)


def test_decode_random_residency(layers):
    _, (L1, H1), _ = layers
    rng = np.random.default_rng(SEED + 1)
    fw = synth.Forward(2048, 512, 17)
    for r in range(3):
        ctx = 900 + r
        xs = synth.ranking_inputs(ctx, 4242 + r)
        dx = Device(xs)
        n = xs.shape[0]
        logits = Device(shape=(n, 512), dtype=np.float32)
        ids, w = Device(shape=(n, 10), dtype=np.int32), Device(shape=(n, 10), dtype=np.float32)
        call("matmul", logits.p, L1.bufs["router"].p, 0, 512, 2048, dx.p, n)
        call("route", ids.p, w.p, logits.p, n)
        resident = synth.resident_ranking(ids.get(), w.get(), 128)
        desc = qg.MoeLayer.from_buffer_copy(L1.desc)
        rdev = Device(resident)
        desc.resident, desc.threshold = rdev.p, 0.10
        saved = L1.desc
        L1.desc = desc
        try:
            for _ in range(4):
                nt = int(rng.integers(1, 18))
                _check_layer(L1, H1, synth.inputs(ctx, nt, 2048, correlated=True), f"resident ctx={ctx} B={nt}",
                             resident=resident, fw=fw)
        finally:
            L1.desc = saved


def test_prefill_random_batches(layers):
    (L0, H0), (L1, H1), (L3, H3) = layers
    rng = np.random.default_rng(SEED + 2)
    for i in range(8):
        big = i % 4 == 3
        nt = int(rng.integers(400, 3000)) if big else int(rng.integers(18, 400))
        corr, seed = bool(rng.integers(0, 2)), 7000 + i
        L, H, name = (L3, H3, "config3") if big else (L1, H1, "config1") if i % 2 else (L0, H0, "config0")
        x = synth.inputs(seed, nt, 2048, correlated=corr)
        fw = P.forward(L, x)
        P.check_routing(fw, H, x)
        P.check_outputs(fw, L, H, x, P.sample_rows(nt, min(24, nt), seed), f"prefill {name} seed={seed} B={nt} corr={corr}")


def test_reference_shape_random_batches(qgl):
    """The reference's own shape, D = 2560 / F = 640 (IQ4_NL down, shared
    expert with an IQ4_NL down): random decode and prefill batch sizes."""
    from test_gpu_dropin import REF, fetcher, host_layer
    L, H = synth.build_layer(REF), host_layer(REF)
    D, Fd = REF.width, REF.ff
    rng = np.random.default_rng(SEED + 3)
    for i in range(10):
        nt = int(rng.integers(1, 18)) if i < 7 else int(rng.integers(18, 700))
        corr, seed = bool(rng.integers(0, 2)), 8000 + i
        x = synth.inputs(seed, nt, D, correlated=corr)
        fw = synth.Forward(D, Fd, nt)
        fw.x.set(x)
        say(f"forward 2560/640 seed={seed} B={nt} corr={corr}")
        fw.run(L, nt)
        call("sync")
        ids, w = O.route(H.logits(x))
        np.testing.assert_array_equal(fw.ids.get()[:nt], ids, err_msg=f"routing ids seed={seed} B={nt}")
        np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), w.view('u4'), err_msg=f"routing weights seed={seed} B={nt}")
        rows = np.arange(nt) if nt <= 40 else P.sample_rows(nt, 24, seed)
        out, *_ = H.forward(x[rows], fetch=fetcher(L))
        maxabs, rel = P.assert_close(fw.out.get()[rows], out, f"2560/640 seed={seed} B={nt}")
        say(f"  2560/640 B={nt}: max-abs {maxabs:.2e} rel-L2 {rel:.2e}")
