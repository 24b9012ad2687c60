"""GPU parity of the full config-2 stack: 48 seeded config-0 layers (Q4_K,
D=2048, F=512, about 43.5 GB of experts resident), one token, each layer
h <- h + MoE(RMSNorm(h)), the whole stack captured into one graph by the C
host driver (libnebula_moe.so) and replayed.

Per layer, in record mode: the routing of the recorded normalised input is
bit-exact against the oracle's, and the layer output is within max-abs 1e-3
and rel-L2 1e-4 of the oracle's layer applied to that input.  The final
hidden state equals the initial one plus the sum of the recorded layer
outputs, added in layer order in fp32.  The seeds are the benchmark's
(9000 + layer).
"""
import ctypes as C
import sys
import time

import numpy as np
import pytest

import oracle as O
from nebula_amd import qg, synth
from nebula_amd.qg import call

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 1e-3, 1e-4
N_LAYERS = 48


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.mark.timeout(900)
def test_stack48_per_layer_parity(qgl):
    layers = []
    t0 = time.time()
    for l in range(N_LAYERS):
        layers.append(synth.build_layer(synth.LayerSpec(seed=9000 + l)))
        if l % 8 == 7:
            call("sync")
            say(f"built layers 0..{l} in {time.time() - t0:.1f} s")
    arr = (qg.MoeLayer * N_LAYERS)(*[L.desc for L in layers])
    h = qg.host()
    stack = h.nm_stack_create(arr, N_LAYERS, 1, 1)
    assert stack, h.nm_last_error()
    try:
        x0 = synth.inputs(31, 1, 2048)
        call("write", h.nm_stack_hidden(stack), x0.ctypes.data, x0.nbytes)
        say("48-layer stack forward (graph capture + replay)")
        assert h.nm_stack_forward(stack, 1, 1) == 0, h.nm_last_error()
        call("sync")
        hfin = np.empty((1, 2048), np.float32)
        call("read", hfin.ctypes.data, h.nm_stack_hidden(stack), hfin.nbytes)
        hcur = x0.copy()
        worst = (0.0, 0.0)
        for l in range(N_LAYERS):
            px, pids, pw, pout = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
            assert h.nm_stack_record(stack, l, C.byref(px), C.byref(pids), C.byref(pw), C.byref(pout)) == 0
            xl, ol = np.empty((1, 2048), np.float32), np.empty((1, 2048), np.float32)
            il, wl = np.empty((1, 10), np.int32), np.empty((1, 10), np.float32)
            for a, p in ((xl, px), (ol, pout), (il, pids), (wl, pw)):
                call("read", a.ctypes.data, p.value, a.nbytes)
            np.testing.assert_allclose(xl, synth.rmsnorm(hcur), rtol=2e-6, atol=2e-6, err_msg=f"layer {l} input")
            H = O.HostLayer(9000 + l)
            out, ids, w, _, _, _ = H.forward(xl, fetch=lambda name, e, L=layers[l]: synth.read_expert(L, name, e))
            np.testing.assert_array_equal(il, ids, err_msg=f"layer {l} ids")
            np.testing.assert_array_equal(wl.view('u4'), w.view('u4'), err_msg=f"layer {l} weights")
            diff = ol.astype(np.float64) - out
            maxabs = float(np.abs(diff).max())
            rel = float(np.linalg.norm(diff) / np.linalg.norm(out))
            assert maxabs <= MAX_ABS and rel <= REL_L2, f"layer {l}: max-abs {maxabs:.3g} rel-L2 {rel:.3g}"
            worst = (max(worst[0], maxabs), max(worst[1], rel))
            hcur = (hcur + ol).astype(np.float32)
            del H
        np.testing.assert_array_equal(hfin, hcur)
        say(f"48 layers: ids bit-exact; worst max-abs {worst[0]:.2e} rel-L2 {worst[1]:.2e}")
    finally:
        h.nm_stack_destroy(stack)
        for L in layers:
            for b in L.bufs.values():
                b.free()
