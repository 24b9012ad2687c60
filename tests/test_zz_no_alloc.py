"""qg_moe_forward_noalloc: the layer with the library's static per-device
workspace (no allocation) equals qg_moe_forward with a caller workspace bit
for bit, on two calls in a row (the second with fewer tokens, so the shared
workspace holds the first call's contents), on the decode and the prefill
paths; layers whose workspace exceeds the static size are rejected; the
entry point captured into a graph (also as its first call in a fresh
process) replays bit-identical to the eager layer."""
import ctypes as C
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from nebula_amd import qg, synth
from nebula_amd.qg import Device, call

pytestmark = pytest.mark.gpu

CFG1 = synth.LayerSpec(seed=210, gate_type=12, up_type=12, down_type=20, shared=True, sh_types=(12, 12, 12))


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.fixture(scope="module")
def layer(qgl):
    say("building config-1 layer on device")
    return synth.build_layer(CFG1)


def run_both(L, x, nt):
    fw = synth.Forward(2048, 512, nt)
    fw.x.set(x)
    fw.run(L, nt)
    out = Device(shape=(nt, 2048), dtype=np.float32)
    ids = Device(shape=(nt, 10), dtype=np.int32)
    w = Device(shape=(nt, 10), dtype=np.float32)
    flags = Device(shape=(nt,), dtype=np.uint8)
    say(f"noalloc forward nt={nt}")
    call("moe_forward_noalloc", out.p, ids.p, w.p, flags.p, None, fw.x.p, nt, C.byref(L.desc))
    call("sync")
    np.testing.assert_array_equal(ids.get(), fw.ids.get()[:nt])
    np.testing.assert_array_equal(w.get().view('u4'), fw.w.get()[:nt].view('u4'))
    np.testing.assert_array_equal(flags.get(), fw.flags.get()[:nt])
    np.testing.assert_array_equal(out.get().view('u4'), fw.out.get()[:nt].view('u4'))


@pytest.mark.parametrize("first,second", [(17, 4), (100, 30), (40, 1)])
def test_noalloc_matches_workspace_entry_point(layer, first, second):
    for nt in (first, second):
        run_both(layer, synth.inputs(600 + nt, nt, 2048, correlated=True), nt)


def test_noalloc_rejects_oversize(layer):
    """2048 tokens need about 250 MB of workspace, beyond the static 16 MiB."""
    nt = 2048
    lib = qg.lib()
    assert lib.qg_moe_workspace_bytes(2048, 512, nt) > (16 << 20)
    out = Device(shape=(nt, 2048), dtype=np.float32)
    ids = Device(shape=(nt, 10), dtype=np.int32)
    w = Device(shape=(nt, 10), dtype=np.float32)
    x = Device(shape=(nt, 2048), dtype=np.float32)
    assert lib.qg_moe_forward_noalloc(out.p, ids.p, w.p, None, None, x.p, nt, C.byref(layer.desc)) != 0
    assert lib.qg_moe_forward_noalloc(out.p, ids.p, w.p, None, None, x.p, 0, C.byref(layer.desc)) != 0
    call("sync")


@pytest.mark.parametrize("nt", [4, 40])
def test_noalloc_graph_replays(layer, nt):
    """qg_moe_forward_noalloc captured (qg_graph_begin/end) and replayed three
    times, with the program's own eager work and a synchronisation between
    replays: every replay equals the eager qg_moe_forward bit for bit."""
    x = synth.inputs(800 + nt, nt, 2048, correlated=True)
    fw = synth.Forward(2048, 512, nt)
    fw.x.set(x)
    fw.run(layer, nt)
    call("sync")
    want = [fw.out.get()[:nt].copy(), fw.ids.get()[:nt].copy(), fw.w.get()[:nt].copy()]
    out = Device(shape=(nt, 2048), dtype=np.float32)
    ids = Device(shape=(nt, 10), dtype=np.int32)
    w = Device(shape=(nt, 10), dtype=np.float32)
    g = C.c_void_p()
    say(f"capture noalloc nt={nt}")
    call("graph_begin", C.byref(g))
    call("moe_forward_noalloc", out.p, ids.p, w.p, None, None, fw.x.p, nt, C.byref(layer.desc))
    call("graph_end", g)
    try:
        for r in range(3):
            call("graph_launch", g)
            call("sync")
            for got, exp in zip((out.get(), ids.get(), w.get()), want):
                np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32), err_msg=f"replay {r}")
            fw.run(layer, nt)
            call("sync")
    finally:
        qg.lib().qg_graph_destroy(g)


def test_noalloc_first_call_under_capture():
    """A fresh process whose first qg_moe_forward_noalloc call is made under
    graph capture (tests/noalloc_capture_child.py), at 4 and 40 tokens."""
    child = Path(__file__).resolve().parent / "noalloc_capture_child.py"
    say("child process: first noalloc call under capture")
    r = subprocess.run([sys.executable, "-u", str(child), "4", "40"], capture_output=True, text=True, timeout=300)
    say(r.stdout.strip())
    assert r.returncode == 0, r.stdout + r.stderr
