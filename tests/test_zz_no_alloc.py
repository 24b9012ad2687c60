"""qg_moe_forward_noalloc: the layer with the library's static per-device
workspace (no allocation) equals qg_moe_forward with a caller workspace bit
for bit, on two calls in a row (the second with fewer tokens, so the shared
workspace holds the first call's contents), on the decode and the prefill
paths; layers whose workspace exceeds the static size are rejected."""
import ctypes as C
import sys

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
