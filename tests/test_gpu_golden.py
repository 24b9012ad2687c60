"""The device path against the committed golden fixtures (tests/golden/):
the device generator writes the recorded bytes (SHA-256), qg_moe_forward
gives the recorded routing, weights and flags bit for bit and the recorded
outputs within max-abs 1e-3 / rel-L2 1e-4 (rows computed on the device,
flag < 2), and qg_moe_dispatch gives the recorded CSR bit for bit.  The
production-shape fixtures run the benchmark's kernels without the oracle
library: D = 2048 at one token the inline-routing gate/up and the fused
down+combine, at 17 tokens the one-expert-per-workgroup gate/up, the down and
the combine; D = 2560 the register-weight gate/up at 1 and 4 tokens."""
import ctypes as C
import hashlib
import sys

import numpy as np
import pytest

from nebula_amd import qg, synth
from nebula_amd.qg import Device, call
from test_golden import CASES, fixture_inputs, load

pytestmark = pytest.mark.gpu


def sha(v):
    return hashlib.sha256(np.ascontiguousarray(v).view(np.uint8).tobytes()).hexdigest()


@pytest.mark.parametrize("name", CASES)
def test_device_matches_fixture(qgl, name):
    meta, a = load(name)
    print(f"golden {name}", flush=True, file=sys.stderr)
    spec = synth.LayerSpec(seed=meta["seed"], width=meta["width"], ff=meta["ff"], gate_type=meta["gate_type"],
                           up_type=meta["up_type"], down_type=meta["down_type"], shared=meta["shared"],
                           sh_types=tuple(meta["shared_types"]))
    L = synth.build_layer(spec, resident=a.get("resident"), threshold=0.10)
    for key, h in meta["sha256"].items():
        if "." in key:
            t, e = key.split(".")
            got = sha(synth.read_expert(L, t, int(e)))
        else:
            got = sha(L.bufs[{"sh_inp": "sh_inp"}.get(key, key)].get())
        assert got == h, key
    nt, D = meta["tokens"], meta["width"]
    fw = synth.Forward(D, meta["ff"], nt)
    fw.x.set(fixture_inputs(meta, a))
    fw.run(L, nt)
    call("sync")
    np.testing.assert_array_equal(fw.ids.get()[:nt], a["ids"])
    np.testing.assert_array_equal(fw.w.get()[:nt].view('u4'), a["weights"].view('u4'))
    np.testing.assert_array_equal(fw.flags.get()[:nt], a["flags"])
    keep = a["flags"] < 2
    got = fw.out.get()[:nt][keep].astype(np.float64)
    want = a["out"][keep].astype(np.float64)
    diff = got - want
    assert np.abs(diff).max() <= 1e-3 and np.linalg.norm(diff) <= 1e-4 * np.linalg.norm(want)
    ids = Device(a["ids"])
    off = Device(shape=(513,), dtype=np.int32)
    tok, slot = Device(shape=(10 * nt,), dtype=np.int32), Device(shape=(10 * nt,), dtype=np.int32)
    st = Device(shape=(1,), dtype=np.int32)
    call("moe_dispatch", off.p, tok.p, slot.p, st.p, ids.p, nt)
    n = len(a["row_token"])
    np.testing.assert_array_equal(off.get(), a["offsets"])
    np.testing.assert_array_equal(tok.get()[:n], a["row_token"])
    np.testing.assert_array_equal(slot.get()[:n], a["row_slot"])
    assert st.get()[0] == 0
