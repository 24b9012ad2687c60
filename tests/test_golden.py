"""The committed golden fixtures (tests/golden/, written by make_golden.py)
against the oracle: the CPU generator still produces the recorded bytes
(SHA-256 of the router, the shared expert and every routed expert) and the
oracle's layer still reproduces the recorded logits, routing, flags, CSR
dispatch, prune counters and outputs bit for bit."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from nebula_amd import synth

HERE = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem for p in HERE.glob("*.json"))


def load(name):
    meta = json.loads((HERE / f"{name}.json").read_text())
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    return meta, arrays


def fixture_inputs(meta, arrays):
    """The fixture's input rows: stored, or (production shapes) regenerated
    from the seed and checked against the stored SHA-256."""
    import hashlib
    x = synth.inputs(meta["input_seed"], meta["tokens"], meta["width"], correlated=meta["correlated"])
    if "x" in arrays:
        np.testing.assert_array_equal(x.view('u4'), arrays["x"].view('u4'))
    else:
        assert hashlib.sha256(np.ascontiguousarray(x).view(np.uint8).tobytes()).hexdigest() == meta["x_sha256"]
    return x


def test_fixtures_present():
    assert len(CASES) >= 9, CASES
    # the production shapes of the benchmark's kernels are among them
    widths = {load(c)[0]["width"] for c in CASES}
    assert {256, 2048, 2560} <= widths, widths


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    import hashlib
    meta, a = load(name)
    H = O.HostLayer(meta["seed"], width=meta["width"], ff=meta["ff"], gt=meta["gate_type"], ut=meta["up_type"],
                    dt=meta["down_type"], shared=meta["shared"], sh_types=tuple(meta["shared_types"]))
    x = fixture_inputs(meta, a)
    out, ids, w, logits, flags, st = H.forward(x, a.get("resident"))
    sha = lambda v: hashlib.sha256(np.ascontiguousarray(v).view(np.uint8).tobytes()).hexdigest()
    for key, h in meta["sha256"].items():
        if "." in key:
            t, e = key.split(".")
            per = H.per[t]
            got = sha(getattr(H, t)[int(e) * per:(int(e) + 1) * per])
        else:
            got = sha(getattr(H, key))
        assert got == h, key
    for k, v in (("logits", logits), ("weights", w), ("out", out)):
        np.testing.assert_array_equal(v.view('u4'), a[k].view('u4'), err_msg=k)
    np.testing.assert_array_equal(ids, a["ids"])
    np.testing.assert_array_equal(flags, a["flags"])
    off, tok, slot = O.dispatch(ids)
    for k, v in (("offsets", off), ("row_token", tok), ("row_slot", slot)):
        np.testing.assert_array_equal(v, a[k], err_msg=k)
    if meta["prune_stats"]:
        assert [st.token_layers, st.missing_selections, st.skipped_selections, st.avoided_token_handoffs] == meta["prune_stats"][:4]
        assert st.skipped_mass == meta["prune_stats"][4]
