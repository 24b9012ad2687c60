"""Child process of test_zz_no_alloc.py: in a fresh process, the first call of
qg_moe_forward_noalloc is made under graph capture (so its one-time set-up,
the workspace address and the device query, runs while capturing); the
graph is replayed three times, with eager work and a synchronisation between
replays, and every replay must equal qg_moe_forward bit for bit.  Exit code 0
on success.  Arguments: token counts."""
import ctypes as C
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
from nebula_amd import qg, synth  # noqa: E402
from nebula_amd.qg import Device, call  # noqa: E402


def main() -> int:
    spec = synth.LayerSpec(seed=210, gate_type=12, up_type=12, down_type=20, shared=True, sh_types=(12, 12, 12))
    L = synth.build_layer(spec)
    for nt in [int(a) for a in sys.argv[1:]]:
        x = synth.inputs(700 + nt, nt, 2048, correlated=True)
        fw = synth.Forward(2048, 512, nt)
        fw.x.set(x)
        out, ids, w = Device(shape=(nt, 2048), dtype=np.float32), Device(shape=(nt, 10), dtype=np.int32), \
            Device(shape=(nt, 10), dtype=np.float32)
        g = C.c_void_p()
        print(f"capture noalloc nt={nt}", flush=True)
        call("graph_begin", C.byref(g))
        call("moe_forward_noalloc", out.p, ids.p, w.p, None, None, fw.x.p, nt, C.byref(L.desc))
        call("graph_end", g)
        fw.run(L, nt)  # eager reference with a caller workspace
        call("sync")
        want = fw.out.get()[:nt].copy(), fw.ids.get()[:nt].copy(), fw.w.get()[:nt].copy()
        for r in range(3):
            call("graph_launch", g)
            call("sync")
            got = out.get(), ids.get(), w.get()
            for a, b, what in zip(got, want, ("out", "ids", "weights")):
                if not np.array_equal(a.view(np.uint32), b.view(np.uint32)):
                    print(f"nt={nt} replay {r}: {what} differs", flush=True)
                    return 1
            fw.run(L, nt)  # the program's own eager work between replays
            call("sync")
        qg.lib().qg_graph_destroy(g)
        print(f"nt={nt}: 3 replays equal the eager layer", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
