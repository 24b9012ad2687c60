"""GPU tests of the qwen_* MoE surface (include/qwen_moe.h): a model opened
from a COB_QWEN_INDEX_V1 index written here (one target layer and the MTP
layer, D=2048, F=512, Q4_K gate/up, IQ4_NL down, shared expert).

- Cache mode (no hotlist): qwen_moe runs the reference's grouped_moe over an
  LRU expert cache (qwen.c:558-570,633-707); outputs against the oracle's
  layer, upload counts against the same LRU policy simulated here, and the
  QROUTE1 trace (qwen.c:86-94,638-646) byte for byte against a file built
  from the oracle's ids and weights.
- Hotlist mode: qwen_set_hotlist's validation (qwen.c:571-602), then the
  device layer with the resident mask and the CPU handoff of flagged tokens
  through the registered CPU MoE; every row against the oracle's full
  layer, prune counters bit-exact, cpu stats and the handoff profile.
- The MTP layer (all experts resident).
"""
import ctypes as C
import struct
import sys

import numpy as np
import pytest

import oracle as O
from index_writer import moe_layer_tensors, write_index
from nebula_amd import qg, synth
from nebula_amd.qg import Device, call

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 1e-3, 1e-4
D, F = 2048, 512
SPEC0 = synth.LayerSpec(seed=520, down_type=20, shared=True, sh_types=(12, 12, 12))
SPEC_MTP = synth.LayerSpec(seed=568, down_type=20, shared=True, sh_types=(12, 12, 12))
TYPES = dict(gate=12, up=12, down=20, sh_gate=12, sh_up=12, sh_down=12)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def assert_close(got, want, what=""):
    g, w = np.asarray(got, np.float64), np.asarray(want, np.float64)
    diff = g - w
    maxabs = float(np.abs(diff).max()) if diff.size else 0.0
    rel = float(np.linalg.norm(diff) / max(np.linalg.norm(w), 1e-30))
    assert maxabs <= MAX_ABS and rel <= REL_L2, f"{what}: max-abs {maxabs:.3g} rel-L2 {rel:.3g}"
    return maxabs, rel


def layer_arrays(spec):
    L = synth.build_layer(spec)
    out = {k: b.get() for k, b in L.bufs.items()}
    for b in L.bufs.values():
        b.free()
    return out


class Host:
    """Oracle layer whose expert bytes are the index file's."""

    def __init__(self, spec, arrays):
        self.H = O.HostLayer(spec.seed, gt=12, ut=12, dt=20, shared=True, sh_types=(12, 12, 12))
        self.a = arrays
        per = {"gate": F * qg.row_bytes(12, D), "up": F * qg.row_bytes(12, D), "down": D * qg.row_bytes(20, F)}
        self.fetch = lambda name, e: arrays[name][e * per[name]:(e + 1) * per[name]]
        np.testing.assert_array_equal(self.H.router.view(np.uint8), arrays["router"])

    def forward(self, x, resident=None):
        return self.H.forward(x, resident, fetch=self.fetch)


@pytest.fixture(scope="module")
def model_index(qgl, tmp_path_factory):
    say("writing a 2-layer index (target layer 0 + MTP layer 48)")
    a0, am = layer_arrays(SPEC0), layer_arrays(SPEC_MTP)
    files = [moe_layer_tensors(0, D, F, TYPES, a0, qg.row_bytes), moe_layer_tensors(48, D, F, TYPES, am, qg.row_bytes)]
    idx = write_index(tmp_path_factory.mktemp("qwen"), files)
    return idx, Host(SPEC0, a0), Host(SPEC_MTP, am)


def open_model(idx, resident, capacity=32):
    lib = qg.qwen()
    m = lib.qwen_open(str(idx).encode(), 4096, resident, capacity)
    assert m, lib.qwen_last_error().decode()
    return m


def run_moe(m, il, x, pos):
    nt = x.shape[0]
    xd, out = Device(x), Device(shape=(nt, D), dtype=np.float32)
    lib = qg.qwen()
    assert lib.qwen_moe(m, il, out.p, xd.p, nt, pos) == 0, lib.qwen_last_error().decode()
    return out.get()


def simulate_lru(calls, slots):
    """Upload count, hit count and calls with an upload under the cache
    policy of qwen.c:558-570,683-697 (resident experts first, then cold ones
    in ascending id; a free slot, else the least recently used unprotected)."""
    ids_of = [-1] * slots
    age = [0] * slots
    clock = uploads = hits = calls_with_upload = 0
    for ids in calls:
        ids = ids.ravel()
        needed = set(int(e) for e in ids)
        resident = set(e for e in ids_of if e >= 0)
        hits += sum(int(e) in resident for e in ids)
        order = sorted(e for e in needed if e in resident) + sorted(e for e in needed if e not in resident)
        before = uploads
        for e in order:
            if e in ids_of:
                j = ids_of.index(e)
            else:
                j, oldest = -1, None
                for k in range(slots):
                    if ids_of[k] < 0:
                        j = k
                        break
                    if ids_of[k] not in needed and (oldest is None or age[k] < oldest):
                        oldest, j = age[k], k
                assert j >= 0
                ids_of[j] = e
                uploads += 1
            clock += 1
            age[j] = clock
            needed.discard(e)
        calls_with_upload += uploads != before
    return uploads, hits, calls_with_upload


def test_cache_mode_trace_and_mtp(model_index, tmp_path):
    idx, H0, HM = model_index
    lib = qg.qwen()
    m = open_model(idx, resident=24)
    try:
        dims = [C.c_int() for _ in range(4)]
        assert lib.qwen_moe_shape(m, *[C.byref(d) for d in dims]) == 0
        assert [d.value for d in dims] == [D, F, 1, 1]
        trace = tmp_path / "routes.bin"
        assert lib.qwen_profile_routes(m, str(trace).encode()) == 0
        expected = [b"QROUTE1\n"]
        routed = []
        pos = 0
        for nt, seed in ((1, 1), (4, 2), (17, 3), (17, 4), (3, 5)):
            x = synth.inputs(8100 + seed, nt, D, correlated=True)
            say(f"qwen_moe cache mode nt={nt}")
            got = run_moe(m, 0, x, pos)
            want, ids, w, *_ = H0.forward(x)
            maxabs, rel = assert_close(got, want, f"cache mode nt={nt}")
            say(f"  cache mode nt={nt}: unique {len(np.unique(ids))} max-abs {maxabs:.2e} rel-L2 {rel:.2e}")
            expected.append(struct.pack("<3I", 0, pos, nt) + ids.astype("<i4").tobytes() + w.astype("<f4").tobytes())
            routed.append(ids)
            pos += nt
        assert lib.qwen_profile_routes(m, None) == 0
        assert trace.read_bytes() == b"".join(expected)
        st = qg.QwenStats()
        lib.qwen_get_stats(m, C.byref(st))
        uploads, hits, with_upload = simulate_lru(routed, 24)
        assert st.expert_handoffs == uploads and st.expert_hits == hits, (st.expert_handoffs, uploads, st.expert_hits, hits)
        assert st.expert_requests == 10 * pos and st.target_position == pos
        assert st.expert_upload_bytes == uploads * (2 * F * qg.row_bytes(12, D) + D * qg.row_bytes(20, F))
        prof = qg.QwenHandoffProfile()
        lib.qwen_get_handoff_profile(m, C.byref(prof))
        assert prof.layer_calls[0] == len(routed) and prof.layer_handoffs[0] == with_upload
        say(f"  cache: {uploads} uploads, {hits} hits over {len(routed)} calls")
        # without a hotlist there are no prune counters
        assert lib.qwen_get_prune_stats(m, C.byref(qg.PruneStats())) == -1
        # the MTP layer: every expert resident, the device layer without a mask
        for nt in (1, 17, 24):
            x = synth.inputs(8200 + nt, nt, D, correlated=True)
            say(f"qwen_moe MTP nt={nt}")
            got = run_moe(m, 48, x, 0)
            want, *_ = HM.forward(x)
            assert_close(got, want, f"MTP nt={nt}")
        assert lib.qwen_moe(m, 1, None, None, 1, 0) == -1
        assert lib.qwen_moe(m, 0, Device(nbytes=64).p, Device(nbytes=64).p, 33, 0) == -1  # above capacity
    finally:
        lib.qwen_close(m)


HOT_CALLS = ((17, 1), (4, 2), (1, 3), (17, 4))


def hotlist_for(H, count):
    """Every expert the first three calls route to (their tokens are then
    fully resident: no handoff), filled up to `count` with experts the last
    call does not route to (so its tokens miss much of their mass)."""
    first, last = [], set()
    for i, (nt, seed) in enumerate(HOT_CALLS):
        ids, _ = O.route(H.H.logits(synth.inputs(8300 + seed, nt, D, correlated=True)))
        if i < 3:
            for e in ids.ravel():
                if int(e) not in first:
                    first.append(int(e))
        else:
            last = set(int(e) for e in ids.ravel())
    fill = [e for e in range(512) if e not in first and e not in last]
    assert len(first) <= count <= len(first) + len(fill)
    return np.array(first + fill[:count - len(first)], np.int32)


def test_hotlist_mode_handoff_and_stats(model_index):
    idx, H0, HM = model_index
    lib = qg.qwen()
    R = 96
    m = open_model(idx, resident=R)
    calls = []

    def cpu_moe(ctx, out, xp, idp, wp, n, g, gt, u, ut, d, dt):
        try:
            calls.append(n)
            return O.lib().nbo_moe(out, xp, idp, wp, n, D, F, g, gt, u, ut, d, dt)
        except Exception as exc:  # noqa: BLE001 - reported through the return code
            say(f"callback failed: {exc!r}")
            return -1
    cb = qg.QWEN_CPU_MOE_FN(cpu_moe)
    try:
        hot = hotlist_for(H0, R)
        hp = hot.ctypes.data
        # validation (qwen.c:572-577)
        assert lib.qwen_set_hotlist(m, hp, R - 1, 4) == -1 and b"matching capacity" in lib.qwen_last_error()
        assert lib.qwen_set_hotlist(m, hp, R, 0) == -1 and lib.qwen_set_hotlist(m, hp, R, 29) == -1
        dup = hot.copy()
        dup[5] = dup[4]
        assert lib.qwen_set_hotlist(m, dup.ctypes.data, R, 4) == -1 and b"duplicate" in lib.qwen_last_error()
        bad = hot.copy()
        bad[0] = 512
        assert lib.qwen_set_hotlist(m, bad.ctypes.data, R, 4) == -1 and b"invalid" in lib.qwen_last_error()
        assert lib.qwen_set_cpu_threads(m, 4) == -1  # before the hotlist
        assert lib.qwen_set_cpu_moe(m, cb, None) == 0
        say("qwen_set_hotlist")
        assert lib.qwen_set_hotlist(m, hp, R, 8) == 0, lib.qwen_last_error().decode()
        assert lib.qwen_cpu_threads(m) == 8 and lib.qwen_set_cpu_threads(m, 4) == 0 and lib.qwen_cpu_threads(m) == 4
        assert lib.qwen_set_cpu_threads(m, 29) == -1
        assert lib.qwen_set_hotlist(m, hp, R, 8) == -1  # once per model
        resident = np.zeros(512, np.uint8)
        resident[hot] = 1
        st0 = qg.QwenStats()
        lib.qwen_get_stats(m, C.byref(st0))
        assert st0.expert_handoffs == R  # the pinning uploads
        total = O.PruneStats()
        flagged = layers_with = hits = missing = 0
        pos = 0
        host = qg.host()
        for i, (nt, seed) in enumerate(HOT_CALLS):
            x = synth.inputs(8300 + seed, nt, D, correlated=True)
            say(f"qwen_moe hotlist nt={nt}")
            before = len(calls)
            reads = host.nm_device_reads()
            got = run_moe(m, 0, x, pos)
            reads = host.nm_device_reads() - reads
            want, ids, w, _, flags, st = H0.forward(x, resident)
            # the reference's hit count over the pruned ids (qwen.c:656-657)
            hits += int(((ids >= 0) & (resident[np.clip(ids, 0, 511)] == 1)).sum())
            missing += int(((ids >= 0) & (resident[np.clip(ids, 0, 511)] == 0)).sum())
            ok = flags < 3
            maxabs, rel = assert_close(got[ok], want[ok], f"hotlist nt={nt}")
            n2 = int((flags == 2).sum())
            assert (len(calls) - before) == (1 if n2 else 0) and (not n2 or calls[-1] == n2)
            say(f"  hotlist nt={nt}: flags {np.bincount(flags, minlength=4).tolist()} max-abs {maxabs:.2e} rel-L2 {rel:.2e}")
            assert (n2 == 0) == (i < 3), flags
            # no device-to-host read for a layer without a flag-2 token; the
            # packed rows, ids and weights (three reads) for one with
            assert reads == (3 if n2 else 0), reads
            flagged += n2
            layers_with += n2 > 0
            for k in ("token_layers", "missing_selections", "skipped_selections", "avoided_token_handoffs"):
                setattr(total, k, getattr(total, k) + getattr(st, k))
            pos += nt
        assert layers_with == 1
        ps = qg.PruneStats()
        assert lib.qwen_get_prune_stats(m, C.byref(ps)) == 0
        assert (ps.token_layers, ps.missing_selections, ps.skipped_selections, ps.avoided_token_handoffs) == (
            total.token_layers, total.missing_selections, total.skipped_selections, total.avoided_token_handoffs)
        cs = qg.QwenCpuStats()
        lib.qwen_get_cpu_stats(m, C.byref(cs))
        assert cs.token_layers == flagged and cs.layer_handoffs == layers_with
        assert cs.activation_bytes == flagged * (D * 8 + 40) and cs.handoff_seconds > 0
        # compute_seconds is the CPU MoE call alone (qwen.c:663-668)
        assert 0 < cs.compute_seconds < cs.handoff_seconds
        assert cs.missing_selections == missing
        prof = qg.QwenHandoffProfile()
        lib.qwen_get_handoff_profile(m, C.byref(prof))
        assert prof.layer_calls[0] == 4 and prof.layer_handoffs[0] == layers_with
        st = qg.QwenStats()
        lib.qwen_get_stats(m, C.byref(st))
        assert st.expert_handoffs == R and st.expert_requests == 10 * pos  # no uploads after pinning
        assert st.expert_hits == hits, (st.expert_hits, hits)
        # the MTP layer is unaffected by the hotlist
        x = synth.inputs(8400, 5, D, correlated=True)
        assert_close(run_moe(m, 48, x, 0), HM.forward(x)[0], "MTP after hotlist")
    finally:
        lib.qwen_close(m)


def q8_0_random(rows: int, cols: int, experts: int, seed: int) -> np.ndarray:
    """GGML Q8_0 bytes (34 per 32 columns: fp16 scale, 32 int8) of random
    rows: scale 0.02/64, values uniform in [-127, 127]."""
    rng = np.random.default_rng(seed)
    blocks = experts * rows * (cols // 32)
    b = np.empty((blocks, 34), np.uint8)
    b[:, :2] = np.frombuffer(np.float16(0.02 / 64).tobytes(), np.uint8)
    b[:, 2:] = rng.integers(-127, 128, (blocks, 32), dtype=np.int8).view(np.uint8)
    return b.ravel()


def test_layers_of_different_expert_sizes(qgl, tmp_path):
    """Cache mode over a 2-layer model whose layer 1 keeps its down experts
    in Q8_0 (1.89x the IQ4_NL bytes of layer 0): the pinned uploader holds the
    largest expert of any layer (qwen.c:365-367), so layer 1's uploads go
    through and its outputs match the oracle.  The same model is refused a
    hotlist at a batch capacity above 17 (layer 1's format has no batch
    kernels), and an MTP layer in that format is refused at open."""
    Dm, Fm = 1024, 256
    s0 = synth.LayerSpec(seed=610, width=Dm, ff=Fm, down_type=20, shared=True, sh_types=(12, 12, 12))
    s1 = synth.LayerSpec(seed=611, width=Dm, ff=Fm, down_type=20, shared=True, sh_types=(12, 12, 12))
    a0, a1 = layer_arrays(s0), layer_arrays(s1)
    a1 = dict(a1, down=q8_0_random(Dm, Fm, 512, 612))
    t0 = dict(TYPES)
    t1 = dict(TYPES, down=8)
    files = [moe_layer_tensors(0, Dm, Fm, t0, a0, qg.row_bytes) + moe_layer_tensors(1, Dm, Fm, t1, a1, qg.row_bytes)]
    (tmp_path / "two").mkdir()
    idx = write_index(tmp_path / "two", files)
    lib = qg.qwen()
    m = lib.qwen_open(str(idx).encode(), 4096, 16, 4)
    assert m, lib.qwen_last_error().decode()
    try:
        H1 = O.HostLayer(611, width=Dm, ff=Fm, gt=12, ut=12, dt=8, shared=True, sh_types=(12, 12, 12))
        per = {"gate": Fm * qg.row_bytes(12, Dm), "up": Fm * qg.row_bytes(12, Dm), "down": Dm * qg.row_bytes(8, Fm)}
        fetch = lambda name, e: a1[name][e * per[name]:(e + 1) * per[name]]
        for il, nt in ((1, 4), (0, 3), (1, 1)):
            x = synth.inputs(700 + il * 10 + nt, nt, Dm, correlated=True)
            xd, out = Device(x), Device(shape=(nt, Dm), dtype=np.float32)
            say(f"qwen_moe cache mode, layer {il}, nt={nt}")
            assert lib.qwen_moe(m, il, out.p, xd.p, nt, 0) == 0, lib.qwen_last_error().decode()
            if il == 1:
                want = H1.forward(x, fetch=fetch)[0]
                assert_close(out.get(), want, f"layer 1 (Q8_0 down) nt={nt}")
        st = qg.QwenStats()
        lib.qwen_get_stats(m, C.byref(st))
        largest = 2 * Fm * qg.row_bytes(12, Dm) + Dm * qg.row_bytes(8, Fm)
        assert st.host_staging_bytes == 2 * largest, (st.host_staging_bytes, largest)
    finally:
        lib.qwen_close(m)
    # a hotlist at capacity 24 needs the batch kernels' formats in every layer
    m = lib.qwen_open(str(idx).encode(), 4096, 16, 24)
    assert m, lib.qwen_last_error().decode()
    try:
        hot = np.tile(np.arange(16, dtype=np.int32), 2)
        assert lib.qwen_set_cpu_moe(m, qg.QWEN_CPU_MOE_FN(lambda *a: -1), None) == 0
        assert lib.qwen_set_hotlist(m, hot.ctypes.data, 32, 4) == -1
        assert b"layer 1" in lib.qwen_last_error(), lib.qwen_last_error()
    finally:
        lib.qwen_close(m)
    # an MTP layer (blk.48) with Q8_0 down: refused above 17 tokens at open,
    # accepted at 17 (its tensors are zero: nothing is computed here)
    mtp = [(name.replace("blk.1.", "blk.48."), typ, dims, np.asarray(data).nbytes)
           for name, typ, dims, data in moe_layer_tensors(1, Dm, Fm, t1, a1, qg.row_bytes)]
    (tmp_path / "mtp").mkdir()
    idx2 = write_index(tmp_path / "mtp", [files[0], mtp])
    assert not lib.qwen_open(str(idx2).encode(), 4096, 16, 24)
    assert b"MTP" in lib.qwen_last_error(), lib.qwen_last_error()
    m = lib.qwen_open(str(idx2).encode(), 4096, 16, 17)
    assert m, lib.qwen_last_error().decode()
    lib.qwen_close(m)
