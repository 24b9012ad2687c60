"""ctypes binding of the CPU oracle: TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  Loads this directory's libnb_oracle.so (the C
restatement) and, when built, _ref/libqwen_cpu_<W>.so (the reference's own
cpu.c compiled in place; see Makefile).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
P, I, F, D64, U64 = C.c_void_p, C.c_int, C.c_float, C.c_double, C.c_uint64
EXPERTS, TOP = 512, 10


class PruneStats(C.Structure):
    _fields_ = [(k, C.c_uint64) for k in ("token_layers", "missing_selections", "skipped_selections", "avoided_token_handoffs")] + [
        ("skipped_mass", C.c_double)]


class LayerDesc(C.Structure):
    _fields_ = [("D", I), ("F", I), ("router", P), ("gate", P), ("up", P), ("down", P), ("gt", I), ("ut", I), ("dt", I),
                ("sh_gate", P), ("sh_up", P), ("sh_down", P), ("sgt", I), ("sut", I), ("sdt", I), ("sh_inp", P),
                ("router_bias", P)]


_SIG = {
    "nbo_row_bytes": ([I, I], C.c_size_t), "nbo_half": ([P], F), "nbo_weight_at": ([P, I, I], F),
    "nbo_matmul": ([P, P, I, I, I, P, I], I), "nbo_exp_d": ([D64], D64), "nbo_expf": ([F], F),
    "nbo_route": ([P, P, P, I], None), "nbo_prune": ([P, P, P, I, D64, P], None),
    "nbo_coverage": ([P, P, P, P, P, I], None), "nbo_moe_map": ([P, P, P, I], None),
    "nbo_dispatch": ([P, P, P, P, I], I),
    "nbo_moe": ([P, P, P, P, I, I, I, P, I, P, I, P, I], I),
    "nbo_shared": ([P, P, I, I, I, P, I, P, I, P, I, P], I),
    "nbo_layer": ([P, P, P, P, P, P, P, I, P, D64, P], I),
    "nbo_rmsnorm": ([P, P, I, I, F], None),
    "nbs_hash": ([U64, U64, U64], U64), "nbs_gauss": ([U64, U64, U64], D64),
    "nbs_f32_to_f16": ([F], C.c_uint16), "nbs_f16_to_f32": ([C.c_uint16], F),
    "nbs_encode_q4k": ([P, P], None), "nbs_encode_iq4nl": ([P, P], None),
    "nbs_fill_matrix": ([P, I, U64, U64, I, I, F], I), "nbs_stream": ([I, I], U64),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        path = HERE / "libnb_oracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} not built (make -C oracle own)")
        h = C.CDLL(str(path))
        for name, (a, r) in _SIG.items():
            fn = getattr(h, name)
            fn.argtypes, fn.restype = a, r
        _lib = h
    return _lib


def ref_lib(width: int = 2048):
    """The reference's cpu.c built for WIDTH=width (2048/512 or 2560/640), or None."""
    path = HERE / "_ref" / f"libqwen_cpu_{width}.so"
    if not path.exists():
        return None
    h = C.CDLL(str(path))
    h.qc_backend_name.restype = C.c_char_p
    h.qc_backend_available.argtypes = [C.c_char_p]
    h.qc_matmul.argtypes = [P, P, I, I, I, P, I, I]
    h.qc_matmul.restype = I
    h.qc_create.argtypes, h.qc_create.restype = [I, I], P
    h.qc_destroy.argtypes = [P]
    h.qc_moe.argtypes = [P, P, P, P, P, I, P, I, P, I, P, I]
    h.qc_moe.restype = I
    h.qc_weight_at.argtypes, h.qc_weight_at.restype = [P, I, I], F
    return h


def row_bytes(typ: int, cols: int) -> int:
    return int(lib().nbo_row_bytes(typ, cols))


def matmul(w: np.ndarray, typ: int, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    out = np.empty((x.shape[0], rows), np.float32)
    assert lib().nbo_matmul(out.ctypes.data, np.ascontiguousarray(w).ctypes.data, typ, rows, cols, x.ctypes.data, x.shape[0]) == 0
    return out


def route(logits: np.ndarray):
    logits = np.ascontiguousarray(logits, np.float32).reshape(-1, EXPERTS)
    nt = logits.shape[0]
    ids = np.empty((nt, TOP), np.int32)
    w = np.empty((nt, TOP), np.float32)
    lib().nbo_route(ids.ctypes.data, w.ctypes.data, logits.ctypes.data, nt)
    return ids, w


def prune(ids, w, resident, threshold=0.10):
    ids = np.array(ids, np.int32, copy=True)
    w = np.array(w, np.float32, copy=True)
    st = PruneStats()
    lib().nbo_prune(ids.ctypes.data, w.ctypes.data, np.ascontiguousarray(resident, np.uint8).ctypes.data, ids.shape[0], threshold, C.byref(st))
    return ids, w, st


def coverage(ids, w, resident):
    ids = np.ascontiguousarray(ids, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    nt = ids.shape[0]
    flags = np.empty(nt, np.uint8)
    mass = np.empty(nt, np.float64)
    lib().nbo_coverage(flags.ctypes.data, mass.ctypes.data, ids.ctypes.data, w.ctypes.data,
                       np.ascontiguousarray(resident, np.uint8).ctypes.data, nt)
    return flags, mass


def moe_map(ids):
    ids = np.ascontiguousarray(ids, np.int32)
    nt = ids.shape[0]
    m = np.zeros((EXPERTS, nt), np.int32)
    counts = np.empty(EXPERTS, np.int32)
    lib().nbo_moe_map(m.ctypes.data, counts.ctypes.data, ids.ctypes.data, nt)
    return m, counts


def dispatch(ids):
    ids = np.ascontiguousarray(ids, np.int32)
    nt = ids.shape[0]
    off = np.empty(EXPERTS + 1, np.int32)
    tok = np.empty(nt * TOP, np.int32)
    slot = np.empty(nt * TOP, np.int32)
    n = lib().nbo_dispatch(off.ctypes.data, tok.ctypes.data, slot.ctypes.data, ids.ctypes.data, nt)
    if n < 0:
        return None
    return off, tok[:n], slot[:n]


def fill_matrix(typ: int, seed: int, strm: int, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    out = np.empty(rows * row_bytes(typ, cols), np.uint8)
    assert lib().nbs_fill_matrix(out.ctypes.data, typ, seed, strm, rows, cols, F(sigma)) == 0
    return out


class HostLayer:
    """The oracle's copy of a synthetic layer: full-size per-tensor arrays in
    which only the experts that are needed get generated (CPU generator) or
    copied (from the device)."""

    def __init__(self, seed, width=2048, ff=512, gt=12, ut=12, dt=12, shared=False, sh_types=(12, 12, 12), router_bias=None):
        self.seed, self.D, self.F = seed, width, ff
        self.router_bias = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32).reshape(EXPERTS)
        self.gt, self.ut, self.dt = gt, ut, dt
        self.per = {"gate": ff * row_bytes(gt, width), "up": ff * row_bytes(ut, width), "down": width * row_bytes(dt, ff)}
        self.gate = np.zeros(EXPERTS * self.per["gate"], np.uint8)
        self.up = np.zeros(EXPERTS * self.per["up"], np.uint8)
        self.down = np.zeros(EXPERTS * self.per["down"], np.uint8)
        self.have = set()
        self.router = fill_matrix(0, seed, 1 << 32, EXPERTS, width).view(np.float32)
        self.shared = shared
        if shared:
            sg, su, sd = sh_types
            self.sh_types = sh_types
            self.sh_gate = fill_matrix(sg, seed, 5 << 32, ff, width)
            self.sh_up = fill_matrix(su, seed, 6 << 32, ff, width)
            self.sh_down = fill_matrix(sd, seed, 7 << 32, width, ff)
            self.sh_inp = fill_matrix(0, seed, 8 << 32, 1, width).view(np.float32)

    def ensure(self, experts, fetch=None) -> None:
        """Make the listed experts' matrices present: generated on the CPU, or
        fetch(name, e) -> bytes (a copy of the device's, whose generator is
        checked equal to this one's separately)."""
        for e in sorted(set(int(v) for v in np.ravel(experts) if 0 <= v < EXPERTS) - self.have):
            for name, tensor, typ, rows, cols in (("gate", 2, self.gt, self.F, self.D), ("up", 3, self.ut, self.F, self.D),
                                                  ("down", 4, self.dt, self.D, self.F)):
                per = self.per[name]
                getattr(self, name)[e * per:(e + 1) * per] = (
                    fetch(name, e) if fetch is not None else fill_matrix(typ, self.seed, (tensor << 32) | e, rows, cols))
            self.have.add(e)

    def desc(self) -> LayerDesc:
        d = LayerDesc(self.D, self.F, self.router.ctypes.data, self.gate.ctypes.data, self.up.ctypes.data, self.down.ctypes.data,
                      self.gt, self.ut, self.dt)
        if self.shared:
            d.sh_gate, d.sh_up, d.sh_down = self.sh_gate.ctypes.data, self.sh_up.ctypes.data, self.sh_down.ctypes.data
            d.sgt, d.sut, d.sdt = self.sh_types
            d.sh_inp = self.sh_inp.ctypes.data
        if self.router_bias is not None:
            d.router_bias = self.router_bias.ctypes.data
        return d

    def logits(self, x):
        """Router logits (+ the optional bias) of the rows of x."""
        logits = matmul(self.router, 0, EXPERTS, self.D, np.ascontiguousarray(x, np.float32))
        if self.router_bias is not None:
            logits += self.router_bias
        return logits

    def forward(self, x, resident=None, threshold=0.10, fetch=None):
        """The reference's layer on the CPU: (out, ids, weights, logits, flags, stats)."""
        x = np.ascontiguousarray(x, np.float32)
        nt = x.shape[0]
        logits = self.logits(x)
        ids, w = route(logits)
        self.ensure(ids, fetch)
        out = np.empty((nt, self.D), np.float32)
        oids = np.empty((nt, TOP), np.int32)
        ow = np.empty((nt, TOP), np.float32)
        flags = np.zeros(nt, np.uint8)
        st = PruneStats()
        res = np.ascontiguousarray(resident, np.uint8) if resident is not None else None
        d = self.desc()
        rc = lib().nbo_layer(out.ctypes.data, oids.ctypes.data, ow.ctypes.data, None, flags.ctypes.data, C.byref(d),
                             x.ctypes.data, nt, res.ctypes.data if res is not None else None, threshold, C.byref(st))
        assert rc == 0
        return out, oids, ow, logits, flags, st

    def routed(self, x, ids, w, fetch=None):
        """The routed part alone (qc_moe, cpu.c:235-261) of the rows of x with
        the given routing: what the host computes for handed-off tokens
        (qwen.c:658-678)."""
        x = np.ascontiguousarray(x, np.float32)
        ids, w = np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(w, np.float32)
        self.ensure(ids, fetch)
        out = np.empty((x.shape[0], self.D), np.float32)
        rc = lib().nbo_moe(out.ctypes.data, x.ctypes.data, ids.ctypes.data, w.ctypes.data, x.shape[0], self.D, self.F,
                           self.gate.ctypes.data, self.gt, self.up.ctypes.data, self.ut, self.down.ctypes.data, self.dt)
        assert rc == 0
        return out

    def shared_part(self, x):
        """The sigmoid-gated shared expert alone (qwen.c:708-713, added to a zero
        row): a handed-off token's device row.  Zero without a shared expert."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros((x.shape[0], self.D), np.float32)
        if self.shared:
            sg, su, sd = self.sh_types
            rc = lib().nbo_shared(out.ctypes.data, x.ctypes.data, x.shape[0], self.D, self.F, self.sh_gate.ctypes.data, sg,
                                  self.sh_up.ctypes.data, su, self.sh_down.ctypes.data, sd, self.sh_inp.ctypes.data)
            assert rc == 0
        return out
