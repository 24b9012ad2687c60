"""Synthetic routed-MoE layers for the benchmark and the parity tests.

Weights are generated on the device (qg_synth_matrix): tensor `t` of expert
`e` in a layer with seed `s` holds sigma*N(0,1) values from stream
(t << 32 | e), encoded to GGML Q4_K / IQ4_NL / F32.  The test oracle states the
same generator on the CPU (oracle/nb_synth.c), so both sides see identical
bytes.  Inputs x are numpy-seeded and RMS-normalised on the host.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import qg

ROUTER, GATE, UP, DOWN, SH_GATE, SH_UP, SH_DOWN, SH_INP = 1, 2, 3, 4, 5, 6, 7, 8
EXPERTS, TOP = 512, 10
SIGMA = 0.02


def stream(tensor: int, expert: int = 0) -> int:
    return (tensor << 32) | expert


def rmsnorm(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + eps)).astype(np.float32)


def inputs(seed: int, tokens: int, width: int, correlated: bool = False) -> np.ndarray:
    """Config 0: RMSNorm(N(0,1)) rows.  Config 1 (correlated): RMSNorm(base + 0.3*noise_t)."""
    rng = np.random.default_rng(seed)
    if correlated:
        base = rng.standard_normal(width)
        x = base[None, :] + 0.3 * rng.standard_normal((tokens, width))
    else:
        x = rng.standard_normal((tokens, width))
    return rmsnorm(x)


RANKING_TOKENS, RANKING_CONTEXTS = 4096, 8


def ranking_inputs(batch_seed: int, noise_seed: int, tokens: int = RANKING_TOKENS, width: int = 2048,
                   contexts: int = RANKING_CONTEXTS) -> np.ndarray:
    """Config 4's ranking set: `tokens` rows from `contexts` correlated
    contexts, RMSNorm(base_c + 0.3*noise), token i in context i % contexts.
    Context 0's base is the verify batch's own (inputs(batch_seed, ...,
    correlated=True) draws the same base first); the other bases and all the
    noise come from `noise_seed`, so no ranking row equals a batch row.  With
    one context the top 128 experts cover every selection of the batch (every
    token flag 0); with 8 the batch's frequent experts are resident and some
    of its rare ones are not, so its tokens mix flags 0, 1 and 2."""
    base0 = np.random.default_rng(batch_seed).standard_normal(width)
    rng = np.random.default_rng(noise_seed)
    bases = np.concatenate([base0[None, :], rng.standard_normal((contexts - 1, width))])
    x = bases[np.arange(tokens) % contexts] + 0.3 * rng.standard_normal((tokens, width))
    return rmsnorm(x)


def resident_ranking(ids: np.ndarray, weights: np.ndarray, count: int = 128) -> np.ndarray:
    """The resident mask of the `count` best-ranked experts over routed
    selections (ids, weights [tokens, 10]): activation count descending, then
    accumulated router weight descending, then expert id ascending, the
    reference's expert ranking (qwen/README.md:38).  Ids outside 0..511 are
    ignored."""
    ids = np.asarray(ids).ravel()
    w = np.asarray(weights).ravel().astype(np.float64)
    ok = (ids >= 0) & (ids < EXPERTS)
    hits = np.bincount(ids[ok], minlength=EXPERTS)
    mass = np.zeros(EXPERTS)
    np.add.at(mass, ids[ok], w[ok])
    order = np.lexsort((np.arange(EXPERTS), -mass, -hits))
    mask = np.zeros(EXPERTS, np.uint8)
    mask[order[:count]] = 1
    return mask


@dataclass
class LayerSpec:
    seed: int
    width: int = 2048
    ff: int = 512
    gate_type: int = 12
    up_type: int = 12
    down_type: int = 12
    shared: bool = False
    sh_types: tuple = (12, 12, 12)
    bias_seed: int | None = None   # Zipf(1.1) router bias (config 3) from this seed


@dataclass
class DeviceLayer:
    spec: LayerSpec
    bufs: dict = field(default_factory=dict)
    desc: qg.MoeLayer = None

    @property
    def expert_bytes(self) -> int:
        s = self.spec
        return s.ff * (qg.row_bytes(s.gate_type, s.width) + qg.row_bytes(s.up_type, s.width)) + s.width * qg.row_bytes(s.down_type, s.ff)


ZIPF_TEMPERATURE = 3.0


def zipf_bias(seed: int, s: float = 1.1) -> np.ndarray:
    """Config 3's router bias: bias[e] = log p(pi(e)) / 3, p(r) proportional
    to r**-s over ranks r = 1..512, pi a seeded permutation of the experts.
    The 1/3 calibrates for deterministic top-10 selection over logits whose
    own spread is ~0.9: the realised per-expert counts of a 2048-token batch
    then follow the Zipf expectation 20480*p(r) near the head (rank 10 ~310)
    and range from 0 to ~800 (an unscaled log p sends ~2000 tokens to the
    rank-1 expert and none to 370 experts)."""
    ranks = np.random.default_rng(seed).permutation(EXPERTS) + 1
    p = np.arange(1, EXPERTS + 1, dtype=np.float64) ** -s
    p /= p.sum()
    return (np.log(p[ranks - 1]) / ZIPF_TEMPERATURE).astype(np.float32)


def _synth(buf: qg.Device, offset: int, typ: int, seed: int, strm: int, rows: int, cols: int) -> None:
    qg.call("synth_matrix", buf.p + offset, typ, seed, strm, rows, cols, qg.F(SIGMA))


def build_layer(spec: LayerSpec, resident: np.ndarray | None = None, threshold: float = 0.10) -> DeviceLayer:
    D, Fd = spec.width, spec.ff
    L = DeviceLayer(spec)
    rb = {k: qg.row_bytes(t, c) for k, t, c in (("g", spec.gate_type, D), ("u", spec.up_type, D), ("d", spec.down_type, Fd))}
    L.bufs["router"] = qg.Device(nbytes=EXPERTS * D * 4)
    _synth(L.bufs["router"], 0, 0, spec.seed, stream(ROUTER), EXPERTS, D)
    for name, tensor, typ, rows, cols, key in (("gate", GATE, spec.gate_type, Fd, D, "g"), ("up", UP, spec.up_type, Fd, D, "u"),
                                               ("down", DOWN, spec.down_type, D, Fd, "d")):
        per = rows * rb[key]
        buf = qg.Device(nbytes=EXPERTS * per)
        qg.call("synth_experts", buf.p, typ, spec.seed, tensor, EXPERTS, rows, cols, qg.F(SIGMA))
        L.bufs[name] = buf
    desc = qg.MoeLayer()
    desc.width, desc.ff = D, Fd
    desc.router, desc.gate, desc.up, desc.down = L.bufs["router"].p, L.bufs["gate"].p, L.bufs["up"].p, L.bufs["down"].p
    desc.gate_type, desc.up_type, desc.down_type = spec.gate_type, spec.up_type, spec.down_type
    if spec.shared:
        sg, su, sd = spec.sh_types
        for name, tensor, typ, rows, cols in (("sh_gate", SH_GATE, sg, Fd, D), ("sh_up", SH_UP, su, Fd, D), ("sh_down", SH_DOWN, sd, D, Fd)):
            buf = qg.Device(nbytes=rows * qg.row_bytes(typ, cols))
            _synth(buf, 0, typ, spec.seed, stream(tensor), rows, cols)
            L.bufs[name] = buf
        L.bufs["sh_inp"] = qg.Device(nbytes=D * 4)
        _synth(L.bufs["sh_inp"], 0, 0, spec.seed, stream(SH_INP), 1, D)
        desc.sh_gate, desc.sh_up, desc.sh_down = L.bufs["sh_gate"].p, L.bufs["sh_up"].p, L.bufs["sh_down"].p
        desc.sh_gate_type, desc.sh_up_type, desc.sh_down_type = sg, su, sd
        desc.sh_gate_inp = L.bufs["sh_inp"].p
    if spec.bias_seed is not None:
        L.bufs["router_bias"] = qg.Device(zipf_bias(spec.bias_seed))
        desc.router_bias = L.bufs["router_bias"].p
    if resident is not None:
        L.bufs["resident"] = qg.Device(np.asarray(resident, np.uint8))
        desc.resident = L.bufs["resident"].p
        desc.threshold = threshold
    L.desc = desc
    return L


def read_expert(L: DeviceLayer, name: str, expert: int) -> np.ndarray:
    """Bytes of one expert's matrix (gate/up/down) copied back to the host."""
    s = L.spec
    typ, rows, cols = {"gate": (s.gate_type, s.ff, s.width), "up": (s.up_type, s.ff, s.width), "down": (s.down_type, s.width, s.ff)}[name]
    per = rows * qg.row_bytes(typ, cols)
    out = np.empty(per, np.uint8)
    qg.call("read", out.ctypes.data, L.bufs[name].p + expert * per, per)
    return out


class Forward:
    """Device buffers for qg_moe_forward at up to `tokens` tokens."""

    def __init__(self, width: int, ff: int, tokens: int):
        self.tokens, self.width = tokens, width
        self.ws_bytes = qg.lib().qg_moe_workspace_bytes(width, ff, tokens)
        if not self.ws_bytes:
            raise ValueError("unsupported shape for qg_moe_forward")
        self.ws = qg.Device(nbytes=self.ws_bytes)
        self.x = qg.Device(nbytes=tokens * width * 4)
        self.out = qg.Device(shape=(tokens, width), dtype=np.float32)
        self.ids = qg.Device(shape=(tokens, TOP), dtype=np.int32)
        self.w = qg.Device(shape=(tokens, TOP), dtype=np.float32)
        self.flags = qg.Device(shape=(tokens,), dtype=np.uint8)
        self.stats = qg.Device(nbytes=qg.C.sizeof(qg.PruneStats))

    def run(self, layer: DeviceLayer, nt: int, x_dev=None) -> None:
        qg.call("moe_forward", self.out.p, self.ids.p, self.w.p, self.flags.p, self.stats.p,
                x_dev if x_dev is not None else self.x.p, nt, qg.C.byref(layer.desc), self.ws.p, self.ws_bytes)
