"""Writer of COB_QWEN_INDEX_V1 indexes (the format qwen.c:108-146 reads):
test infrastructure for the qwen_* surface.

An index is: the version line, "VERIFIED 1", 36 whitespace-separated
integers (3 id multipliers, 16 head offsets, 16 nonzero head vocab sizes,
the PLE end-of-sequence id), then FILE lines (id, bytes, path) and TENSOR
lines (name, file, offset, bytes, GGML type, dims[4]), tab-separated.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

HEADER_NUMBERS = [3, 5, 7] + list(range(16)) + [1000 + i for i in range(16)] + [2]


def tensor_line(name, file, offset, nbytes, typ, dims):
    d = list(dims) + [1] * (4 - len(dims))
    return "TENSOR\t" + "\t".join(str(v) for v in (name, file, offset, nbytes, typ, *d)) + "\n"


def write_index(directory: Path, files: list[list[tuple]], numbers=None, sparse: bool = False) -> Path:
    """files: per file, a list of (name, type, dims, data or byte count);
    each tensor starts 32-byte aligned.  A byte count in place of data (or
    sparse: every tensor given so) leaves the tensor's bytes zero without
    writing them (the file is only sized over them)."""
    directory = Path(directory)
    lines = ["COB_QWEN_INDEX_V1\n", "VERIFIED 1\n", " ".join(str(v) for v in (numbers or HEADER_NUMBERS)) + "\n"]
    tensor_lines = []
    for fid, tensors in enumerate(files):
        path = directory / f"weights{fid}.bin"
        off = 0
        with open(path, "wb") as f:
            for name, typ, dims, data in tensors:
                zero = sparse or isinstance(data, (int, np.integer))
                nbytes = int(data) if zero else np.asarray(data).nbytes
                off = (off + 31) // 32 * 32
                if not zero:
                    f.seek(off)
                    f.write(np.ascontiguousarray(data).tobytes())
                tensor_lines.append(tensor_line(name, fid, off, nbytes, typ, dims))
                off += nbytes
            f.truncate(off)
        lines.append(f"FILE\t{fid}\t{off}\t{path}\n")
    index = directory / "model.index"
    index.write_text("".join(lines + tensor_lines))
    return index


def moe_layer_tensors(il: int, D: int, F: int, types: dict, arrays: dict | None = None, row_bytes=None) -> list[tuple]:
    """The eight MoE tensors of layer il with GGML dims (qwen.c:157-161,
    D/F general).  types: gate/up/down/sh_gate/sh_up/sh_down GGML types.
    arrays: the bytes of each tensor (router, gate, up, down, sh_gate, sh_up,
    sh_down, sh_inp), or None for byte counts (sparse files)."""
    rb = row_bytes
    spec = [("ffn_gate_inp.weight", 0, (D, 512), "router", 512 * D * 4),
            ("ffn_gate_exps.weight", types["gate"], (D, F, 512), "gate", 512 * F * rb(types["gate"], D)),
            ("ffn_up_exps.weight", types["up"], (D, F, 512), "up", 512 * F * rb(types["up"], D)),
            ("ffn_down_exps.weight", types["down"], (F, D, 512), "down", 512 * D * rb(types["down"], F)),
            ("ffn_gate_shexp.weight", types["sh_gate"], (D, F), "sh_gate", F * rb(types["sh_gate"], D)),
            ("ffn_up_shexp.weight", types["sh_up"], (D, F), "sh_up", F * rb(types["sh_up"], D)),
            ("ffn_down_shexp.weight", types["sh_down"], (F, D), "sh_down", D * rb(types["sh_down"], F)),
            ("ffn_gate_inp_shexp.weight", 0, (D,), "sh_inp", D * 4)]
    return [(f"blk.{il}.{name}", typ, dims, arrays[key] if arrays is not None else nbytes)
            for name, typ, dims, key, nbytes in spec]
