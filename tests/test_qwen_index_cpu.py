"""CPU tests of the qwen_* surface (include/qwen_moe.h) that need no GPU:
the COB_QWEN_INDEX_V1 preflight (qwen_validate_index, the rules of
qwen.c:108-146 plus the MoE tensor shapes of qwen.c:157-161), the constants
native.py probes (qwen_max_draft()==16, qwen_handoff_version()==1,
native.py:84-101) and the ABI-visible struct layouts (qwen.h:11-21,68-71,
80-84).  Index files are sparse (sized, not written): the preflight never
reads weight payloads."""
import ctypes as C
import re
from pathlib import Path

import pytest

from index_writer import moe_layer_tensors, write_index

ROOT = Path(__file__).resolve().parent.parent
LIBS = [ROOT / "nebula_amd" / "lib" / n for n in ("libqwen_gpu.so", "libnebula_moe.so")]
pytestmark = pytest.mark.skipif(not all(p.exists() for p in LIBS), reason="native libraries not built")

D, F = 256, 32
TYPES = dict(gate=12, up=12, down=20, sh_gate=12, sh_up=12, sh_down=20)


def rb(typ, cols):
    from nebula_amd import qg
    return qg.row_bytes(typ, cols)


def q():
    from nebula_amd import qg
    return qg.qwen()


def layer(il, **over):
    ts = moe_layer_tensors(il, D, F, TYPES, None, rb)
    out = []
    for name, typ, dims, nbytes in ts:
        key = name.split(".", 2)[2]
        if key in over:
            typ, dims, nbytes = over[key]
        out.append((name, typ, dims, nbytes))
    return out


def validate(path):
    rc = q().qwen_validate_index(str(path).encode())
    return rc, q().qwen_last_error().decode()


def test_constants_and_struct_layouts():
    from nebula_amd import qg
    lib = q()
    assert lib.qwen_max_draft() == 16 and lib.qwen_handoff_version() == 1
    assert C.sizeof(qg.QwenStats) == 14 * 8 + 7 * 8 + 4 * 4
    assert C.sizeof(qg.QwenHandoffProfile) == 2 * 48 * 8
    assert C.sizeof(qg.QwenCpuStats) == 4 * 8 + 2 * 8
    assert C.sizeof(qg.PruneStats) == 4 * 8 + 8
    # the header declares the reference's field order (qwen.h:11-21,68-71,80-84)
    text = (ROOT / "include" / "qwen_moe.h").read_text()
    for fields in ("gpu_weight_bytes, gpu_state_bytes, gpu_workspace_bytes, gpu_arena_bytes",
                   "target_position, mtp_position, context, resident_per_layer",
                   "uint64_t layer_calls[48], layer_handoffs[48]",
                   "layer_handoffs, token_layers, missing_selections, activation_bytes",
                   "token_layers, missing_selections, skipped_selections, avoided_token_handoffs"):
        assert fields in text, fields


def test_every_declared_qwen_symbol_is_exported():
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "qwen_moe.h").read_text(), flags=re.S)
    names = set(re.findall(r"\b(qwen_[a-z_0-9]+)\s*\(", text))
    lib = C.CDLL(str(LIBS[1]))
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # every name native.py binds for the MoE path (native.py:84-117)
    for n in ("qwen_set_hotlist", "qwen_get_prune_stats", "qwen_get_cpu_stats", "qwen_handoff_version",
              "qwen_get_handoff_profile", "qwen_max_draft", "qwen_last_error", "qwen_get_stats",
              "qwen_set_cpu_threads", "qwen_cpu_threads", "qwen_open", "qwen_close", "qwen_validate_index"):
        assert n in names, n


def test_validate_good_index(tmp_path):
    idx = write_index(tmp_path, [layer(0) + layer(1), layer(48) + [("output_norm.weight", 0, (D,), D * 4)]], sparse=True)
    rc, msg = validate(idx)
    assert rc == 0, msg


@pytest.mark.parametrize("case,message", [
    ("version", "invalid Qwen index version"),
    ("unverified", "SHA256 verification"),
    ("zero_vocab", "malformed"),
    ("short_numbers", "malformed"),
    ("file_size", "weights missing/incomplete"),
    ("tensor_bytes", "malformed"),
    ("duplicate", "malformed"),
    ("past_end", "malformed"),
    ("bad_file_id", "malformed"),
    ("unknown_line", "malformed"),
    ("router_shape", "invalid MoE layer 0"),
    ("down_shape", "invalid MoE layer 1"),
    ("no_layer0", "no MoE layer 0"),
    ("widths", "unsupported MoE widths"),
])
def test_validate_rejects(tmp_path, case, message):
    idx = write_index(tmp_path, [layer(0) + layer(1)], sparse=True)
    text = idx.read_text()
    lines = text.splitlines(keepends=True)
    tensor = [i for i, l in enumerate(lines) if l.startswith("TENSOR")]
    filel = [i for i, l in enumerate(lines) if l.startswith("FILE")][0]
    if case == "version":
        lines[0] = "COB_QWEN_INDEX_V2\n"
    elif case == "unverified":
        lines[1] = "VERIFIED 0\n"
    elif case == "zero_vocab":
        nums = lines[2].split()
        nums[19] = "0"
        lines[2] = " ".join(nums) + "\n"
    elif case == "short_numbers":
        lines[2] = " ".join(lines[2].split()[:20]) + "\n"
    elif case == "file_size":
        f = lines[filel].split("\t")
        f[2] = str(int(f[2]) + 1)
        lines[filel] = "\t".join(f)
    elif case == "tensor_bytes":
        t = lines[tensor[1]].split("\t")
        t[4] = str(int(t[4]) - 144)
        lines[tensor[1]] = "\t".join(t)
    elif case == "duplicate":
        lines.append(lines[tensor[0]])
    elif case == "past_end":
        t = lines[tensor[-1]].split("\t")
        t[3] = str(int(t[3]) + 64)
        lines[tensor[-1]] = "\t".join(t)
    elif case == "bad_file_id":
        t = lines[tensor[0]].split("\t")
        t[2] = "3"
        lines[tensor[0]] = "\t".join(t)
    elif case == "unknown_line":
        lines.append("BOGUS\t1\n")
    elif case == "router_shape":
        idx = write_index(tmp_path, [layer(0, **{"ffn_gate_inp.weight": (0, (D, 511), 511 * D * 4)}) + layer(1)], sparse=True)
        lines = idx.read_text().splitlines(keepends=True)
    elif case == "down_shape":
        idx = write_index(tmp_path, [layer(0) + layer(1, **{"ffn_down_exps.weight": (20, (F, D, 256), 256 * D * rb(20, F))})],
                          sparse=True)
        lines = idx.read_text().splitlines(keepends=True)
    elif case == "no_layer0":
        idx = write_index(tmp_path, [layer(1)], sparse=True)
        lines = idx.read_text().splitlines(keepends=True)
    elif case == "widths":
        ts = moe_layer_tensors(0, 2048, 40, dict(TYPES, down=0, sh_down=0), None, rb)
        idx = write_index(tmp_path, [ts], sparse=True)
        lines = idx.read_text().splitlines(keepends=True)
    idx.write_text("".join(lines))
    rc, msg = validate(idx)
    assert rc == -1 and message in msg, (case, msg)


def test_validate_missing_file_and_bad_arguments(tmp_path):
    rc, msg = validate(tmp_path / "absent.index")
    assert rc == -1 and "open index" in msg
    lib = q()
    assert lib.qwen_validate_index(None) == -1
    assert lib.qwen_open(None, 1, 1, 1) is None
    idx = write_index(tmp_path, [layer(0)], sparse=True)
    for args in ((0, 32, 17), (64, 0, 17), (64, 513, 17), (64, 32, 0), (64, 32, 8193)):
        assert lib.qwen_open(str(idx).encode(), *args) is None
        assert "invalid open arguments" in lib.qwen_last_error().decode()
    # calls on a null model fail cleanly
    assert lib.qwen_get_prune_stats(None, None) == -1
    assert lib.qwen_set_hotlist(None, None, 0, 1) == -1
    assert lib.qwen_cpu_threads(None) == 0
    assert lib.qwen_moe(None, 0, None, None, 1, 0) == -1
    assert lib.qwen_profile_routes(None, None) == -1
