"""Write tests/golden/tensor_maps.json: the record indices of every tensor in the
reference's static tensor maps, read as text from the reference tree.

The maps are archive-format data (where each tensor's tiles sit in a .chpe
archive); the engine and the oracle compute them by formula, and the tests pin
those formulas against this fixture.

Sources (read as text, nothing is executed):
  src/qwen3b_tensor_map.zig:21-531   3B cell-archive table (36 layers)
  src/qwen35_tensor_map.zig:53-1015  9B table (32 layers)
  src/qwen72b_tensor_map.zig:89-112  72B invariants asserted by its own test
  src/qwen3b_geometry.zig:48-79      3B raw-archive offsets

Usage: python tests/golden/make_tensor_maps.py [/root/reference]
"""
import json
import re
import sys
from pathlib import Path

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).with_name("tensor_maps.json")


def parse_const(text, name):
    m = re.search(r"pub const %s: usize = (\d+);" % re.escape(name), text)
    return int(m.group(1)) if m else None


def parse_layer_blocks(text):
    """Return a list of dicts, one per `.{ ... }` layer literal inside LAYERS."""
    start = text.index("pub const LAYERS")
    body = text[start:]
    blocks = []
    depth = 0
    cur = None
    i = body.index("{", body.index("=")) + 1  # skip the array's own brace
    while i < len(body):
        ch = body[i]
        if ch == "{":
            depth += 1
            if depth == 1:
                cur = i + 1
        elif ch == "}":
            if depth == 0:
                break
            depth -= 1
            if depth == 0:
                blocks.append(body[cur:i])
        i += 1
    layers = []
    for b in blocks:
        d = {}
        for key, val in re.findall(r"\.(\w+)\s*=\s*([^,\n]+)", b):
            val = val.strip()
            if val in ("true", "false"):
                d[key] = val == "true"
            elif re.fullmatch(r"\d+", val):
                d[key] = int(val)
            else:
                d[key] = float(val)
        layers.append(d)
    return layers


def main():
    t3 = (REF / "src/qwen3b_tensor_map.zig").read_text()
    t9 = (REF / "src/qwen35_tensor_map.zig").read_text()
    t72 = (REF / "src/qwen72b_tensor_map.zig").read_text()
    g3 = (REF / "src/qwen3b_geometry.zig").read_text()

    out = {
        "qwen3b_cell": {
            "embed_records": parse_const(t3, "EMBED_TOKENS_RECORDS"),
            "final_norm": parse_const(t3, "FINAL_NORM_RECORD"),
            "total": parse_const(t3, "TOTAL_RECORDS"),
            "layers": parse_layer_blocks(t3),
        },
        "qwen35_9b": {
            "embed_tiles": parse_const(t9, "EMBED_TOKENS_TILES"),
            "final_norm": parse_const(t9, "FINAL_NORM_TILE"),
            "lm_head": parse_const(t9, "LM_HEAD_TILE"),
            "lm_head_tiles": parse_const(t9, "LM_HEAD_TILES"),
            "total": parse_const(t9, "TOTAL_TILES"),
            "layers": parse_layer_blocks(t9),
        },
        "qwen72b": {
            # the values asserted by the reference's own test block
            "asserts": [int(x) for x in re.findall(
                r"expectEqual\(@as\(usize, (\d+)\)", t72)],
        },
        "qwen3b_raw": {
            k: parse_const(g3, k) for k in (
                "EMBED_TOKENS_RECORDS", "RECORDS_PER_LAYER", "FINAL_NORM_RECORD",
                "TOTAL_RECORDS", "Q_PROJ_TILES", "K_PROJ_TILES", "V_PROJ_TILES",
                "O_PROJ_TILES", "GATE_PROJ_TILES", "UP_PROJ_TILES", "DOWN_PROJ_TILES")
        },
    }
    # per-layer offsets of the raw map: `layerBase(l) + K` in Bf16LayerOffsets
    out["qwen3b_raw"]["offsets"] = {
        name: int(off) for name, off in re.findall(
            r"pub fn (\w+)\(l: usize\) usize \{ return layerBase\(l\) \+ (\d+); \}", g3)
    }
    assert len(out["qwen3b_cell"]["layers"]) == 36
    assert len(out["qwen35_9b"]["layers"]) == 32
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
