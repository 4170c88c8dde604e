"""The permuted code copy of the matrix-core flat GEMV (k_xm_layout; gemvCellFlat,
src/chpe_engine.zig:584-729).  The engine writes the gate/up and LM head codes once more in the
kernel's load order, and the kernel then reads each lane's bytes from the copy instead of the
records (4-bit: 16 bytes per set; 2-bit: the 8 bytes of two sets in one 16-byte load; 2-bit
archives copy every decode launch's codes, the residual launches included).  The copy holds the
same bytes for the same lanes, so the outputs must be bit for bit those of the records path:
each case runs here (copy) and in a child process started with CHPE_XM_LAYOUT=0 (records, read
once per process), on the same inputs.  Both are also checked against the oracle by
test_gpu_gemv_flat.py.  The multi-part q/k/v launch, which the one-launch hook cannot express,
is covered with the whole 72B 2-bit model (test_gpu_models.py: decode steps with and without
the copies, bit for bit)."""
import os
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

import chpe_amd as ca

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
TILE = 32768

CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import chpe_amd as ca
d = np.load(sys.argv[2])
mode = str(d["mode"])
up = d["up"] if d["up"].size else None
g = d["gamma"] if d["gamma"].size else None
y0 = d["y0"] if d["y0"].size else None
r = ca.gpu_gemv_flat(mode, int(d["rows"]), int(d["cols"]), d["cells"], d["x"], tiles_up=up, gamma=g, eps=1e-6, y=y0)
y = r[0] if mode == "logits" else r
extra = np.array([r[1], np.float32(r[2]).view(np.uint32)] if mode == "logits" else [], np.uint32)
np.save(sys.argv[3], np.concatenate([y.view(np.uint32), extra]))
"""


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_tiles(rng, rows, cols, bits=4):
    n = rows * cols
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    hot = rng.choice(n, size=max(1, n // 2000), replace=False)
    w[hot] = (rng.standard_normal(hot.size) * 0.5).astype(np.float32)
    n_tiles = (n + TILE - 1) // TILE
    w = np.concatenate([w, np.zeros(n_tiles * TILE - n, np.float32)])
    return np.stack([ca.pack_flat(w[t * TILE:(t + 1) * TILE], bits=bits, n_outliers=64) for t in range(n_tiles)])


CASES = [  # (mode, bits, rows, cols): every one on the matrix-core kernel with the copy
    ("swiglu", 4, 8192, 8192),   # 4096 units at 4 waves, 2 workgroups per CU
    ("logits", 4, 300, 8192),
    ("logits", 4, 90, 4096),     # 2 waves
    ("swiglu", 2, 8192, 8192),   # 2-bit: two sets per 16-byte load
    ("logits", 2, 130, 4096),
    ("accum", 2, 512, 8192),     # 2-bit residual launches (o) read their copy too
    ("accum", 2, 96, 29568),     # the down shape: 15 waves, the last one's columns partly empty
]


@pytest.mark.parametrize("mode,bits,rows,cols", CASES)
def test_permuted_codes_match_records(mode, bits, rows, cols):
    rng = np.random.default_rng(rows + cols + bits)
    say(f"xm layout mode={mode} bits={bits} rows={rows} cols={cols}")
    cells = make_tiles(rng, rows, cols, bits)
    up = make_tiles(rng, rows, cols, bits) if mode == "swiglu" else None
    x = rng.standard_normal(cols).astype(np.float32)
    gamma = (rng.standard_normal(cols) * 0.2 + 1.0).astype(np.float32)
    y0 = rng.standard_normal(rows).astype(np.float32) if mode == "accum" else None
    r = ca.gpu_gemv_flat(mode, rows, cols, cells, x, tiles_up=up, gamma=gamma if mode in ("swiglu", "logits") else None,
                         eps=1e-6, y=y0)
    y = r[0] if mode == "logits" else r
    got = np.concatenate([y.view(np.uint32),
                          np.array([r[1], np.float32(r[2]).view(np.uint32)] if mode == "logits" else [], np.uint32)])
    with tempfile.TemporaryDirectory() as td:
        inp, out = os.path.join(td, "in.npz"), os.path.join(td, "out.npy")
        np.savez(inp, mode=np.array(mode), rows=np.array(rows), cols=np.array(cols), cells=cells, x=x,
                 up=up if up is not None else np.zeros(0, np.uint8),
                 gamma=gamma if mode in ("swiglu", "logits") else np.zeros(0, np.float32),
                 y0=y0 if y0 is not None else np.zeros(0, np.float32))
        # (2 workgroups per CU as with the copy, so that the launches differ in the code source only)
        env = dict(os.environ, CHPE_XM_LAYOUT="0", CHPE_GEMV_XM_WPC="2,2,2,1")
        say("  records path in a child process")
        subprocess.run([sys.executable, "-c", CHILD, str(ROOT / "chpe-qwen-engine_amd"), inp, out], env=env,
                       check=True, timeout=300)
        want = np.load(out)
    assert got.shape == want.shape
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} outputs differ, first at {int(bad[0])}"
