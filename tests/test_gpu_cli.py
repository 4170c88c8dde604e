"""The chpe_fwd command line (the reference's src/main.zig contract) on the GPU.

The LAMBADA harness (scripts/eval_lambada_fidelity.py:126-164) writes the prompt as raw
little-endian u32 (`--tokens-file`), runs `chpe_fwd --archive A --tokens-file P --arch X
--out-logits L`, fails on a non-zero exit code and reads L as raw f32[vocab]; the parity script
(tests/verify_baseline_parity.sh:59-66) greps the receipt for the argmax.  Here:
  * the logits file holds the vocab_size floats of chpe_forward_tokens on the same prompt, bit
    for bit (the same engine and kernels), and their argmax is the oracle's;
  * the receipt lines (main.zig:189-196) parse, and carry the C ABI's last-result values;
  * --bench N runs the prompt N times from position 0 (main.zig:169-184) with the same result;
  * the spoke JSON (main.zig:211-246) is written when run/spoke_outbox exists;
  * error exits: a missing archive (FileNotFound), an empty tokens file (EmptyTokensFile),
    --hybrid on an archive that is not Qwen3.5-9B.
"""
import json
import re
import subprocess
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

CLI = ca.PKG_DIR / "chpe_fwd"
RECEIPT = {
    "argmax": (r"^Argmax Decoded Token ID : (\d+)$", int),
    "max_logit": (r"^Maximum Vocab Logit     : (-?[\d.]+|nan|inf|-inf)$", float),
    "token0_logit": (r"^Token 0 Logit           : (-?[\d.]+|nan|inf|-inf)$", float),
    "hidden_norm": (r"^Final Hidden Vector Norm: (-?[\d.]+|nan|inf)$", float),
    "latency_ms": (r"^Mean Latency            : ([\d.]+) ms \(([\d.]+) s\)$", float),
    "throughput": (r"^Throughput              : ([\d.]+) tokens/sec$", float),
    "sound": (r"^Numerical Soundness     : (.*)$", str),
}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_cli(args, cwd):
    say("chpe_fwd " + " ".join(map(str, args)))
    p = subprocess.run([str(CLI)] + [str(a) for a in args], cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                       text=True, timeout=300)
    return p.returncode, p.stderr


def receipt(text):
    out = {}
    for k, (pat, conv) in RECEIPT.items():
        m = re.search(pat, text, re.M)
        assert m, (k, text[-2000:])
        out[k] = conv(m.group(1))
    return out


def test_cli_tokens_file_out_logits_and_receipt(w4_archive, tmp_path):
    assert CLI.exists(), f"{CLI} is not built"
    toks = np.random.default_rng(21).integers(0, 151936, 12).astype(np.uint32)
    tf = tmp_path / "prompt.bin"
    tf.write_bytes(toks.astype("<u4").tobytes())
    lf = tmp_path / "logits.bin"
    (tmp_path / "run" / "spoke_outbox").mkdir(parents=True)
    rc, err = run_cli(["--archive", w4_archive, "--tokens-file", tf, "--arch", "qwen2_5_3b", "--out-logits", lf,
                       "--max-seq-len", 64], tmp_path)
    assert rc == 0, err
    r = receipt(err)
    assert f"Prompt Tokens  : Loaded {toks.size} tokens from '{tf}'" in err
    assert f"Exported Logits Binary  : {lf} (151936 floats, {151936 * 4} bytes)" in err
    assert r["sound"] == "100% FINITE (Zero NaN / Zero Inf)"
    logits = np.fromfile(lf, dtype="<f4")
    assert logits.size == 151936 and np.isfinite(logits).all()
    # the same prompt through the C ABI: the file is chpe_forward_tokens' logits, bit for bit
    e = ca.Engine(w4_archive, arch=0, max_seq_len=64)
    try:
        am, lg = e.forward_tokens(toks, want_logits=True)
        last = e.last()
    finally:
        e.close()
    assert np.array_equal(logits.view(np.uint32), lg.view(np.uint32))
    assert r["argmax"] == am == int(np.argmax(logits))
    for k in ("max_logit", "token0_logit", "hidden_norm"):
        assert r[k] == pytest.approx(last[k], abs=5e-6 + 1e-6 * abs(last[k])), k  # (printed with 6 decimals)
    # and the oracle's forward of the same prompt
    o = orc.Oracle(w4_archive, arch=0, max_seq_len=64, threads=16)
    try:
        for pos, t in enumerate(toks):
            res = o.forward(int(t), pos)
        assert res.argmax_token == r["argmax"]
        assert float(np.abs(logits.astype(np.float64) - o.logits()).max()) <= 2e-3
    finally:
        o.close()
    # the spoke telemetry (main.zig:211-246)
    spoke = json.loads((tmp_path / "run" / "spoke_outbox" / "metal.chpe_fwd.result.json").read_text())
    assert spoke["tokens_evaluated"] == toks.size and spoke["argmax_token"] == r["argmax"]
    assert spoke["all_finite"] is True and spoke["model"] == "Qwen2.5-3B"


def test_cli_bench_iterations_restart(w4_archive, tmp_path):
    toks = np.array([151644, 872, 198], np.uint32)
    tf = tmp_path / "p.bin"
    tf.write_bytes(toks.astype("<u4").tobytes())
    rc1, err1 = run_cli([w4_archive, "--tokens-file", tf, "--bench", 3, "--max-seq-len", 16], tmp_path)
    rc2, err2 = run_cli([w4_archive, "--tokens-file", tf, "--max-seq-len", 16], tmp_path)
    assert rc1 == 0 and rc2 == 0, (err1, err2)
    assert len(re.findall(r"^  \[Iter \d/3\] Latency: [\d.]+ ms$", err1, re.M)) == 3
    a, b = receipt(err1), receipt(err2)
    for k in ("argmax", "max_logit", "token0_logit", "hidden_norm"):
        assert a[k] == b[k], k


def test_cli_error_exits(w4_archive, tmp_path):
    rc, err = run_cli(["--archive", tmp_path / "missing.chpe"], tmp_path)
    assert rc == 1 and "FileNotFound" in err
    empty = tmp_path / "empty.bin"
    empty.write_bytes(b"")
    rc, err = run_cli(["--archive", w4_archive, "--tokens-file", empty], tmp_path)
    assert rc == 1 and "EmptyTokensFile" in err
    rc, err = run_cli(["--archive", w4_archive, "--hybrid"], tmp_path)
    assert rc == 1 and "--hybrid needs a Qwen3.5-9B archive" in err
    rc, err = run_cli(["-h"], tmp_path)
    assert rc == 0 and "--tokens-file <path>" in err and "--hybrid" in err
