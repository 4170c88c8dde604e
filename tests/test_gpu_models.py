"""Whole-model decode on the Qwen2.5-72B and Qwen3.5-9B archives against the oracle (GPU).

The archives are the seeded writer's (include/chpe_pack.h): 72B with 4-bit and 2-bit flat
tiles (qwen72b_tensor_map), 9B with 4-bit flat tiles at the INT8 map's indices, decoded the
way the reference's engine decodes them (the 9B linear-attention layers aliased onto GQA:
q <- in_proj_qkv, k <- in_proj_z, v <- in_proj_a with one tile, o <- out_proj,
src/chpe_engine.zig:1107-1131).  Contexts are short because the oracle reads 37 GB per 72B step on the host.

Bars:
  * greedy token streams (f32 KV cache, as the reference keeps it) identical, a difference
    allowed only after an oracle step whose top-2 logit gap is below 1e-3 (a tie at f32
    precision); single-step logits within 2e-4 * max|logit| and cosine >= 0.9999;
  * the fp16 KV cache (the configs' cache) against the oracle's kv-f16 mode: logits within
    1.5e-3 * max|logit|, cosine >= 0.9999, same argmax.  Every k / v element is rounded to
    fp16, and an element whose f32 value differs from the oracle's in the last bits (another
    summation order) rounds to the neighbouring fp16 value: a 2^-11 relative step that the
    following layers carry to the logits (80 layers and a residual of norm ~6600 for 72B).

Each archive is written into $CHPE_ARCHIVE_DIR when first needed and removed after its module
(a 72B archive is 38.6 GB).
"""
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def threads():
    return max(1, min(16, len(os.sched_getaffinity(0))))


def check_stream(gpu, ref, gaps, tag):
    for i, (a, b) in enumerate(zip(gpu, ref)):
        if a != b:
            assert gaps[i] < 1e-3, (tag, i, int(a), int(b), float(gaps[i]))
            return i
    return len(ref)


def compare_logits(lg, ol, tag, rel):
    d = np.abs(lg.astype(np.float64) - ol)
    cos = float(lg.astype(np.float64) @ ol / np.linalg.norm(lg) / np.linalg.norm(ol))
    scale = float(np.abs(ol).max())
    say(f"  {tag}: max|dlogit| {d.max():.3e} ({d.max() / scale:.2e} of max|logit| {scale:.3f}) cos {cos:.9f}")
    assert np.all(np.isfinite(lg)) and np.all(np.isfinite(ol))
    assert d.max() <= rel * scale and cos >= 0.9999, (tag, float(d.max()), cos)


def archive(kind):
    os.environ["CHPE_PACK_PROGRESS"] = "1"
    say(f"writing archive kind {kind} ({ca.archive_size(kind) / 1e9:.1f} GB)")
    p = ca.ensure_archive(kind, seed=0, threads=threads())
    say(f"archive {p}")
    return p


@pytest.fixture(scope="module", params=[ca.PACK_72B_W4, ca.PACK_72B_W2], ids=["w4", "w2"])
def a72(request):
    p = archive(request.param)
    yield p
    p.unlink(missing_ok=True)


@pytest.fixture(scope="module")
def a9():
    p = archive(ca.PACK_9B_W4)
    yield p
    p.unlink(missing_ok=True)


def run_model(path, arch, vocab, n_prompt, n_gen, seed):
    prompt = np.random.default_rng(seed).integers(0, vocab, n_prompt).astype(np.uint32)
    e = ca.Engine(path, arch=arch, max_seq_len=64, kv_f16=False)
    o = orc.Oracle(path, arch=arch, max_seq_len=64, kv_f16=False, threads=threads())
    try:
        steps = []
        for pos in range(2):
            say(f"f32 KV step pos={pos} token={int(prompt[pos])}")
            am, lg = e.decode_step(int(prompt[pos]), pos)
            r = o.forward(int(prompt[pos]), pos)
            ol = o.logits()
            compare_logits(lg, ol, f"pos {pos}", 2e-4)
            assert am == r.argmax_token and r.all_finite
            assert e.last()["hidden_norm"] == pytest.approx(r.hidden_norm, rel=1e-4)
            steps.append((lg.astype(np.float64), ol.astype(np.float64)))
        # the steps' dependence on their input: the change of the logits from one teacher-forced
        # token to the next is at least 20 times the two steps' measured deviations from the
        # oracle, so the comparisons above resolve it -- a step that ignored its token (or the
        # context) would deviate by that change.  This holds where the argmax does not move:
        # the 2-bit model's greedy stream repeats one token (its logits change by ~4e-3 between
        # positions against deviations of ~7e-6)
        (g0, o0), (g1, o1) = steps
        err = float(np.abs(g0 - o0).max() + np.abs(g1 - o1).max())
        dd, dref = float(np.abs((g1 - g0) - (o1 - o0)).max()), float(np.abs(o1 - o0).max())
        say(f"  logit change pos 0 -> 1: max {dref:.4g}, gpu vs oracle {dd:.2e}, step deviations {err:.2e}")
        assert dd <= err + 1e-12 and dref >= 20 * err
        say(f"stream (f32 KV): {n_prompt} prompt + {n_gen} generated")
        g = e.generate(prompt, n_gen)
        ref, gaps = o.generate(prompt, n_gen)
        say(f"  gpu {list(map(int, g))} oracle {list(map(int, ref))} top-2 gaps {[round(float(x), 4) for x in gaps]}")
        assert check_stream(g, ref, gaps, f"arch {arch}") == n_gen
        assert np.all(np.isfinite(gaps))  # finite logits all along (no NaN layer break)
    finally:
        e.close()
        o.close()
    e = ca.Engine(path, arch=arch, max_seq_len=64, kv_f16=True)
    o = orc.Oracle(path, arch=arch, max_seq_len=64, kv_f16=True, threads=threads())
    try:
        for pos in range(3):
            say(f"fp16 KV step pos={pos} token={int(prompt[pos])}")
            am, lg = e.decode_step(int(prompt[pos]), pos)
            r = o.forward(int(prompt[pos]), pos)
            compare_logits(lg, o.logits(), f"kv-f16 pos {pos}", 1.5e-3)
            assert am == r.argmax_token
    finally:
        e.close()
        o.close()


@pytest.mark.timeout(1500)
def test_72b_stream_matches_oracle(a72):
    run_model(a72, 2, 152064, 6, 4, seed=3)


@pytest.mark.timeout(900)
def test_9b_compat_stream_matches_oracle(a9):
    run_model(a9, 1, 248320, 8, 6, seed=2)


def top2_gap(lg):
    t = np.sort(lg.astype(np.float64))
    return float(t[-1] - t[-2])


def run_block(path, arch, vocab, seed, oracle_check, block=True):
    """The block step (every weight read once for up to 32 tokens; no reference code, defined as
    the decode steps it replaces) against the decode step on the same engine: chpe_prefill vs
    chpe_forward_tokens (the last position's logits, then one decode step on each cache, so the
    KV rows agree; 11 tokens: one block of the 512-column ranges with 3 token quads; 43 tokens:
    a full block of 32 and one of 11), chpe_verify of 8 drafts vs 8 decode steps (every argmax,
    the last logits; the 2048-column ranges).
    Bars: 2e-4 * max|logit| with the f32 cache, as for the decode step against the oracle;
    3e-3 with the fp16 cache, twice the single-step bar: the two paths sum in different orders,
    so k / v elements near an fp16 rounding boundary round differently, and here 19 cached
    positions (not 3) carry such flips through 80 layers.  An argmax may differ only where the
    decode step's top-2 gap is below twice the bar.  oracle_check: the prefill's logits against
    the oracle's forward as well; block: whether the archive runs the block step (flat 4- and
    2-bit tiles do)."""
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, vocab, 11).astype(np.uint32)
    drafts = rng.integers(0, vocab, 8).astype(np.uint32)
    n = len(prompt)
    for kv16, rel in ((False, 2e-4), (True, 3e-3)):
        e = ca.Engine(path, arch=arch, max_seq_len=64, kv_f16=kv16)
        try:
            assert e.block_ready() == block
            if not e.block_ready():  # no block step: prefill and verify are the decode steps, bit for bit
                _, lseq = e.forward_tokens(prompt, want_logits=True)
                _, lblk = e.prefill(prompt, want_logits=True)
                assert np.array_equal(lseq.view(np.uint32), lblk.view(np.uint32))
                seq = [e.decode_step(int(d), n + i)[0] for i, d in enumerate(drafts[:4])]
                assert list(e.verify(drafts[:4], n)) == seq
                continue
            say(f"block step arch {arch} kv_f16={kv16}: sequential reference")
            _, lseq = e.forward_tokens(prompt, want_logits=True)
            seq = [e.decode_step(int(d), n + i) for i, d in enumerate(drafts)]
            say("  prefill of 11 positions (one block)")
            _, lblk = e.prefill(prompt, want_logits=True)
            compare_logits(lblk, lseq, "prefill vs forward_tokens", rel)
            am, lg = e.decode_step(int(drafts[0]), n)
            compare_logits(lg, seq[0][1], "decode step after prefill", rel)
            say("  prefill of 43 positions (a block of 32 + 11) vs forward_tokens")
            long = rng.integers(0, vocab, 43).astype(np.uint32)
            _, lseq2 = e.forward_tokens(long, want_logits=True)
            _, lblk2 = e.prefill(long, want_logits=True)
            compare_logits(lblk2, lseq2, "prefill 43 vs forward_tokens", rel)
            e.forward_tokens(prompt)  # (the context of the verify below)
            say("  verify 8 drafts")
            got = e.verify(drafts, n)
            for i in range(8):
                ref_am, ref_lg = seq[i]
                if got[i] != ref_am:
                    assert top2_gap(ref_lg) < 2 * rel * float(np.abs(ref_lg).max()), (i, int(got[i]), int(ref_am))
            compare_logits(e.logits(), seq[7][1], "verify: last draft", rel)
            if oracle_check and not kv16:
                o = orc.Oracle(path, arch=arch, max_seq_len=64, kv_f16=False, threads=threads())
                try:
                    for pos, tok in enumerate(prompt):
                        o.forward(int(tok), pos)
                    compare_logits(lblk, o.logits(), "prefill vs oracle", rel)
                    # verify of 4 drafts (the batch-4 configuration) against the oracle's
                    # sequential steps: every argmax, the last draft's logits
                    e.prefill(prompt)
                    say("  verify 4 drafts vs the oracle")
                    got4 = e.verify(drafts[:4], n)
                    lv4 = e.logits()
                    for i in range(4):
                        r = o.forward(int(drafts[i]), n + i)
                        if int(got4[i]) != r.argmax_token:
                            ol = o.logits()
                            assert top2_gap(ol) < 2 * rel * float(np.abs(ol).max()), (i, int(got4[i]), r.argmax_token)
                    compare_logits(lv4, o.logits(), "verify 4: last draft vs oracle", rel)
                    # the device state continues where the sequential steps would leave it:
                    # the last draft's argmax at position n + 4 (one step launched from it)
                    e.time_steps(1)
                    o.forward(int(got4[3]), n + 4)
                    compare_logits(e.logits(), o.logits(), "step continuing after verify 4 vs oracle", rel)
                finally:
                    o.close()
        finally:
            e.close()


@pytest.mark.timeout(1200)
def test_72b_block_step_matches_decode_steps(a72):
    run_block(a72, 2, 152064, seed=5, oracle_check=True)


STEPS_CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import chpe_amd as ca
e = ca.Engine(sys.argv[2], arch=2, max_seq_len=16, kv_f16=True)
out = [e.decode_step(int(t), p)[1] for p, t in enumerate(np.load(sys.argv[3]))]
e.close()
np.save(sys.argv[4], np.stack(out))
"""


@pytest.mark.timeout(900)
def test_72b_w2_permuted_copies_bit_identical(a72):
    """A 2-bit archive's decode launches all read a permuted copy of their codes (the 3-part
    q/k/v launch, o, gate/up, down, the LM head): decode steps with the copies (here) and
    without them (a child process started with CHPE_XM_LAYOUT=0, the codes read from the
    records) give the same logits bit for bit -- the copies hold the same bytes for the same
    lanes, whatever the launch's parts and modes."""
    if "-w2-" not in a72.name:
        pytest.skip("4-bit archives copy gate/up and the LM head only (test_gpu_xm_layout.py)")
    toks = np.array([151643, 9707, 11], np.uint32)
    say("72B 2-bit: decode steps with the permuted copies")
    e = ca.Engine(a72, arch=2, max_seq_len=16, kv_f16=True)
    try:
        got = np.stack([e.decode_step(int(t), p)[1] for p, t in enumerate(toks)])
    finally:
        e.close()
    with tempfile.TemporaryDirectory() as td:
        tf, out = os.path.join(td, "t.npy"), os.path.join(td, "l.npy")
        np.save(tf, toks)
        say("  the same steps from the records (CHPE_XM_LAYOUT=0, child process)")
        subprocess.run([sys.executable, "-c", STEPS_CHILD, str(ca.PKG_DIR), str(a72), tf, out],
                       env=dict(os.environ, CHPE_XM_LAYOUT="0"), check=True, timeout=600)
        want = np.load(out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.timeout(900)
def test_9b_compat_block_step_matches_decode_steps(a9):
    run_block(a9, 1, 248320, seed=6, oracle_check=True)


@pytest.mark.timeout(900)
def test_9b_break_in_block_and_decode_steps(a9):
    """forwardDecode's non-finite break (src/chpe_engine.zig:1753-1764) in the block step (per
    token) and in the decode step: layer 1's down projection with one outlier weight set to +inf
    (outliers replace weights, :632-646) makes a hidden row infinite after layer 1 at every
    position, so the reference leaves the layer loop there; its hidden norm is +inf, its logits
    NaN (argmax 0, all_finite false), and layers 2-31 write no KV rows.  Without the break (the
    oracle's set_break(False), a planted deviation) the hidden norm turns NaN."""
    import tempfile
    from test_gpu_nonfinite import inf_outlier_edit
    li = orc.layer_info(2, 1)
    off, b = inf_outlier_edit(a9, li["down_proj"], li["down_tiles"])
    data = np.fromfile(a9, dtype=np.uint8)
    data[off:off + 2] = np.frombuffer(b, np.uint8)
    fd, path = tempfile.mkstemp(suffix=".chpe", prefix="qwen3.5-9b-mod-", dir=os.path.dirname(str(a9)))
    os.close(fd)
    data.tofile(path)
    prompt = np.random.default_rng(8).integers(0, 248320, 11).astype(np.uint32)
    try:
        e = ca.Engine(path, arch=1, max_seq_len=64, kv_f16=False)
        o = orc.Oracle(data=data, arch=1, max_seq_len=64, threads=threads())
        nb = orc.Oracle(data=data, arch=1, max_seq_len=64, threads=threads())
        nb.set_break(False)
        try:
            assert e.block_ready()
            say("9B break: prefill of 11 positions (one block)")
            am, lg = e.prefill(prompt, want_logits=True)
            for pos, tok in enumerate(prompt):
                r = o.forward(int(tok), pos)
                rn = nb.forward(int(tok), pos)
            last = e.last()
            say(f"  gpu argmax {am} hidden_norm {last['hidden_norm']} | oracle {r.argmax_token} {r.hidden_norm} "
                f"| without the break {rn.hidden_norm}")
            assert am == r.argmax_token == 0 and not r.all_finite and np.isnan(lg).all()
            assert np.isinf(last["hidden_norm"]) and np.isinf(r.hidden_norm) and np.isnan(rn.hidden_norm)
            for i in range(2):
                pos = len(prompt) + i
                am, lg = e.decode_step(int(prompt[i]), pos)
                r = o.forward(int(prompt[i]), pos)
                last = e.last()
                say(f"  decode pos {pos}: gpu argmax {am} hidden_norm {last['hidden_norm']} | oracle {r.argmax_token} {r.hidden_norm}")
                assert am == r.argmax_token and np.isnan(lg).all() and not r.all_finite
                assert np.isinf(last["hidden_norm"]) and np.isinf(r.hidden_norm)
        finally:
            e.close()
            o.close()
            nb.close()
    finally:
        os.unlink(path)
