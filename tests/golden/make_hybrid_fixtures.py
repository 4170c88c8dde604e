"""Writes tests/golden/hybrid_fixtures.npz: the hidden state after the first four layers of the
Qwen3.5-9B hybrid (three gated-DeltaNet layers, then a gated full-attention layer) at positions
0, 1, 2 of a three-token prompt, computed by the third-party library that defines the model
(transformers 5.15.0, models/qwen3_5/modeling_qwen3_5.py: Qwen3_5DecoderLayer :740-793 with
Qwen3_5GatedDeltaNet :387-543 and Qwen3_5Attention :629-701, Qwen3_5TextRotaryEmbedding
:84-165) with the weights of the seeded 9B archive (libchpe_pack.so, kind qwen3.5-9b-w4,
seed 0), dequantised tile by tile by the oracle's gemvCellFlat dequantisation and read from its
norm / bf16 vector records.

The library runs the prompt as one sequence (the chunked delta rule, the conv over the whole
prompt, a causal mask), which equals three consecutive decode steps; its RMSNorm multiplies by
1 + weight, so the archive's gains g (the effective gain the engine and the oracle use) enter
as weight = g - 1; the gated norm's weight is used as stored.

Run where transformers is installed (no network needed): the fixture is data, the library never
ships.  The archive is written (3.7 GB) if it is not cached.
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "chpe-qwen-engine_amd"), str(ROOT / "oracle")]
import chpe_amd as ca  # noqa: E402
import oracle as orc  # noqa: E402
from transformers.models.qwen3_5 import modeling_qwen3_5 as m  # noqa: E402
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig  # noqa: E402

OUT = Path(__file__).with_name("hybrid_fixtures.npz")
CELL, P = 17408, 64 + 16384
TOKENS = [151643, 9707, 248000]
N_LAYERS = 4


def q35_records(l):
    """Record offsets of layer l (qwen35_tensor_map.zig:62-1015)."""
    full = lambda i: i % 4 == 3
    b = 62080 + sum(12804 if full(i) else 13337 for i in range(l))
    r = {"input_norm": b}
    if full(l):
        r.update(q_proj=b + 1, k_proj=b + 2049, v_proj=b + 2305, o_proj=b + 2561, q_norm=b + 3585, k_norm=b + 3586,
                 post_norm=b + 3587)
    else:
        r.update(in_proj_qkv=b + 1, in_proj_z=b + 2049, in_proj_a=b + 3073, in_proj_b=b + 3081, conv1d=b + 3089,
                 a_log=b + 3093, dt_bias=b + 3094, linear_norm=b + 3095, out_proj=b + 3096, post_norm=b + 4120)
    r["gate_proj"] = r["post_norm"] + 1
    r["up_proj"] = r["gate_proj"] + 3072
    r["down_proj"] = r["up_proj"] + 3072
    return r


def main():
    path = ca.ensure_archive(ca.PACK_9B_W4, 0)
    data = np.memmap(path, dtype=np.uint8, mode="r")
    cell = lambda rec: np.array(data[4096 + rec * CELL:4096 + (rec + 1) * CELL])

    def flat(rec, rows, cols):
        n = (rows * cols + 32767) // 32768
        w = np.concatenate([orc.flat_tile_weights(cell(rec + t)) for t in range(n)])
        return torch.from_numpy(w[:rows * cols].reshape(rows, cols).copy())

    def f32vec(rec, n):
        return torch.from_numpy(np.frombuffer(cell(rec)[64:64 + 4 * n].tobytes(), np.float32).copy())

    def bf16vec(rec, n):
        raw = np.concatenate([cell(rec + i)[64:64 + 16384] for i in range((n + 8191) // 8192)])
        h = np.frombuffer(raw.tobytes(), np.uint16)[:n].astype(np.uint32) << 16
        return torch.from_numpy(h.view(np.float32).copy())

    cfg = Qwen3_5TextConfig(vocab_size=248320, hidden_size=4096, intermediate_size=12288, num_hidden_layers=N_LAYERS,
                            num_attention_heads=16, num_key_value_heads=4, head_dim=256, rms_norm_eps=1e-6,
                            linear_conv_kernel_dim=4, linear_key_head_dim=128, linear_value_head_dim=128,
                            linear_num_key_heads=16, linear_num_value_heads=32,
                            rope_parameters={"rope_type": "default", "rope_theta": 1000000.0,
                                             "partial_rotary_factor": 0.25})
    cfg._attn_implementation = "eager"
    assert cfg.layer_types == ["linear_attention"] * 3 + ["full_attention"]
    layers = []
    with torch.no_grad():
        for l in range(N_LAYERS):
            r = q35_records(l)
            L = m.Qwen3_5DecoderLayer(cfg, l).float().eval()
            L.input_layernorm.weight.copy_(f32vec(r["input_norm"], 4096) - 1.0)
            L.post_attention_layernorm.weight.copy_(f32vec(r["post_norm"], 4096) - 1.0)
            L.mlp.gate_proj.weight.copy_(flat(r["gate_proj"], 12288, 4096))
            L.mlp.up_proj.weight.copy_(flat(r["up_proj"], 12288, 4096))
            L.mlp.down_proj.weight.copy_(flat(r["down_proj"], 4096, 12288))
            if l % 4 == 3:
                A = L.self_attn
                A.q_proj.weight.copy_(flat(r["q_proj"], 8192, 4096))
                A.k_proj.weight.copy_(flat(r["k_proj"], 1024, 4096))
                A.v_proj.weight.copy_(flat(r["v_proj"], 1024, 4096))
                A.o_proj.weight.copy_(flat(r["o_proj"], 4096, 4096))
                A.q_norm.weight.copy_(bf16vec(r["q_norm"], 256) - 1.0)
                A.k_norm.weight.copy_(bf16vec(r["k_norm"], 256) - 1.0)
            else:
                G = L.linear_attn
                G.in_proj_qkv.weight.copy_(flat(r["in_proj_qkv"], 8192, 4096))
                G.in_proj_z.weight.copy_(flat(r["in_proj_z"], 4096, 4096))
                G.in_proj_a.weight.copy_(flat(r["in_proj_a"], 32, 4096))
                G.in_proj_b.weight.copy_(flat(r["in_proj_b"], 32, 4096))
                G.conv1d.weight.copy_(bf16vec(r["conv1d"], 8192 * 4).reshape(8192, 1, 4))
                G.A_log.copy_(bf16vec(r["a_log"], 32))
                G.dt_bias.copy_(bf16vec(r["dt_bias"], 32))
                G.norm.weight.copy_(bf16vec(r["linear_norm"], 128))
                G.out_proj.weight.copy_(flat(r["out_proj"], 4096, 4096))
            layers.append(L)
        o = orc.Oracle(path, arch=1, max_seq_len=8)
        emb = torch.from_numpy(np.stack([o.embed_row(t) for t in TOKENS]))[None]  # (1, T, D)
        o.close()
        T = len(TOKENS)
        pos = torch.arange(T)[None]
        rot = m.Qwen3_5TextRotaryEmbedding(cfg)
        cos, sin = rot(emb, pos)
        causal = torch.full((T, T), float("-inf")).triu(1)[None, None]
        h = emb
        for l, L in enumerate(layers):
            mask = causal if l % 4 == 3 else None
            h = L(h, position_embeddings=(cos, sin), attention_mask=mask, position_ids=pos)
            if isinstance(h, tuple):
                h = h[0]
    np.savez_compressed(OUT, tokens=np.array(TOKENS, np.uint32), n_layers=N_LAYERS,
                        hidden=h[0].numpy().astype(np.float32), archive=str(Path(path).name))
    print(f"wrote {OUT}: hidden after {N_LAYERS} layers at positions 0..{T - 1} (archive {Path(path).name})")


if __name__ == "__main__":
    main()
