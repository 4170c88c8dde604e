"""Writes tests/golden/deltanet_fixtures.npz: inputs and outputs of the gated-DeltaNet decode
step as computed by the routines of the third-party library that defines the Qwen3.5 layer
(transformers 5.15.0, models/qwen3_5/modeling_qwen3_5.py): causal_conv1d_update (:200-217),
torch_recurrent_gated_delta_rule (:331-380, l2norm inside, :242-245), Qwen3_5RMSNormGated
(:168-184), and the layer's beta/g formulas (:497-499) and head repetition (:500-502).

Run in a container where transformers is installed (no network needed); the fixtures are
data, the library never ships.  Small shapes: 4 value heads, 2 key heads, head dim 16,
3 consecutive steps from a random initial state; a conv of 24 channels x 4 taps.
"""
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F
from transformers.models.qwen3_5 import modeling_qwen3_5 as m

OUT = Path(__file__).with_name("deltanet_fixtures.npz")


def main():
    g = torch.Generator().manual_seed(7)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).float()
    fx = {}
    # conv: 3 steps of one token
    ch, taps = 24, 4
    w = r(ch, taps, sc=0.5)
    state = r(1, ch, taps - 1)
    fx["conv_w"], fx["conv_state0"] = w.numpy(), state[0].numpy().copy()
    xs, outs = [], []
    for t in range(3):
        x = r(1, ch, 1)
        y = m.causal_conv1d_update(x, state, w, None, "silu")
        xs.append(x[0, :, 0].numpy()), outs.append(y[0, :, 0].numpy())
    fx["conv_x"], fx["conv_out"], fx["conv_state3"] = np.stack(xs), np.stack(outs), state[0].numpy().copy()
    # gated delta rule: 3 steps
    nv, nk, d = 4, 2, 16
    A_log, dt_bias = torch.log(torch.rand(nv, generator=g) * 16 + 0.1), r(nv, sc=0.5)
    S = r(1, nv, d, d, sc=0.3)
    fx["A_log"], fx["dt_bias"], fx["S0"] = A_log.numpy(), dt_bias.numpy(), S[0].numpy().copy()
    qs, ks, vs, as_, bs, os_ = [], [], [], [], [], []
    for t in range(3):
        q, k, v, a, b = r(1, 1, nk, d), r(1, 1, nk, d), r(1, 1, nv, d), r(1, 1, nv), r(1, 1, nv)
        beta = b.sigmoid()
        gg = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
        qq = q.repeat_interleave(nv // nk, dim=2)
        kk = k.repeat_interleave(nv // nk, dim=2)
        o, S = m.torch_recurrent_gated_delta_rule(qq, kk, v, g=gg, beta=beta, initial_state=S,
                                                  output_final_state=True, use_qk_l2norm_in_kernel=True)
        for lst, tsr in ((qs, q), (ks, k), (vs, v), (as_, a), (bs, b), (os_, o)):
            lst.append(tsr[0, 0].numpy())
    fx["q"], fx["k"], fx["v"], fx["a"], fx["b"] = (np.stack(t) for t in (qs, ks, vs, as_, bs))
    fx["o"], fx["S3"] = np.stack(os_), S[0].numpy()
    # gated RMSNorm over heads
    norm = m.Qwen3_5RMSNormGated(d, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(r(d, sc=0.5) + 1.0)
    x, z = r(nv, d), r(nv, d)
    with torch.no_grad():
        y = norm(x, z)
    fx["gn_w"], fx["gn_x"], fx["gn_z"], fx["gn_out"] = norm.weight.detach().numpy(), x.numpy(), z.numpy(), y.numpy()
    np.savez(OUT, **fx)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
