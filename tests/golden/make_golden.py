"""Writes the golden fixtures of tests/golden/ (run from the repo root).

cfg1_small.npz  a reduced config-1 case (fp32, B=2, S=32, d=64, E=8, top-2,
                F=64): inputs, weights, and the expected outputs of the
                op-for-op torch-CPU port of the reference path
                (oracle/torch_port.py: softmax/topk router, stable-argsort
                dispatch, padded bmm SwiGLU, index_add_ combine, aux losses).
e4m3_kat.npz    fp32 inputs and their e4m3fn codes from torch's
                float8_e4m3fn cast after clamping to +-448.
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import torch_port as P  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def cfg1_small():
    g = torch.Generator().manual_seed(1)
    B, S, d, E, k, F_ = 2, 32, 64, 8, 2, 64
    x = torch.randn(B, S, d, generator=g)
    w_in = torch.randn(128, d, generator=g) * 0.1
    w_out = torch.randn(E, 128, generator=g) * 0.1
    w1 = torch.randn(E, d, F_, generator=g) * 0.1
    w2 = torch.randn(E, d, F_, generator=g) * 0.1
    w3 = torch.randn(E, F_, d, generator=g) * 0.1
    w, idx, logits = P.router_tc(x, w_in, w_out, k)
    y, aux = P.moe_layer_tc(x, w_in, w_out, w1, w2, w3, k)
    counts = torch.bincount(idx.reshape(-1), minlength=E)
    np.savez_compressed(os.path.join(OUT, "cfg1_small.npz"), x=x.reshape(-1, d).numpy(), w_in=w_in.numpy(),
                        w_out=w_out.numpy(), w1=w1.numpy(), w2=w2.numpy(), w3=w3.numpy(), k=k,
                        idx=idx.reshape(-1, k).numpy(), counts=counts.numpy(), y=y.reshape(-1, d).numpy(),
                        aux=np.float64(aux), logits=logits.reshape(-1, E).numpy())


def e4m3_kat():
    vals = np.concatenate([np.linspace(-500, 500, 2001), np.geomspace(1e-5, 448, 3000),
                           -np.geomspace(1e-5, 448, 3000), [0.0, -0.0, 2 ** -9, 2 ** -10, 3 * 2 ** -10]])
    vals = vals.astype(np.float32)
    codes = torch.from_numpy(vals).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.savez_compressed(os.path.join(OUT, "e4m3_kat.npz"), inputs=vals, codes=codes)


if __name__ == "__main__":
    cfg1_small()
    e4m3_kat()
    print("wrote", sorted(f for f in os.listdir(OUT) if f.endswith(".npz")))
