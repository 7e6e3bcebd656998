"""Writes the golden fixtures of tests/test_oracle.py from torch's own CPU routines (not from the oracle).

The reference ships no tests or vectors; its paths for these ops are torch expressions (softmax/baseline.py:13, the
rmsnorm and rope wrappers' docstrings, a stable descending sort for top-k). These fixtures freeze what the installed
torch computes for them on small seeded inputs, with the torch version recorded, so the oracle stays pinned even if
torch changes. Run: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import torch_paths  # noqa: E402  (the torch expressions only; no C oracle involved)


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    ver = np.array(torch.__version__)
    g = torch.Generator().manual_seed(2024)

    x = torch.randn(8, 333, generator=g) * 3
    xb = (torch.randn(8, 333, generator=g) * 3).bfloat16()
    np.savez(os.path.join(HERE, "softmax.npz"), torch_version=ver, x=x.numpy(),
             y64=torch.softmax(x.double(), -1).numpy(), y32=torch_paths.softmax(x).numpy(),
             xb=bits(xb), yb=bits(torch.softmax(xb.double(), -1).bfloat16()))

    xr = torch.randn(64, 512, generator=g).bfloat16()
    w = (torch.rand(512, generator=g) + 0.5).bfloat16()
    inv = torch.rsqrt(xr.float().pow(2).mean(-1) + 1e-6).to(torch.bfloat16)
    np.savez(os.path.join(HERE, "rmsnorm.npz"), torch_version=ver, x=bits(xr), w=bits(w),
             y=bits(torch_paths.rmsnorm(xr, w, 1e-6)), inv_torch=bits(inv))

    q = torch.randn(16, 4, 64, generator=g).bfloat16()
    k = torch.randn(16, 2, 64, generator=g).bfloat16()
    ids = torch.randint(0, 64, (16,), generator=g)
    cos, sin = torch_paths.rope_cache(64, 64)
    np.savez(os.path.join(HERE, "rope.npz"), torch_version=ver, q=bits(q), k=bits(k), cos=cos.numpy(),
             sin=sin.numpy(), ids=ids.numpy(), q_out=bits(torch_paths.rope(q, cos, sin, ids)),
             k_out=bits(torch_paths.rope(k, cos, sin, ids)))

    xt = torch.randn(4, 2048, generator=g) * 2
    xt[1, ::7] = 1.5  # planted ties
    xt[2, :] = torch.randint(0, 4, (2048,), generator=g).float()
    out = {}
    for kk in (1, 50, 1024):
        v, i = torch_paths.topk(xt, kk)
        out[f"v{kk}"], out[f"i{kk}"] = v.numpy(), i.numpy()
    np.savez(os.path.join(HERE, "topk.npz"), torch_version=ver, x=xt.numpy(), **out)
    print("fixtures written with torch", torch.__version__)


if __name__ == "__main__":
    main()
