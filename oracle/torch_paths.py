"""The reference's own PyTorch paths for the four ops, evaluated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). These are the torch expressions the reference names for each op;
they pin the C restatement in oracle.c and serve as the timed CPU baseline.

  softmax  softmax/baseline.py:12-13        torch.softmax(x, dim=-1)
  rmsnorm  rmsnorm/candidate.py:3-4          x * rsqrt(mean(x^2) + eps).to(x.dtype)   (kernel.cu:1-8)
  rope     rope/candidate.py:3-5             x * cos + rotate_half(x) * sin, fp32, one rounding (kernel.cu:1-11)
  topk     topk/kernel.cu:1-3                largest k, sorted, ties by lowest index (stable descending sort)
"""

import torch


def softmax(x):
    """softmax/baseline.py:13."""
    return torch.softmax(x, dim=-1)


def rmsnorm(x, weight=None, eps=1e-6):
    """rmsnorm/kernel.cu:1-8: inv = rsqrt(mean(x^2) + eps) rounded to x's dtype, y = x * inv; weighted: w * y."""
    inv = torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps).to(x.dtype)
    y = x * inv
    return y if weight is None else weight * y


def rmsnorm_add(x, residual, weight=None, eps=1e-6):
    """Fused residual add + RMSNorm as torch eager evaluates it on dtype tensors: h = x + residual, y = rmsnorm(h)."""
    h = x + residual
    return rmsnorm(h, weight, eps), h


def inv_freq(head_dim, theta=10000.0):
    """The HF/Llama inverse frequencies: 1 / theta ** (arange(0, D, 2) / D) in fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rope_cache(positions, head_dim, theta=10000.0, dtype=torch.float32):
    """cos/sin cache [positions, D]: emb = cat(outer(pos, inv_freq), same) (HF LlamaRotaryEmbedding)."""
    pos = torch.arange(positions, dtype=torch.int64).float()
    freqs = torch.outer(pos, inv_freq(head_dim, theta))
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope(x, cos, sin, ids):
    """rope/kernel.cu:1-11 for x [B, S, H, D] (or [tokens, H, D]) with cos/sin rows gathered by ids: fp32 math, each
    product and the sum rounded (torch eager), one rounding to x's dtype."""
    c = cos[ids].float().unsqueeze(-2)
    s = sin[ids].float().unsqueeze(-2)
    xf = x.float()
    return (xf * c + rotate_half(xf) * s).to(x.dtype)


def topk(x, k):
    """Largest k per row, sorted descending, ties by lowest index (a stable descending sort)."""
    v, i = torch.sort(x, dim=-1, descending=True, stable=True)
    return v[..., :k], i[..., :k]
