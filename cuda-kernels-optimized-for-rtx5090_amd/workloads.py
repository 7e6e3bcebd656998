"""The named workloads the kernels are measured and checked on: shapes, seeds and input recipes.

Inputs are drawn on the CPU from a seeded torch.Generator (so every run and every machine sees the same values) and
moved to the device by the caller. `algorithmic_bytes` is the minimum HBM traffic of one call: every input element
read once and every output element written once (cos/sin are computed on the fly for RoPE, except in the cache
workload, which reads each cache entry once; workspaces excluded).
"""

import torch

THETA = 10000.0
EPS = 1e-6


def softmax_4096x4096():
    """Softmax fp32 over the last dim of x[4096, 4096] ~ N(0, 3^2), seed 0."""
    g = torch.Generator().manual_seed(0)
    return {"x": torch.randn(4096, 4096, generator=g) * 3}


def rmsnorm_16384x4096():
    """RMSNorm bf16: x[16384, 4096] ~ N(0, 1), weight[4096] ~ U(0.5, 1.5), eps 1e-6, seed 0."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16384, 4096, generator=g).bfloat16()
    w = (torch.rand(4096, generator=g) + 0.5).bfloat16()
    return {"x": x, "weight": w, "eps": EPS}


def rmsnorm_add_16384x4096():
    """Fused residual add + RMSNorm bf16 (the step before a decoder layer's norm): x, residual [16384, 4096] ~ N(0, 1),
    weight[4096] ~ U(0.5, 1.5), eps 1e-6, seed 2."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(16384, 4096, generator=g).bfloat16()
    r = torch.randn(16384, 4096, generator=g).bfloat16()
    w = (torch.rand(4096, generator=g) + 0.5).bfloat16()
    return {"x": x, "residual": r, "weight": w, "eps": EPS}


def rope_inv_freq(head_dim=128, theta=THETA):
    """HF/Llama inverse frequencies 1 / theta ** (arange(0, D, 2) / D), fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rope_4x4096_32q_8kv_128():
    """RoPE bf16 in place: q[4, 4096, 32, 128], k[4, 4096, 8, 128] ~ N(0, 1), positions 0..4095 per sequence,
    theta 1e4, rotate-half pairing, seed 0."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(4, 4096, 32, 128, generator=g).bfloat16()
    k = torch.randn(4, 4096, 8, 128, generator=g).bfloat16()
    pos = torch.arange(4096, dtype=torch.int64).view(1, 4096).expand(4, 4096).contiguous()
    return {"q": q, "k": k, "position_ids": pos, "inv_freq": rope_inv_freq(128)}


def rope_kv_4x4096_32q_8kv_128():
    """RoPE fused with the KV-cache write, bf16: the rope_4x4096_32q_8kv_128 inputs plus v[4, 4096, 8, 128] and a
    16384-slot cache [16384, 8, 128] for k and v; the tokens' slots are a seeded permutation (a paged cache's blocks
    in any order), seed 3."""
    inp = rope_4x4096_32q_8kv_128()
    g = torch.Generator().manual_seed(3)
    inp["v"] = torch.randn(4, 4096, 8, 128, generator=g).bfloat16()
    inp["slot_mapping"] = torch.randperm(16384, generator=g).view(4, 4096)
    inp["k_cache"] = torch.zeros(16384, 8, 128, dtype=torch.bfloat16)
    inp["v_cache"] = torch.zeros(16384, 8, 128, dtype=torch.bfloat16)
    return inp


def rope_cache_4x4096_32q_8kv_128():
    """RoPE bf16 in place through the reference's ABI `launch`, cos/sin read from an fp32 cache [4096, 128] built by
    HF's formula (emb = cat(outer(pos, inv_freq)) twice, cos and sin in fp32), over the rope_4x4096_32q_8kv_128
    inputs."""
    inp = rope_4x4096_32q_8kv_128()
    freqs = torch.outer(torch.arange(4096, dtype=torch.int64).float(), inp["inv_freq"])
    emb = torch.cat((freqs, freqs), dim=-1)
    inp["cos"], inp["sin"] = emb.cos(), emb.sin()
    return inp


def softmax_64x262144():
    """Long-row softmax fp32: x[64, 262144] ~ N(0, 5^2) with exactly 1% of the entries set to +20, seed 1."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 262144, generator=g) * 5
    n = x.numel()
    idx = torch.randperm(n, generator=g)[: n // 100]
    x.view(-1)[idx] = 20.0
    return {"x": x}


def topk_128x128256():
    """Top-k over fp32 logits x[128, 128256] ~ N(0, 2^2), seed 0 (k = 1, 50, 1024)."""
    g = torch.Generator().manual_seed(0)
    return {"x": torch.randn(128, 128256, generator=g) * 2}


def topk_sample_128x128256():
    """Top-k (k = 50) and a draw from it per row (temperature 0.8, top_p 0.9) over the top-k workload's logits, with
    seeded uniforms, seed 4 (one launch: topk_launch_sample)."""
    inp = topk_128x128256()
    g = torch.Generator().manual_seed(4)
    inp.update({"k": 50, "temperature": 0.8, "top_p": 0.9, "uniforms": torch.rand(128, generator=g)})
    return inp


def algorithmic_bytes(name, k=50):
    if name == "softmax_4096x4096":
        return 2 * 4096 * 4096 * 4
    if name == "softmax_64x262144":
        return 2 * 64 * 262144 * 4
    if name == "rmsnorm_16384x4096":
        return 2 * 16384 * 4096 * 2 + 4096 * 2
    if name == "rmsnorm_add_16384x4096":
        return 4 * 16384 * 4096 * 2 + 4096 * 2
    if name == "rope_kv_4x4096_32q_8kv_128":
        # q read and written; k and v read, their cache rows written; int64 positions and slots read
        return 2 * (4 * 4096 * 32 * 128 + 2 * 4 * 4096 * 8 * 128) * 2 + 2 * 4 * 4096 * 8
    if name == "rope_4x4096_32q_8kv_128":
        return 2 * (4 * 4096 * 32 * 128 + 4 * 4096 * 8 * 128) * 2 + 4 * 4096 * 8
    if name == "rope_cache_4x4096_32q_8kv_128":
        # the on-the-fly workload's bytes plus the fp32 cos and sin caches [4096, 128], each read once
        return algorithmic_bytes("rope_4x4096_32q_8kv_128") + 2 * 4096 * 128 * 4
    if name == "topk_sample_128x128256":
        # the logits read once, the uniforms read, the top-k list (fp32 values, int64 indices) and the drawn int64
        # indices written; the draw reads the list from the launch's own LDS or L2, not from HBM
        return 128 * 128256 * 4 + 128 * 4 + 128 * 50 * (4 + 8) + 128 * 8
    if name == "topk_128x128256":
        return 128 * 128256 * 4 + 128 * k * (4 + 8)
    raise KeyError(name)


WORKLOADS = {
    "softmax_4096x4096": softmax_4096x4096,
    "rmsnorm_16384x4096": rmsnorm_16384x4096,
    "rope_4x4096_32q_8kv_128": rope_4x4096_32q_8kv_128,
    "softmax_64x262144": softmax_64x262144,
    "topk_128x128256": topk_128x128256,
    "rmsnorm_add_16384x4096": rmsnorm_add_16384x4096,
    "rope_kv_4x4096_32q_8kv_128": rope_kv_4x4096_32q_8kv_128,
    "rope_cache_4x4096_32q_8kv_128": rope_cache_4x4096_32q_8kv_128,
    "topk_sample_128x128256": topk_sample_128x128256,
}
