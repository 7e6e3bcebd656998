"""CPU checks of the PyTorch-ROCm operators (torch.ops.ckopt.*, build/torch/libckopt_torch.so): the library loads into
torch and registers every operator with its schema, the meta shape functions give the outputs' shapes and dtypes
without data (what tracing sees), and a CPU tensor is refused (there is no CPU path)."""

import pytest
import torch

# operator: (argument names, the arguments it writes, number of returns)
SCHEMAS = {
    "softmax": (["x"], [], 1),
    "rmsnorm": (["x", "weight", "eps"], [], 1),
    "rmsnorm_add": (["x", "residual", "weight", "eps"], [], 2),
    "rmsnorm_add_": (["x", "residual", "weight", "eps"], ["residual"], 1),
    "rope": (["q", "k", "cos", "sin", "position_ids"], [], 2),
    "rope_": (["q", "k", "position_ids", "inv_freq"], ["q", "k"], 0),
    "rope_kv_": (["q", "k", "v", "position_ids", "inv_freq", "k_cache", "v_cache", "slot_mapping"],
                 ["q", "k_cache", "v_cache"], 0),
    "topk": (["x", "k"], [], 2),
    "topk_and_sample": (["x", "k", "uniforms", "temperature", "top_p"], [], 3),
    "topk_sample": (["values", "indices", "uniforms", "temperature", "top_p"], [], 1),
}


@pytest.fixture(scope="module")
def ckopt(pkg):
    return pkg.ops()


@pytest.mark.parametrize("name", sorted(SCHEMAS))
def test_operator_registered(ckopt, name):
    schema = getattr(ckopt, name).default._schema
    names, written, returns = SCHEMAS[name]
    assert schema.name == "ckopt::" + name
    assert [a.name for a in schema.arguments] == names
    assert [a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write] == written
    assert len(schema.returns) == returns


def test_meta_shapes(ckopt):
    meta = dict(device="meta")
    x = torch.empty(6, 300, **meta)
    assert ckopt.softmax(x).shape == (6, 300)
    xb = torch.empty(6, 256, dtype=torch.bfloat16, **meta)
    y, h = ckopt.rmsnorm_add(xb, torch.empty_like(xb), None, 1e-6)
    assert y.shape == h.shape == (6, 256) and y.dtype == torch.bfloat16
    q, k = torch.empty(1, 4, 8, 64, **meta), torch.empty(1, 4, 2, 64, **meta)
    qo, ko = ckopt.rope(q, k, torch.empty(16, 64, **meta), torch.empty(16, 64, **meta),
                        torch.empty(1, 4, dtype=torch.long, **meta))
    assert qo.shape == q.shape and ko.shape == k.shape
    v, i = ckopt.topk(x, 50)
    assert v.shape == i.shape == (6, 50) and i.dtype == torch.int64 and v.dtype == torch.float32
    v, i, d = ckopt.topk_and_sample(x, 7, torch.empty(6, **meta), 0.8, 0.9)
    assert d.shape == (6,) and d.dtype == torch.int64


def test_cpu_tensors_refused(ckopt):
    with pytest.raises((NotImplementedError, RuntimeError)):
        ckopt.softmax(torch.zeros(2, 8))
    with pytest.raises((NotImplementedError, RuntimeError)):
        ckopt.topk(torch.zeros(2, 8), 3)
