"""encode_gguf's layer-group size (host logic, no GPU): the largest layer count whose
estimated footprint -- 28 B per weight plus 40 n^2 B per tensor -- fits in half the free
device memory, at least one."""
import pytest
import torch

from perm_amd import ef


class _T:
    def __init__(self, ne):
        self.shape = ne  # GGUF ne order: [ne0 (input), ne1 (rows)]


def _model(layers, layer_shapes):
    f16, sel = {}, []
    for b in range(layers):
        for kind, (n, rows) in layer_shapes.items():
            name = f"blk.{b}.{kind}.weight"
            f16[name] = _T([n, rows])
            sel.append((name, "Q2_K"))
    f16["token_embd.weight"] = _T([1024, 151936])
    sel.append(("token_embd.weight", "Q6_K"))
    return f16, sel


def _block_of(name):
    return int(name.split(".")[1]) if name.startswith("blk.") else -1


QWEN3_06B = {"attn_q": (1024, 2048), "attn_k": (1024, 1024), "attn_v": (1024, 1024),
             "attn_output": (2048, 1024), "ffn_gate": (1024, 3072), "ffn_up": (1024, 3072),
             "ffn_down": (3072, 1024)}
LLAMA3_8B = {"attn_q": (4096, 4096), "attn_k": (4096, 1024), "attn_v": (4096, 1024),
             "attn_output": (4096, 4096), "ffn_gate": (4096, 14336), "ffn_up": (4096, 14336),
             "ffn_down": (14336, 4096)}


def _per_layer(shapes):
    return sum(28 * n * r + 40 * n * n for n, r in shapes.values())


@pytest.mark.parametrize("shapes,layers", [(QWEN3_06B, 28), (LLAMA3_8B, 32)])
def test_layers_per_pass_from_free_memory(monkeypatch, shapes, layers):
    free = 288 * 2**30
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda *a: (free, free))
    f16, sel = _model(layers, shapes)
    got = ef._auto_layers_per_pass(f16, sel, _block_of)
    assert got == max(1, int(0.5 * free // _per_layer(shapes)))
    if shapes is QWEN3_06B:
        assert got >= layers          # the whole model in one pass
    else:
        assert 1 <= got < layers      # split, each group within half the memory
        assert got * _per_layer(shapes) <= 0.5 * free


def test_layers_per_pass_at_least_one(monkeypatch):
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda *a: (1 << 20, 1 << 20))
    f16, sel = _model(2, LLAMA3_8B)
    assert ef._auto_layers_per_pass(f16, sel, _block_of) == 1
