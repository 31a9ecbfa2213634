"""The built-in module -> GGUF tensor name map of collect_hessians (host logic, no GPU).

The reference maps HF module names with gguf's TensorNameMap (hessians.py:64-82), which
is not installed here; the expected names below are the GGUF tensor names llama.cpp's
converter writes for these modules (token_embd, blk.N.attn_q/k/v/output,
blk.N.ffn_gate/up/down, output)."""
import pytest

from conftest import tiny_hf_decoder


def _expected(n_layers):
    out = {"model.embed_tokens": "token_embd", "lm_head": "output"}
    for l in range(n_layers):
        for hf, g in [("self_attn.q_proj", "attn_q"), ("self_attn.k_proj", "attn_k"),
                      ("self_attn.v_proj", "attn_v"), ("self_attn.o_proj", "attn_output"),
                      ("mlp.gate_proj", "ffn_gate"), ("mlp.up_proj", "ffn_up"),
                      ("mlp.down_proj", "ffn_down")]:
            out[f"model.layers.{l}.{hf}"] = f"blk.{l}.{g}"
    return out


@pytest.mark.parametrize("kind,arch", [("qwen3", "qwen3"), ("llama", "llama"), ("llama", "qwen2")])
def test_name_map_of_the_hf_decoder(kind, arch):
    from perm_amd import hessians as hs
    model = tiny_hf_decoder(kind, n_layers=3)
    assert hs.build_name_map(model, arch, 3) == _expected(3)
    # blocks past n_layers are not in the map (TensorNameMap is built for n_layers blocks)
    assert hs.build_name_map(model, arch, 2) == _expected(2)


def test_name_map_refuses_an_unknown_arch():
    from perm_amd import hessians as hs
    with pytest.raises(ValueError, match="name map"):
        hs.build_name_map(tiny_hf_decoder(), "gpt2", 2)


def test_collect_refuses_a_shape_mismatch_before_any_hook():
    """hessians.py:126-135: the mismatch is found while planning, so no hook is left on
    the model and nothing reaches a device."""
    from perm_amd import hessians as hs
    model = tiny_hf_decoder()
    ne0 = {g + ".weight": 64 for g in _expected(2).values()}
    ne0["blk.1.ffn_down.weight"] = 96
    ne0["blk.0.attn_q.weight"] = 999
    with pytest.raises(ValueError, match="mis-key"):
        hs.collect_hessians(model, [], ne0, "qwen3", 2, log=lambda *_: None)
    assert all(not m._forward_hooks for m in model.modules())
