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


def test_plan_classifies_like_the_reference():
    """plan_targets (hessians.py:108-135): every mapped Linear of the shard is a target with
    its GGUF name and width; a module without a name, or whose tensor the GGUF lacks, is
    unmapped; the embedding and other shards' tensors are neither; output goes with the
    shard that starts at block 0. The refusal message matches the reference test's pattern
    (test_hessians.py:43)."""
    import re

    from perm_amd import hessians as hs
    model = tiny_hf_decoder()
    names = hs.build_name_map(model, "qwen3", 2)
    ne0 = {g + ".weight": 96 if g.endswith("ffn_down") else 64 for g in names.values()}
    del ne0["blk.1.attn_k.weight"]
    names = dict(names)
    del names["model.layers.0.mlp.up_proj"]
    t0, un0 = hs.plan_targets(model, names, ne0, 0, 1)
    t1, un1 = hs.plan_targets(model, names, ne0, 1, 2)
    assert un0 == un1
    assert "model.layers.0.mlp.up_proj" in un0
    assert "model.layers.1.self_attn.k_proj (-> blk.1.attn_k.weight, not in the GGUF)" in un0
    assert {t.gguf_name for t in t0} == {f"blk.0.{k}.weight" for k in
                                        ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate",
                                         "ffn_down")} | {"output.weight"}
    assert {t.gguf_name for t in t1} == {f"blk.1.{k}.weight" for k in
                                        ("attn_q", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                         "ffn_down")}
    for t in t0 + t1:
        assert t.width == t.module.in_features == ne0[t.gguf_name]
        assert names[t.module_name] + ".weight" == t.gguf_name
    ne0["blk.1.ffn_up.weight"] = 65
    hs.plan_targets(model, names, ne0, 0, 1)  # another shard's conflict is not this shard's
    with pytest.raises(ValueError) as e:
        hs.plan_targets(model, names, ne0, 1, 2)
    assert re.search(r"ne\[0\]|mis-key|MISMATCH", str(e.value))
    assert "model.layers.1.mlp.up_proj" in str(e.value)
