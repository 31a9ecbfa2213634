"""Shared fixtures and markers.

``gpu`` tests run the HIP library on a real device; everything else runs on the
CPU (the oracle against the golden vectors, host-side logic, and the C-ABI
library's load/export check)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "kquant_golden.npz")
TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
CODEC_TYPES = TYPES + ["Q8_0"]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def heavy_tailed(nrow, n, seed):
    """Cubed normals with a per-row U(0.2, 3) scale (the reference's tests/conftest.py:8-13)."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((nrow, n)) ** 3).astype(np.float32)
    x *= rng.uniform(0.2, 3.0, size=(nrow, 1)).astype(np.float32)
    return x


def correlated_hessian(n, T, seed):
    """X^T X of correlated Gaussian rows (the reference's tests/test_ef_synthetic.py:12-18)."""
    rng = np.random.default_rng(seed)
    mix = rng.standard_normal((n, n)) / np.sqrt(n)
    mix += 1.5 * np.eye(n)
    X = rng.standard_normal((T, n)) @ mix.T
    return (X.T @ X).astype(np.float64)


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN)


# The reference optimizer test's model (test_perm_optimize.py:14-42): 2 layers,
# d_model 256, d_ffn 512, vocab 512, 4 q heads / 2 kv heads of 64, f16 weights.
OPT_DIMS = {"d_model": 256, "d_ffn": 512, "n_layers": 2, "n_heads": 4, "n_kv": 2, "head_dim": 64}


def small_qwen3_model(seed=0):
    D, FFN, V, HD, NKV, NH = 256, 512, 512, 64, 2, 4
    shapes = {"token_embd.weight": (V, D), "output.weight": (V, D)}
    for l in range(2):
        shapes[f"blk.{l}.attn_q.weight"] = (NH * HD, D)
        shapes[f"blk.{l}.attn_k.weight"] = (NKV * HD, D)
        shapes[f"blk.{l}.attn_v.weight"] = (NKV * HD, D)
        shapes[f"blk.{l}.attn_output.weight"] = (D, NH * HD)
        shapes[f"blk.{l}.ffn_gate.weight"] = (FFN, D)
        shapes[f"blk.{l}.ffn_up.weight"] = (FFN, D)
        shapes[f"blk.{l}.ffn_down.weight"] = (D, FFN)
    rng = np.random.default_rng(seed)
    return {n: (rng.standard_normal(s) ** 3 * 0.1).astype(np.float16) for n, s in shapes.items()}


def tiny_hf_decoder(kind="qwen3", n_layers=2, tie=False, seed=0):
    """A random-init HF decoder of the llama family on the CPU, float32: hidden 64,
    4 q heads / 2 kv heads of 16, FFN 96, vocab 128 (the reference tests' tiny_qwen3
    shape class, built offline from a config)."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM
    kw = dict(vocab_size=128, hidden_size=64, intermediate_size=96, num_hidden_layers=n_layers,
              num_attention_heads=4, num_key_value_heads=2, head_dim=16, tie_word_embeddings=tie)
    torch.manual_seed(seed)
    if kind == "qwen3":
        model = Qwen3ForCausalLM(Qwen3Config(**kw))
    else:
        model = LlamaForCausalLM(LlamaConfig(**kw))
    return model.eval()


TINY_DIMS = {"d_model": 64, "d_ffn": 96, "n_layers": 2, "n_heads": 4, "n_kv": 2, "head_dim": 16}
