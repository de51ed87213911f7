"""Pins the oracle's decoder pieces (RMSNorm, SwiGLU, rotary embedding, the
whole Llama-style causal LM) against the transformers Llama modules run on
the CPU -- the modules the reference's infer.py runs under KuiperMode -- and
against closed forms.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import kuiops_oracle as O

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM  # noqa: E402
from transformers.models.llama.modeling_llama import (LlamaRMSNorm, LlamaRotaryEmbedding,  # noqa: E402
                                                      apply_rotary_pos_emb)

TINY = dict(vocab=512, d=256, ffn=512, layers=2, hq=4, hkv=2, eps=1e-5, theta=10000.0)


def hf_config(c):
    return LlamaConfig(vocab_size=c["vocab"], hidden_size=c["d"], intermediate_size=c["ffn"],
                       num_hidden_layers=c["layers"], num_attention_heads=c["hq"],
                       num_key_value_heads=c["hkv"], max_position_embeddings=1024,
                       rms_norm_eps=c["eps"], rope_theta=c["theta"], tie_word_embeddings=False,
                       attn_implementation="eager")


def f(t):
    return t.detach().float().numpy()


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def frac_equal(a, b):
    return float(np.mean(a == b))


def test_rmsnorm_matches_llama_module():
    x, w = bf((16, 256), 1), bf((256,), 2)
    mod = LlamaRMSNorm(256, eps=1e-5).to(torch.bfloat16)
    with torch.no_grad():
        mod.weight.copy_(w)
        ref = f(mod(x))
    y, h = O.rmsnorm(f(x), f(w), 1e-5)
    np.testing.assert_array_equal(h, f(x))
    # fp32 variance vs the oracle's fp64 one flips a rare bf16 rounding
    assert frac_equal(y, ref) > 0.99
    assert O.within(y, ref, 1e-2, 1e-2)


def test_rmsnorm_residual_and_closed_form():
    x, r, w = bf((4, 64), 3), bf((4, 64), 4), bf((64,), 5)
    y, h = O.rmsnorm(f(x), f(w), 1e-6, residual=f(r))
    np.testing.assert_array_equal(h, f((x + r)))                    # bf16 add, rounded once
    # a constant row c normalises to sign(c) / sqrt(1 + eps / c^2) ~ sign(c)
    c = np.full((1, 64), -3.0, dtype=np.float32)
    y, _ = O.rmsnorm(c, f(w), 1e-6)
    np.testing.assert_allclose(y[0], O.round_bf16(-f(w)), rtol=0, atol=0)


def test_silu_mul_matches_llama_mlp_activation():
    g, u = bf((8, 128), 6), bf((8, 128), 7)
    ref = f(torch.nn.functional.silu(g) * u)
    out = O.silu_mul(np.concatenate([f(g), f(u)], -1))
    assert frac_equal(out, ref) > 0.99 and O.within(out, ref, 1e-2, 1e-2)


def test_rope_matches_llama_rotary():
    cfg = hf_config(TINY)
    rot = LlamaRotaryEmbedding(config=cfg)
    hd = TINY["d"] // TINY["hq"]
    np.testing.assert_allclose(O.rope_inv_freq(hd, TINY["theta"]), rot.inv_freq.numpy(), rtol=1e-6)
    q, k = bf((1, 4, 40, hd), 8), bf((1, 2, 40, hd), 9)
    pos = torch.arange(100, 140)[None]
    cos, sin = rot(q, pos)
    rq, rk = apply_rotary_pos_emb(q, k, cos, sin)
    inv = O.rope_inv_freq(hd, TINY["theta"])
    oq = O.rope(f(q), pos[0].numpy(), inv)
    ok = O.rope(f(k), pos[0].numpy(), inv)
    for o, r in ((oq, f(rq)), (ok, f(rk))):
        assert frac_equal(o, r) > 0.99 and O.within(o, r, 1e-2, 1e-2)


def test_rope_closed_forms():
    x = f(bf((3, 5, 64), 10))
    inv = O.rope_inv_freq(64, 10000.0)
    np.testing.assert_array_equal(O.rope(x, np.zeros(5), inv), x)   # position 0: identity
    y = O.rope(x, np.arange(1000, 1005), inv)
    n0 = x[..., :32] ** 2 + x[..., 32:] ** 2
    n1 = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=3e-2, atol=1e-2)        # a rotation keeps pair norms


@pytest.fixture(scope="module")
def tiny_model():
    torch.manual_seed(0)
    m = LlamaForCausalLM(hf_config(TINY))
    inv = m.model.rotary_emb.inv_freq.clone()
    m = m.to(torch.bfloat16).eval()
    m.model.rotary_emb.inv_freq = inv           # fp32, as from_pretrained(torch_dtype=bf16) keeps it
    return m


def test_llama_forward_matches_transformers(tiny_model):
    p = {k: f(v) for k, v in tiny_model.state_dict().items()}
    toks = torch.randint(0, TINY["vocab"], (24,), generator=torch.Generator().manual_seed(11))
    with torch.no_grad():
        ref = f(tiny_model(toks[None]).logits[0])
    out = O.llama_forward(p, toks.numpy(), TINY)
    assert out.shape == ref.shape
    assert O.within(out, ref, 2e-2, 2e-2)
    # argmax agrees wherever the reference's top two logits are not within tolerance
    srt = np.sort(ref, -1)
    clear = (srt[:, -1] - srt[:, -2]) > 4e-2
    assert clear.sum() >= 12
    assert np.array_equal(out.argmax(-1)[clear], ref.argmax(-1)[clear])
