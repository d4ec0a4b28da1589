"""The decode oracle's composition against an independent implementation of the same
model: transformers' Qwen3ForCausalLM (the reference's decode step follows the same
architecture, ironmule/dense_cpu.py:188-220), built here from a Qwen3Config with random
weights (no download), on the CPU.

The oracle's dequantised float64 weights are loaded into the transformers model; the
oracle then decodes a prompt one token at a time (each step writing its own KV pools and
attending over them), and its logits at every position must match the transformers
model's logits for the whole sequence (one causal forward, no cache) at the fp32 rounding
level (transformers computes its RMSNorms in fp32).  Mutant compositions that a property
test of the oracle alone would not notice (rotary skipped, q/k-norm skipped, the MLP fed
from the residual stream instead of its RMSNorm) miss the same bar by orders of magnitude.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

HIDDEN, INTER, LAYERS, HEADS, KV_HEADS, HEAD_DIM, VOCAB = 256, 512, 2, 4, 2, 128, 512
EPS, THETA = 1e-6, 1e6
BAR = 1e-6  # max |logit - ref| / max |ref|: fp32 rounding level (observed about 1e-7)


def _weights(orc):
    """Dequantised 4-bit weights (float64) of every projection and the tied embedding,
    from the oracle's synthetic format, and norm weights near 1."""
    rng = np.random.default_rng(20261215)

    def deq(n, k, seed):
        pr = orc.synthetic(n, k, 1, seed=seed)
        return orc.dequant_f32(pr.w, pr.s, pr.b).astype(np.float64)

    def norm(n):
        return rng.uniform(0.8, 1.2, n)

    layers = []
    for i in range(LAYERS):
        s = 1000 + 10 * i
        layers.append(dict(wq=deq(HEADS * HEAD_DIM, HIDDEN, s), wk=deq(KV_HEADS * HEAD_DIM, HIDDEN, s + 1),
                           wv=deq(KV_HEADS * HEAD_DIM, HIDDEN, s + 2), wo=deq(HIDDEN, HEADS * HEAD_DIM, s + 3),
                           wg=deq(INTER, HIDDEN, s + 4), wu=deq(INTER, HIDDEN, s + 5),
                           wd=deq(HIDDEN, INTER, s + 6), input_norm=norm(HIDDEN),
                           post_norm=norm(HIDDEN), q_norm=norm(HEAD_DIM), k_norm=norm(HEAD_DIM)))
    # the synthetic weights have a positive mean; centring the embedding keeps the logits'
    # scale moderate (any matrix works: it only has to be the same in both models)
    embed = deq(VOCAB, HIDDEN, 999)
    embed -= embed.mean()
    return layers, embed, norm(HIDDEN)


def _hf_model(layers, embed, final_norm):
    cfg = transformers.Qwen3Config(vocab_size=VOCAB, hidden_size=HIDDEN, intermediate_size=INTER,
                                   num_hidden_layers=LAYERS, num_attention_heads=HEADS,
                                   num_key_value_heads=KV_HEADS, head_dim=HEAD_DIM,
                                   rms_norm_eps=EPS, rope_theta=THETA, tie_word_embeddings=True,
                                   attention_bias=False, max_position_embeddings=256,
                                   hidden_act="silu")
    cfg._attn_implementation = "eager"
    model = transformers.Qwen3ForCausalLM(cfg).double().eval()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(t(embed))
        model.model.norm.weight.copy_(t(final_norm))
        for lay, L in zip(model.model.layers, layers):
            lay.self_attn.q_proj.weight.copy_(t(L["wq"]))
            lay.self_attn.k_proj.weight.copy_(t(L["wk"]))
            lay.self_attn.v_proj.weight.copy_(t(L["wv"]))
            lay.self_attn.o_proj.weight.copy_(t(L["wo"]))
            lay.self_attn.q_norm.weight.copy_(t(L["q_norm"]))
            lay.self_attn.k_norm.weight.copy_(t(L["k_norm"]))
            lay.mlp.gate_proj.weight.copy_(t(L["wg"]))
            lay.mlp.up_proj.weight.copy_(t(L["wu"]))
            lay.mlp.down_proj.weight.copy_(t(L["wd"]))
            lay.input_layernorm.weight.copy_(t(L["input_norm"]))
            lay.post_attention_layernorm.weight.copy_(t(L["post_norm"]))
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    return model


def _oracle_logits(do, layers, embed, final_norm, tokens, slot=1, slots=3):
    """The oracle decodes `tokens` one step at a time in KV slot `slot`; logits per step."""
    model = do.Model(layers=[do.Layer(**L) for L in layers], embed=embed, norm=final_norm,
                     heads=HEADS, kv_heads=KV_HEADS, eps=EPS, theta=THETA)
    keys = [np.full((slots, KV_HEADS, len(tokens), HEAD_DIM), np.nan) for _ in range(LAYERS)]
    values = [np.full_like(k, np.nan) for k in keys]
    out = []
    for pos, tok in enumerate(tokens):
        out.append(do.decode_step(model, keys, values, [tok], [slot], [pos], round_bf16=False)[0])
    return np.stack(out)


@pytest.fixture(scope="module")
def setup():
    from oracle import decode_oracle as do
    from oracle import oracle as orc
    orc.lib()
    layers, embed, final_norm = _weights(orc)
    model = _hf_model(layers, embed, final_norm)
    tokens = [3, 511, 17, 17, 200, 5, 64, 300, 9, 1, 450, 77]
    with torch.no_grad():
        ref = model(torch.tensor([tokens])).logits[0].numpy()
    return do, layers, embed, final_norm, tokens, ref


def _rel(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


def test_decode_oracle_matches_transformers_qwen3(setup):
    do, layers, embed, final_norm, tokens, ref = setup
    got = _oracle_logits(do, layers, embed, final_norm, tokens)
    rel = _rel(got, ref)
    print(f"max |oracle - transformers| / max |logit| = {rel:.2e} over {len(tokens)} positions")
    assert rel <= BAR, rel


@pytest.mark.parametrize("mutant", ["no_rope", "no_qk_norm", "mlp_from_residual"])
def test_mutant_compositions_miss_the_bar(setup, monkeypatch, mutant):
    do, layers, embed, final_norm, tokens, ref = setup
    if mutant == "no_rope":
        monkeypatch.setattr(do, "rope", lambda x, positions, theta: np.asarray(x, np.float64))
        L = layers
    elif mutant == "no_qk_norm":
        L = [dict(l, q_norm=np.ones(HEAD_DIM), k_norm=np.ones(HEAD_DIM)) for l in layers]
        real = do.rms_norm
        # q/k-norm skipped: the per-head RMSNorm (last axis HEAD_DIM) becomes the identity
        monkeypatch.setattr(do, "rms_norm", lambda x, w, eps: np.asarray(x, np.float64)
                            if np.shape(x)[-1] == HEAD_DIM else real(x, w, eps))
    else:
        real = do.rms_norm
        # the post-attention RMSNorm returns the residual stream unnormalised
        monkeypatch.setattr(do, "rms_norm", lambda x, w, eps: np.asarray(x, np.float64) * w
                            if w is layers[0]["post_norm"] or w is layers[1]["post_norm"]
                            else real(x, w, eps))
        L = layers
    with np.errstate(over="ignore"):
        got = _oracle_logits(do, L, embed, final_norm, tokens)
    assert _rel(got, ref) > 100 * BAR
