"""The decode oracle's Gemma 3 composition against transformers' Gemma3ForCausalLM, built
from a Gemma3TextConfig with random weights (no download), on the CPU.

The reference's paired decode step composes Gemma 3 (ironmule/paired_research.py:177-215).
The oracle's dequantised float64 weights are loaded into the transformers model; the oracle
decodes a prompt one token at a time and its logits at every position must match one causal
forward of the transformers model at the fp32 rounding level.  The configuration makes every
Gemma-specific choice visible: two sliding-window layers with a window shorter than the prompt
and one global layer, different rotary bases for the two kinds, a query_pre_attn_scalar that is
not the head dimension, norm weights away from zero (the 1 + w form), and an embedding scale of
sqrt(hidden).  Mutant compositions (the plain-w norm, no sliding window, one rotary base, the
head-dimension scale, no post-attention norm, SiLU for the tanh GELU) miss the bar by orders of
magnitude.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

HIDDEN, INTER, HEADS, KV_HEADS, HEAD_DIM, VOCAB = 256, 512, 2, 1, 128, 512
LAYERS, PATTERN, WINDOW = 3, 3, 4
EPS, THETA_GLOBAL, THETA_LOCAL, QUERY_SCALAR = 1e-6, 1e6, 1e4, 96
BAR = 1e-6  # max |logit - ref| / max |ref| (fp32 rounding level)


def _weights(orc):
    rng = np.random.default_rng(20261216)

    def deq(n, k, seed):
        pr = orc.synthetic(n, k, 1, seed=seed)
        w = orc.dequant_f32(pr.w, pr.s, pr.b).astype(np.float64)
        return w - w.mean()  # centred: moderate activations through three layers

    def norm(n):
        return rng.uniform(-0.3, 0.3, n)  # the w of Gemma's 1 + w

    layers = []
    for i in range(LAYERS):
        s = 2000 + 10 * i
        layers.append(dict(wq=deq(HEADS * HEAD_DIM, HIDDEN, s), wk=deq(KV_HEADS * HEAD_DIM, HIDDEN, s + 1),
                           wv=deq(KV_HEADS * HEAD_DIM, HIDDEN, s + 2), wo=deq(HIDDEN, HEADS * HEAD_DIM, s + 3),
                           wg=deq(INTER, HIDDEN, s + 4), wu=deq(INTER, HIDDEN, s + 5),
                           wd=deq(HIDDEN, INTER, s + 6), input_norm=norm(HIDDEN), post_attn_norm=norm(HIDDEN),
                           pre_ff_norm=norm(HIDDEN), post_ff_norm=norm(HIDDEN), q_norm=norm(HEAD_DIM),
                           k_norm=norm(HEAD_DIM)))
    return layers, deq(VOCAB, HIDDEN, 1999), norm(HIDDEN)


def _hf_model(layers, embed, final_norm):
    types = ["full_attention" if i % PATTERN == PATTERN - 1 else "sliding_attention" for i in range(LAYERS)]
    cfg = transformers.Gemma3TextConfig(
        vocab_size=VOCAB, hidden_size=HIDDEN, intermediate_size=INTER, num_hidden_layers=LAYERS,
        num_attention_heads=HEADS, num_key_value_heads=KV_HEADS, head_dim=HEAD_DIM, rms_norm_eps=EPS,
        sliding_window=WINDOW, layer_types=types, query_pre_attn_scalar=QUERY_SCALAR,
        rope_parameters={"sliding_attention": {"rope_type": "default", "rope_theta": THETA_LOCAL},
                         "full_attention": {"rope_type": "default", "rope_theta": THETA_GLOBAL}},
        hidden_activation="gelu_pytorch_tanh", tie_word_embeddings=True, max_position_embeddings=256,
        final_logit_softcapping=None, attn_logit_softcapping=None)
    cfg._attn_implementation = "eager"
    model = transformers.Gemma3ForCausalLM(cfg).double().eval()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(t(embed))
        model.model.norm.weight.copy_(t(final_norm))
        for lay, L in zip(model.model.layers, layers):
            a = lay.self_attn
            for name, key in (("q_proj", "wq"), ("k_proj", "wk"), ("v_proj", "wv"), ("o_proj", "wo")):
                getattr(a, name).weight.copy_(t(L[key]))
            a.q_norm.weight.copy_(t(L["q_norm"]))
            a.k_norm.weight.copy_(t(L["k_norm"]))
            lay.mlp.gate_proj.weight.copy_(t(L["wg"]))
            lay.mlp.up_proj.weight.copy_(t(L["wu"]))
            lay.mlp.down_proj.weight.copy_(t(L["wd"]))
            lay.input_layernorm.weight.copy_(t(L["input_norm"]))
            lay.post_attention_layernorm.weight.copy_(t(L["post_attn_norm"]))
            lay.pre_feedforward_layernorm.weight.copy_(t(L["pre_ff_norm"]))
            lay.post_feedforward_layernorm.weight.copy_(t(L["post_ff_norm"]))
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    return model


def _oracle_logits(do, layers, embed, final_norm, tokens, *, window=WINDOW, theta_local=THETA_LOCAL,
                   query_scalar=QUERY_SCALAR, slot=1, slots=3):
    model = do.Gemma3Model(layers=[do.Gemma3Layer(**L) for L in layers], embed=embed, norm=final_norm,
                           heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM, eps=EPS,
                           theta_global=THETA_GLOBAL, theta_local=theta_local, window=window,
                           pattern=PATTERN, query_scalar=query_scalar)
    keys = [np.full((slots, KV_HEADS, len(tokens), HEAD_DIM), np.nan) for _ in range(LAYERS)]
    values = [np.full_like(k, np.nan) for k in keys]
    return np.stack([do.gemma3_decode_step(model, keys, values, [tok], [slot], [pos], round_bf16=False)[0]
                     for pos, tok in enumerate(tokens)])


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


def test_gemma3_oracle_matches_transformers(setup):
    do, layers, embed, final_norm, tokens, ref = setup
    rel = _rel(_oracle_logits(do, layers, embed, final_norm, tokens), ref)
    print(f"max |oracle - transformers| / max |logit| = {rel:.2e} over {len(tokens)} positions")
    assert rel <= BAR, rel


@pytest.mark.parametrize("mutant", ["plain_w_norm", "no_window", "one_rope_base", "head_dim_scale",
                                    "no_post_attention_norm", "silu_mlp"])
def test_gemma3_mutant_compositions_miss_the_bar(setup, monkeypatch, mutant):
    do, layers, embed, final_norm, tokens, ref = setup
    kw = {}
    if mutant == "plain_w_norm":
        real = do.rms_norm
        monkeypatch.setattr(do, "gemma_norm", lambda x, w, eps, r=None: real(x, w, eps))
    elif mutant == "no_window":
        kw["window"] = 10 ** 6
    elif mutant == "one_rope_base":
        kw["theta_local"] = THETA_GLOBAL
    elif mutant == "head_dim_scale":
        kw["query_scalar"] = HEAD_DIM
    elif mutant == "no_post_attention_norm":
        real = do.gemma_norm
        post = {id(L["post_attn_norm"]) for L in layers}
        monkeypatch.setattr(do, "gemma_norm", lambda x, w, eps, r=lambda a: np.asarray(a, np.float64):
                            np.asarray(x, np.float64) if id(w) in post else real(x, w, eps, r))
    else:
        monkeypatch.setattr(do, "gelu_tanh", lambda x: np.asarray(x, np.float64) / (1.0 + np.exp(-np.asarray(x, np.float64))))
    with np.errstate(over="ignore"):
        got = _oracle_logits(do, layers, embed, final_norm, tokens, **kw)
    assert _rel(got, ref) > 100 * BAR, mutant
