"""Pins the oracle's whole forward pass (LlamaModel.Forward, and
QwenModel.Forward for the Qwen2 variant) against the float64 restatement
npref.Llama64 on a tiny model, for every weight mix."""
import numpy as np
import pytest

import npref
import oracle
from chatnet_amd import TINY_TEST, _native, synth


@pytest.mark.parametrize("mix", ["q4_0", "q4_k_m"])
def test_tiny_model_logits_match_float64(mix):
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=11, mix=mix)
    ora = oracle.OracleLlama(cfg, ck)
    ref = npref.Llama64(cfg, ck)
    toks = synth.tokens(11, "prompt", 6, cfg.vocab_size)
    for pos, t in enumerate(toks):
        a = ora.forward([t], pos)
        b = ref.forward([t], pos)
        assert np.max(np.abs(a - b)) < 1e-4 * max(1.0, np.max(np.abs(b)))
    # KV cache contents follow LlamaModel.cs:150-153 (post-RoPE K, raw V)
    for l in range(cfg.n_layers):
        np.testing.assert_allclose(ora.kv(l, 3, 0), ref.kc[l, 3], atol=1e-5)
        np.testing.assert_allclose(ora.kv(l, 3, 1), ref.vc[l, 3], atol=1e-5)


@pytest.mark.parametrize("bias,tied", [(True, False), (False, False), (True, True)])
def test_tiny_qwen2_logits_match_float64(bias, tied):
    # QwenModel.Forward (QwenModel.cs:69-178): biases, split-half RoPE, tied LM head
    cfg = TINY_TEST.replace(arch=_native.ARCH_QWEN2, rope_freq_base=1e6)
    emb = _native.GGML_Q8_0 if tied else _native.GGML_F32
    ck = synth.llama_checkpoint(cfg, seed=14, mix="q8_0", qkv_bias=bias, with_output=not tied, embedding=emb)
    ora = oracle.OracleLlama(cfg, ck)
    ref = npref.Llama64(cfg, ck)
    toks = synth.tokens(14, "prompt", 6, cfg.vocab_size)
    for pos, t in enumerate(toks):
        a = ora.forward([t], pos)
        b = ref.forward([t], pos)
        assert np.max(np.abs(a - b)) < 1e-4 * max(1.0, np.max(np.abs(b)))
    for l in range(cfg.n_layers):
        np.testing.assert_allclose(ora.kv(l, 3, 0), ref.kc[l, 3], atol=1e-5)
        np.testing.assert_allclose(ora.kv(l, 3, 1), ref.vc[l, 3], atol=1e-5)


def test_qwen2_bias_and_rope_change_the_result():
    # the restatement is not Llama's in disguise: dropping the bias or using
    # interleaved RoPE moves the logits
    cfg = TINY_TEST.replace(arch=_native.ARCH_QWEN2)
    ck = synth.llama_checkpoint(cfg, seed=15, mix="q8_0")
    toks = synth.tokens(15, "prompt", 4, cfg.vocab_size)
    a = oracle.OracleLlama(cfg, ck).forward(toks, 0)
    nb = {k: v for k, v in ck.items() if not k.endswith(".bias")}
    b = oracle.OracleLlama(cfg, nb).forward(toks, 0)
    c = oracle.OracleLlama(cfg.replace(arch=_native.ARCH_LLAMA), nb).forward(toks, 0)
    assert np.max(np.abs(a - b)) > 1e-3 and np.max(np.abs(b - c)) > 1e-3


def test_span_forward_equals_token_by_token():
    # IModel.Forward over a span: LM head only for the last token (LlamaModel.cs:207)
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=12)
    toks = synth.tokens(12, "prompt", 5, cfg.vocab_size)
    a = oracle.OracleLlama(cfg, ck)
    la = a.forward(toks, 0)
    b = oracle.OracleLlama(cfg, ck)
    for i, t in enumerate(toks):
        lb = b.forward([t], i)
    assert np.array_equal(la, lb)


def test_greedy_loop_respects_context_limit():
    # InferenceEngine.cs:295-298: emission stops once position reaches ctx-1
    cfg = TINY_TEST.replace(context_length=10)
    ck = synth.llama_checkpoint(cfg, seed=13)
    toks, margins = oracle.OracleLlama(cfg, ck).generate_greedy([1, 2, 3, 4], 50)
    assert len(toks) == 10 - 4
    assert len(margins) == len(toks)
