"""GPU parity of the whole forward pass (chatnet_forward / chatnet_generate_greedy)
against the oracle's LlamaModel.Forward on identical seeded checkpoints.

Bars: logits max-abs error <= 1e-2; greedy tokens identical to the oracle's
(a step whose oracle top-1/top-2 margin is below 1e-3 is reported and the
comparison is teacher-forced from there)."""
import numpy as np
import pytest

import oracle
from chatnet_amd import TINY_TEST, TINYLLAMA_1B, HipLlamaModel, _native, synth
from chatnet_amd.engine import GreedySampler, generate
from gpu_util import announce, compare_greedy

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(16)
    yield
    oracle.set_threads(1)


@pytest.mark.parametrize("mix,kv", [("q4_0", _native.KV_F32), ("q4_k_m", _native.KV_F32),
                                    ("q4_0", _native.KV_F16), ("q8_0", _native.KV_F32),
                                    ("q5_k_m", _native.KV_F32)])
def test_tiny_model_logits_token_by_token(mix, kv):
    cfg = TINY_TEST.replace(kv_dtype=kv)
    ck = synth.llama_checkpoint(cfg, seed=21, mix=mix)
    ora = oracle.OracleLlama(cfg, ck)
    toks = synth.tokens(21, "prompt", 12, cfg.vocab_size)
    announce(f"tiny model mix={mix} kv={kv}")
    with HipLlamaModel(cfg, ck) as m:
        for pos, t in enumerate(toks):
            g = m.forward([t], pos)
            r = ora.forward([t], pos)
            tol = LOGIT_TOL if kv == _native.KV_F32 else 2 * LOGIT_TOL
            assert np.max(np.abs(g - r)) <= tol, (pos, float(np.max(np.abs(g - r))))
        assert m.argmax() == GreedySampler().sample(g)


# -- Qwen2 variant (QwenModel.Forward): QKV biases, split-half RoPE, tied LM head --
TINY_QWEN = TINY_TEST.replace(arch=_native.ARCH_QWEN2, rope_freq_base=1e6, rms_norm_eps=1e-6)


@pytest.mark.parametrize("mix,bias,tied", [("q8_0", True, False), ("q4_0", False, False), ("q4_k_m", True, False),
                                           ("q4_0", True, True)])
def test_tiny_qwen2_logits_token_by_token(mix, bias, tied):
    cfg = TINY_QWEN
    emb = _native.GGML_Q8_0 if tied else _native.GGML_F32
    ck = synth.llama_checkpoint(cfg, seed=41, mix=mix, qkv_bias=bias, with_output=not tied, embedding=emb)
    ora = oracle.OracleLlama(cfg, ck)
    toks = synth.tokens(41, "prompt", 12, cfg.vocab_size)
    announce(f"tiny qwen2 mix={mix} bias={bias} tied={tied}")
    with HipLlamaModel(cfg, ck) as m:
        for pos, t in enumerate(toks):
            g = m.forward([t], pos)
            r = ora.forward([t], pos)
            assert np.max(np.abs(g - r)) <= LOGIT_TOL, (pos, float(np.max(np.abs(g - r))))


def test_qwen2_span_and_greedy_match_oracle():
    """A 40-token Qwen2 span on the batched path (bias and split-half RoPE in
    the span kernels), a continuing 8-token span, then 32 greedy tokens from
    the device loop."""
    cfg = SPAN_SMALL.replace(arch=_native.ARCH_QWEN2, rope_freq_base=1e6, context_length=128)
    ck = synth.llama_checkpoint(cfg, seed=42, mix="q4_0")
    toks = synth.tokens(42, "prompt", 48, cfg.vocab_size)
    announce("qwen2 span 40 + 8, greedy 32")
    with HipLlamaModel(cfg, ck) as m:
        g = m.forward(toks[:40], 0).copy()
        g2 = m.forward(toks[40:], 40).copy()
        gt = list(m.decode_greedy(32))
    ora = oracle.OracleLlama(cfg, ck)
    r = ora.forward(toks[:40], 0)
    r2 = ora.forward(toks[40:], 40)
    assert np.max(np.abs(g - r)) <= LOGIT_TOL and np.max(np.abs(g2 - r2)) <= LOGIT_TOL
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(toks), 32)
    compare_greedy(gt, o, margins, "qwen2 span 40+8, greedy 32", resume=(cfg, ck, list(toks)))


def test_qwen2_iq3_s_rows_keep_the_file_order():
    """IQ3_S q/k matrices of a Qwen2 model: each row's last block reads the
    next row of the file (DequantIQ.cs:255-283), while the device keeps q/k in
    its per-head pair order; decode and a span against the oracle."""
    cfg = SPAN_SMALL.replace(arch=_native.ARCH_QWEN2, rope_freq_base=1e6, context_length=64)
    ck = synth.llama_checkpoint(cfg, seed=45, mix="iq_b")
    toks = synth.tokens(45, "prompt", 20, cfg.vocab_size)
    announce("qwen2 iq_b: 12-token span + 8 decode steps")
    ora = oracle.OracleLlama(cfg, ck)
    with HipLlamaModel(cfg, ck) as m:
        g = m.forward(toks[:12], 0)
        r = ora.forward(toks[:12], 0)
        assert np.max(np.abs(g - r)) <= LOGIT_TOL
        for i, t in enumerate(toks[12:]):
            g = m.forward([t], 12 + i)
            r = ora.forward([t], 12 + i)
            assert np.max(np.abs(g - r)) <= LOGIT_TOL, (i, float(np.max(np.abs(g - r))))


def test_qwen2_from_gguf_matches_uploaded_checkpoint(tmp_path):
    from chatnet_amd import gguf
    cfg = TINY_QWEN
    ck = synth.llama_checkpoint(cfg, seed=43, mix="q8_0", with_output=False, embedding=_native.GGML_Q8_0)
    path = str(tmp_path / "qwen.gguf")
    gguf.write_llama(path, cfg, ck)
    toks = synth.tokens(43, "prompt", 10, cfg.vocab_size)
    announce("qwen2 gguf load")
    with HipLlamaModel.from_gguf(path) as m:
        assert m.config.arch == _native.ARCH_QWEN2
        g = m.forward(toks, 0).copy()
    with HipLlamaModel(cfg, ck) as m2:
        r = m2.forward(toks, 0).copy()
    assert np.array_equal(g, r)
    o = oracle.OracleLlama(cfg, ck).forward(toks, 0)
    assert np.max(np.abs(g - o)) <= LOGIT_TOL


def test_qwen2_upload_rules():
    cfg = TINY_QWEN
    ck = synth.llama_checkpoint(cfg, seed=44, mix="q4_0")
    announce("qwen2 upload rules")
    qb = ck["blk.0.attn_q.bias"]
    with HipLlamaModel(TINY_TEST) as m:   # Llama has no biases (LlamaWeights.cs:105-144)
        with pytest.raises(_native.ChatnetKeyNotFound):
            m.upload_tensor("blk.0.attn_q.bias", qb.type, qb.dims, qb.data)
    with HipLlamaModel(cfg) as m:
        with pytest.raises(_native.ChatnetNotSupported):
            m.upload_tensor("blk.0.attn_q.bias", _native.GGML_F16, qb.dims, qb.data[: qb.data.size // 2])
        with pytest.raises(_native.ChatnetSizeMismatch):
            m.upload_tensor("blk.0.attn_k.bias", qb.type, qb.dims, qb.data)   # dim floats where kv_dim are due
        for name, t in ck.items():
            if name not in ("blk.1.attn_k.bias", "blk.1.attn_v.bias"):
                m.upload_tensor(name, t.type, t.dims, t.data)
        with pytest.raises(_native.ChatnetKeyNotFound):   # q bias without k/v (QwenWeights.cs:164-169)
            m.forward([1], 0)
        for name in ("blk.1.attn_k.bias", "blk.1.attn_v.bias"):
            t = ck[name]
            m.upload_tensor(name, t.type, t.dims, t.data)
        r = oracle.OracleLlama(cfg, ck).forward([1, 2], 0)
        assert np.max(np.abs(m.forward([1, 2], 0) - r)) <= LOGIT_TOL


# Every weight type MatVecMulByType dispatches here (LlamaModel.cs:470-567),
# embeddings of each type LoadEmbedding reads (LlamaModel.cs:365-394), and the
# tied LM head on the embedding of any type (LlamaWeights.cs:89-98).  "mixed"
# gives every matrix its own type, ffn_gate and ffn_up different
# (LlamaModel.cs:175-179: each dispatched on its own type).
@pytest.mark.parametrize("mix,emb,tied", [
    ("q4_0", _native.GGML_F16, False), ("q4_0", _native.GGML_Q4_0, False), ("q4_0", _native.GGML_Q4_0, True),
    ("q8_0", _native.GGML_Q8_0, True), ("f32", _native.GGML_F32, False), ("f32", _native.GGML_F32, True),
    ("f16", _native.GGML_F16, False), ("f16", _native.GGML_F16, True), ("mixed", _native.GGML_Q8_0, False),
    ("mixed", _native.GGML_F32, True), ("q4_k_m", _native.GGML_F16, True),
    # the types read as packed units, as matrices, embeddings and tied LM heads
    ("legacy_blocks", _native.GGML_Q5_1, False), ("legacy_blocks", _native.GGML_Q4_1, True),
    ("q3_k_m", _native.GGML_Q3_K, False), ("q3_k_m", _native.GGML_Q5_0, True),
    ("q2_k", _native.GGML_Q2_K, True), ("q2_k", _native.GGML_Q8_K, False),
    ("q4_k_m", _native.GGML_Q4_K, True), ("q4_0", _native.GGML_Q6_K, False), ("q8_0", _native.GGML_Q5_K, True),
    # the IQ family (DequantIQ.cs decoders)
    ("iq_a", _native.GGML_IQ4_NL, False), ("iq_a", _native.GGML_IQ4_XS, True), ("iq_b", _native.GGML_IQ2_S, False),
    ("iq_b", _native.GGML_IQ1_M, True), ("iq_a", _native.GGML_IQ3_XXS, False), ("iq_b", _native.GGML_IQ2_XS, True),
    ("iq_a", _native.GGML_IQ2_XXS, True), ("iq_b", _native.GGML_IQ1_S, False),
])
def test_weight_and_embedding_types_match_oracle(mix, emb, tied):
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=27, mix=mix, with_output=not tied, embedding=emb)
    toks = synth.tokens(27, "prompt", 6, cfg.vocab_size)
    announce(f"types mix={mix} embedding={emb} tied={tied}")
    ora = oracle.OracleLlama(cfg, ck)
    with HipLlamaModel(cfg, ck) as m:
        for pos, t in enumerate(toks):
            g = m.forward([t], pos)
            r = ora.forward([t], pos)
            assert np.max(np.abs(g - r)) <= LOGIT_TOL, (pos, float(np.max(np.abs(g - r))))
        gt = list(m.decode_greedy(16))
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(toks), 16)
    compare_greedy(gt, o, margins, f"types mix={mix} embedding={emb} tied={tied}", resume=(cfg, ck, list(toks)))


@pytest.mark.parametrize("tie_rows,nan_rows,expect,vocab", [
    ((7, 1030, 1031, 3000, 4095), (), 7, 4096),  # ties across threads and waves: lowest index wins
    ((1024, 2048, 9), (), 9, 4096),              # same thread (stride 1024) and across waves
    ((7, 3000), (0,), 0, 4096),                  # NaN at index 0 never loses (GreedySampler.cs:16-24)
    ((7, 3000), (5, 2999), 7, 4096),             # NaN elsewhere never wins
    ((40002, 32769, 40001), (), 32769, 40003),   # second round of loads, the 3 tail elements
    ((40002,), (1,), 40002, 40003),              # the maximum in the tail only
])
def test_device_argmax_ties_and_nan(tie_rows, nan_rows, expect, vocab):
    cfg = TINY_TEST.replace(vocab_size=vocab)
    ck = synth.llama_checkpoint(cfg, seed=28)
    prompt = [3, 1, 4, 1, 5]
    bpr = cfg.dim // 32 * 18
    announce(f"argmax ties {tie_rows} nan {nan_rows}")
    base = oracle.OracleLlama(cfg, ck).forward(prompt, 0)
    src = int(np.argmax(base))
    assert base[src] > 0
    w = ck["output.weight"].data.reshape(cfg.vocab_size, bpr).copy()
    zero = np.zeros(bpr, np.uint8).reshape(-1, 18)
    zero[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)  # d = 1, every q = 8: weight 0
    zero[:, 2:] = 0x88
    row_src = w[src].copy()
    w[:] = zero.ravel()
    for r in tie_rows:
        w[r] = row_src
    for r in nan_rows:
        w[r, 0:2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)  # fp16 NaN scale
    ck["output.weight"] = synth.SynthTensor(ck["output.weight"].type, ck["output.weight"].dims, w.ravel())
    ref = oracle.OracleLlama(cfg, ck).forward(prompt, 0)
    assert oracle.argmax(ref) == expect
    with HipLlamaModel(cfg, ck) as m:
        g = m.forward(prompt, 0).copy()
        assert np.all(g[list(tie_rows)] == g[tie_rows[0]])  # identical rows give identical logits
        assert m.argmax() == expect
        assert GreedySampler().sample(g) == expect
        assert list(m.generate_greedy(prompt, 1)) == [expect]  # the decode loop's first pick


def test_eos_stops_before_forwarding_and_a_continued_decode_resumes():
    """InferenceEngine.cs:258-261: Generate breaks on EOS before forwarding it.
    With EOS set to the k-th greedy token the device loop returns the k tokens
    before it and leaves the cache, position and logits of the (k-1)-th, so a
    continued decode without EOS picks EOS again and then follows the
    uninterrupted sequence."""
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=29)
    prompt = synth.tokens(29, "prompt", 6, cfg.vocab_size)
    announce("eos mid-stream, continued decode")
    with HipLlamaModel(cfg, ck) as m:
        full = [int(t) for t in m.generate_greedy(prompt, 30)]
        k = next(i for i in range(2, 30) if full[i] not in full[:i])
        eos = full[k]
        cut = [int(t) for t in m.generate_greedy(prompt, 30, eos_token=eos)]
        assert cut == full[:k]
        lg = m.get_logits()
        rest = [int(t) for t in m.decode_greedy(30 - k)]
        assert rest == full[k:30]
        # the host loop over IModel.Forward stops at the same place
        h = generate(m, prompt, 30, GreedySampler(), eos_token=eos)
        assert list(h) == full[:k]
    r = oracle.OracleLlama(cfg, ck).forward(list(prompt) + full[:k], 0)
    assert np.max(np.abs(lg - r)) <= LOGIT_TOL
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 30)
    compare_greedy(full, o[:30], margins, "eos run, uninterrupted 6+30", resume=(cfg, ck, list(prompt)))


@pytest.mark.parametrize("n_prompt,expect_len", [(12, 1), (11, 1), (10, 2), (4, 8)])
def test_prompt_filling_the_context(n_prompt, expect_len):
    """InferenceEngine.cs:256-298: the first token is emitted before the context
    check, so a prompt that fills the cache still yields one token."""
    cfg = TINY_TEST.replace(context_length=12)
    ck = synth.llama_checkpoint(cfg, seed=30)
    prompt = synth.tokens(30, "prompt", n_prompt, cfg.vocab_size)
    announce(f"context fill: prompt {n_prompt} of 12")
    with HipLlamaModel(cfg, ck) as m:
        g = [int(t) for t in m.generate_greedy(prompt, 5 if n_prompt > 4 else 100)]
        h = generate(m, prompt, 5 if n_prompt > 4 else 100, GreedySampler())
    assert len(g) == expect_len and list(h) == g
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 5 if n_prompt > 4 else 100)
    compare_greedy(g, o, margins, f"context fill {n_prompt}/12", resume=(cfg, ck, list(prompt)))


def test_span_forward_matches_oracle_span():
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=22)
    toks = synth.tokens(22, "prompt", 9, cfg.vocab_size)
    announce("tiny model span forward")
    with HipLlamaModel(cfg, ck) as m:
        g = m.forward(toks, 0)
        g2 = m.forward(toks[:3], 9)  # continue the same sequence at position 9
    ora = oracle.OracleLlama(cfg, ck)
    r = ora.forward(toks, 0)
    r2 = ora.forward(toks[:3], 9)
    assert np.max(np.abs(g - r)) <= LOGIT_TOL
    assert np.max(np.abs(g2 - r2)) <= LOGIT_TOL


def test_tiny_greedy_generation_matches_oracle():
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=23)
    prompt = synth.tokens(23, "prompt", 8, cfg.vocab_size)
    announce("tiny greedy generation")
    with HipLlamaModel(cfg, ck) as m:
        g = m.generate_greedy(prompt, 32)
        # the host loop over IModel.Forward gives the same tokens as the device loop
        h = generate(m, prompt, 32, GreedySampler())
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 32)
    compare_greedy(list(g), o, margins, "tiny greedy 8+32", resume=(cfg, ck, list(prompt)))
    assert list(g) == list(h)


def test_from_gguf_matches_uploaded_checkpoint(tmp_path):
    """A GGUF file written by chatnet_amd.gguf and loaded with
    HipLlamaModel.from_gguf (InferenceEngine.LoadFromGguf's path) gives the
    same logits and greedy tokens, bit for bit, as the checkpoint uploaded
    directly, and matches the oracle."""
    from chatnet_amd import gguf
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=39, mix="q4_k_m")
    path = str(tmp_path / "tiny.gguf")
    gguf.write_llama(path, cfg, ck)
    toks = synth.tokens(39, "prompt", 10, cfg.vocab_size)
    announce("gguf load")
    with HipLlamaModel.from_gguf(path) as m:
        assert m.config == cfg.replace(rms_norm_eps=float(np.float32(cfg.rms_norm_eps)))
        g = m.forward(toks, 0).copy()
        gt = list(m.decode_greedy(16))
    with HipLlamaModel(cfg, ck) as m2:
        r = m2.forward(toks, 0).copy()
        rt = list(m2.decode_greedy(16))
    assert np.array_equal(g, r) and gt == rt
    o = oracle.OracleLlama(cfg, ck).forward(toks, 0)
    assert np.max(np.abs(g - o)) <= LOGIT_TOL


def test_context_limit_and_eos():
    cfg = TINY_TEST.replace(context_length=12)
    ck = synth.llama_checkpoint(cfg, seed=24)
    prompt = [5, 6, 7, 8]
    announce("context limit / eos")
    with HipLlamaModel(cfg, ck) as m:
        g = m.generate_greedy(prompt, 100)
        assert len(g) == 12 - 4  # InferenceEngine.cs:295-298
        cut = m.generate_greedy(prompt, 100, eos_token=int(g[3]))
        assert list(cut) == list(g[: list(g).index(g[3])])
        assert len(m.generate_greedy(prompt, 0)) == 0


def test_tinyllama_q4_0_greedy_32_steps_match_oracle():
    """TinyLlama-1.1B-shaped Q4_0: 16 seeded prompt tokens, 32 greedy steps."""
    cfg = TINYLLAMA_1B.replace(context_length=64)
    announce("tinyllama checkpoint generation")
    ck = synth.llama_checkpoint(cfg, seed=1234, mix="q4_0")
    prompt = synth.tokens(1234, "prompt", 16, cfg.vocab_size)
    announce("tinyllama greedy on gpu")
    with HipLlamaModel(cfg, ck) as m:
        g = m.generate_greedy(prompt, 32)
        logits_g = m.get_logits()
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 32)
    n = compare_greedy(list(g), o, margins, "tinyllama 16+32 (live oracle)", resume=(cfg, ck, list(prompt)))
    print(f"tinyllama: {n}/32 greedy tokens identical; min margin {min(margins):.3g}", flush=True)
    if n == 32:
        # the last decode step forwarded token 32 at position 16+31; compare its logits
        ora = oracle.OracleLlama(cfg, ck)
        seq = list(prompt) + list(o)
        r = ora.forward(seq, 0)
        assert np.max(np.abs(logits_g - r)) <= LOGIT_TOL


def test_error_paths():
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=25)
    announce("error paths")
    with HipLlamaModel(cfg) as m:
        with pytest.raises(_native.ChatnetKeyNotFound):
            m.forward([1], 0)  # nothing uploaded: KeyNotFoundException
        t = ck["blk.0.attn_q.weight"]
        with pytest.raises(_native.ChatnetSizeMismatch):
            m.upload_tensor("blk.0.attn_q.weight", t.type, t.dims, t.data[:-18])
        with pytest.raises(_native.ChatnetSizeMismatch):
            m.upload_tensor("blk.0.attn_q.weight", t.type, (cfg.dim, cfg.dim // 2), t.data[: t.data.size // 2])
        with pytest.raises(_native.ChatnetNotSupported):  # Q8_1: no MatVecMulByType branch
            m.upload_tensor("blk.0.attn_q.weight", 9, t.dims, np.zeros(cfg.dim * cfg.dim // 32 * 36, np.uint8))
        with pytest.raises(_native.ChatnetOutOfRange):  # IQ3S.Dequantize reads past an embedding row
            m.upload_tensor("token_embd.weight", _native.GGML_IQ3_S, (cfg.dim, cfg.vocab_size),
                            np.zeros(cfg.vocab_size * cfg.dim // 256 * 110, np.uint8))
        with pytest.raises(_native.ChatnetKeyNotFound):
            m.upload_tensor("blk.9.attn_q.weight", t.type, t.dims, t.data)
        for name, tt in ck.items():
            m.upload_tensor(name, tt.type, tt.dims, tt.data)
        with pytest.raises(_native.ChatnetOutOfRange):
            m.forward([1], cfg.context_length)
        with pytest.raises(_native.ChatnetOutOfRange):
            m.forward([cfg.vocab_size], 0)
        m.forward([1, 2], 0)  # still usable after errors


# -- batched spans (>= 8 tokens: MFMA GEMM projections + causal span attention) --
SPAN_SMALL = TINY_TEST.replace(dim=256, hidden_dim=512, n_heads=4, n_kv_heads=2, head_dim=64,
                               context_length=1100)


def span_case(cfg, seed, n_prompt, n_next=8, mix="q4_0", ck=None, check_batched=False):
    """A span of n_prompt tokens and a continuing span of n_next, logits
    against the oracle.  check_batched: the same prompt on the per-token
    schedule must give different bits (the batched GEMM rounds differently),
    i.e. the span really ran batched."""
    if ck is None:
        ck = synth.llama_checkpoint(cfg, seed=seed, mix=mix)
    toks = synth.tokens(seed, "prompt", n_prompt + n_next, cfg.vocab_size)
    with HipLlamaModel(cfg, ck) as m:
        g = m.forward(toks[:n_prompt], 0).copy()
        g2 = m.forward(toks[n_prompt:], n_prompt)  # a second span continuing the sequence
    if check_batched:
        import os
        os.environ["CHATNET_SPAN_BATCH"] = "0"
        try:
            with HipLlamaModel(cfg, ck) as m:
                h = m.forward(toks[:n_prompt], 0).copy()
        finally:
            del os.environ["CHATNET_SPAN_BATCH"]
        assert not np.array_equal(g, h), "the span ran on the per-token schedule"
    ora = oracle.OracleLlama(cfg, ck)
    r = ora.forward(toks[:n_prompt], 0)
    r2 = ora.forward(toks[n_prompt:], n_prompt)
    tol = LOGIT_TOL if cfg.kv_dtype == _native.KV_F32 else 2 * LOGIT_TOL
    e1, e2 = float(np.max(np.abs(g - r))), float(np.max(np.abs(g2 - r2)))
    print(f"span logits max-abs err {e1:.3g} / {e2:.3g} (logit scale {float(np.max(np.abs(r))):.3g})", flush=True)
    assert e1 <= tol and e2 <= tol


def test_span_tinyllama_layers_match_oracle():
    announce("span: tinyllama-shaped 2 layers, 24 + 8 tokens")
    span_case(TINYLLAMA_1B.replace(n_layers=2, context_length=128), 31, 24)


def test_span_llama7b_layer_matches_oracle():
    from chatnet_amd import LLAMA2_7B
    announce("span: llama-7b-shaped 1 layer, 16 + 8 tokens")
    span_case(LLAMA2_7B.replace(n_layers=1, context_length=64), 32, 16)


def test_span_fp16_kv_matches_oracle():
    announce("span: fp16 kv cache")
    span_case(SPAN_SMALL.replace(kv_dtype=_native.KV_F16, context_length=96), 33, 40)


def test_span_longer_than_batch_cap_matches_oracle_and_token_schedule(monkeypatch):
    """600 tokens run as batches of 512 + 88; logits and the greedy tokens that
    follow agree with the oracle and with the per-token schedule."""
    cfg = SPAN_SMALL
    ck = synth.llama_checkpoint(cfg, seed=34, mix="q4_0")
    toks = synth.tokens(34, "prompt", 600, cfg.vocab_size)
    announce("span: 600 tokens (two batches)")
    with HipLlamaModel(cfg, ck) as m:
        g = m.forward(toks, 0)
        gt = m.decode_greedy(16)
    monkeypatch.setenv("CHATNET_SPAN_BATCH", "0")
    announce("span: 600 tokens per-token schedule")
    with HipLlamaModel(cfg, ck) as m:
        h = m.forward(toks, 0)
    ora = oracle.OracleLlama(cfg, ck)
    r = ora.forward(toks, 0)
    assert np.max(np.abs(g - r)) <= LOGIT_TOL
    assert np.max(np.abs(h - r)) <= LOGIT_TOL
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(toks), 16)
    compare_greedy(list(gt), o, margins, "span 600 tokens, greedy 16", resume=(cfg, ck, list(toks)))


@pytest.mark.parametrize("mix", ["q4_k_m", "q5_k_m", "q8_0", "q6_k", "q4_k", "mixed_blocks", "legacy_blocks",
                                 "q3_k_m", "q2_k", "iq_a", "iq_b"])
def test_span_block_type_mixes_match_oracle(mix):
    """Spans of models with other block types run batched on packed weights
    (every matrix re-encoded once, types mixed freely, ffn_gate and ffn_up of
    different types in mixed_blocks)."""
    announce(f"span: mix {mix}, 40 + 8 tokens")
    span_case(SPAN_SMALL.replace(context_length=96), 39, 40, mix=mix, check_batched=True)


@pytest.mark.parametrize("mix", ["f16", "f32", "float_mix"])
def test_span_float_weight_mixes_match_oracle(mix):
    """Spans of models with F16 or F32 projections run batched: F16 rows meet
    x's fp16 hi + lo planes directly (two products per step, exact weights),
    F32 rows are split into fp16 hi + lo as they are read (three products);
    float_mix runs F16 attention, Q4_0 gate/up and an F32 down projection in
    one span, each GEMM on its own weight format."""
    announce(f"span: float mix {mix}, 40 + 8 tokens")
    span_case(SPAN_SMALL.replace(context_length=96), 41, 40, mix=mix, check_batched=True)


def test_span_f16_llama7b_layer_matches_oracle():
    """A 7B-shaped layer with F16 projections as a 16-token span."""
    from chatnet_amd import LLAMA2_7B
    announce("span: llama-7b-shaped f16 layer, 16 + 8 tokens")
    span_case(LLAMA2_7B.replace(n_layers=1, context_length=64), 42, 16, mix="f16", check_batched=True)


def test_span_q4_k_m_llama7b_layer_matches_oracle():
    """A 7B-shaped Q4_K_M layer (Q4_K attention and gate/up, Q6_K down, Q6_K
    LM head) as a 16-token span."""
    from chatnet_amd import LLAMA2_7B
    announce("span: llama-7b-shaped q4_k_m layer, 16 + 8 tokens")
    span_case(LLAMA2_7B.replace(n_layers=1, context_length=64), 40, 16, mix="q4_k_m", check_batched=True)


def test_span_qwen2_0_5b_layer_matches_oracle():
    """Qwen2-0.5B-shaped layer (14 query heads over 2 kv heads: kv_mul 7, 9
    tokens x 7 heads per span-attention workgroup, one padding row) with Q8_0
    weights, biases and the tied Q8_0 embedding, as a 40-token span."""
    from chatnet_amd import QWEN2_0_5B
    cfg = QWEN2_0_5B.replace(n_layers=1, context_length=64)
    ck = synth.llama_checkpoint(cfg, seed=47, mix="q8_0", with_output=False, embedding=_native.GGML_Q8_0)
    announce("span: qwen2-0.5b layer, 40 + 8 tokens")
    span_case(cfg, 47, 40, ck=ck, check_batched=True)


@pytest.mark.parametrize("head_dim,n_heads,n_kv,kv", [
    (64, 8, 2, _native.KV_F32),    # kv_mul 4: 16 tokens per workgroup
    (64, 16, 1, _native.KV_F32),   # kv_mul 16: 4 tokens per workgroup
    (128, 4, 4, _native.KV_F32),   # head_dim 128 without grouping
    (128, 8, 2, _native.KV_F16),   # head_dim 128, kv_mul 4, fp16 cache
    (64, 14, 2, _native.KV_F32),   # kv_mul 7: 9 tokens per workgroup, one padding row
    (128, 12, 4, _native.KV_F16),  # kv_mul 3: 21 tokens per workgroup, one padding row
    (64, 10, 2, _native.KV_F32),   # kv_mul 5: 12 tokens per workgroup, four padding rows
])
def test_span_attention_layouts_match_oracle(head_dim, n_heads, n_kv, kv):
    """Causal span attention across GQA ratios and head sizes: a 150-token
    span (three chunks of 64 positions, ragged last workgroup) and a 37-token
    span continuing at position 150."""
    cfg = TINY_TEST.replace(dim=head_dim * n_heads, hidden_dim=512, n_heads=n_heads, n_kv_heads=n_kv,
                            head_dim=head_dim, context_length=256, kv_dtype=kv)
    announce(f"span attention layout hd={head_dim} heads={n_heads} kv={n_kv} kvtype={kv}")
    span_case(cfg, 38, 150, n_next=37)


def test_long_context_decode_attention_matches_oracle():
    """2000-token prompt, then greedy decode: the decode attention runs with up
    to 64 position splits (63 active at 2000 positions, merged in rounds)."""
    cfg = SPAN_SMALL.replace(context_length=2100)
    ck = synth.llama_checkpoint(cfg, seed=35, mix="q4_0")
    toks = synth.tokens(35, "prompt", 2000, cfg.vocab_size)
    announce("decode attention: 2000-token context, 64 splits")
    with HipLlamaModel(cfg, ck) as m:
        m.forward(toks, 0)
        gt = m.decode_greedy(8)
        logits_g = m.get_logits()
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(toks), 8)
    n = compare_greedy(list(gt), o, margins, "2000-token context, greedy 8", resume=(cfg, ck, list(toks)))
    if n == 8:
        # the 8th decode step forwarded the 8th token at position 2007
        r = oracle.OracleLlama(cfg, ck).forward(list(toks) + list(o), 0)
        assert np.max(np.abs(logits_g - r)) <= LOGIT_TOL


# -- decode attention layouts: the four waves of a workgroup split the query
# heads of a kv head (kv_mul >= 4: 1, 2 or 4 heads per wave), or split the
# positions and fold through LDS (kv_mul 1, 2); buckets of one chunk write the
# output directly, larger ones merge chunks.  The prompt runs as one span and
# the decode crosses the 64 and 128 position buckets.
@pytest.mark.parametrize("head_dim,n_heads,n_kv,kv", [
    (128, 4, 4, _native.KV_F32),   # kv_mul 1: positions over four waves
    (128, 4, 2, _native.KV_F32),   # kv_mul 2: two head waves x two position waves
    (64, 8, 2, _native.KV_F32),    # kv_mul 4: one head per wave
    (64, 16, 1, _native.KV_F32),   # kv_mul 16: four heads per wave
    (32, 8, 1, _native.KV_F32),    # kv_mul 8, head_dim 32
    (64, 14, 2, _native.KV_F32),   # kv_mul 7 (Qwen2-0.5B): a ragged second pass of heads
    (128, 4, 4, _native.KV_F16),
])
def test_decode_attention_layouts_match_oracle(head_dim, n_heads, n_kv, kv):
    cfg = TINY_TEST.replace(dim=head_dim * n_heads, hidden_dim=512, n_heads=n_heads, n_kv_heads=n_kv,
                            head_dim=head_dim, context_length=300, kv_dtype=kv)
    ck = synth.llama_checkpoint(cfg, seed=36, mix="q4_0")
    prompt = synth.tokens(36, "prompt", 60, cfg.vocab_size)
    announce(f"decode attention layout hd={head_dim} heads={n_heads} kv={n_kv} kvtype={kv}")
    with HipLlamaModel(cfg, ck) as m:
        m.forward(prompt, 0)
        g = m.decode_greedy(80)
        logits_g = m.get_logits()
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 80)
    n = compare_greedy(list(g), o, margins, f"decode attention hd={head_dim} heads={n_heads} kv={n_kv} kvtype={kv}", resume=(cfg, ck, list(prompt)))
    if n == 80:
        r = oracle.OracleLlama(cfg, ck).forward(list(prompt) + list(o), 0)
        tol = LOGIT_TOL if kv == _native.KV_F32 else 2 * LOGIT_TOL
        assert np.max(np.abs(logits_g - r)) <= tol


def test_qwen2_0_5b_layer_decode_matches_oracle():
    """Qwen2-0.5B-shaped layer (dim 896, 14 heads over 2 kv heads, QKV biases,
    split-half RoPE at base 1e6) with Q8_0 weights and the tied Q8_0 embedding
    as a 151936-row LM head."""
    from chatnet_amd import QWEN2_0_5B
    cfg = QWEN2_0_5B.replace(n_layers=1, context_length=64)
    ck = synth.llama_checkpoint(cfg, seed=46, mix="q8_0", with_output=False, embedding=_native.GGML_Q8_0)
    prompt = synth.tokens(46, "prompt", 8, cfg.vocab_size)
    announce("qwen2-0.5b layer decode")
    with HipLlamaModel(cfg, ck) as m:
        m.forward(prompt, 0)
        g = m.decode_greedy(8)
        lg = m.get_logits()
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 8)
    n = compare_greedy(list(g), o, margins, "qwen2-0.5b layer, greedy 8", resume=(cfg, ck, list(prompt)))
    if n == 8:
        r = oracle.OracleLlama(cfg, ck).forward(list(prompt) + list(o), 0)
        assert np.max(np.abs(lg - r)) <= LOGIT_TOL


def test_llama7b_layer_decode_matches_oracle():
    """7B-shaped layer decode: QKV 12288x4096, O, gate/up 22016x4096, down
    4096x11008 and the LM head at their real shapes; tokens and logits match
    the oracle."""
    from chatnet_amd import LLAMA2_7B
    cfg = LLAMA2_7B.replace(n_layers=1, context_length=64)
    ck = synth.llama_checkpoint(cfg, seed=37, mix="q4_0")
    prompt = synth.tokens(37, "prompt", 8, cfg.vocab_size)
    announce("7b layer decode")
    with HipLlamaModel(cfg, ck) as m:
        m.forward(prompt, 0)
        g = m.decode_greedy(8)
        lg = m.get_logits()
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 8)
    n = compare_greedy(list(g), o, margins, "7b layer, greedy 8", resume=(cfg, ck, list(prompt)))
    if n == 8:
        r = oracle.OracleLlama(cfg, ck).forward(list(prompt) + list(o), 0)
        assert np.max(np.abs(lg - r)) <= LOGIT_TOL


@pytest.mark.parametrize("mix", ["q4_0", "q5_k_m"])
def test_wide_rows_in_paired_epilogues_match_oracle(mix):
    """dim 8448: the QKV and gate/up GEMVs read rows of 8192 < K <= 12288,
    where the store and add launches run one row per lane; the RoPE and SwiGLU
    epilogues take a lane's rows in pairs and keep two rows per lane."""
    cfg = TINY_TEST.replace(dim=8448, hidden_dim=512, n_layers=1, n_heads=66, n_kv_heads=66, head_dim=128,
                            context_length=32)
    ck = synth.llama_checkpoint(cfg, seed=38, mix=mix)
    prompt = synth.tokens(38, "prompt", 4, cfg.vocab_size)
    announce(f"wide rows mix={mix}")
    with HipLlamaModel(cfg, ck) as m:
        m.forward(prompt, 0)
        g = m.decode_greedy(4)
        lg = m.get_logits()
    o, margins = oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt), 4)
    n = compare_greedy(list(g), o, margins, f"wide rows mix={mix}, greedy 4", resume=(cfg, ck, list(prompt)))
    if n == 4:
        r = oracle.OracleLlama(cfg, ck).forward(list(prompt) + list(o), 0)
        assert np.max(np.abs(lg - r)) <= LOGIT_TOL
