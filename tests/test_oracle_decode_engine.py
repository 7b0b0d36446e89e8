"""Pins oracle/decode.py's composition of the decode step to the reference's
own engine: UnifiedEngine::forward_token (asdsl/kernels/native/unified_engine.cpp:1339-1688),
compiled unchanged into oracle/_ref/_native_unified.so by oracle/Makefile and
constructed through its pybind11 constructor (unified_engine.cpp:2272-2445,
2662-2675), on two synthetic profiles:

* C0 (every projection and the lm_head preq2 g32, fused activation
  quantization);
* C0.1 (ASDSL_C01=1: qkv/o preq2 g32, gate_up/down as 66-byte Q4_128
  blocks run by gemv_q4_128_preq_avx2 after a group-128 activation
  quantization, unified_engine.cpp:1532-1538,1592-1598; the lm_head is an
  fp16 output projection the engine quantizes to Q4_128 at load,
  unified_engine.cpp:413-461, run after rmsnorm_quantize_f32 at group 128,
  unified_engine.cpp:1651-1653).  The oracle runs the same weights as
  preq2-g128 (the lossless Q4_128 repack) and the engine's lm_head rule
  restated (oracle.decode.quantize_lm_head_q4_128).

The engine keeps K/V as int8 per 64 dims (set_kv_cache, 859-920), so the
oracle runs its int8 cache.  What this pins beyond the GEMV pins: which norm
weight feeds which GEMV, the residual order, RoPE on q and k, the int8 cache
rule, GQA head mapping, online-softmax attention across 64-position tiles,
SwiGLU with the polynomial exp, the final norm and the lm_head, and for C0.1
the group-128 activation quantization of the MLP and lm_head inputs and the
engine's lm_head quantizer.

Bars, per case: C0 every step within 1e-2 relative L2 of the engine's
logits; C0.1 median below 1.5e-2 and every step below 2e-2; the same greedy
token at >= 95 % of the steps; pooled over the one-layer cases of either
profile, median <= 1e-5.  Measured here (max relative L2 per case): C0
3.9e-3, 3.4e-3, 1.2e-3, 4.2e-3, 7.8e-3 with 98.6 % token agreement in the
worst case (1, 4, 4); C0.1 1.9e-3, 5.0e-3, 9.4e-3, 9.6e-3 with every token
agreeing.  The one-layer medians are at float32 rounding (2e-7 to 3e-7);
the maxima are one-level int8 flips of a GEMV input (the two sides sum in
different orders), carried forward by the K/V rows they write, so the
multi-layer medians sit at 6e-3 (C0 four layers, C0.1 two layers) to 9e-3
(C0.1 four layers).  No restatement that is not bit-exact holds 1e-3 at
depth.  Planted composition mistakes (RoPE sign, swapped norm weights) miss
the bars (test_c01_bars_fail_planted_mistakes).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from asdsl.quantization import synthetic as syn
from conftest import rel_l2
from oracle import decode as od

REF = oracle.reference_available("_native_unified")
pytestmark = pytest.mark.skipif(not REF, reason="oracle/_ref not built (reference tree not mounted)")


def _model(n_layers, n_heads, n_kv, ffn, vocab, max_seq, seed, fatrelu=0.0):
    from asdsl.engine import DecodeConfig, rope_tables

    hd = 128
    cfg = DecodeConfig(hidden=n_heads * hd, ffn=ffn, vocab=vocab, n_layers=n_layers, n_heads=n_heads,
                       n_kv_heads=n_kv, head_dim=hd, rotary_dim=96, max_seq=max_seq, gs_attn=32, gs_ffn=32,
                       gs_lm=32)
    rng = np.random.default_rng(seed)
    layers, ref_layers = [], {}
    shapes = {"qkv": ("qkv_proj", cfg.qkv_dim, cfg.hidden), "o": ("o_proj", cfg.hidden, cfg.hidden),
              "gu": ("gate_up_proj", 2 * ffn, cfg.hidden), "down": ("down_proj", cfg.hidden, ffn)}
    for li in range(n_layers):
        L, R = {}, {}
        for n, (name, M, K) in shapes.items():
            w = syn.gaussian_weights(M, K, seed * 1000 + li * 10 + len(name))
            meta, quant = syn.preq2(w, 32)
            L[n] = (meta, quant)
            R[name] = syn.preq_blocks(w)  # the engine's preq blocks (unused while preq2 is bound)
            R[name + "_meta"], R[name + "_quant"] = meta, quant
        L["rms_att"] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        L["rms_ffn"] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        R["rms_att"], R["rms_ffn"] = L["rms_att"], L["rms_ffn"]
        if fatrelu > 0:
            R["fatrelu_threshold"] = float(fatrelu)
        layers.append(L)
        ref_layers[li] = R
    embed = rng.standard_normal((vocab, cfg.hidden)).astype(np.float16)
    rms_out = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    lm_meta, lm_quant = syn.preq2(syn.gaussian_weights(vocab, cfg.hidden, seed + 7), 32)
    cos, sin = rope_tables(max_seq, cfg.rotary_dim)
    model = {"cfg": cfg, "layers": layers, "embed": embed, "rms_out": rms_out, "lm_meta": lm_meta,
             "lm_quant": lm_quant, "rope_cos": cos, "rope_sin": sin, "fatrelu_threshold": fatrelu}

    ue = oracle.load_reference("_native_unified")
    ec = ue.EngineConfig()
    ec.num_layers, ec.hidden_size, ec.num_heads, ec.num_kv_heads = n_layers, cfg.hidden, n_heads, n_kv
    ec.head_dim, ec.intermediate_size, ec.vocab_size, ec.rms_norm_eps = hd, ffn, vocab, cfg.rms_eps
    ec.group_size, ec.lm_head_group_size, ec.max_seq_len, ec.rotary_dim, ec.weight_format = 32, 0, max_seq, 96, 0
    engine = ue.UnifiedEngine(ec, embed, rms_out, None, cos, sin, ref_layers, lm_meta, lm_quant)
    return model, engine


def _q8_caches(cfg):
    shape = (cfg.n_kv_heads, cfg.max_seq, cfg.head_dim)
    mk = lambda: (np.zeros(shape, np.int8), np.ones(shape[:2] + (cfg.head_dim // 64,), np.float32))  # noqa: E731
    return [mk() for _ in range(cfg.n_layers)], [mk() for _ in range(cfg.n_layers)]


# (layers, query heads, KV heads, steps, FATReLU threshold, seed)
CASES = [(1, 6, 2, 70, 0.0, 1), (1, 4, 4, 70, 0.0, 2), (1, 6, 2, 70, 0.05, 3), (2, 6, 2, 40, 0.0, 5),
         (4, 6, 2, 20, 0.0, 7)]


@pytest.fixture(scope="module")
def runs():
    """Every case: greedy steps from position 0 (70 steps cross the engine's
    64-position attention tiles), hidden heads*128, FFN 2048, vocab 2048;
    both sides get the oracle's token at every step.  Per step: the relative
    L2 of the engine's logits against the oracle's, and whether the greedy
    tokens agree."""
    out = {}
    for case in CASES:
        n_layers, n_heads, n_kv, steps, fatrelu, seed = case
        model, engine = _model(n_layers, n_heads, n_kv, 2048, 2048, 96, seed=seed, fatrelu=fatrelu)
        kc, vc = _q8_caches(model["cfg"])
        tok, errs, agree = 5, [], []
        for pos in range(steps):
            want, nxt = od.decode_step(model, tok, pos, kc, vc)
            got = np.array(engine.forward_token(tok, pos), copy=True)
            errs.append(rel_l2(got, want))
            agree.append(int(np.argmax(got)) == nxt)
            tok = nxt
        assert engine.get_kv_seq_len() == steps
        out[case] = (np.array(errs), np.array(agree))
    return out


@pytest.mark.parametrize("case", CASES)
def test_oracle_decode_matches_reference_engine(runs, case):
    """Every step within 1e-2 and the greedy tokens agree at >= 95 % of the
    steps.  The two sides sum in different orders, so a GEMV input element
    sitting at an int8 rounding boundary can round to neighbouring levels
    (one level of one element moves that GEMV's output by ~1e-3), and a
    flipped K/V row stays in the cache for the later steps: two correct
    restatements differ by up to ~8e-3 (measured here between the oracle
    and the same oracle summing in float32).  A wrong composition (a norm
    weight, a residual, a head mapping, a RoPE sign) moves every step by
    far more."""
    errs, agree = runs[case]
    assert errs.max() < 1e-2, errs
    assert agree.mean() >= 0.95, agree


def test_single_layer_steps_are_exact_but_for_rounding_flips(runs):
    """Pooled over the one-layer cases, most steps agree to float32 rounding
    (median <= 1e-5): the composition of a layer, the int8 cache rule and the
    attention tiles are the reference's, not just close to them."""
    errs = np.concatenate([runs[c][0] for c in CASES if c[0] == 1])
    assert np.median(errs) <= 1e-5, np.sort(errs)


# ------------------------------------------------------------------ C0.1
def tie_rows_matrix(vocab: int, hidden: int, rng) -> np.ndarray:
    """fp16 [vocab][hidden] ~ N(0, 1) whose every fourth row holds, in each
    128-group, one element of +-7 and others at +-k.5 (k < 7): the group's
    amax is 7, so the lm_head quantizer's inverse scale is exactly 1 and
    those elements are ties, which round half away from zero in the engine
    (std::round) and half to even in repack_q4_128.py."""
    e = rng.standard_normal((vocab, hidden)).astype(np.float32)
    tie_rows = np.arange(0, vocab, 4)
    t = (rng.integers(0, 7, (tie_rows.size, hidden)) + 0.5) * rng.choice([-1.0, 1.0], (tie_rows.size, hidden))
    t[:, ::128] = 7.0 * rng.choice([-1.0, 1.0], (tie_rows.size, hidden // 128))
    e[tie_rows] = t
    return e.astype(np.float16)


def model_c01(n_layers, n_heads, n_kv, ffn, vocab, max_seq, seed):
    """C0.1 weights for both sides.  Oracle: qkv/o preq2 g32, gate_up/down/
    lm_head preq2-g128 (repacked from the Q4_128 blocks), int8 KV.  Engine:
    the same qkv/o preq2 arrays, gate_up/down Q4_128 blocks, an fp16 output
    projection it quantizes at load (lm_head_group_size 128).  The output
    projection is drawn apart from the embedding: with random weights a
    tied one makes every greedy step repeat its input token."""
    from asdsl.engine import DecodeConfig, rope_tables
    from asdsl.quantization.repack import repack_q4_128_blocks_to_preq2

    hd = 128
    cfg = DecodeConfig(hidden=n_heads * hd, ffn=ffn, vocab=vocab, n_layers=n_layers, n_heads=n_heads,
                       n_kv_heads=n_kv, head_dim=hd, rotary_dim=96, max_seq=max_seq, gs_attn=32, gs_ffn=128,
                       gs_lm=128, kv_format="int8")
    rng = np.random.default_rng(seed)
    layers, ref_layers = [], {}
    shapes = {"qkv": ("qkv_proj", cfg.qkv_dim, cfg.hidden), "o": ("o_proj", cfg.hidden, cfg.hidden),
              "gu": ("gate_up_proj", 2 * ffn, cfg.hidden), "down": ("down_proj", cfg.hidden, ffn)}
    for li in range(n_layers):
        L, R = {}, {}
        for n, (name, M, K) in shapes.items():
            w = syn.gaussian_weights(M, K, seed * 1000 + li * 10 + len(name))
            if n in ("qkv", "o"):
                L[n] = syn.preq2(w, 32)
                R[name + "_meta"], R[name + "_quant"] = L[n]
            else:
                blocks = syn.q4_128_blocks(w)
                L[n] = repack_q4_128_blocks_to_preq2(blocks, M, K)
                R[name + "_g128"] = blocks
            R[name] = np.zeros(M * K // 32 * 20, np.uint8)  # preq blocks: bound, never read in this profile
        L["rms_att"] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        L["rms_ffn"] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        R["rms_att"], R["rms_ffn"] = L["rms_att"], L["rms_ffn"]
        layers.append(L)
        ref_layers[li] = R
    embed = rng.standard_normal((vocab, cfg.hidden)).astype(np.float16)
    lm_w = tie_rows_matrix(vocab, cfg.hidden, rng)
    rms_out = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    lm_blocks = od.quantize_lm_head_q4_128(lm_w.astype(np.float32))
    lm_meta, lm_quant = repack_q4_128_blocks_to_preq2(lm_blocks, vocab, cfg.hidden)
    cos, sin = rope_tables(max_seq, cfg.rotary_dim)
    model = {"cfg": cfg, "layers": layers, "embed": embed, "rms_out": rms_out, "lm_meta": lm_meta,
             "lm_quant": lm_quant, "rope_cos": cos, "rope_sin": sin, "lm_w": lm_w}

    ue = oracle.load_reference("_native_unified")
    ec = ue.EngineConfig()
    ec.num_layers, ec.hidden_size, ec.num_heads, ec.num_kv_heads = n_layers, cfg.hidden, n_heads, n_kv
    ec.head_dim, ec.intermediate_size, ec.vocab_size, ec.rms_norm_eps = hd, ffn, vocab, cfg.rms_eps
    ec.group_size, ec.lm_head_group_size, ec.max_seq_len, ec.rotary_dim, ec.weight_format = 32, 128, max_seq, 96, 0
    engine = ue.UnifiedEngine(ec, embed, rms_out, lm_w, cos, sin, ref_layers)
    return model, engine, lm_blocks


# (layers, query heads, KV heads, steps, seed)
CASES_C01 = [(1, 6, 2, 70, 11), (1, 4, 4, 70, 12), (2, 6, 2, 40, 13), (4, 6, 2, 20, 14)]


@pytest.fixture(scope="module")
def runs_c01():
    """As `runs`, on the C0.1 profile with ASDSL_C01=1 set while the engine
    steps (the engine reads it at every call).  Also keeps, per case, the
    first step's final stream and both sides' first logits."""
    import os

    prev = os.environ.get("ASDSL_C01")
    os.environ["ASDSL_C01"] = "1"
    out = {}
    try:
        for case in CASES_C01:
            n_layers, n_heads, n_kv, steps, seed = case
            model, engine, lm_blocks = model_c01(n_layers, n_heads, n_kv, 2048, 2048, 96, seed)
            kc, vc = _q8_caches(model["cfg"])
            tok, errs, agree, first = 5, [], [], None
            for pos in range(steps):
                trace = [] if pos == 0 else None
                want, nxt = od.decode_step(model, tok, pos, kc, vc, trace=trace)
                got = np.array(engine.forward_token(tok, pos), copy=True)
                if pos == 0:
                    first = {"h": trace[-1]["h"], "want": want, "got": got}
                errs.append(rel_l2(got, want))
                agree.append(int(np.argmax(got)) == nxt)
                tok = nxt
            out[case] = (np.array(errs), np.array(agree), model, first)
    finally:
        if prev is None:
            os.environ.pop("ASDSL_C01", None)
        else:
            os.environ["ASDSL_C01"] = prev
    return out


# C0.1 bars: median < 1.5e-2 and max < 2e-2 relative L2 per case, greedy
# tokens agree at >= 95 % of the steps.  Measured here: max 1.9e-3 / 5.0e-3
# (one layer, medians 2e-7), 9.4e-3 (two layers, median 5.9e-3), 9.6e-3
# (four layers, median 8.7e-3): a one-level flip at an early step stays in
# the K/V rows it wrote.  The planted mistakes of
# test_c01_bars_fail_planted_mistakes land at medians of 2.9e-2 and above.
C01_MEDIAN_BAR, C01_MAX_BAR = 1.5e-2, 2e-2


@pytest.mark.parametrize("case", CASES_C01)
def test_oracle_decode_matches_reference_engine_c01(runs_c01, case):
    errs, agree = runs_c01[case][:2]
    assert np.median(errs) < C01_MEDIAN_BAR and errs.max() < C01_MAX_BAR, errs
    assert agree.mean() >= 0.95, agree


def test_c01_bars_fail_planted_mistakes():
    """The C0.1 bars have power: on the two-layer case the oracle with a
    planted composition mistake -- RoPE's rotation sign, or the two norm
    weights of each layer swapped -- misses the median bar against the
    engine, while the correct composition meets it (above)."""
    import os

    n_layers, n_heads, n_kv, _, seed = CASES_C01[2]

    def rope_sign(m):
        m["rope_sin"] = -m["rope_sin"]

    def swap_norms(m):
        for L in m["layers"]:
            L["rms_att"], L["rms_ffn"] = L["rms_ffn"], L["rms_att"]

    prev = os.environ.get("ASDSL_C01")
    os.environ["ASDSL_C01"] = "1"
    try:
        for plant in (rope_sign, swap_norms):
            model, engine, _ = model_c01(n_layers, n_heads, n_kv, 2048, 2048, 96, seed)
            plant(model)
            kc, vc = _q8_caches(model["cfg"])
            tok, errs = 5, []
            for pos in range(12):
                want, _ = od.decode_step(model, tok, pos, kc, vc)
                got = np.array(engine.forward_token(tok, pos), copy=True)
                errs.append(rel_l2(got, want))
                tok = int(np.argmax(got))
            assert np.median(errs) > C01_MEDIAN_BAR, (plant.__name__, errs)
    finally:
        if prev is None:
            os.environ.pop("ASDSL_C01", None)
        else:
            os.environ["ASDSL_C01"] = prev


def test_single_layer_steps_c01_exact_but_for_rounding_flips(runs_c01):
    """Pooled over the one-layer C0.1 cases the median step agrees to float32
    rounding (median <= 1e-5): the group-128 quantizations, the Q4_128
    GEMVs (as preq2-g128) and the lm_head quantizer are the engine's."""
    errs = np.concatenate([runs_c01[c][0] for c in CASES_C01 if c[0] == 1])
    assert np.median(errs) <= 1e-5, np.sort(errs)


def test_lm_head_quantizer_is_the_engines(runs_c01):
    """The engine's lm_head quantizer, not repack_q4_128.py's: on the first
    step of the one-layer case the oracle's logits with
    quantize_lm_head_q4_128 match the engine's to float32 rounding, while
    the same logits with the tie rows rounded half to even (the repack
    quantizer) differ by far more.  The tie rows make the two rules differ."""
    from asdsl.quantization.repack import repack_q4_128_blocks_to_preq2

    case = CASES_C01[0]
    model, first = runs_c01[case][2], runs_c01[case][3]
    c = model["cfg"]
    assert rel_l2(first["got"], first["want"]) < 1e-5
    alt = dict(model)
    alt["lm_meta"], alt["lm_quant"] = repack_q4_128_blocks_to_preq2(
        syn.q4_128_blocks(model["lm_w"].astype(np.float32)), c.vocab, c.hidden)
    rne = od.lm_head_forward(alt, first["h"])
    assert rel_l2(rne, first["got"]) > 1e-3
    # the two quantizers agree except at ties
    a = od.quantize_lm_head_q4_128(model["lm_w"][1::4].astype(np.float32))
    b = syn.q4_128_blocks(model["lm_w"][1::4].astype(np.float32))
    assert np.mean(a != b) < 1e-3


def test_kv_q8_rule_known_blocks():
    """set_kv_cache's int8 rule on hand-made blocks: +-amax -> +-127 with
    scale amax*(1/127); a zero block keeps scale 1e-12 and zeros; halves
    round to even; every value within half a step of the original."""
    x = np.zeros((3, 128), np.float32)
    x[0, :64] = np.linspace(-2.0, 2.0, 64, dtype=np.float32)
    x[0, 64:] = 0.0
    x[1, :] = np.float32(1.0)
    x[1, 5] = np.float32(-1.0)
    x[2, :64] = np.float32(127.0)
    x[2, 1] = np.float32(0.5)
    x[2, 2] = np.float32(1.5)
    x[2, 3] = np.float32(-2.5)
    x[2, 64:] = np.random.default_rng(1).standard_normal(64).astype(np.float32)
    q, s = od.kv_quantize_q8(x)
    assert q[0, 0] == -127 and q[0, 63] == 127
    assert s[0, 0] == np.float32(np.float32(2.0) * np.float32(1.0 / 127.0))
    assert s[0, 1] == np.float32(1e-12) and np.all(q[0, 64:] == 0)
    assert np.all(q[1, :] == np.where(np.arange(128) == 5, -127, 127))
    # scale 127 * (1/127) rounds to 1.0: 0.5 -> 0 (even), 1.5 -> 2, -2.5 -> -2
    assert s[2, 0] == np.float32(1.0) and q[2, 1] == 0 and q[2, 2] == 2 and q[2, 3] == -2
    deq = od.kv_dequant_q8(q, s)
    assert np.all(np.abs(deq - x) <= 0.5 * np.repeat(s, 64, axis=1) * (1 + 1e-6))


def test_lm_head_g32_quantizer_is_the_engines():
    """At lm_head_group_size 32 the engine quantizes an fp16 output
    projection itself (unified_engine.cpp:320-398: symmetric levels in preq
    blocks with zero 8.0, copied into its preq2 lm_head).  The preq2 lm_head
    it exports (export_lm_head_preq2) equals the oracle's restatement
    (quantize_lm_head_preq_g32, repacked) byte for byte, tie rows included,
    and none of its tie nibbles is the round-half-even one."""
    import torch

    from asdsl.quantization.repack import repack_preq_blocks_to_preq2
    from decode_c01 import tie_rows_torch

    n_layers, n_heads, n_kv, vocab = 1, 6, 2, 2048
    model, _ = _model(n_layers, n_heads, n_kv, 2048, vocab, 96, seed=21)
    c = model["cfg"]
    lm_w = tie_rows_torch(vocab, c.hidden, torch.Generator().manual_seed(21), "cpu").numpy()
    ue = oracle.load_reference("_native_unified")
    ec = ue.EngineConfig()
    ec.num_layers, ec.hidden_size, ec.num_heads, ec.num_kv_heads = n_layers, c.hidden, n_heads, n_kv
    ec.head_dim, ec.intermediate_size, ec.vocab_size, ec.rms_norm_eps = 128, 2048, vocab, c.rms_eps
    ec.group_size, ec.lm_head_group_size, ec.max_seq_len, ec.rotary_dim, ec.weight_format = 32, 32, 96, 96, 0
    ref_layers = {}
    for li, L in enumerate(model["layers"]):
        R = {"rms_att": L["rms_att"], "rms_ffn": L["rms_ffn"]}
        for n, name in (("qkv", "qkv_proj"), ("o", "o_proj"), ("gu", "gate_up_proj"), ("down", "down_proj")):
            R[name + "_meta"], R[name + "_quant"] = L[n]
            R[name] = np.zeros(len(L[n][0]) // 4 * 20, np.uint8)
        ref_layers[li] = R
    engine = ue.UnifiedEngine(ec, model["embed"], model["rms_out"], lm_w, model["rope_cos"], model["rope_sin"],
                              ref_layers)
    meta, quant = engine.export_lm_head_preq2()
    blocks = od.quantize_lm_head_preq_g32(lm_w.astype(np.float32))
    want = repack_preq_blocks_to_preq2(blocks, vocab, c.hidden, 32)
    assert np.array_equal(meta, np.ravel(want[0])) and np.array_equal(quant, np.ravel(want[1]))
    w = lm_w[0::4].astype(np.float32).reshape(-1, 32)  # tie rows: amax 7 in the group of each +-7
    v = w * (np.float32(7.0) / np.abs(w).max(axis=1, keepdims=True))
    ties = np.abs(v - np.trunc(v)) == 0.5
    b = blocks.reshape(vocab, -1, 20)[0::4].reshape(-1, 20)[:, 4:]
    lv = np.empty((b.shape[0], 32), np.int64)
    lv[:, 0::2], lv[:, 1::2] = b & 0xF, b >> 4
    assert ties.sum() > 1000 and np.all(lv[ties] - 8 == (np.trunc(v) + np.sign(v))[ties])


def test_factored_norm_form_is_the_same_map_up_to_rounding():
    """The oracle's factored norm form (the GEMV quantizes x * w and scales
    its outputs by 1/rms) computes the same step as the reference order up
    to int8 rounding flips: with the activation scale's 1/rms factored out
    the two forms quantize the same vector to the same levels except where
    a value sits on a rounding boundary.  The norm factor is 1/rms; a step's
    logits agree within 5e-3 (one int8 level flip moves a 2-layer model's
    logits by ~3e-3) and their median within 1e-5 (measured: 1.1e-7 to
    1.5e-7, no flips in these four steps)."""
    from oracle import decode as od

    rng = np.random.default_rng(3)
    x = rng.standard_normal(3072).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(3072)).astype(np.float32)
    xw, inv = od.rmsnorm_factored(x, w, 1e-5)
    ref = od.rmsnorm(x, w, 1e-5)
    assert np.array_equal(xw, (x * w).astype(np.float32))
    assert abs(float(inv) * np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) - 1) < 1e-6
    assert rel_l2(xw * inv, ref) < 1e-6

    model, _, _ = model_c01(2, 8, 2, 1024, 1024, 64, seed=9)
    fmodel = dict(model, factored_norm=True)
    shape = (2, 64, model["cfg"].head_dim)
    caches = [[np.zeros(shape, np.float16) for _ in range(2)] for _ in range(4)]
    errs = []
    for pos, t in enumerate([5, 77, 300, 12]):
        a, _ = od.decode_step(model, t, pos, caches[0], caches[1])
        b, _ = od.decode_step(fmodel, t, pos, caches[2], caches[3])
        errs.append(rel_l2(b, a))
    assert max(errs) < 5e-3 and np.median(errs) < 1e-5, errs
