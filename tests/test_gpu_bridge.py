"""The reference bridge's entry points on a weight store
(asdsl.inference.unified_bridge): build_unified_engine from reference-format
blocks (preq Q4_32 for every projection, Q4_128 for gate_up/down under
ASDSL_C01, the tied embedding as the lm_head), cpp_generate against serial
greedy decoding, unified_forward_token against the oracle's decode step, and
cpp_generate's stop rule (the stop token is returned, then generation ends:
UnifiedEngine::generate, unified_engine.cpp:1736-1756)."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from asdsl.quantization import synthetic as syn
from conftest import rel_l2

pytestmark = pytest.mark.gpu

PROMPT = [11, 523, 97, 1800, 42, 7, 1333, 64]


def _store(seed: int):
    import torch
    from asdsl.engine import DecodeConfig

    cfg = DecodeConfig(hidden=768, ffn=2048, vocab=2048, n_layers=2, n_heads=6, n_kv_heads=2, max_seq=512)
    rng = np.random.default_rng(seed)
    shapes = {"qkv_proj": (cfg.qkv_dim, cfg.hidden), "o_proj": (cfg.hidden, cfg.hidden),
              "gate_up_proj": (2 * cfg.ffn, cfg.hidden), "down_proj": (cfg.hidden, cfg.ffn)}
    blocks, g128, norms = {}, {}, {}
    for li in range(cfg.n_layers):
        for name, (M, K) in shapes.items():
            w = syn.gaussian_weights(M, K, seed * 100 + li * 10 + len(name))
            blocks[(li, name)] = syn.preq_blocks(w)
            if name in ("gate_up_proj", "down_proj"):
                g128[(li, name)] = syn.q4_128_blocks(w)
        for name in ("input_layernorm", "post_attention_layernorm"):
            norms[(li, name)] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    return SimpleNamespace(decode_config=cfg, group_size=32, _preq_blocks_np=blocks, _preq_gs128_np=g128,
                           _norm_np=norms, lm_head=None,
                           embed_f16=torch.from_numpy(rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float16)),
                           final_norm=torch.from_numpy((1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)))


@pytest.mark.parametrize("c01", ["0", "1"])
def test_cpp_generate_equals_greedy(gpu, monkeypatch, c01):
    from asdsl.inference import unified_bridge as ub

    monkeypatch.setenv("ASDSL_C01", c01)
    store = _store(5)
    eng = ub.get_or_build_unified_engine(store)
    assert ub.get_or_build_unified_engine(store) is eng  # built once
    assert eng.cfg.gs_ffn == (128 if c01 == "1" else 32) and eng.cfg.gs_attn == 32 and eng.cfg.gs_lm == 32
    got = ub.cpp_generate(store, PROMPT, 40)
    want = ub.greedy_generate(store, PROMPT, 40)
    assert len(got) == 40 and got == want[len(PROMPT):]


def test_unified_forward_token_matches_oracle(gpu):
    """The engine the bridge builds holds the store's weights byte for byte
    (preq2 repacked from its preq blocks, the lm_head quantized from the
    embedding by the engine rule, the norms), and its steps follow the
    oracle's decode step: every step within 2e-2 relative L2 (a one-level
    int8 flip moves a 2-layer random model's logits by ~3e-3; a wrong weight
    or norm by far more) with the same greedy token."""
    import torch

    from asdsl.inference import unified_bridge as ub
    from asdsl.quantization.lm_head import quantize_output_projection
    from asdsl.quantization.repack import repack_preq_blocks_to_preq2
    from oracle import decode as od

    store = _store(6)
    ub.reset_unified_session(store)
    eng = ub.get_or_build_unified_engine(store)
    c = eng.cfg
    names = {"qkv": ("qkv_proj", c.qkv_dim, c.hidden), "o": ("o_proj", c.hidden, c.hidden),
             "gu": ("gate_up_proj", 2 * c.ffn, c.hidden), "down": ("down_proj", c.hidden, c.ffn)}
    for li, L in enumerate(eng.layers):
        for n, (name, M, K) in names.items():
            meta, quant = repack_preq_blocks_to_preq2(store._preq_blocks_np[(li, name)], M, K, 32)
            assert np.array_equal(L[n][0].cpu().numpy(), np.ravel(meta)), (li, n)
            assert np.array_equal(L[n][1].cpu().numpy(), np.ravel(quant)), (li, n)
        assert np.array_equal(L["rms_att"].cpu().numpy(), store._norm_np[(li, "input_layernorm")])
        assert np.array_equal(L["rms_ffn"].cpu().numpy(), store._norm_np[(li, "post_attention_layernorm")])
    lm = quantize_output_projection(store.embed_f16, 32)
    assert torch.equal(eng.lm_meta.cpu(), lm[0]) and torch.equal(eng.lm_quant.cpu(), lm[1])
    model = od.host_model(eng)
    shape = (c.n_kv_heads, c.max_seq, c.head_dim)
    kc = [np.zeros(shape, np.float16) for _ in range(c.n_layers)]
    vc = [np.zeros(shape, np.float16) for _ in range(c.n_layers)]
    for pos, t in enumerate(PROMPT):
        want, want_next = od.decode_step(model, t, pos, kc, vc)
        if pos % 2:
            assert ub.unified_forward_token(store, t, pos, need_logits=False) is None
            continue
        got = ub.unified_forward_token(store, t, pos)
        assert isinstance(got, np.ndarray) and got.dtype == np.float32 and got.shape == (c.vocab,)
        assert rel_l2(got, want) < 2e-2 and int(np.argmax(got)) == want_next, pos
    assert eng.get_kv_seq_len() == len(PROMPT)


def test_cpp_generate_stops_after_a_stop_token(gpu):
    from asdsl.inference import unified_bridge as ub

    store = _store(7)
    free = ub.cpp_generate(store, PROMPT, 20, stop_ids=[])
    stop = free[5]
    first = free.index(stop)
    got = ub.cpp_generate(store, PROMPT, 20, stop_ids=[stop])
    assert got == free[:first + 1]


def _state(eng):
    """Position, KV length, device token and every layer's K/V rows."""
    return (eng._host_pos, int(eng.pos.item()), eng.get_kv_seq_len(), int(eng.token.item()),
            [(L["k_cache"].clone(), L["v_cache"].clone()) for L in eng.layers])


def _same_state(a, b):
    import torch

    assert a[:4] == b[:4], (a[:4], b[:4])
    for (ka, va), (kb, vb) in zip(a[4], b[4]):
        assert torch.equal(ka, kb) and torch.equal(va, vb)


@pytest.mark.parametrize("max_new,stop_at", [(1, None), (16, None), (17, None), (40, None), (40, 5), (40, 21),
                                             (40, 0)])
def test_chunked_generation_is_the_per_token_loop(gpu, max_new, stop_at):
    """greedy_generate and cpp_generate run their steps in chunks of 16 on
    the device (decode_steps, one read per chunk).  Against the one step per
    token loop (forward_token, next_token): the same tokens, and the engine
    left in the same state (position, KV length, device token, K/V rows),
    whether the generation ends on max_new_tokens inside or on a chunk's
    end, or on a stop token inside a chunk (stop_at: index of the free run's
    token used as the stop token)."""
    from asdsl.inference import unified_bridge as ub

    store = _store(8)
    eng = ub.get_or_build_unified_engine(store)
    free = ub.cpp_generate(store, PROMPT, 45, stop_ids=[])
    stop = [] if stop_at is None else [free[stop_at]]

    def per_token(include_stop: bool):
        eng.reset_session()
        for i, t in enumerate(PROMPT):
            eng.forward_token(t, i)
        out, pos = [], len(PROMPT)
        for _ in range(max_new):
            cur = eng.next_token()
            if cur in stop:
                if include_stop:
                    out.append(cur)
                break
            out.append(cur)
            eng.forward_token(cur, pos)
            pos += 1
        return out

    want_g = per_token(False)
    st_g = _state(eng)
    got_g = ub.greedy_generate(store, PROMPT, max_new, eos=stop)
    assert got_g[len(PROMPT):] == want_g
    _same_state(_state(eng), st_g)

    want_c = per_token(True)
    st_c = _state(eng)
    got_c = ub.cpp_generate(store, PROMPT, max_new, stop_ids=stop or [-1])
    assert got_c == want_c
    _same_state(_state(eng), st_c)