"""Full-size decode parity anchored to the reference's own engine.

Three implementations of one greedy decode step run side by side on the
same weights, each with its own int8 KV cache:

* the GPU engine (asdsl.engine.DecodeEngine, int8 cache);
* the reference's UnifiedEngine::forward_token
  (asdsl/kernels/native/unified_engine.cpp:1339-1688), compiled unchanged
  into oracle/_ref/_native_unified.so, on its C0.1 profile (ASDSL_C01=1:
  gate_up/down through gemv_q4_128_preq_avx2, 1532-1538 and 1592-1598; the
  lm_head quantized by the engine at load, 413-461, run through
  gemv_q4_128_preq_avx2 after rmsnorm_quantize_f32, 1651-1653);
* the oracle (oracle/decode.py) with its own GEMVs.

Model: 32 layers, hidden 3072, FFN 8192, vocab 200064, 24/8 heads.  qkv/o
are preq2 g32 (the same meta/quant arrays on all three); gate_up/down are
Q4_128 blocks of N(0, 0.02) weights, which the reference runs as they are
and the GPU and the oracle run as preq2-g128 (the lossless Q4_128 repack);
the output projection is an fp16 matrix that the reference quantizes at
load and that the GPU and the oracle get quantized by the same rule
(asdsl.quantization.lm_head.quantize_output_projection on the device, a
slice of it checked here against oracle.decode.quantize_lm_head_q4_128).

Each side prefills positions 0..ctx-1 with the same seeded tokens (the
reference with forward_token_prefill; the oracle with the reference's
compiled GEMV kernels for speed -- gemv_preq2_fused_avx2, and
quantize_activation_avx2 + gemv_q4_128_preq_avx2 on the Q4_128 blocks, which
the oracle's own GEMVs match to 1e-6 -- and without the lm_head), then runs
16 steps teacher forced by the reference's greedy token, the oracle with its
own GEMVs.  Per step: relative L2 and top-1 agreement of GPU vs reference,
oracle vs reference and GPU vs oracle.

Bar: the GPU is no further from the reference than the oracle is -- median
relative L2 of GPU vs reference within 2x that of oracle vs reference +
1e-3, top-1 agreement with the reference at most 0.1 below the oracle's.
Every independent restatement of this random 32-layer model drifts from the
reference by a few 1e-2 (one-level int8 flips amplified over depth), so the
absolute 1e-3 is not the bar here; tests/test_gpu_decode_full.py holds it per
layer.  Set ASDSL_DECODE_PARITY_LOG to a file path to get one JSON line per
step and a summary per context.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from decode_c01 import tie_rows_torch

pytestmark = pytest.mark.gpu

CTXS = (128, 1024)
STEPS = 16
MAX_SEQ = CTXS[-1] + STEPS + 16
REF = oracle.reference_available("_native_unified") and oracle.reference_available("_native_gemv")


def _log(rows):
    path = os.environ.get("ASDSL_DECODE_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            for r in rows:
                f.write(json.dumps(r) + "\n")


class _C01:
    """The three sides and their shared position."""


@pytest.fixture(scope="module")
def c01(gpu):
    if not REF:
        pytest.skip("oracle/_ref not built (reference tree not mounted when the tree was built)")
    import torch
    from asdsl import _hip
    from asdsl.engine import DecodeConfig, DecodeEngine, _layer_mats
    from asdsl.quantization.lm_head import quantize_output_projection
    from asdsl.quantization.repack import repack_q4_128_blocks_to_preq2
    from asdsl.quantization.synthetic import preq2_from_weights_torch, q4_128_from_weights_torch
    from oracle import decode as od

    cfg = DecodeConfig(max_seq=MAX_SEQ, kv_format="int8")
    dev = _hip.device()
    gen = torch.Generator(device=dev).manual_seed(31)

    def host(t):
        return t.cpu().numpy()

    def norm_w():
        return 1.0 + 0.1 * torch.randn(cfg.hidden, generator=gen, device=dev, dtype=torch.float32)

    layers, host_layers, ref_layers, q4 = [], [], {}, {}
    mats = _layer_mats(cfg)
    names = {"qkv": "qkv_proj", "o": "o_proj", "gu": "gate_up_proj", "down": "down_proj"}
    for li in range(cfg.n_layers):
        L, H, R = {}, {}, {}
        for n, name in names.items():
            rows, cols, gs = mats[n]
            w = torch.randn((rows, cols), generator=gen, device=dev, dtype=torch.float32) * 0.02
            if gs == 32:
                L[n] = preq2_from_weights_torch(w, 32)
                H[n] = (host(L[n][0]), host(L[n][1]))
                R[name + "_meta"], R[name + "_quant"] = H[n]
            else:
                blocks = q4_128_from_weights_torch(w)
                L[n] = repack_q4_128_blocks_to_preq2(blocks, rows, cols)
                H[n] = (host(L[n][0]), host(L[n][1]))
                R[name + "_g128"] = host(blocks)
                q4[id(H[n][1])] = R[name + "_g128"]
            del w
            # the engine binds a preq-block array per projection; this profile
            # never reads them (zero pages, not resident)
            R[name] = np.zeros(rows * cols // 32 * 20, np.uint8)
        L["rms_att"], L["rms_ffn"] = norm_w(), norm_w()
        H["rms_att"], H["rms_ffn"] = host(L["rms_att"]), host(L["rms_ffn"])
        R["rms_att"], R["rms_ffn"] = H["rms_att"], H["rms_ffn"]
        layers.append(L)
        host_layers.append(H)
        ref_layers[li] = R
    embed = torch.randn((cfg.vocab, cfg.hidden), generator=gen, device=dev, dtype=torch.float32).half()
    lm_w = tie_rows_torch(cfg.vocab, cfg.hidden, gen, dev)
    lm_meta, lm_quant = quantize_output_projection(lm_w, 128)
    G = cfg.hidden // 128
    want = repack_q4_128_blocks_to_preq2(od.quantize_lm_head_q4_128(host(lm_w[:4096].float())), 4096, cfg.hidden)
    assert np.array_equal(host(lm_meta[:4096 * G * 4]), np.ravel(want[0]))
    assert np.array_equal(host(lm_quant[:1024 * G * 256]), np.ravel(want[1]))
    rms_out = norm_w()
    eng = DecodeEngine(cfg, layers, embed, rms_out, lm_meta, lm_quant)

    s = _C01()
    s.cfg, s.eng = cfg, eng
    s.model = {"cfg": cfg, "layers": host_layers, "embed": host(embed), "rms_out": host(rms_out),
               "lm_meta": host(lm_meta), "lm_quant": host(lm_quant), "rope_cos": host(eng.rope_cos),
               "rope_sin": host(eng.rope_sin)}

    ue = oracle.load_reference("_native_unified")
    ec = ue.EngineConfig()
    ec.num_layers, ec.hidden_size, ec.num_heads, ec.num_kv_heads = (cfg.n_layers, cfg.hidden, cfg.n_heads,
                                                                    cfg.n_kv_heads)
    ec.head_dim, ec.intermediate_size, ec.vocab_size, ec.rms_norm_eps = cfg.head_dim, cfg.ffn, cfg.vocab, cfg.rms_eps
    ec.group_size, ec.lm_head_group_size, ec.max_seq_len = 32, 128, MAX_SEQ
    ec.rotary_dim, ec.weight_format = cfg.rotary_dim, 0
    s.prev_c01 = os.environ.get("ASDSL_C01")
    os.environ["ASDSL_C01"] = "1"
    s.ref = ue.UnifiedEngine(ec, s.model["embed"], s.model["rms_out"], host(lm_w), s.model["rope_cos"].copy(),
                             s.model["rope_sin"].copy(), ref_layers)
    del lm_w
    s.ref_layers = ref_layers

    ng = oracle.load_reference("_native_gemv")

    def ref_gemv(meta, quant, x, M, K, gs):
        """The reference's compiled GEMVs in the oracle's gemv signature."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(M, np.float32)
        if gs == 32:
            ng.gemv_preq2_fused_avx2(meta, quant, x, y, M, K, 32)
        else:
            xq = np.empty(K, np.int8)
            xs = np.empty(K // 128, np.float32)
            ng.quantize_activation_avx2(x, xq, xs, K, 128)
            ng.gemv_q4_128_preq_avx2(q4[id(quant)], xq, xs, y, M, K, 128)
        return y

    s.ref_gemv = ref_gemv
    shape = (cfg.n_kv_heads, MAX_SEQ, cfg.head_dim)

    def q8():
        return np.zeros(shape, np.int8), np.ones(shape[:2] + (cfg.head_dim // 64,), np.float32)

    s.kc = [q8() for _ in range(cfg.n_layers)]
    s.vc = [q8() for _ in range(cfg.n_layers)]
    s.tokens = np.random.default_rng(7).integers(0, cfg.vocab, MAX_SEQ)
    s.pos = 0
    yield s
    if s.prev_c01 is None:
        os.environ.pop("ASDSL_C01", None)
    else:
        os.environ["ASDSL_C01"] = s.prev_c01


def _prefill_to(s, ctx):
    from oracle import decode as od

    while s.pos < ctx:
        t = int(s.tokens[s.pos])
        s.eng.forward_token(t, s.pos)
        s.ref.forward_token_prefill(t, s.pos)
        od.decode_step(s.model, t, s.pos, s.kc, s.vc, gemv=s.ref_gemv, lm_head=False)
        s.pos += 1
        if s.pos % 128 == 0:
            _log([{"test": "c01_reference_prefill", "pos": s.pos}])


@pytest.mark.parametrize("ctx", CTXS)
def test_decode_against_reference_engine(c01, ctx):
    from oracle import decode as od

    s = c01
    assert s.pos <= ctx, "contexts run in increasing order on one module fixture"
    _prefill_to(s, ctx)
    tok = int(s.tokens[s.pos])
    rows = []
    for _ in range(STEPS):
        g = s.eng.forward_token(tok, s.pos).cpu().numpy()
        r = np.array(s.ref.forward_token(tok, s.pos), copy=True)
        o, o_next = od.decode_step(s.model, tok, s.pos, s.kc, s.vc)
        rt, gt = int(np.argmax(r)), int(np.argmax(g))
        rows.append({"test": "c01_reference", "ctx": ctx, "pos": s.pos, "gpu_ref": rel_l2(g, r),
                     "orc_ref": rel_l2(o, r), "gpu_orc": rel_l2(g, o), "gpu_ref_agree": gt == rt,
                     "orc_ref_agree": o_next == rt, "gpu_orc_agree": gt == o_next})
        tok = rt
        s.pos += 1
    summary = {"test": "c01_reference_summary", "ctx": ctx}
    for k in ("gpu_ref", "orc_ref", "gpu_orc"):
        v = np.array([r[k] for r in rows])
        summary[k] = {"median": float(np.median(v)), "max": float(v.max()), "min": float(v.min()),
                      "agree": float(np.mean([r[k + "_agree"] for r in rows]))}
    _log(rows + [summary])
    g, o = summary["gpu_ref"], summary["orc_ref"]
    assert g["median"] <= 2.0 * o["median"] + 1e-3, summary
    assert g["agree"] >= o["agree"] - 0.1, summary
