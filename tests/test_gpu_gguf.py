"""HIP parity for the GGUF path: ggml Q2_K .. Q6_K, Q4_0, Q4_1, Q5_0, Q5_1 and Q8_0 decoding
(random blocks against the oracle, the hand-worked known-answer blocks), the Q4_K ->
ASDSL Q4_K rearrangement, the symmetric Q4 requantization (bit for bit
against the oracle, up to the full Phi-4 projection shapes), the Q4_K GEMV
on real-layout GGUF blocks, and a GGUF file loaded into the decode engine:
every operand equal to the oracle pipeline's bytes and greedy steps within
the decode bars of the oracle's step on them."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import decode as od
from conftest import rel_l2
from gguf_writer import ARRAY, FLOAT32, STRING, UINT32, write_gguf

pytestmark = pytest.mark.gpu


def _f16_bytes(v) -> np.ndarray:
    return np.asarray(v, np.float16).view(np.uint8).reshape(-1, 2)


def q4k_blocks(n, rng, scale=3e-5) -> np.ndarray:
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    b[:, 2:4] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    return b.reshape(-1)


def q6k_blocks(n, rng, scale=5e-6) -> np.ndarray:
    b = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    b[:, 208:210] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    return b.reshape(-1)


def q5k_blocks(n, rng, scale=3e-5) -> np.ndarray:
    b = rng.integers(0, 256, (n, 176), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    b[:, 2:4] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    return b.reshape(-1)


def q8_0_blocks(n, rng, scale=2e-4) -> np.ndarray:
    b = rng.integers(0, 256, (n, 34), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    return b.reshape(-1)


def legacy_blocks(kind, scale=2e-3):
    """Random ggml legacy blocks with d (and m) drawn around `scale`."""
    nb = oracle.LEGACY_BLOCK_BYTES[kind]

    def make(n, rng) -> np.ndarray:
        b = rng.integers(0, 256, (n, nb), dtype=np.uint8)
        b[:, 0:2] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
        if nb in (20, 24):
            b[:, 2:4] = _f16_bytes(-rng.uniform(0.5, 1.5, n) * 8 * scale)
        return b.reshape(-1)
    return make


def q2k_blocks(n, rng, scale=1e-3) -> np.ndarray:
    b = rng.integers(0, 256, (n, 84), dtype=np.uint8)
    b[:, 80:82] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    b[:, 82:84] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    return b.reshape(-1)


def q3k_blocks(n, rng, scale=1e-4) -> np.ndarray:
    b = rng.integers(0, 256, (n, 110), dtype=np.uint8)
    b[:, 108:110] = _f16_bytes(rng.uniform(0.5, 1.5, n) * scale)
    return b.reshape(-1)


def _legacy_decoder(kind):
    return lambda raw, n: oracle.dequant_gguf_legacy(kind, raw, n)


# ggml type id -> (weights per block, block maker, oracle decoder)
KINDS = {12: (256, q4k_blocks, oracle.dequant_gguf_q4k), 13: (256, q5k_blocks, oracle.dequant_gguf_q5k),
         14: (256, q6k_blocks, oracle.dequant_gguf_q6k), 8: (32, q8_0_blocks, oracle.dequant_gguf_q8_0),
         10: (256, q2k_blocks, oracle.dequant_gguf_q2k), 11: (256, q3k_blocks, oracle.dequant_gguf_q3k),
         2: (32, legacy_blocks("q4_0"), _legacy_decoder("q4_0")), 3: (32, legacy_blocks("q4_1"), _legacy_decoder("q4_1")),
         6: (32, legacy_blocks("q5_0"), _legacy_decoder("q5_0")), 7: (32, legacy_blocks("q5_1"), _legacy_decoder("q5_1"))}
TYPE_ID = {"q4_k": 12, "q5_k": 13, "q6_k": 14, "q8_0": 8, "q2_k": 10, "q3_k": 11, "q4_0": 2, "q4_1": 3, "q5_0": 6,
           "q5_1": 7}
# the decoders added beside Q4_K/Q5_K/Q6_K/Q8_0: ggml type -> C-ABI decoder
MORE_DECODERS = {"q2_k": "asdsl_dequant_gguf_q2k", "q3_k": "asdsl_dequant_gguf_q3k",
                 "q4_0": "asdsl_dequant_gguf_q4_0", "q4_1": "asdsl_dequant_gguf_q4_1",
                 "q5_0": "asdsl_dequant_gguf_q5_0", "q5_1": "asdsl_dequant_gguf_q5_1"}


def _decode(tid, raw, n_weights):
    per, _, dec = KINDS[tid]
    return dec(raw, n_weights // per)


def _dev(a):
    from asdsl import _hip

    return _hip.to_device(np.ascontiguousarray(a), a.dtype)


def _run(fn, *args):
    from asdsl import _hip

    _hip.call(fn, *args, _hip.stream_handle())


@pytest.mark.parametrize("rows,cols", [(1, 256), (5, 512), (5120, 3072), (3072, 8192)])
def test_dequant_q4k_bit_exact(gpu, rows, cols):
    import torch

    rng = np.random.default_rng(rows + cols)
    n = rows * cols // 256
    blocks = q4k_blocks(n, rng)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    _run("asdsl_dequant_gguf_q4k", gpu.ptr(_dev(blocks)), gpu.ptr(out), rows, cols)
    want = oracle.dequant_gguf_q4k(blocks, n).reshape(rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 768), (3072, 8192), (200064 // 16, 3072)])
def test_dequant_q6k_bit_exact(gpu, rows, cols):
    import torch

    rng = np.random.default_rng(rows * 3 + cols)
    n = rows * cols // 256
    blocks = q6k_blocks(n, rng)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    _run("asdsl_dequant_gguf_q6k", gpu.ptr(_dev(blocks)), gpu.ptr(out), rows, cols)
    want = oracle.dequant_gguf_q6k(blocks, n).reshape(rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 256), (5, 512), (3072, 8192)])
def test_dequant_q5k_bit_exact(gpu, rows, cols):
    import torch

    rng = np.random.default_rng(rows * 5 + cols)
    n = rows * cols // 256
    blocks = q5k_blocks(n, rng)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    _run("asdsl_dequant_gguf_q5k", gpu.ptr(_dev(blocks)), gpu.ptr(out), rows, cols)
    want = oracle.dequant_gguf_q5k(blocks, n).reshape(rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 96), (3072, 3072)])
def test_dequant_q8_0_bit_exact(gpu, rows, cols):
    import torch

    rng = np.random.default_rng(rows * 7 + cols)
    n = rows * cols // 32
    blocks = q8_0_blocks(n, rng)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    _run("asdsl_dequant_gguf_q8_0", gpu.ptr(_dev(blocks)), gpu.ptr(out), rows, cols)
    want = oracle.dequant_gguf_q8_0(blocks, n).reshape(rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # 34-byte blocks: a tensor may start 2-byte aligned
    seven = q8_0_blocks(7, rng)
    buf = _dev(np.concatenate([np.zeros(2, np.uint8), seven]))
    out2 = torch.empty((7, 32), dtype=torch.float32, device="cuda")
    _run("asdsl_dequant_gguf_q8_0", gpu.ptr(buf) + 2, gpu.ptr(out2), 7, 32)
    assert np.array_equal(out2.cpu().numpy().reshape(-1).view(np.uint32),
                          oracle.dequant_gguf_q8_0(seven, 7).view(np.uint32))


@pytest.mark.parametrize("kind", sorted(MORE_DECODERS))
@pytest.mark.parametrize("rows,blocks_per_row", [(1, 1), (7, 3), (3072, 12)])
def test_dequant_more_types_bit_exact(gpu, kind, rows, blocks_per_row):
    """Random blocks of each added type, up to the o_proj shape 3072 x 3072
    (96 legacy or 12 K-quant blocks a row), against the oracle bit for bit;
    and a tensor that starts 2-byte aligned."""
    import torch

    per, make, dec = KINDS[TYPE_ID[kind]]
    if per == 32:
        blocks_per_row *= 8  # legacy rows of 32-weight blocks: 8, 24, 96 blocks
    cols = per * blocks_per_row
    rng = np.random.default_rng(rows * 13 + cols + TYPE_ID[kind])
    n = rows * blocks_per_row
    blocks = make(n, rng)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    _run(MORE_DECODERS[kind], gpu.ptr(_dev(blocks)), gpu.ptr(out), rows, cols)
    want = dec(blocks, n).reshape(rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    if rows == 7:
        buf = _dev(np.concatenate([np.zeros(2, np.uint8), blocks]))
        out2 = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
        _run(MORE_DECODERS[kind], gpu.ptr(buf) + 2, gpu.ptr(out2), rows, cols)
        assert np.array_equal(out2.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", ["q4k", "q5k", "q6k", "q8_0", "q2k", "q3k", "q4_0", "q4_1", "q5_0", "q5_1"])
def test_known_answer_blocks_on_the_gpu(gpu, kind):
    """The hand-worked blocks of test_oracle_gguf.py through the kernels."""
    import torch

    from test_oracle_gguf import KNOWN

    make, _, n = KNOWN[kind]
    blk, want = make()
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    fn = {"q4k": "asdsl_dequant_gguf_q4k", "q5k": "asdsl_dequant_gguf_q5k", "q6k": "asdsl_dequant_gguf_q6k",
          "q8_0": "asdsl_dequant_gguf_q8_0", "q2k": "asdsl_dequant_gguf_q2k", "q3k": "asdsl_dequant_gguf_q3k",
          **{k: MORE_DECODERS[k] for k in ("q4_0", "q4_1", "q5_0", "q5_1")}}[kind]
    _run(fn, gpu.ptr(_dev(blk.copy())), gpu.ptr(out), 1, n)
    w = out.cpu().numpy().reshape(-1)
    for i, v in want.items():
        assert w[i] == np.float32(v), (kind, i, w[i], v)


def test_dequant_q6k_blocks_at_odd_offsets(gpu):
    """Q6_K blocks are 210 bytes: a tensor may start 2-byte aligned."""
    import torch

    rng = np.random.default_rng(11)
    blocks = q6k_blocks(6, rng)
    buf = _dev(np.concatenate([np.zeros(2, np.uint8), blocks]))
    out = torch.empty((2, 768), dtype=torch.float32, device="cuda")
    _run("asdsl_dequant_gguf_q6k", gpu.ptr(buf) + 2, gpu.ptr(out), 2, 768)
    assert np.array_equal(out.cpu().numpy().reshape(-1), oracle.dequant_gguf_q6k(blocks, 6))


@pytest.mark.parametrize("rows,cols", [(3, 256), (16384, 3072)])
def test_q4k_to_q4km_bit_exact_and_gemv(gpu, rows, cols):
    import torch

    rng = np.random.default_rng(rows)
    n = rows * cols // 256
    blocks = q4k_blocks(n, rng)
    out = torch.empty(n * 144, dtype=torch.uint8, device="cuda")
    _run("asdsl_repack_gguf_q4k_to_q4km", gpu.ptr(_dev(blocks)), gpu.ptr(out), rows, cols)
    want = oracle.repack_gguf_q4k_to_q4km(blocks, n)
    got = out.cpu().numpy()
    assert np.array_equal(got, want)
    if rows > 3:
        return
    # the ASDSL Q4_K GEMV on the rearranged blocks computes ggml's weights
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    _run("asdsl_gemv_q4km_q8", gpu.ptr(out), gpu.ptr(_dev(x)), gpu.ptr(y), rows, cols)
    xq, xs = oracle.quantize_activation_q4k(x)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    w = oracle.dequant_gguf_q4k(blocks, n).reshape(rows, cols).astype(np.float64)
    assert rel_l2(y.cpu().numpy(), w @ xd) < 1e-5


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("rows,cols", [(3, 256), (5120, 3072)])
def test_quantize_q4_symmetric_bit_exact(gpu, gs, rows, cols):
    import torch

    rng = np.random.default_rng(gs + rows)
    w = (rng.standard_normal((rows, cols)) * rng.uniform(1e-6, 0.1, (rows, 1))).astype(np.float32)
    w[0, :gs] = 0.0
    if rows > 3:
        w[1, :gs] = ((rng.integers(0, 16, gs) - 7.5) * 0.25).astype(np.float32)  # ties and exact codes
    groups = rows * cols // gs
    packed = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
    scales = torch.empty(groups, dtype=torch.float32, device="cuda")
    biases = torch.empty(groups, dtype=torch.float32, device="cuda")
    _run("asdsl_quantize_q4_symmetric", gpu.ptr(_dev(w)), gpu.ptr(packed), gpu.ptr(scales), gpu.ptr(biases), rows,
         cols, gs)
    p, s, b = oracle.quantize_q4_symmetric(w, gs)
    assert np.array_equal(packed.cpu().numpy(), p)
    assert np.array_equal(scales.cpu().numpy(), s) and np.array_equal(biases.cpu().numpy(), b)


def test_argument_errors(gpu):
    from asdsl import _hip

    with pytest.raises(ValueError, match="multiple of 256"):
        _run("asdsl_dequant_gguf_q4k", 16, 16, 2, 100)
    with pytest.raises(ValueError, match="multiple of 256"):
        _run("asdsl_dequant_gguf_q3k", 16, 16, 2, 100)
    with pytest.raises(ValueError, match="multiple of 32"):
        _run("asdsl_dequant_gguf_q5_1", 16, 16, 2, 48)
    with pytest.raises(ValueError, match="2-byte"):
        _run("asdsl_dequant_gguf_q4_0", 17, 32, 1, 32)
    with pytest.raises(ValueError, match="group_size"):
        _run("asdsl_quantize_q4_symmetric", 16, 16, 16, 16, 2, 96, 48)
    with pytest.raises(ValueError, match="16-byte aligned"):
        _run("asdsl_repack_gguf_q4k_to_q4km", 18, 32, 1, 256)
    assert _hip.last_error()


# ------------------------------------------------------------ whole model
# tensor -> ggml type of the two mixes: "q4" (Q4_K with Q6_K down and
# embedding, as a Q4_K_M file) and "q5" (Q5_K and Q8_0 beside Q6_K)
MIXES = {"q4": {"qkv": "q4_k", "o": "q4_k", "gu": "q4_k", "gate": "q4_k", "up": "q6_k", "down": "q6_k",
                "embd": "q6_k", "out": "q4_k"},
         "q5": {"qkv": "q5_k", "o": "q8_0", "gu": "q5_k", "gate": "q8_0", "up": "q5_k", "down": "q6_k",
                "embd": "q8_0", "out": "q5_k"},
         "legacy": {"qkv": "q4_0", "o": "q5_0", "gu": "q4_1", "gate": "q5_1", "up": "q3_k", "down": "q2_k",
                    "embd": "q5_1", "out": "q4_0"}}


def _write_model(path, cfg, rng, gate_up_split=False, mix="q4"):
    """A Phi-4-shaped GGUF with the projections, token_embd and output in
    the types of MIXES[mix], F32 norms, phi3 metadata."""
    H, F, V = cfg.hidden, cfg.ffn, cfg.vocab
    qkv_rows = cfg.qkv_dim
    tensors = []
    kinds = MIXES[mix]

    def add(name, rows, cols, what):
        tid = TYPE_ID[kinds[what]]
        per, make, _ = KINDS[tid]
        tensors.append((name, tid, (cols, rows), make(rows * cols // per, rng)))

    for i in range(cfg.n_layers):
        p = f"blk.{i}."
        add(p + "attn_qkv.weight", qkv_rows, H, "qkv")
        add(p + "attn_output.weight", H, H, "o")
        if gate_up_split:
            add(p + "ffn_gate.weight", F, H, "gate")
            add(p + "ffn_up.weight", F, H, "up")
        else:
            add(p + "ffn_up.weight", 2 * F, H, "gu")
        add(p + "ffn_down.weight", H, F, "down")
        for n in ("attn_norm.weight", "ffn_norm.weight"):
            tensors.append((p + n, 0, (H,), (1 + 0.1 * rng.standard_normal(H)).astype(np.float32).view(np.uint8)))
    add("token_embd.weight", V, H, "embd")
    tensors.append(("output_norm.weight", 0, (H,), (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
                    .view(np.uint8)))
    add("output.weight", V, H, "out")
    meta = [("general.architecture", STRING, "phi3"), ("phi3.embedding_length", UINT32, H),
            ("phi3.feed_forward_length", UINT32, F), ("phi3.block_count", UINT32, cfg.n_layers),
            ("phi3.attention.head_count", UINT32, cfg.n_heads),
            ("phi3.attention.head_count_kv", UINT32, cfg.n_kv_heads),
            ("phi3.rope.dimension_count", UINT32, cfg.rotary_dim), ("phi3.context_length", UINT32, cfg.max_seq),
            ("phi3.attention.layer_norm_rms_epsilon", FLOAT32, cfg.rms_eps),
            ("phi3.rope.freq_base", FLOAT32, cfg.rope_theta),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(V)]))]
    write_gguf(path, tensors, meta)
    return {name: (tid, raw) for name, tid, _, raw in tensors}


def _oracle_preq2(tid, raw, rows, cols, gs):
    w = _decode(tid, raw, rows * cols)
    p, s, b = oracle.quantize_q4_symmetric(w, gs)
    return oracle.repack_asym_to_preq2(p, s, b, rows, cols, gs)


@pytest.mark.parametrize("split,mix", [(False, "q4"), (True, "q4"), (False, "q5"), (True, "q5"), (False, "legacy"),
                                       (True, "legacy")])
def test_gguf_model_loads_and_decodes(gpu, tmp_path, split, mix):
    """2 Phi-4-shaped layers, vocab 4096, from a GGUF file: the config from
    its metadata; every preq2 operand, norm and the fp16 embedding equal to
    the oracle pipeline (decode, requantize, repack) bit for bit; three
    greedy steps from a 100-position random KV prefix within 1e-3 of the
    oracle's step with the same tokens."""
    import torch

    from asdsl.engine import DecodeConfig, DecodeEngine, _layer_mats

    cfg0 = DecodeConfig(n_layers=2, vocab=4096, max_seq=512)
    rng = np.random.default_rng(5 + split)
    path = tmp_path / "m.gguf"
    raw = _write_model(path, cfg0, rng, gate_up_split=split, mix=mix)
    eng = DecodeEngine.from_gguf(path)
    cfg = eng.cfg
    assert (cfg.hidden, cfg.ffn, cfg.vocab, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.rotary_dim,
            cfg.max_seq) == (3072, 8192, 4096, 2, 24, 8, 96, 512)

    host = lambda t: t.cpu().numpy()  # noqa: E731
    mats = _layer_mats(cfg)
    names = {"qkv": "attn_qkv.weight", "o": "attn_output.weight", "down": "ffn_down.weight"}
    layers = []
    for i, L in enumerate(eng.layers):
        ol = {}
        for n, (rows, cols, gs) in mats.items():
            if n == "gu" and split:
                g = _decode(*raw[f"blk.{i}.ffn_gate.weight"], rows // 2 * cols)
                u = _decode(*raw[f"blk.{i}.ffn_up.weight"], rows // 2 * cols)
                p, s, b = oracle.quantize_q4_symmetric(np.concatenate([g, u]), gs)
                want = oracle.repack_asym_to_preq2(p, s, b, rows, cols, gs)
            else:
                tid, r = raw[f"blk.{i}." + names.get(n, "ffn_up.weight")]
                want = _oracle_preq2(tid, r, rows, cols, gs)
            got = (host(L[n][0]).reshape(-1), host(L[n][1]).reshape(-1))
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), (i, n)
            ol[n] = want
        for n, key in (("rms_att", "attn_norm.weight"), ("rms_ffn", "ffn_norm.weight")):
            ol[n] = raw[f"blk.{i}.{key}"][1].view(np.float32)
            assert np.array_equal(host(L[n]), ol[n])
        layers.append(ol)
    emb = _decode(*raw["token_embd.weight"], cfg.vocab * cfg.hidden)
    emb16 = emb.astype(np.float16).reshape(cfg.vocab, cfg.hidden)
    assert np.array_equal(host(eng.embed), emb16)
    lm = _oracle_preq2(*raw["output.weight"], cfg.vocab, cfg.hidden, cfg.gs_lm)
    assert np.array_equal(host(eng.lm_meta).reshape(-1), lm[0]) and np.array_equal(host(eng.lm_quant).reshape(-1), lm[1])
    rms_out = raw["output_norm.weight"][1].view(np.float32)
    assert np.array_equal(host(eng.rms_out), rms_out)

    model = {"cfg": cfg, "layers": layers, "embed": emb16, "rms_out": rms_out, "lm_meta": lm[0],
             "lm_quant": lm[1], "rope_cos": host(eng.rope_cos), "rope_sin": host(eng.rope_sin)}
    ctx = 100
    eng.prefill_kv_random(ctx, seed=4)
    kc = [host(L["k_cache"]) for L in eng.layers]
    vc = [host(L["v_cache"]) for L in eng.layers]
    tok = 77
    eng.token.fill_(tok)
    for step in range(3):
        want_logits, want_next = od.decode_step(model, tok, ctx + step, kc, vc)
        eng._queue_step(int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert rel_l2(host(eng.logits), want_logits) < 1e-3, step
        assert eng.next_token() == want_next, step
        tok = want_next
