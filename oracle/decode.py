"""CPU oracle of one batch-1 decode step — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's UnifiedEngine::forward_token
(asdsl/kernels/native/unified_engine.cpp:1339-1688) on the fused-preq path, with
the GEMVs taken from the oracle's C restatement (oracle.gemv_preq2_fused):

    h = embed[token]                                        (load_embed_row_f32, 181-197)
    per layer:
        x   = rmsnorm(h, rms_att)                           (rmsnorm_f32, 499-524)
        qkv = gemv_preq2_fused(qkv, x)                      (1399-1401)
        q, k = rope(q), rope(k)                             (rope_apply_inplace, 768-801)
        cache[pos] = k, v (fp16, or int8 per 64 as the reference: set_kv_cache, 859-920)
        att = softmax(q.K / sqrt(128)) V over 0..pos         (compute_attention_flash_q8, 922-1027)
        h   = h + gemv_preq2_fused(o, att)                  (1487-1489, residual_add_rmsnorm_f32 651-688)
        gu  = gemv_preq2_fused(gate_up, rmsnorm(h, rms_ffn))
        h   = h + gemv_preq2_fused(down, swiglu(gate, up))  (swiglu_inplace 803-857, vec_add 487-497)
    logits = gemv_preq2_fused(lm_head, rmsnorm(h, rms_out)); next = argmax (207-233)

Every array is float32 as in the reference; the new K/V are stored in the
cache (rounded to fp16, or quantized to int8 per 64 dims) before attention,
which reads them back from there, as the reference does.
"""

from __future__ import annotations

import numpy as np

import oracle

F32 = np.float32


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """rmsnorm_f32: inv = 1/sqrt(sum(x^2)/n + eps); out = (x*inv)*w, fp32."""
    x = x.astype(F32)
    ss = F32(np.dot(x.astype(np.float64), x.astype(np.float64)))
    inv = F32(1.0) / np.sqrt(ss / F32(x.size) + F32(eps), dtype=F32)
    return ((x * inv) * w.astype(F32)).astype(F32)


def fma32(a, b, c) -> np.ndarray:
    """float32 fused multiply-add: a*b is exact in float64, the sum is rounded
    to float64 and then to float32 (the double rounding can differ from one
    rounding only when the float64 sum lands exactly halfway between two
    float32 values)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def rope(heads: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    """Half-split rotation of the first 2*len(cos_row) dims of every head row,
    as rope_apply_inplace forms it (unified_engine.cpp:777-786):
    x_i' = fma(x_i, c, -(x_{i+h} s)), x_{i+h}' = fma(x_i, s, x_{i+h} c)."""
    out = heads.astype(F32).copy()
    h = cos_row.size
    xf = heads[:, :h].astype(F32)
    xs = heads[:, h:2 * h].astype(F32)
    out[:, :h] = fma32(xf, cos_row, -(xs * sin_row).astype(F32))
    out[:, h:2 * h] = fma32(xf, sin_row, (xs * cos_row).astype(F32))
    return out


def fast_exp_parts(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fast_exp_avx2 (unified_engine.cpp:803-825) as exp(x) = p * 2^i: clamp to
    +-87.3, t = x*log2(e) rounded to float32, i = round-half-even(t), f = t - i,
    p = the degree-5 polynomial in f by fused multiply-adds (_mm256_fmadd_ps);
    returns (p, 2^i)."""
    x = np.clip(x.astype(F32), F32(-87.3), F32(87.3))
    t = (x * F32(1.4426950408889634)).astype(F32)
    fi = np.rint(t).astype(F32)
    f = (t - fi).astype(F32)
    p = fma32(F32(0.001333838100523091), f, F32(0.009618129107628477))
    p = fma32(p, f, F32(0.05550410866482158))
    p = fma32(p, f, F32(0.2402265069591007))
    p = fma32(p, f, F32(0.6931471805599453))
    p = fma32(p, f, F32(1.0))
    two_i = ((fi.astype(np.int32) + 127) << 23).astype(np.int32).view(F32)
    return p, two_i


def fast_exp(x: np.ndarray) -> np.ndarray:
    p, two_i = fast_exp_parts(x)
    return (p * two_i).astype(F32)


def swiglu(gate: np.ndarray, up: np.ndarray, threshold: float = 0.0) -> np.ndarray:
    """swiglu_inplace (unified_engine.cpp:827-857) as the reference's build
    evaluates it: sigmoid = 1 / fma(p, 2^i, 1) with (p, 2^i) = fast_exp_parts(-g)
    (GCC fuses the polynomial's last product into the 1 + exp add), v = (g *
    sigmoid) * u; |v| < threshold -> 0.  The quotient is correctly rounded here;
    the reference build forms it with a reciprocal estimate and one Newton
    step, which moves the last bits and depends on the CPU's estimate table."""
    g = gate.astype(F32)
    p, two_i = fast_exp_parts(-g)
    sig = (F32(1.0) / fma32(p, two_i, F32(1.0))).astype(F32)
    v = ((g * sig).astype(F32) * up.astype(F32)).astype(F32)
    if threshold > 0.0:
        v[np.abs(v) < F32(threshold)] = F32(0.0)
    return v


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_kv: int) -> np.ndarray:
    """q [n_heads][d]; k, v [n_kv][T][d] (fp16 or the fp16-rounded floats).
    out[h] = softmax(q_h . k / sqrt(d)) v of kv head h // (n_heads / n_kv),
    in float64 (the query heads of one KV head share its converted rows)."""
    n_heads, d = q.shape
    g = n_heads // n_kv
    out = np.empty((n_heads, d), F32)
    for j in range(n_kv):
        kk = k[j].astype(np.float64)
        vv = v[j].astype(np.float64)
        qq = q[j * g:(j + 1) * g].astype(np.float64)
        s = kk @ qq.T / np.sqrt(d)              # [T][g]
        w = np.exp(s - s.max(axis=0))
        out[j * g:(j + 1) * g] = ((w.T @ vv) / w.sum(axis=0)[:, None]).astype(F32)
    return out


KV_QBLOCK = 64


def kv_quantize_q8(rows: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """set_kv_cache (unified_engine.cpp:859-920) on rows [n][d] (d a multiple of
    64), as built with -ffast-math: per 64-dim block amax; scale =
    amax * f32(1/127) (the constant division becomes a reciprocal multiply)
    when amax > 1e-12, else 1e-12; inv = 1 / scale; q = clip(rne(x * inv),
    -127, 127).  Returns int8 [n][d] and float32 scales [n][d / 64]."""
    x = np.ascontiguousarray(rows, F32).reshape(rows.shape[0], -1, KV_QBLOCK)
    amax = np.abs(x).max(axis=2)
    scale = np.where(amax > F32(1e-12), (amax * F32(1.0 / 127.0)).astype(F32), F32(1e-12)).astype(F32)
    inv = (F32(1.0) / scale).astype(F32)
    q = np.clip(np.rint((x * inv[:, :, None]).astype(F32)), -127, 127).astype(np.int8)
    return q.reshape(rows.shape), scale


def kv_dequant_q8(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """float(q) * scale per 64-dim block in fp32, as compute_attention_flash_q8
    forms each K/V element (unified_engine.cpp:948-951,981-983)."""
    lead = q.shape[:-1]
    qq = q.reshape(*lead, -1, KV_QBLOCK).astype(F32)
    return (qq * scale.reshape(*lead, -1, 1).astype(F32)).astype(F32).reshape(q.shape)


def argmax_first(x: np.ndarray) -> int:
    """argmax_f32_avx2: the first index of the maximum."""
    return int(np.argmax(x))


def _lm_head_levels(w: np.ndarray, gs: int):
    """The engine's symmetric load-time rule per gs-group (see
    quantize_lm_head_q4_128): returns (q uint8 [rows][G][gs] in 0..15,
    fp16 scale bits [rows][G]) with q = 8 and scale 0 for amax < 1e-12."""
    x = np.ascontiguousarray(w, F32)
    rows, cols = x.shape
    g = x.reshape(rows, cols // gs, gs)
    amax = np.abs(g).max(axis=2)
    tiny = amax < F32(1e-12)
    safe = np.where(tiny, F32(1.0), amax).astype(F32)
    scale = (safe * F32(1.0 / 7.0)).astype(F32)
    inv = (F32(7.0) / safe).astype(F32)
    v = (g * inv[:, :, None]).astype(F32)
    t = np.trunc(v)
    r = t + np.where(np.abs(v - t) >= F32(0.5), np.sign(v), F32(0.0))  # half away from zero, exact in float32
    q = np.clip(r + F32(8.0), 0, 15).astype(np.uint8)
    q[tiny] = 8
    s16 = np.where(tiny, F32(0.0), scale).astype(np.float16).view(np.uint16)
    return q, s16


def quantize_lm_head_q4_128(w: np.ndarray) -> np.ndarray:
    """The engine's load-time Q4_128 quantization of the output projection
    (UnifiedEngine constructor, unified_engine.cpp:413-461, lm_head_group_size
    128) on float32 rows [rows][cols] (cols a multiple of 128), as built with
    -ffast-math: per 128-group amax; amax < 1e-12 -> scale 0 and nibbles 0x88;
    else scale = amax * f32(1/7) (the constant division becomes a reciprocal
    multiply) stored as fp16 (round to nearest even), inv = 7.0f / amax (a
    true float32 division), q = round-half-away(x * inv) + 8 clamped to
    [0, 15] (std::round).  Differs from repack_q4_128.py's quantizer in the
    rounding of ties (half away, not half even) and in forming the scale in
    float32.  Returns flat 66-byte blocks (uint8)."""
    q, s16 = _lm_head_levels(w, 128)
    n = q.shape[0] * q.shape[1]
    q = q.reshape(n, 128)
    blocks = np.empty((n, 66), np.uint8)
    blocks[:, 0] = (s16.reshape(n) & 0xFF).astype(np.uint8)
    blocks[:, 1] = (s16.reshape(n) >> 8).astype(np.uint8)
    blocks[:, 2:] = q[:, 0::2] | (q[:, 1::2] << 4)
    return blocks.reshape(-1)


def quantize_lm_head_preq_g32(w: np.ndarray) -> np.ndarray:
    """The engine's load-time quantization of the output projection at
    lm_head_group_size 32 (unified_engine.cpp:320-372): the same symmetric
    rule per 32-group, stored as 20-byte preq blocks with zero-point fp16 8.0
    (0x4800): [fp16 scale | fp16 8.0 | 16 B nibbles]; an all-zero group is
    scale 0, zero 8.0, nibbles 0x88.  The engine then copies them into its
    preq2 lm_head byte for byte (unified_engine.cpp:374-398).  Returns flat
    blocks (uint8)."""
    q, s16 = _lm_head_levels(w, 32)
    n = q.shape[0] * q.shape[1]
    q = q.reshape(n, 32)
    blocks = np.empty((n, 20), np.uint8)
    blocks[:, 0] = (s16.reshape(n) & 0xFF).astype(np.uint8)
    blocks[:, 1] = (s16.reshape(n) >> 8).astype(np.uint8)
    blocks[:, 2] = 0x00
    blocks[:, 3] = 0x48
    blocks[:, 4:] = q[:, 0::2] | (q[:, 1::2] << 4)
    return blocks.reshape(-1)


def rmsnorm_factored(x: np.ndarray, w: np.ndarray, eps: float) -> tuple[np.ndarray, np.float32]:
    """The factored form of rmsnorm_f32 that the GPU's norm-fed GEMVs take
    on request: (x * w, inv_rms) -- the GEMV quantizes x * w and its outputs
    are scaled by inv_rms afterwards (1/rms is one positive factor of the
    whole input)."""
    x = x.astype(F32)
    ss = F32(np.dot(x.astype(np.float64), x.astype(np.float64)))
    inv = F32(1.0) / np.sqrt(ss / F32(x.size) + F32(eps), dtype=F32)
    return (x * w.astype(F32)).astype(F32), inv


def _norm_gemv(gemv, meta, quant, h, w, eps, M, K, gs, factored):
    """gemv(rmsnorm(h, w)), or in the factored form gemv(h * w) * inv_rms."""
    if not factored:
        x = rmsnorm(h, w, eps)
        return x, gemv(meta, quant, x, M, K, gs)
    x, inv = rmsnorm_factored(h, w, eps)
    return x, (gemv(meta, quant, x, M, K, gs) * inv).astype(F32)


def layer_forward(model: dict, li: int, h: np.ndarray, pos: int, k_cache: list, v_cache: list,
                  trace: dict | None = None, gemv=None) -> np.ndarray:
    """Decoder layer li at position pos on the residual stream h (float32
    [hidden]); returns the next residual stream.  The layer's K/V row at pos is
    written into k_cache[li]/v_cache[li] (see decode_step).  trace (a dict),
    when given, receives this layer's intermediate values: x_att (the normed
    qkv input), qkv, att, o, h_mid (the stream after the attention residual),
    x_ffn, gu, s (the SwiGLU output) and down.  gemv replaces
    oracle.gemv_preq2_fused (same signature)."""
    c = model["cfg"]
    gemv = gemv or oracle.gemv_preq2_fused
    fact = bool(model.get("factored_norm", False))
    hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
    cos_row, sin_row = model["rope_cos"][pos], model["rope_sin"][pos]
    L = model["layers"][li]
    x, qkv = _norm_gemv(gemv, *L["qkv"], h, L["rms_att"], c.rms_eps, c.qkv_dim, c.hidden, c.gs_attn, fact)
    q = rope(qkv[: nh * hd].reshape(nh, hd), cos_row, sin_row)
    k = rope(qkv[nh * hd:(nh + nkv) * hd].reshape(nkv, hd), cos_row, sin_row)
    v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
    if isinstance(k_cache[li], tuple):  # int8 per 64 dims
        (kq, ks), (vq, vs) = k_cache[li], v_cache[li]
        kq[:, pos], ks[:, pos] = kv_quantize_q8(k)
        vq[:, pos], vs[:, pos] = kv_quantize_q8(v)
        att = attention(q, kv_dequant_q8(kq[:, :pos + 1], ks[:, :pos + 1]),
                        kv_dequant_q8(vq[:, :pos + 1], vs[:, :pos + 1]), nkv)
    else:
        k_cache[li][:, pos] = k.astype(np.float16)
        v_cache[li][:, pos] = v.astype(np.float16)
        att = attention(q, k_cache[li][:, :pos + 1], v_cache[li][:, :pos + 1], nkv)
    o = gemv(*L["o"], att.reshape(-1), c.hidden, nh * hd, c.gs_attn)
    h_mid = (h + o).astype(F32)
    x_ffn, gu = _norm_gemv(gemv, *L["gu"], h_mid, L["rms_ffn"], c.rms_eps, 2 * c.ffn, c.hidden, c.gs_ffn, fact)
    sw = swiglu(gu[: c.ffn], gu[c.ffn:], model.get("fatrelu_threshold", 0.0))
    down = gemv(*L["down"], sw, c.hidden, c.ffn, c.gs_ffn)
    if trace is not None:
        trace.update(x_att=x, qkv=qkv, att=att.reshape(-1), o=o, h_mid=h_mid, x_ffn=x_ffn, gu=gu, s=sw, down=down)
    return (h_mid + down).astype(F32)


def lm_head_forward(model: dict, h: np.ndarray, gemv=None) -> np.ndarray:
    """logits = lm_head(rmsnorm(h, rms_out)) (unified_engine.cpp:1634-1648)."""
    c = model["cfg"]
    gemv = gemv or oracle.gemv_preq2_fused
    return _norm_gemv(gemv, model["lm_meta"], model["lm_quant"], h, model["rms_out"], c.rms_eps, c.vocab, c.hidden,
                      c.gs_lm, bool(model.get("factored_norm", False)))[1]


def decode_step(model: dict, token: int, pos: int, k_cache: list, v_cache: list, trace: list | None = None,
                gemv=None, lm_head: bool = True) -> tuple[np.ndarray, int]:
    """One greedy step.  model: host copies of the engine's weights
    (host_model; model["factored_norm"] = True takes the norm-fed GEMVs'
    factored form, rmsnorm_factored); k_cache/v_cache: per layer either an fp16 array
    [n_kv][max_seq][128] or, for the int8 cache, a pair (int8
    [n_kv][max_seq][128], float32 scales [n_kv][max_seq][2]); updated at
    `pos` in place.  trace (a list), when given, receives per layer a dict
    with the layer's input stream "h" and the values layer_forward traces,
    then {"h": final stream}.  gemv replaces oracle.gemv_preq2_fused.
    lm_head=False stops after the layers (the K/V rows written, no logits:
    the reference's forward_token_prefill) and returns (None, None)."""
    h = model["embed"][token].astype(F32)
    for li in range(len(model["layers"])):
        t = {"h": h} if trace is not None else None
        h = layer_forward(model, li, h, pos, k_cache, v_cache, t, gemv)
        if trace is not None:
            trace.append(t)
    if trace is not None:
        trace.append({"h": h})
    if not lm_head:
        return None, None
    logits = lm_head_forward(model, h, gemv)
    return logits, argmax_first(logits)


def host_model(eng) -> dict:
    """Host copies of a DecodeEngine's weights in the layout decode_step reads
    (tensors copied with .cpu().numpy(); nothing else of the engine is used)."""
    def h(t):
        return t.cpu().numpy()

    layers = []
    for L in eng.layers:
        layers.append({n: (h(L[n][0]), h(L[n][1])) for n in ("qkv", "o", "gu", "down")} |
                      {"rms_att": h(L["rms_att"]), "rms_ffn": h(L["rms_ffn"])})
    return {"cfg": eng.cfg, "layers": layers, "embed": h(eng.embed), "rms_out": h(eng.rms_out),
            "lm_meta": h(eng.lm_meta), "lm_quant": h(eng.lm_quant),
            "rope_cos": h(eng.rope_cos), "rope_sin": h(eng.rope_sin)}
