"""CPU oracle of one batch-1 decode step — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's UnifiedEngine::forward_token
(asdsl/kernels/native/unified_engine.cpp:1339-1688) on the fused-preq path, with
the GEMVs taken from the oracle's C restatement (oracle.gemv_preq2_fused):

    h = embed[token]                                        (load_embed_row_f32, 181-197)
    per layer:
        x   = rmsnorm(h, rms_att)                           (rmsnorm_f32, 499-524)
        qkv = gemv_preq2_fused(qkv, x)                      (1399-1401)
        q, k = rope(q), rope(k)                             (rope_apply_inplace, 768-801)
        cache[pos] = k, v (fp16 here; int8 per 64 in the reference, 859-920)
        att = softmax(q.K / sqrt(128)) V over 0..pos         (compute_attention_flash_q8, 922-1027)
        h   = h + gemv_preq2_fused(o, att)                  (1487-1489, residual_add_rmsnorm_f32 651-688)
        gu  = gemv_preq2_fused(gate_up, rmsnorm(h, rms_ffn))
        h   = h + gemv_preq2_fused(down, swiglu(gate, up))  (swiglu_inplace 803-857, vec_add 487-497)
    logits = gemv_preq2_fused(lm_head, rmsnorm(h, rms_out)); next = argmax (207-233)

Every array is float32 as in the reference; the new K/V are rounded to fp16
before attention, as if read back from the cache.
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


def rope(heads: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    """Half-split rotation of the first 2*len(cos_row) dims of every head row:
    (x_i, x_{i+h}) -> (x_i c - x_{i+h} s, x_i s + x_{i+h} c)."""
    out = heads.astype(F32).copy()
    h = cos_row.size
    xf = heads[:, :h].astype(F32)
    xs = heads[:, h:2 * h].astype(F32)
    out[:, :h] = xf * cos_row - xs * sin_row
    out[:, h:2 * h] = xf * sin_row + xs * cos_row
    return out


def fast_exp(x: np.ndarray) -> np.ndarray:
    """fast_exp_avx2 (unified_engine.cpp:781-801): clamp to +-87.3, x*log2(e) =
    i + f with i = round-half-even(x*log2(e)), 2^f by a degree-5 polynomial."""
    x = np.clip(x.astype(F32), F32(-87.3), F32(87.3))
    x = (x * F32(1.4426950408889634)).astype(F32)
    fi = np.rint(x).astype(F32)
    f = (x - fi).astype(F32)
    p = F32(0.001333838100523091) * f + F32(0.009618129107628477)
    p = p * f + F32(0.05550410866482158)
    p = p * f + F32(0.2402265069591007)
    p = p * f + F32(0.6931471805599453)
    p = p * f + F32(1.0)
    two_i = ((fi.astype(np.int32) + 127) << 23).astype(np.int32).view(F32)
    return (p.astype(F32) * two_i).astype(F32)


def swiglu(gate: np.ndarray, up: np.ndarray, threshold: float = 0.0) -> np.ndarray:
    """swiglu_inplace: v = (g * 1/(1 + fast_exp(-g))) * u; |v| < threshold -> 0."""
    g = gate.astype(F32)
    sig = F32(1.0) / (F32(1.0) + fast_exp(-g))
    v = ((g * sig) * up.astype(F32)).astype(F32)
    if threshold > 0.0:
        v[np.abs(v) < F32(threshold)] = F32(0.0)
    return v


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_kv: int) -> np.ndarray:
    """q [n_heads][d]; k, v [n_kv][T][d] (already fp16-rounded floats).
    out[h] = softmax(q_h . k / sqrt(d)) v of kv head h // (n_heads / n_kv)."""
    n_heads, d = q.shape
    g = n_heads // n_kv
    out = np.empty((n_heads, d), F32)
    for h in range(n_heads):
        kk = k[h // g].astype(np.float64)
        s = kk @ q[h].astype(np.float64) / np.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w @ v[h // g].astype(np.float64) / w.sum()).astype(F32)
    return out


def argmax_first(x: np.ndarray) -> int:
    """argmax_f32_avx2: the first index of the maximum."""
    return int(np.argmax(x))


def decode_step(model: dict, token: int, pos: int, k_cache: list, v_cache: list) -> tuple[np.ndarray, int]:
    """One greedy step.  model: host copies of the engine's weights (see
    tests/test_gpu_decode.py); k_cache/v_cache: per layer fp16 arrays
    [n_kv][max_seq][128], updated at `pos` in place."""
    c = model["cfg"]
    hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
    cos_row, sin_row = model["rope_cos"][pos], model["rope_sin"][pos]
    h = model["embed"][token].astype(F32)
    for li, L in enumerate(model["layers"]):
        x = rmsnorm(h, L["rms_att"], c.rms_eps)
        qkv = oracle.gemv_preq2_fused(*L["qkv"], x, c.qkv_dim, c.hidden, c.gs_attn)
        q = rope(qkv[: nh * hd].reshape(nh, hd), cos_row, sin_row)
        k = rope(qkv[nh * hd:(nh + nkv) * hd].reshape(nkv, hd), cos_row, sin_row)
        v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
        k_cache[li][:, pos] = k.astype(np.float16)
        v_cache[li][:, pos] = v.astype(np.float16)
        att = attention(q, k_cache[li][:, :pos + 1].astype(F32), v_cache[li][:, :pos + 1].astype(F32), nkv)
        h = (h + oracle.gemv_preq2_fused(*L["o"], att.reshape(-1), c.hidden, nh * hd, c.gs_attn)).astype(F32)
        gu = oracle.gemv_preq2_fused(*L["gu"], rmsnorm(h, L["rms_ffn"], c.rms_eps), 2 * c.ffn, c.hidden, c.gs_ffn)
        s = swiglu(gu[: c.ffn], gu[c.ffn:], model.get("fatrelu_threshold", 0.0))
        h = (h + oracle.gemv_preq2_fused(*L["down"], s, c.hidden, c.ffn, c.gs_ffn)).astype(F32)
    logits = oracle.gemv_preq2_fused(model["lm_meta"], model["lm_quant"], rmsnorm(h, model["rms_out"], c.rms_eps),
                                     c.vocab, c.hidden, c.gs_lm)
    return logits, argmax_first(logits)
