"""HIP parity for the decode step (A13): the fused GEMV prologues (residual add
+ RMSNorm, SwiGLU), the argmax epilogue, RoPE + KV write + attention over an
fp16 cache, and whole greedy steps of a Phi-4-shaped model, all against
oracle/decode.py.

Bars (written here as in the task statement): every GEMV and the attention
output within 1e-4 relative L2 of the oracle; the residual stream written by
the fused prologue bit-exact; the decode step's logits within 1e-3 relative L2
with the same greedy tokens; a captured graph replays bitwise equal to the
eager step.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from oracle import decode as od
from asdsl.quantization import synthetic as syn
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _packed(M, K, gs, seed):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn((M, K), generator=g, device="cuda") * 0.02
    return syn.preq2_from_weights_torch(w, gs)


def _host(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("gs,M,K", [(32, 5120, 3072), (128, 16384, 3072), (128, 1000, 640)])
def test_rmsnorm_gemv_matches_oracle(gpu, gs, M, K):
    import torch
    from asdsl import _hip

    meta, quant = _packed(M, K, gs, M + K)
    rng = np.random.default_rng(K)
    h = rng.standard_normal(K).astype(np.float32) * 3
    d = rng.standard_normal(K).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    dh, dd, dw = (torch.from_numpy(a).cuda() for a in (h, d, w))
    hout = torch.empty(K, device="cuda")
    y = torch.empty(M, device="cuda")
    _hip.call("asdsl_gemv_preq2_rmsnorm", _hip.ptr(meta), _hip.ptr(quant), _hip.ptr(dh), _hip.ptr(dd), _hip.ptr(dw),
              _hip.ptr(hout), _hip.ptr(y), M, K, gs, 1e-5, None, _hip.stream_handle())
    torch.cuda.synchronize()
    assert np.array_equal(_host(hout).view(np.uint32), (h + d).view(np.uint32))
    want = oracle.gemv_preq2_fused(_host(meta), _host(quant), od.rmsnorm(h + d, w, 1e-5), M, K, gs)
    assert rel_l2(_host(y), want) < TOL


def test_argmax_epilogue_first_row_on_ties(gpu):
    """Rows 700 and 900 are identical copies of the largest row: the key must
    name row 700; without delta, h_out untouched."""
    import torch
    from asdsl import _hip

    M, K, gs = 2000, 3072, 128
    g = torch.Generator(device="cuda").manual_seed(3)
    w = torch.randn((M, K), generator=g, device="cuda") * 0.02
    x = torch.randn(K, generator=g, device="cuda")
    nw = torch.ones(K, device="cuda")
    w[700] = x * 0.05
    w[900] = w[700]
    meta, quant = syn.preq2_from_weights_torch(w, gs)
    y = torch.empty(M, device="cuda")
    key = torch.zeros(1, dtype=torch.int64, device="cuda")
    _hip.call("asdsl_gemv_preq2_rmsnorm", _hip.ptr(meta), _hip.ptr(quant), _hip.ptr(x), None, _hip.ptr(nw), None,
              _hip.ptr(y), M, K, gs, 1e-5, _hip.ptr(key), _hip.stream_handle())
    torch.cuda.synchronize()
    yh = _host(y)
    row = 0xFFFFFFFF - (int(key.item()) & 0xFFFFFFFF)
    assert row == od.argmax_first(yh) == 700
    assert yh[700] == yh[900]


@pytest.mark.parametrize("gs,F,K,thr", [(128, 8192, 3072, 0.0), (32, 8192, 3072, 0.05), (128, 1024, 640, 0.0)])
def test_gateup_swiglu_epilogue(gpu, gs, F, K, thr):
    """gate_up with the residual + RMSNorm prologue and SwiGLU epilogue: the
    residual stream bit-exact, s bit for bit swiglu of the plain norm-fed
    GEMV's [gate | up] outputs (same rows, same per-row arithmetic), and
    within 1e-4 of the oracle."""
    import torch
    from asdsl import _hip

    meta, quant = _packed(2 * F, K, gs, F + K + gs)
    rng = np.random.default_rng(F)
    h = rng.standard_normal(K).astype(np.float32) * 3
    d = rng.standard_normal(K).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    dh, dd, dw = (torch.from_numpy(a).cuda() for a in (h, d, w))
    hout = torch.empty(K, device="cuda")
    s_out = torch.empty(F, device="cuda")
    gu = torch.empty(2 * F, device="cuda")
    P, st = _hip.ptr, _hip.stream_handle()
    _hip.call("asdsl_gemv_preq2_rmsnorm_swiglu", P(meta), P(quant), P(dh), P(dd), P(dw), P(hout), P(s_out), F, K, gs,
              1e-5, thr, st)
    _hip.call("asdsl_gemv_preq2_rmsnorm", P(meta), P(quant), P(dh), P(dd), P(dw), None, P(gu), 2 * F, K, gs, 1e-5,
              None, st)
    torch.cuda.synchronize()
    assert np.array_equal(_host(hout).view(np.uint32), (h + d).view(np.uint32))
    g = _host(gu)
    assert np.array_equal(_host(s_out).view(np.uint32), od.swiglu(g[:F], g[F:], thr).view(np.uint32))
    want_gu = oracle.gemv_preq2_fused(_host(meta), _host(quant), od.rmsnorm(h + d, w, 1e-5), 2 * F, K, gs)
    assert rel_l2(_host(s_out), od.swiglu(want_gu[:F], want_gu[F:], thr)) < TOL


@pytest.mark.parametrize("gs,thr", [(128, 0.0), (32, 0.0), (128, 0.05)])
def test_swiglu_gemv_matches_oracle(gpu, gs, thr):
    import torch
    from asdsl import _hip

    M, K = 3072, 8192
    meta, quant = _packed(M, K, gs, 77 + gs)
    gu = (np.random.default_rng(5).standard_normal(2 * K) * 2).astype(np.float32)
    y = torch.empty(M, device="cuda")
    dgu = torch.from_numpy(gu).cuda()
    _hip.call("asdsl_gemv_preq2_swiglu", _hip.ptr(meta), _hip.ptr(quant), _hip.ptr(dgu), _hip.ptr(y), M, K, gs, thr,
              _hip.stream_handle())
    torch.cuda.synchronize()
    want = oracle.gemv_preq2_fused(_host(meta), _host(quant), od.swiglu(gu[:K], gu[K:], thr), M, K, gs)
    assert rel_l2(_host(y), want) < TOL


@pytest.mark.parametrize("pos,max_seq", [(0, 1600), (1, 1600), (127, 1600), (128, 1600), (129, 1600), (383, 1600),
                                         (1500, 1600), (4100, 4224), (9000, 9100)])
def test_attention_rope_kv_matches_oracle(gpu, pos, max_seq):
    """RoPE, the KV write and attention at 1 to 141 splits of 64 positions
    (past 16 splits the combine folds runs of splits in up to 8 parallel
    groups; at 141 each group takes two chunks)."""
    import torch
    from asdsl import _hip
    from asdsl.engine import rope_tables

    nh, nkv, hd, rot = 24, 8, 128, 96
    rng = np.random.default_rng(pos)
    qkv = rng.standard_normal((nh + 2 * nkv) * hd).astype(np.float32)
    kc = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    vc = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    cos, sin = rope_tables(max_seq, rot)
    d = {k: torch.from_numpy(v).cuda() for k, v in dict(qkv=qkv, kc=kc, vc=vc, cos=cos, sin=sin).items()}
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    att = torch.empty(nh * hd, device="cuda")
    work = torch.zeros(_hip.LIB.asdsl_attention_work_floats(nh, max_seq), device="cuda")
    _hip.call("asdsl_attention_f16kv", _hip.ptr(d["qkv"]), _hip.ptr(d["kc"]), _hip.ptr(d["vc"]), _hip.ptr(d["cos"]),
              _hip.ptr(d["sin"]), _hip.ptr(dpos), _hip.ptr(att), _hip.ptr(work), nh, nkv, hd, rot, max_seq,
              _hip.stream_handle())
    torch.cuda.synchronize()
    q = od.rope(qkv[: nh * hd].reshape(nh, hd), cos[pos], sin[pos])
    k = od.rope(qkv[nh * hd:(nh + nkv) * hd].reshape(nkv, hd), cos[pos], sin[pos])
    v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, pos], vc2[:, pos] = k.astype(np.float16), v.astype(np.float16)
    got_k, got_v = _host(d["kc"]), _host(d["vc"])
    # the written rows: fp16 of the rotated k (one fp16 ulp: the kernel fuses
    # the rotation's multiply-add) and of v (exact); other rows untouched
    np.testing.assert_allclose(got_k[:, pos].astype(np.float32), kc2[:, pos].astype(np.float32), rtol=1e-3, atol=1e-3)
    assert np.array_equal(got_v[:, pos], vc2[:, pos])
    mask = np.ones(max_seq, bool)
    mask[pos] = False
    assert np.array_equal(got_k[:, mask], kc[:, mask]) and np.array_equal(got_v[:, mask], vc[:, mask])
    want = od.attention(q, got_k[:, : pos + 1].astype(np.float32), got_v[:, : pos + 1].astype(np.float32), nkv)
    assert rel_l2(_host(att), want.reshape(-1)) < TOL


def _small_engine(n_layers=2, vocab=8192, max_seq=512, seed=0):
    from asdsl.engine import DecodeConfig, DecodeEngine

    cfg = DecodeConfig(n_layers=n_layers, vocab=vocab, max_seq=max_seq)
    return DecodeEngine.synthetic(cfg, seed=seed)


def _oracle_model(eng):
    c = eng.cfg
    layers = []
    for L in eng.layers:
        layers.append({n: (_host(L[n][0]), _host(L[n][1])) for n in ("qkv", "o", "gu", "down")} |
                      {"rms_att": _host(L["rms_att"]), "rms_ffn": _host(L["rms_ffn"])})
    return {"cfg": c, "layers": layers, "embed": _host(eng.embed), "rms_out": _host(eng.rms_out),
            "lm_meta": _host(eng.lm_meta), "lm_quant": _host(eng.lm_quant),
            "rope_cos": _host(eng.rope_cos), "rope_sin": _host(eng.rope_sin)}


def test_decode_steps_match_oracle(gpu):
    """Two Phi-4-shaped layers (hidden 3072, 24/8 heads, FFN 8192, qkv/o at
    gs 32, MLP and lm_head at gs 128), vocab 8192, a 100-position random fp16
    KV prefix, three greedy steps: logits within 1e-3 and the same tokens."""
    import torch

    eng = _small_engine()
    ctx = 100
    eng.prefill_kv_random(ctx, seed=4)
    model = _oracle_model(eng)
    kc = [_host(L["k_cache"]) for L in eng.layers]
    vc = [_host(L["v_cache"]) for L in eng.layers]
    tok = 1234
    eng.token.fill_(tok)
    for step in range(3):
        pos = ctx + step
        want_logits, want_next = od.decode_step(model, tok, pos, kc, vc)
        eng._queue_step(int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        got = _host(eng.logits)
        assert rel_l2(got, want_logits) < 1e-3, step
        assert eng.next_token() == want_next, step
        assert int(eng.pos.item()) == pos + 1
        tok = want_next


@pytest.mark.parametrize("ctx", [127, 129, 2100, 4100])
def test_decode_long_context_matches_oracle(gpu, ctx):
    """One layer at contexts whose attention spans 2, 3, 33 and 65 splits of
    64 positions (the combine folds them in one group, one group, three and
    five parallel groups of at most 16), two steps each: logits within 1e-3
    and the same tokens."""
    import torch

    eng = _small_engine(n_layers=1, vocab=4096, max_seq=4224, seed=ctx)
    eng.prefill_kv_random(ctx, seed=5)
    model = _oracle_model(eng)
    kc = [_host(L["k_cache"]) for L in eng.layers]
    vc = [_host(L["v_cache"]) for L in eng.layers]
    tok = 321
    eng.token.fill_(tok)
    eng.pos.fill_(ctx)
    for step in range(2):
        pos = ctx + step
        want_logits, want_next = od.decode_step(model, tok, pos, kc, vc)
        eng._queue_step(int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert rel_l2(_host(eng.logits), want_logits) < 1e-3, (ctx, step)
        assert eng.next_token() == want_next, (ctx, step)
        tok = want_next


@pytest.mark.parametrize("max_seq,ctx", [(300, 150), (1600, 1400), (3000, 2500)])
def test_graph_replay_matches_eager_steps(gpu, max_seq, ctx):
    """Eager steps, each queued for its position's range as the engine
    captures it (below 512 the splits merged in o_proj's prologue, beyond the
    combine kernel), against a captured graph replayed three times: bitwise
    equal."""
    import torch

    eng = _small_engine(n_layers=1, vocab=4096, max_seq=max_seq, seed=9)
    eng.prefill_kv_random(ctx, seed=2)
    snap = [(L["k_cache"].clone(), L["v_cache"].clone()) for L in eng.layers]
    eng.token.fill_(17)
    eager = []
    for i in range(3):
        eng._queue_step(int(torch.cuda.current_stream().cuda_stream), eng._pos_limit(ctx + i))
        eager.append((eng.logits.clone(), eng.next_token()))
    # reset and replay a captured step three times
    for L, (k, v) in zip(eng.layers, snap):
        L["k_cache"].copy_(k)
        L["v_cache"].copy_(v)
    eng.token.fill_(17)
    eng.pos.fill_(ctx)
    eng.capture()
    for i in range(3):
        eng.step()
        torch.cuda.synchronize()
        assert torch.equal(eng.logits, eager[i][0]), i
        assert eng.next_token() == eager[i][1]
    assert int(eng.pos.item()) == ctx + 3


@pytest.mark.parametrize("ctx", [0, 130, 255])
def test_short_form_gives_the_general_steps_bits(gpu, ctx):
    """A position below 256 through the step queued for positions below 256
    (attention splits merged in o_proj's prologue) and through the general
    step (queued for any position of a 600-position cache: the long form and
    the combine kernel), two layers: the same logits, token and K/V rows bit
    for bit."""
    import torch

    eng = _small_engine(n_layers=2, vocab=4096, max_seq=600, seed=ctx + 1)
    eng.prefill_kv_random(ctx, seed=9)
    snap = [(L["k_cache"].clone(), L["v_cache"].clone()) for L in eng.layers]
    out = []
    for limit in (256, 600):
        for L, (k, v) in zip(eng.layers, snap):
            L["k_cache"].copy_(k)
            L["v_cache"].copy_(v)
        eng.token.fill_(33)
        eng.pos.fill_(ctx)
        eng._queue_step(int(torch.cuda.current_stream().cuda_stream), limit)
        torch.cuda.synchronize()
        out.append((_host(eng.logits), eng.next_token(), [_host(L["k_cache"][:, ctx]) for L in eng.layers]))
    (la, ta, ka), (lb, tb, kb) = out
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)) and ta == tb
    assert all(np.array_equal(x, y) for x, y in zip(ka, kb))


def test_forward_token_api(gpu):
    eng = _small_engine(n_layers=1, vocab=4096, max_seq=256, seed=3)
    eng.prefill_kv_random(10)
    logits = eng.forward_token(5, 10)
    assert tuple(logits.shape) == (4096,) and logits.is_cuda
    assert eng.next_token() == int(logits.argmax().item())
    with pytest.raises(ValueError):
        eng.forward_token(4096, 0)
    with pytest.raises(ValueError):
        eng.forward_token(0, 256)



# Eight greedy steps from position 250 of a two-layer model; the logits of
# every step are saved to OUT (set by the caller).
_FOLD_RUN = """
import numpy as np
import torch
from asdsl.engine import DecodeConfig, DecodeEngine

eng = DecodeEngine.synthetic(DecodeConfig(n_layers=2, vocab=4096, max_seq=512), seed=6)
eng.prefill_kv_random(250, seed=3)
eng.token.fill_(99)
eng.pos.fill_(250)
out = []
for i in range(8):
    eng._queue_step(int(torch.cuda.current_stream().cuda_stream), eng._pos_limit(250 + i))
    torch.cuda.synchronize()
    out.append(eng.logits.cpu().numpy().copy())
np.save(OUT, np.stack(out))
"""


def test_combine_fold_gives_the_combine_kernels_bits(gpu, tmp_path):
    """Positions 250..257 (4 splits of 64, then 5; steps shaped for
    positions below 256, then below 512): the o_proj GEMV's prologue merges
    the attention splits.  A run that leaves the merge to the combine kernel
    everywhere (ASDSL_HIP_NO_COMBINE_FOLD=1, read once per process, so in a
    second process) gives the same logits bit for bit at every position."""
    import os
    import subprocess
    import sys

    from conftest import REPO

    here, there = tmp_path / "fold.npy", tmp_path / "nofold.npy"
    exec(compile(_FOLD_RUN, "fold_run", "exec"), {"OUT": str(here)})
    env = dict(os.environ, ASDSL_HIP_NO_COMBINE_FOLD="1",
               PYTHONPATH=os.pathsep.join([str(REPO), str(REPO / "asdsl-framework_amd"),
                                           os.environ.get("PYTHONPATH", "")]))
    subprocess.run([sys.executable, "-c", f"OUT = {str(there)!r}\n" + _FOLD_RUN], env=env, check=True, timeout=100)
    a, b = np.load(here), np.load(there)
    assert a.shape == (8, 4096) and np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
