"""Weight caches uploaded to the device and turned into the decode step's
operands there: the preq cache at group size 32 (20-byte blocks, qkv/o) and
128 (Q4_128 blocks, gate_up/down), and the lm_head preq2 cache, restored with
``device=`` and repacked by the HIP kernels; the operands byte-equal to the
oracle's repack of the same file, and a decode step on them within the
decode tolerance of the oracle."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

import oracle
from oracle import decode as od
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _host(t):
    return t.cpu().numpy()


def test_caches_to_decode_engine(gpu, tmp_path, monkeypatch):
    import torch

    from asdsl.engine import DecodeConfig, DecodeEngine, PROJ_NAMES, _layer_mats, layers_from_preq_blocks
    from asdsl.quantization import lmhead_preq2_cache as lc
    from asdsl.quantization import preq_cache as pc
    from asdsl.quantization import repack as rp

    monkeypatch.delenv("ASDSL_LMHEAD_GS", raising=False)
    monkeypatch.delenv("PHI4_NO_LMHEAD_PREQ2_CACHE", raising=False)
    cfg = DecodeConfig(n_layers=1, vocab=4096, max_seq=256)
    rng = np.random.default_rng(3)
    st32, st128 = pc.PreqStore(group_size=32), pc.PreqStore(group_size=128)
    for n, (rows, cols, gs) in _layer_mats(cfg).items():
        key = (0, PROJ_NAMES[n])
        if gs == 32:  # asymmetric weights -> 20-byte preq blocks (the reference's cache build)
            q = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
            packed = ((q[:, 1::2] << 4) | q[:, 0::2]).astype(np.uint8)
            sc = rng.uniform(0.0005, 0.002, (rows, cols // 32)).astype(np.float32)
            bi = (-7.5 * sc).astype(np.float32)
            blocks = rp.repack_asymmetric_to_q4_32_blocks(packed, sc, bi, rows, cols).reshape(-1)
            st = st32
        else:  # fp32 weights -> Q4_128 blocks
            w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
            blocks = rp.repack_fp32_to_q4_128_blocks(w, rows, cols).reshape(-1)
            st = st128
        st._quant_shapes[key] = (rows, cols)
        st._preq_blocks_np[key] = blocks
    pc.save_preq_cache(st32, tmp_path / "p32.safetensors")
    pc.save_preq_cache(st128, tmp_path / "p128.safetensors")
    lm_w = (rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.02).astype(np.float32)
    lm_meta_h, lm_quant_h = rp.quantize_preq2(lm_w, 128)
    store_lm = SimpleNamespace(group_size=128, lm_head=lm_w)
    lc.save_lmhead_preq2_cache(store_lm, tmp_path / "lm.safetensors", lm_meta_h, lm_quant_h)

    d32 = pc.PreqStore(group_size=32, _quant_shapes=dict(st32._quant_shapes))
    d128 = pc.PreqStore(group_size=128, _quant_shapes=dict(st128._quant_shapes))
    assert pc.try_restore_preq_cache(d32, tmp_path / "p32.safetensors", device="cuda")
    assert pc.try_restore_preq_cache(d128, tmp_path / "p128.safetensors", device="cuda")
    assert all(t.is_cuda for t in d32._preq_blocks_dev.values())
    lm = lc.try_restore_lmhead_preq2_cache(store_lm, tmp_path / "lm.safetensors", device="cuda")
    assert lm is not None and lm[0].is_cuda
    assert np.array_equal(_host(lm[0]), lm_meta_h) and np.array_equal(_host(lm[1]), lm_quant_h)

    g = torch.Generator(device="cuda").manual_seed(5)
    norms = [(1 + 0.1 * torch.randn(cfg.hidden, generator=g, device="cuda"),
              1 + 0.1 * torch.randn(cfg.hidden, generator=g, device="cuda"))]
    layers = layers_from_preq_blocks(cfg, {**d32._preq_blocks_dev, **d128._preq_blocks_dev}, norms)
    for n, (rows, cols, gs) in _layer_mats(cfg).items():
        hb = (st32 if gs == 32 else st128)._preq_blocks_np[(0, PROJ_NAMES[n])]
        want = oracle.repack_preq_to_preq2(hb, rows, cols) if gs == 32 else \
            oracle.repack_q4_128_to_preq2(hb, rows, cols)
        assert np.array_equal(_host(layers[0][n][0]), want[0]) and np.array_equal(_host(layers[0][n][1]), want[1]), n

    embed = (torch.randn((cfg.vocab, cfg.hidden), generator=g, device="cuda")).half()
    rms_out = 1 + 0.1 * torch.randn(cfg.hidden, generator=g, device="cuda")
    eng = DecodeEngine(cfg, layers, embed, rms_out, lm[0], lm[1])
    eng.prefill_kv_random(40, seed=2)
    model = {"cfg": cfg, "embed": _host(embed), "rms_out": _host(rms_out), "lm_meta": lm_meta_h,
             "lm_quant": lm_quant_h, "rope_cos": _host(eng.rope_cos), "rope_sin": _host(eng.rope_sin),
             "layers": [{n: (_host(layers[0][n][0]), _host(layers[0][n][1])) for n in ("qkv", "o", "gu", "down")} |
                        {"rms_att": _host(norms[0][0]), "rms_ffn": _host(norms[0][1])}]}
    kc, vc = [_host(eng.layers[0]["k_cache"])], [_host(eng.layers[0]["v_cache"])]
    want_logits, want_next = od.decode_step(model, 77, 40, kc, vc)
    eng.token.fill_(77)
    eng._queue_step(int(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rel_l2(_host(eng.logits), want_logits) < 1e-3
    assert eng.next_token() == want_next
