"""Greedy batch-1 decode of a Phi-4-shaped model on the GPU.

Mirrors the reference's UnifiedEngine::forward_token
(asdsl/kernels/native/unified_engine.cpp:1339-1688, driven from Python by
asdsl/inference/unified_bridge.py): one call embeds a token, runs every
decoder layer at a position and produces the logits and the greedy next
token.  The whole step is one C-ABI call (asdsl_decode_token) that queues
6 kernels per layer; the token id and position live in device memory, so a
HIP graph of one step replays token after token.

Weights are preq2 Q4 (attention projections at group size 32, the MLP and
lm_head at 128 by default), norms fp32, embeddings and the KV cache fp16.
``DecodeEngine.synthetic`` builds a model with random weights of the given
shape (W ~ N(0, 0.02) quantized, embeddings ~ N(0, 1), norm weights 1 + N(0, 0.1));
``layers_from_preq_blocks`` builds the layer operands on the device from the
preq blocks of the reference's preq cache (asdsl.quantization.preq_cache).
"""

from __future__ import annotations

import ctypes
import os
import sys
from dataclasses import dataclass

import numpy as np

from asdsl import _hip


@dataclass
class DecodeConfig:
    """Model shape (Phi-4 defaults, experiments/phi4_cpu_run.py:316-334)."""

    hidden: int = 3072
    ffn: int = 8192
    vocab: int = 200064
    n_layers: int = 32
    n_heads: int = 24
    n_kv_heads: int = 8
    head_dim: int = 128
    rotary_dim: int = 96
    max_seq: int = 4352
    gs_attn: int = 32
    gs_ffn: int = 128
    gs_lm: int = 128
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    # "int8": the reference's KV cache (int8 codes, one fp32 scale per 64
    # dims; UnifiedEngine::set_kv_cache); "fp16": fp16 rows
    kv_format: str = "fp16"

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "qkv_meta", "qkv_quant", "o_meta", "o_quant", "gu_meta", "gu_quant", "down_meta", "down_quant",
        "rms_att", "rms_ffn", "k_cache", "v_cache")] + [("fatrelu_threshold", ctypes.c_float)] + [
        (n, ctypes.c_void_p) for n in ("k_scale", "v_scale")]


class _Model(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "hidden", "ffn", "vocab", "n_layers", "n_heads", "n_kv_heads", "head_dim", "rotary_dim", "max_seq",
        "gs_attn", "gs_ffn", "gs_lm")] + [("rms_eps", ctypes.c_float), ("layers", ctypes.POINTER(_Layer))] + [
        (n, ctypes.c_void_p) for n in ("embed", "rms_out", "lm_meta", "lm_quant", "rope_cos", "rope_sin")] + [
        ("kv_format", ctypes.c_int)]

KV_FORMATS = {"fp16": 0, "int8": 1}
KV_QBLOCK = 64  # dims per int8 cache scale


def rope_tables(max_seq: int, rotary_dim: int, theta: float = 10000.0) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin[pos][i] = cos/sin(pos * theta^(-2i/rotary_dim)) computed in float64,
    stored fp32 (the reference's _build_rope_native_tables,
    experiments/phi4_cpu_run.py:3318-3344)."""
    half = rotary_dim // 2
    i = np.arange(half, dtype=np.float64)
    freq = 1.0 / (theta ** (2.0 * i / rotary_dim))
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * freq[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# names of the per-layer matrices: (rows, cols, group size attribute)
def _layer_mats(cfg: DecodeConfig):
    return {"qkv": (cfg.qkv_dim, cfg.hidden, cfg.gs_attn), "o": (cfg.hidden, cfg.n_heads * cfg.head_dim, cfg.gs_attn),
            "gu": (2 * cfg.ffn, cfg.hidden, cfg.gs_ffn), "down": (cfg.hidden, cfg.ffn, cfg.gs_ffn)}


# the reference's projection names (experiments/phi4_cpu_run.py:628)
PROJ_NAMES = {"qkv": "qkv_proj", "o": "o_proj", "gu": "gate_up_proj", "down": "down_proj"}


def layers_from_preq_blocks(cfg: "DecodeConfig", blocks: dict, norms: list) -> list[dict]:
    """Layer operands for DecodeEngine from preq blocks on the device.

    blocks: {(layer, projection name): device uint8 tensor} as
    ``preq_cache.try_restore_preq_cache(store, path, device=...)`` leaves in
    ``store._preq_blocks_dev`` -- 20-byte Q4_32 blocks for projections at
    group size 32, 66-byte Q4_128 blocks at 128 (cfg.gs_attn for qkv/o,
    cfg.gs_ffn for gate_up/down).  norms: per layer (rms_att, rms_ffn) fp32
    device tensors.  The preq2 operands are built by the repack kernels on
    the current stream; nothing passes through host memory."""
    from asdsl.quantization.preq_cache import preq2_from_preq_blocks

    if len(norms) != cfg.n_layers:
        raise ValueError(f"layers_from_preq_blocks: {len(norms)} norm pairs for {cfg.n_layers} layers")
    layers = []
    for li in range(cfg.n_layers):
        L = {}
        for n, (rows, cols, gs) in _layer_mats(cfg).items():
            key = (li, PROJ_NAMES[n])
            if key not in blocks:
                raise ValueError(f"layers_from_preq_blocks: no preq blocks for layer {li} {PROJ_NAMES[n]}")
            L[n] = preq2_from_preq_blocks(blocks[key], rows, cols, gs)
        L["rms_att"], L["rms_ffn"] = norms[li]
        layers.append(L)
    return layers


GGUF_DEFAULT_MAX_SEQ = 4096  # KV positions a GGUF model gets unless max_seq is given


def config_from_gguf(metadata: dict, **overrides) -> DecodeConfig:
    """DecodeConfig from a GGUF file's metadata (``{arch}.embedding_length``,
    ``.feed_forward_length``, ``.block_count``, ``.attention.head_count``,
    ``.attention.head_count_kv``, ``.rope.dimension_count``,
    ``.context_length``, ``.attention.layer_norm_rms_epsilon``,
    ``.rope.freq_base``, with arch = ``general.architecture``); the
    vocabulary from the token list.  The KV cache holds
    min(context_length, GGUF_DEFAULT_MAX_SEQ = 4096) positions unless the
    caller passes max_seq: a file's trained context (131072 for Phi-4-mini)
    would otherwise allocate ~17 GB of fp16 cache and RoPE tables of that
    many rows.  Keyword overrides win."""
    arch = metadata.get("general.architecture", "phi3")

    def get(key, default=None):
        v = metadata.get(f"{arch}.{key}", default)
        if v is None:
            raise ValueError(f"GGUF metadata lacks {arch}.{key}")
        return v

    hidden, n_heads = int(get("embedding_length")), int(get("attention.head_count"))
    tokens = metadata.get("tokenizer.ggml.tokens")
    fields = dict(hidden=hidden, ffn=int(get("feed_forward_length")), n_layers=int(get("block_count")),
                  n_heads=n_heads, n_kv_heads=int(get("attention.head_count_kv", n_heads)),
                  head_dim=hidden // n_heads, rotary_dim=int(get("rope.dimension_count", hidden // n_heads)),
                  max_seq=min(int(get("context_length")), GGUF_DEFAULT_MAX_SEQ),
                  rms_eps=float(get("attention.layer_norm_rms_epsilon", 1e-5)),
                  rope_theta=float(get("rope.freq_base", 10000.0)))
    if tokens is not None:
        fields["vocab"] = len(tokens)
    fields.update(overrides)
    return DecodeConfig(**fields)


def _gguf_projection(info: dict, rows: int, cols: int, gs: int, what: str):
    """One GGUF weight -> preq2 (meta, quant) on the device: decoded to fp32
    (asdsl_dequant_gguf_*: any K-quant from Q2_K to Q6_K, Q4_0, Q4_1, Q5_0,
    Q5_1 or Q8_0), requantized to symmetric Q4 at group
    size gs (asdsl_quantize_q4_symmetric, the reference's load_from_gguf
    rule, experiments/phi4_cpu_run.py:1437-1466) and packed as preq2
    (asdsl_repack_asym_to_preq2, zero 7.5: the requantized weights exactly)."""
    import torch

    from asdsl.io.gguf_loader import dequant_tensor_device
    from asdsl.quantization._device_repack import asym_to_preq2

    got = tuple(info.get("logical_shape", ()))
    if got != (rows, cols):
        raise ValueError(f"GGUF {what}: shape {got}, expected {(rows, cols)}")
    w = dequant_tensor_device(info).contiguous()
    dev = w.device
    packed = torch.empty(rows * cols // 2, dtype=torch.uint8, device=dev)
    scales = torch.empty(rows * cols // gs, dtype=torch.float32, device=dev)
    biases = torch.empty_like(scales)
    _hip.call("asdsl_quantize_q4_symmetric", _hip.ptr(w), _hip.ptr(packed), _hip.ptr(scales), _hip.ptr(biases),
              rows, cols, gs, _hip.stream_handle())
    del w
    return asym_to_preq2(packed, scales, biases, rows, cols, gs)


def layers_from_gguf(cfg: DecodeConfig, tensors: dict) -> tuple[list[dict], dict]:
    """Decode-step operands from the tensors of a GGUF file (read_gguf_tensors).

    Per layer ``blk.{i}.``: attn_qkv, attn_output, the gate and up rows
    (ffn_gate_up, or ffn_up holding both as in Phi-3/4 conversions, or
    ffn_gate + ffn_up stacked), ffn_down -- Q2_K..Q6_K, Q4_0, Q4_1, Q5_0,
    Q5_1, Q8_0 or a float type, decoded and requantized on the GPU
    (_gguf_projection) -- and
    attn_norm / ffn_norm.
    Model-wide: token_embd (decoded, stored fp16), output_norm, and output
    (the embedding when absent: tied weights) as the lm_head at cfg.gs_lm.
    Returns (layers, {"embed", "rms_out", "lm_meta", "lm_quant"})."""
    import torch

    from asdsl.io.gguf_loader import dequant_tensor_device

    def need(name):
        if name not in tensors:
            raise ValueError(f"GGUF lacks {name}")
        return tensors[name]

    def norm(name):
        v = dequant_tensor_device(need(name)).reshape(-1).float().contiguous()
        if v.numel() != cfg.hidden:
            raise ValueError(f"GGUF {name}: {v.numel()} values, expected {cfg.hidden}")
        return v

    mats = _layer_mats(cfg)
    layers = []
    for i in range(cfg.n_layers):
        p = f"blk.{i}."
        L = {}
        for n, tname in (("qkv", "attn_qkv.weight"), ("o", "attn_output.weight"), ("down", "ffn_down.weight")):
            rows, cols, gs = mats[n]
            L[n] = _gguf_projection(need(p + tname), rows, cols, gs, p + tname)
        rows, cols, gs = mats["gu"]
        if p + "ffn_gate_up.weight" in tensors or (p + "ffn_up.weight" in tensors and p + "ffn_gate.weight" not in tensors):
            name = p + ("ffn_gate_up.weight" if p + "ffn_gate_up.weight" in tensors else "ffn_up.weight")
            L["gu"] = _gguf_projection(tensors[name], rows, cols, gs, name)
        else:
            g = dequant_tensor_device(need(p + "ffn_gate.weight"))
            u = dequant_tensor_device(need(p + "ffn_up.weight"))
            stacked = {"type": "f32", "shape": (cols, rows), "logical_shape": (rows, cols),
                       "data": torch.cat([g, u]).cpu().numpy().view(np.uint8).reshape(-1)}
            del g, u
            L["gu"] = _gguf_projection(stacked, rows, cols, gs, p + "ffn_gate+ffn_up")
        L["rms_att"], L["rms_ffn"] = norm(p + "attn_norm.weight"), norm(p + "ffn_norm.weight")
        layers.append(L)
    emb_info = need("token_embd.weight")
    embed = dequant_tensor_device(emb_info)
    if tuple(embed.shape) != (cfg.vocab, cfg.hidden):
        raise ValueError(f"GGUF token_embd.weight: shape {tuple(embed.shape)}, expected {(cfg.vocab, cfg.hidden)}")
    embed = embed.half().contiguous()
    out_info = tensors.get("output.weight", emb_info)
    lm_meta, lm_quant = _gguf_projection(out_info, cfg.vocab, cfg.hidden, cfg.gs_lm, "output.weight")
    return layers, {"embed": embed, "rms_out": norm("output_norm.weight"), "lm_meta": lm_meta, "lm_quant": lm_quant}


class DecodeEngine:
    """Holds the device weights, KV caches and step buffers of one model."""

    def __init__(self, cfg: DecodeConfig, layers: list[dict], embed, rms_out, lm_meta, lm_quant,
                 fatrelu_threshold: float = 0.0):
        import torch

        self.cfg = cfg
        dev = _hip.device()
        self.layers = layers
        self.embed, self.rms_out, self.lm_meta, self.lm_quant = embed, rms_out, lm_meta, lm_quant
        cos, sin = rope_tables(cfg.max_seq, cfg.rotary_dim, cfg.rope_theta)
        self.rope_cos = torch.from_numpy(cos).to(dev)
        self.rope_sin = torch.from_numpy(sin).to(dev)
        if cfg.kv_format not in KV_FORMATS:
            raise ValueError(f"kv_format must be one of {sorted(KV_FORMATS)}")
        self.kv_int8 = cfg.kv_format == "int8"
        for L in layers:
            if "k_cache" not in L:
                shape = (cfg.n_kv_heads, cfg.max_seq, cfg.head_dim)
                L["k_cache"] = torch.zeros(shape, dtype=torch.int8 if self.kv_int8 else torch.float16, device=dev)
                L["v_cache"] = torch.zeros_like(L["k_cache"])
                if self.kv_int8:  # zero_kv_from's state: codes 0, scales 1.0
                    L["k_scale"] = torch.ones(shape[:2] + (cfg.head_dim // KV_QBLOCK,), dtype=torch.float32,
                                              device=dev)
                    L["v_scale"] = torch.ones_like(L["k_scale"])
        self._c_layers = (_Layer * cfg.n_layers)()
        for i, L in enumerate(layers):
            c = self._c_layers[i]
            for n in ("qkv", "o", "gu", "down"):
                setattr(c, f"{n}_meta", _hip.ptr(L[n][0]))
                setattr(c, f"{n}_quant", _hip.ptr(L[n][1]))
            c.rms_att, c.rms_ffn = _hip.ptr(L["rms_att"]), _hip.ptr(L["rms_ffn"])
            c.k_cache, c.v_cache = _hip.ptr(L["k_cache"]), _hip.ptr(L["v_cache"])
            if self.kv_int8:
                c.k_scale, c.v_scale = _hip.ptr(L["k_scale"]), _hip.ptr(L["v_scale"])
            c.fatrelu_threshold = float(fatrelu_threshold)
        m = _Model()
        for n in ("hidden", "ffn", "vocab", "n_layers", "n_heads", "n_kv_heads", "head_dim", "rotary_dim",
                  "max_seq", "gs_attn", "gs_ffn", "gs_lm"):
            setattr(m, n, int(getattr(cfg, n)))
        m.rms_eps = float(cfg.rms_eps)
        m.layers = ctypes.cast(self._c_layers, ctypes.POINTER(_Layer))
        m.embed, m.rms_out = _hip.ptr(embed), _hip.ptr(rms_out)
        m.lm_meta, m.lm_quant = _hip.ptr(lm_meta), _hip.ptr(lm_quant)
        m.rope_cos, m.rope_sin = _hip.ptr(self.rope_cos), _hip.ptr(self.rope_sin)
        m.kv_format = KV_FORMATS[cfg.kv_format]
        self._model = m
        nbytes = _hip.LIB.asdsl_decode_work_bytes(ctypes.byref(m))
        if nbytes == 0:
            raise ValueError(f"invalid decode model: {_hip.last_error()}")
        # zeroed: the step's flags word lives in it (asdsl_decode_flags_offset)
        self.work = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        off = _hip.LIB.asdsl_decode_flags_offset(ctypes.byref(m))
        self._flags = self.work[off:off + 4].view(torch.int32)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.logits = torch.empty(cfg.vocab, dtype=torch.float32, device=dev)
        self._graphs: dict[int, object] = {}
        # HIP graphs of the reference-signature calls (forward_token per
        # position range, forward_batch_all_logits per token count), keyed
        # with the ASDSL_HIP_* switches in force when captured; off with
        # ASDSL_ENGINE_EAGER=1
        self._call_graphs: dict[tuple, object] = {}
        self.graph_calls = os.environ.get("ASDSL_ENGINE_EAGER", "") in ("", "0")
        self._host_pos = 0  # the device position as the host last set or advanced it
        # committed KV length and its snapshot stack (UnifiedEngine::kv_seq_len_,
        # kv_snapshot_stack_), host-side like the reference's
        self.kv_seq_len = 0
        self._kv_snapshots: list[int] = []
        self._verify = None  # work, token, logits and next-token buffers of the verify pass
        # ASDSL_ENGINE_PROFILE / ASDSL_ENGINE_PROFILE_TOKEN, read like the
        # reference's engine_profile_enabled/_target_token
        # (asdsl/kernels/native/unified_engine.cpp:71-87): the target decode
        # step (counted from 1) runs eagerly with per-stage timing.
        flag = os.environ.get("ASDSL_ENGINE_PROFILE", "")
        self._profile_token = int(os.environ.get("ASDSL_ENGINE_PROFILE_TOKEN", "3")) if flag[:1] not in ("", "0") \
            else None
        self._decode_idx = 0
        self.last_profile: dict | None = None

    # ------------------------------------------------------------ building
    @classmethod
    def synthetic(cls, cfg: DecodeConfig, seed: int = 0, fatrelu_threshold: float = 0.0) -> "DecodeEngine":
        import torch

        from asdsl.quantization.synthetic import preq2_from_weights_torch

        dev = _hip.device()
        gen = torch.Generator(device=dev).manual_seed(seed)

        def packed(rows, cols, gs):
            w = torch.randn((rows, cols), generator=gen, device=dev, dtype=torch.float32) * 0.02
            out = preq2_from_weights_torch(w, gs)
            del w
            return out

        def norm_w():
            return 1.0 + 0.1 * torch.randn(cfg.hidden, generator=gen, device=dev, dtype=torch.float32)

        layers = []
        for _ in range(cfg.n_layers):
            L = {n: packed(r, c, g) for n, (r, c, g) in _layer_mats(cfg).items()}
            L["rms_att"], L["rms_ffn"] = norm_w(), norm_w()
            layers.append(L)
        embed = torch.randn((cfg.vocab, cfg.hidden), generator=gen, device=dev, dtype=torch.float32).half()
        lm_meta, lm_quant = packed(cfg.vocab, cfg.hidden, cfg.gs_lm)
        return cls(cfg, layers, embed, norm_w(), lm_meta, lm_quant, fatrelu_threshold)

    @classmethod
    def from_gguf(cls, path, cfg: DecodeConfig | None = None, fatrelu_threshold: float = 0.0,
                  **overrides) -> "DecodeEngine":
        """A model from a GGUF file (its configuration from the file's
        metadata unless cfg is given; overrides such as max_seq, gs_ffn or
        kv_format apply to either).  The reference loads GGUF projections the
        same way (experiments/phi4_cpu_run.py:1316-1466: K-quant decode,
        symmetric Q4 requantization) but keeps the embeddings and norms of
        its HF checkpoint; here they come from the file too."""
        from dataclasses import replace

        from asdsl.io.gguf_loader import GGUFFile, read_gguf_tensors

        cfg = config_from_gguf(GGUFFile(path).metadata, **overrides) if cfg is None else replace(cfg, **overrides)
        layers, rest = layers_from_gguf(cfg, read_gguf_tensors(path))
        return cls(cfg, layers, rest["embed"], rest["rms_out"], rest["lm_meta"], rest["lm_quant"],
                   fatrelu_threshold)

    # A step is shaped for the positions it serves (asdsl_decode_token_upto):
    # below 512 the attention splits are merged in o_proj's prologue, beyond
    # by the combine kernel, and the attention launch covers only the splits
    # its range uses (4, 8, 16, 32).  One graph per range.
    POS_LIMITS = (256, 512, 1024, 2048)

    def _pos_limit(self, pos: int) -> int:
        c = self.cfg
        for limit in self.POS_LIMITS:
            if 0 <= pos < limit < c.max_seq:
                return limit
        return c.max_seq

    def prefill_kv_random(self, ctx: int, seed: int = 1) -> None:
        """Positions [0, ctx) of every layer's cache ~ N(0, 1) (fp16 rows, or
        int8 codes and scales quantized per 64 dims); the rest zeroed as
        truncate_kv leaves it.  The next step decodes at position ctx."""
        import torch

        if not 0 <= ctx < self.cfg.max_seq:
            raise ValueError(f"ctx must be in [0, {self.cfg.max_seq})")
        gen = torch.Generator(device=_hip.device()).manual_seed(seed)
        for L in self.layers:
            for n in ("k", "v"):
                cache = L[f"{n}_cache"]
                cache.zero_()
                if self.kv_int8:
                    L[f"{n}_scale"].fill_(1.0)
                if not ctx:
                    continue
                rows = torch.randn((self.cfg.n_kv_heads, ctx, self.cfg.head_dim), generator=gen,
                                   device=cache.device, dtype=torch.float32)
                if self.kv_int8:
                    cache[:, :ctx], L[f"{n}_scale"][:, :ctx] = kv_quantize_int8(rows)
                else:
                    cache[:, :ctx] = rows.half()
        self.pos.fill_(ctx)
        self._host_pos = ctx
        self.kv_seq_len = ctx

    # ------------------------------------------------------------ stepping
    def _queue_step(self, stream: int, pos_limit: int | None = None) -> None:
        """Queue one step; the device position must be below pos_limit
        (default: max_seq, any position)."""
        limit = self.cfg.max_seq if pos_limit is None else int(pos_limit)
        _hip.check(_hip.LIB.asdsl_decode_token_upto(ctypes.byref(self._model), _hip.ptr(self.token),
                                                    _hip.ptr(self.pos), limit, _hip.ptr(self.logits),
                                                    _hip.ptr(self.work), stream),
                   "asdsl_decode_token_upto")

    def forward_token(self, token_id: int, pos: int):
        """Reference: UnifiedEngine::forward_token(token_id, pos, logits).
        Returns the logits (device tensor); ``next_token()`` is their argmax."""
        if not 0 <= token_id < self.cfg.vocab:
            raise ValueError("forward_token: token_id out of vocab range")
        if not 0 <= pos < self.cfg.max_seq:
            raise ValueError("forward_token: pos out of kv-cache range")
        self.token.fill_(token_id)
        self.pos.fill_(pos)
        limit = self._pos_limit(pos)
        if self._profile_due():
            self._report(self.profile_step(limit))
        else:
            self._graph_call(("step", limit), lambda h: self._queue_step(h, limit))
        self._host_pos = pos + 1
        self.kv_seq_len = max(self.kv_seq_len, pos + 1)
        return self.logits

    # bits of the step's device flags word (include/asdsl_hip.h)
    FLAG_POS_LIMIT, FLAG_POS_RANGE = 1, 2

    def device_flags(self) -> int:
        """The flags the steps raised on the device since they were last
        cleared (0: none); reading waits for the queued steps."""
        return int(self._flags.item())

    def check_device_flags(self) -> None:
        """Raise RuntimeError (and clear the word) if a step ran at a
        position its launch did not cover: a captured graph replayed at or
        past the position range it was shaped for (FLAG_POS_LIMIT), or a
        position outside the KV cache (FLAG_POS_RANGE).  Such a step computed
        zero attention and wrote no K/V row, so its logits and token are not
        the model's.  Called at the engine's sync points (next_token,
        capture)."""
        f = self.device_flags()
        if f:
            self._flags.zero_()
            why = []
            if f & self.FLAG_POS_LIMIT:
                why.append("a step ran at a position past the range its graph was captured for")
            if f & self.FLAG_POS_RANGE:
                why.append("a step ran at a position outside the KV cache")
            raise RuntimeError("decode step: " + "; ".join(why) + f" (device flags 0x{f:x})")

    def next_token(self) -> int:
        import torch

        tok, flags = torch.stack((self.token[0], self._flags[0])).tolist()  # one device read
        if flags:
            self.check_device_flags()
        return int(tok)

    # Below this position the verify pass's columns are the single-token
    # step bit for bit (its attention splits coincide with the step's); from
    # it on the step's deep attention form splits differently.
    EXACT_BATCH_LIMIT = 2048

    def prefill(self, tokens) -> None:
        """The prompt tokens at positions 0, 1, ...: the K/V rows, the device
        token (the greedy token after the last one), the logits of the last
        token and the position that forward_token on each in turn leaves,
        bit for bit; below EXACT_BATCH_LIMIT positions as verify passes of up
        to MAX_VERIFY_TOKENS tokens (one pass instead of one step per token),
        the rest as single steps."""
        toks = [int(t) for t in tokens]
        pos = 0
        while pos < len(toks):
            n = min(self.MAX_VERIFY_TOKENS, len(toks) - pos, self.EXACT_BATCH_LIMIT - pos)
            if n >= 2:
                logits = self.forward_batch_all_logits(toks[pos:pos + n], pos)
                self.logits.copy_(logits[n - 1])
                self.token.copy_(self._verify["next"][n - 1:n])
                pos += n
            else:
                self.forward_token(toks[pos], pos)
                pos += 1

    def decode_steps(self, k: int) -> list[int]:
        """k greedy steps (step(), captured graphs) queued back to back from
        the device token at the device position, each step's token copied to
        a device history; returns the k tokens with one read, where k calls
        of next_token() and step() would read the device k times.  The host
        position advances by k; the caller's position must not pass max_seq."""
        import torch

        k = int(k)
        if k < 1:
            return []
        if self._host_pos + k > self.cfg.max_seq:
            raise ValueError("decode_steps: positions out of kv-cache range")
        hist = getattr(self, "_hist", None)
        if hist is None or hist.numel() < k + 1:
            hist = self._hist = torch.empty(max(k + 1, 64), dtype=torch.int32, device=self.token.device)
        for j in range(k):
            self.step()
            hist[j:j + 1].copy_(self.token)
        hist[k:k + 1].copy_(self._flags)
        out = hist[:k + 1].tolist()  # one device read
        self.kv_seq_len = max(self.kv_seq_len, self._host_pos)
        if out[k]:
            self.check_device_flags()
        return [int(t) for t in out[:k]]

    def capture(self) -> None:
        """HIP graph of one step (token and position advance on the device)
        for the current position's range (POS_LIMITS); the
        host's copy of the position is read back from the device here."""
        import torch

        self.check_device_flags()
        self._host_pos = int(self.pos.item())
        limit = self._pos_limit(self._host_pos)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        tok, pos = self.token.clone(), self.pos.clone()
        with torch.cuda.stream(side):
            self._queue_step(int(side.cuda_stream), limit)  # warm-up (also the library's one-time set-up)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.token.copy_(tok)
        self.pos.copy_(pos)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._queue_step(int(torch.cuda.current_stream().cuda_stream), limit)
        torch.cuda.synchronize()
        self.token.copy_(tok)
        self.pos.copy_(pos)
        self._graphs[limit] = g

    @property
    def _graph(self):
        return self._graphs.get(self._pos_limit(self._host_pos))

    @_graph.setter
    def _graph(self, value) -> None:
        if value is None:
            self._graphs.clear()

    def step(self) -> None:
        """One captured step: consumes self.token at self.pos, leaves the next
        greedy token and pos + 1.  The position is tracked on the host (set by
        prefill, forward_token, the verify pass and the KV bookkeeping, read
        back by capture()); a position set by writing self.pos directly needs
        a capture() before the next step."""
        if self._profile_due():
            self._report(self.profile_step())
            return
        if self._graph is None:
            self.capture()
        self._graph.replay()
        self._host_pos += 1

    def _graph_call(self, key: tuple, queue) -> None:
        """queue(stream) on the current stream: replayed from a HIP graph
        when one was captured for `key` under the same ASDSL_HIP_* switches;
        otherwise queued eagerly and then captured for the next call (the
        capture records the launches without running them).  The launches
        read their token(s) and position from device buffers, so one graph
        serves every call with the same key, with the eager call's bits."""
        import torch

        if not self.graph_calls or torch.cuda.is_current_stream_capturing():
            queue(_hip.stream_handle())
            return
        full = key + tuple(sorted((k, v) for k, v in os.environ.items() if k.startswith("ASDSL_HIP_")))
        g = self._call_graphs.get(full)
        if g is not None:
            g.replay()
            return
        queue(_hip.stream_handle())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            queue(int(torch.cuda.current_stream().cuda_stream))
        self._call_graphs[full] = g

    # ------------------------------------------------------------ profiling
    STAGES = ("embed", "qkv", "attention", "attention_combine", "o_proj", "gate_up", "down", "lm_head", "finalize")

    def profile_step(self, pos_limit: int | None = None) -> dict:
        """One step queued eagerly (the same launches a captured step
        replays; token and position advance on the device) with each launch
        timed by its own dispatch events (asdsl_profile_stages_begin/_end).
        Consumes self.token at the device position like step().  Returns ms
        per stage summed over layers, the launch count, and the span from the
        first launch's start to the last one's end; eager launches sit
        further apart than a graph's, so the span exceeds a replayed step's
        time."""
        limit = self._pos_limit(self._host_pos) if pos_limit is None else int(pos_limit)
        stages, span = _hip.profile_stages(lambda: self._queue_step(_hip.stream_handle(), limit),
                                           max_launches=16 * self.cfg.n_layers + 16)
        self._host_pos += 1
        per: dict[str, float] = {}
        for label, ms in stages:
            per[label] = per.get(label, 0.0) + ms
        return {"stages_ms": per, "launches": len(stages), "span_ms": span}

    def _profile_due(self) -> bool:
        if self._profile_token is None:
            return False
        self._decode_idx += 1
        return self._decode_idx == self._profile_token

    def _report(self, prof: dict) -> None:
        """The reference's ASDSL_ENGINE_PROFILE report
        (asdsl/kernels/native/unified_engine.cpp:1668-1687) on stderr: its
        keys (activation quantization and the norms run inside the GEMV
        prologues here, so those rows are 0), then what "other" holds."""
        st = prof["stages_ms"]
        gemv = {k: st.get(s, 0.0) for k, s in (("gate_up_gemv", "gate_up"), ("down_gemv", "down"),
                                                 ("qkv_gemv", "qkv"), ("o_gemv", "o_proj"))}
        lm = st.get("lm_head", 0.0)
        total = prof["span_ms"]
        other = max(0.0, total - sum(gemv.values()) - lm)
        prof = dict(prof, token=self._decode_idx, other_ms=other)
        self.last_profile = prof
        lines = [f"[ASDSL_ENGINE_PROFILE] decode token {self._decode_idx} (ms, {self.cfg.n_layers} layers):"]
        lines += [f"  {k} {v:.4f}" for k, v in gemv.items()]
        lines += ["  activation_q8 0 (in the GEMV prologues)", "  prep_fused 0 (in the GEMV prologues)",
                  f"  lm_head {lm:.4f}"]
        parts = ", ".join(f"{k} {st[k]:.4f}" for k in ("attention", "attention_combine", "finalize", "embed")
                          if k in st)
        lines += [f"  other {other:.4f} ({parts}; the rest is time between launches)",
                  f"  total {total:.4f} (eager launches, {prof['launches']} kernels)"]
        print("\n".join(lines), file=sys.stderr, flush=True)

    # ------------------------------------------------------------ verify
    MAX_VERIFY_TOKENS = 16

    def forward_batch_all_logits(self, tokens, start_pos: int):
        """Logits of every column of a multi-token pass (the speculative
        verify; the reference's UnifiedEngine::forward_verify_batch and its
        bridge call forward_batch_all_logits): tokens[i] at position
        start_pos + i, K/V written at those positions, the projections as
        batched GEMVs.  Returns a device tensor [n][vocab]; the greedy next
        token of each column is ``verify_next_tokens()``."""
        import torch

        toks = [int(t) for t in tokens]
        n = len(toks)
        c = self.cfg
        if not 1 <= n <= self.MAX_VERIFY_TOKENS:
            raise ValueError(f"forward_batch_all_logits: 1..{self.MAX_VERIFY_TOKENS} tokens, got {n}")
        if any(not 0 <= t < c.vocab for t in toks):
            raise ValueError("forward_batch_all_logits: token_id out of vocab range")
        if not (0 <= start_pos and start_pos + n <= c.max_seq):
            raise ValueError("forward_batch_all_logits: positions out of kv-cache range")
        if self._verify is None:
            dev = self.token.device
            nbytes = _hip.LIB.asdsl_decode_verify_work_bytes(ctypes.byref(self._model), self.MAX_VERIFY_TOKENS)
            if nbytes == 0:
                raise ValueError(f"invalid decode model: {_hip.last_error()}")
            self._verify = {
                "work": torch.empty(nbytes, dtype=torch.uint8, device=dev),
                "tokens": torch.zeros(self.MAX_VERIFY_TOKENS, dtype=torch.int32, device=dev),
                "next": torch.zeros(self.MAX_VERIFY_TOKENS, dtype=torch.int32, device=dev),
                "logits": torch.empty((self.MAX_VERIFY_TOKENS, c.vocab), dtype=torch.float32, device=dev),
            }
        v = self._verify
        v["tokens"][:n].copy_(torch.tensor(toks, dtype=torch.int32))
        self.pos.fill_(start_pos)

        def queue(h, n=n, v=v):
            _hip.check(_hip.LIB.asdsl_decode_verify(ctypes.byref(self._model), _hip.ptr(v["tokens"]), n,
                                                    _hip.ptr(self.pos), _hip.ptr(v["logits"]), _hip.ptr(v["next"]),
                                                    _hip.ptr(v["work"]), h),
                       "asdsl_decode_verify")
        self._graph_call(("verify", n), queue)
        self.pos.fill_(start_pos + n)
        self._host_pos = start_pos + n
        self.kv_seq_len = max(self.kv_seq_len, start_pos + n)
        self._verify_n = n
        return v["logits"][:n]

    forward_verify_batch = forward_batch_all_logits

    def verify_next_tokens(self) -> list[int]:
        """Greedy argmax of each column of the last multi-token pass."""
        return [int(t) for t in self._verify["next"][: self._verify_n].tolist()]

    # ------------------------------------------------------------ KV bookkeeping
    def get_kv_seq_len(self) -> int:
        return self.kv_seq_len

    def truncate_kv(self, new_len: int) -> None:
        """UnifiedEngine::truncate_kv (unified_engine.cpp:1298-1307): clamp to
        [0, max_seq], zero every layer's K/V rows from there on, set the
        committed length (and the device position) to it."""
        c = self.cfg
        new_len = min(max(int(new_len), 0), c.max_seq)
        for L in self.layers:
            if self.kv_int8:
                _hip.check(_hip.LIB.asdsl_kv_zero_from_q8(_hip.ptr(L["k_cache"]), _hip.ptr(L["v_cache"]),
                                                          _hip.ptr(L["k_scale"]), _hip.ptr(L["v_scale"]),
                                                          c.n_kv_heads, c.head_dim, c.max_seq, new_len,
                                                          _hip.stream_handle()),
                           "asdsl_kv_zero_from_q8")
            else:
                _hip.check(_hip.LIB.asdsl_kv_zero_from(_hip.ptr(L["k_cache"]), _hip.ptr(L["v_cache"]),
                                                       c.n_kv_heads, c.head_dim, c.max_seq, new_len,
                                                       _hip.stream_handle()),
                           "asdsl_kv_zero_from")
        self.kv_seq_len = new_len
        self.pos.fill_(new_len)
        self._host_pos = new_len

    def snapshot_kv(self) -> None:
        """Push the committed KV length (unified_engine.cpp:1285-1287)."""
        self._kv_snapshots.append(self.kv_seq_len)

    def restore_kv(self) -> None:
        """Pop the last snapshot and truncate to it; no-op without one
        (unified_engine.cpp:1289-1296)."""
        if self._kv_snapshots:
            self.truncate_kv(self._kv_snapshots.pop())

    def reset_session(self) -> None:
        """Empty KV cache and snapshot stack (unified_engine.cpp:1325-1337)."""
        self.truncate_kv(0)
        self._kv_snapshots.clear()

    # ------------------------------------------------------------ accounting
    def weight_bytes(self) -> int:
        n = 0
        for L in self.layers:
            for k in ("qkv", "o", "gu", "down"):
                n += L[k][0].numel() + L[k][1].numel()
            n += 2 * 4 * self.cfg.hidden
        return n + self.lm_meta.numel() + self.lm_quant.numel() + 4 * self.cfg.hidden

    def bytes_per_token(self, pos: int) -> int:
        """HBM bytes one step must move at position pos: every weight once,
        the K and V cache rows of positions 0..pos (fp16: 2 bytes a dim; int8:
        1 byte a dim and 4 bytes per 64 dims), one embedding row; activations
        and logits are included for completeness."""
        c = self.cfg
        row = c.head_dim + 4 * (c.head_dim // KV_QBLOCK) if self.kv_int8 else 2 * c.head_dim
        kv = c.n_layers * 2 * c.n_kv_heads * (pos + 1) * row
        return self.weight_bytes() + kv + 2 * c.hidden + 4 * c.vocab


def kv_quantize_int8(rows):
    """set_kv_cache's rule (unified_engine.cpp:859-920) on a float32 device
    tensor [..., d] (d a multiple of 64): per 64-dim block scale = amax *
    float32(1/127) (1e-12 when amax <= 1e-12), code = round-half-even(x *
    (1/scale)) clamped to [-127, 127].  Returns (int8 codes [..., d], float32
    scales [..., d/64])."""
    import torch

    x = rows.float().reshape(*rows.shape[:-1], -1, KV_QBLOCK)
    amax = x.abs().amax(dim=-1)
    scale = torch.where(amax > 1e-12, amax * float(np.float32(1.0 / 127.0)), torch.full_like(amax, 1e-12))
    inv = 1.0 / scale
    q = torch.round(x * inv.unsqueeze(-1)).clamp_(-127, 127).to(torch.int8)
    return q.reshape(rows.shape), scale


def ideal_tokens_per_s(bytes_per_token: int, peak_gbs: float = 8000.0) -> float:
    return peak_gbs * 1e9 / bytes_per_token
