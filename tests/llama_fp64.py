"""A float64 Llama forward pass and a small-checkpoint writer, for tests.

Test infrastructure: the independent reference the CPU oracle's whole-model
composition (and the GPU model's) is checked against. It is written from the
Llama architecture as published (Hugging Face's LlamaForCausalLM: pre-norm
decoder layers, RMSNorm, rotate-half RoPE with Llama 3 frequency scaling,
grouped-query attention with a causal mask, SwiGLU MLP, tied embeddings), not
from the oracle's code, and keeps every activation in float64: it has no
rounding points at all, so its distance to a bf16 implementation is that
implementation's rounding noise, and a structural mistake on either side
(wrong head mapping, RoPE pairing, residual, norm weight, mask) shows up as a
distance orders of magnitude larger.

`mistake` plants one such error in this model, to show the bounds used by
the tests catch it.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

import oracle

MISTAKES = ("rope_interleaved", "kv_head_modulo", "no_attention_residual", "no_post_norm_weight",
            "swiglu_swapped", "no_causal_mask", "no_final_norm", "rope_on_queries_only")


def tiny_config(**overrides) -> dict:
    cfg = {
        "architectures": ["LlamaForCausalLM"], "model_type": "llama", "hidden_act": "silu",
        "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
        "num_attention_heads": 8, "num_key_value_heads": 2, "head_dim": 64,
        "vocab_size": 512, "rms_norm_eps": 1e-5, "rope_theta": 500000.0,
        "rope_scaling": {"factor": 32.0, "high_freq_factor": 4.0, "low_freq_factor": 1.0,
                         "original_max_position_embeddings": 8192, "rope_type": "llama3"},
        "tie_word_embeddings": True, "torch_dtype": "bfloat16", "max_position_embeddings": 131072,
        "bos_token_id": 1, "eos_token_id": 2,
    }
    cfg.update(overrides)
    return cfg


def write_checkpoint(directory, cfg: dict, seed: int = 7) -> dict:
    """Writes config.json and a BF16 model.safetensors with seeded weights.
    Norm weights are 1 + N(0, 0.25) (not all ones, so a misplaced norm weight
    changes the result); q/k projections are scaled so that attention scores
    have a spread of a few units (a flat softmax would hide mask and scale
    mistakes). Returns the float32 values of every tensor."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    r = np.random.default_rng(seed)
    H, F, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    nh, nkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    tensors = {"model.embed_tokens.weight": r.normal(0, 0.1, (V, H)),
               "model.norm.weight": 1 + r.normal(0, 0.25, H)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        tensors[p + "input_layernorm.weight"] = 1 + r.normal(0, 0.25, H)
        tensors[p + "post_attention_layernorm.weight"] = 1 + r.normal(0, 0.25, H)
        tensors[p + "self_attn.q_proj.weight"] = r.normal(0, 0.09, (nh * hd, H))
        tensors[p + "self_attn.k_proj.weight"] = r.normal(0, 0.09, (nkv * hd, H))
        tensors[p + "self_attn.v_proj.weight"] = r.normal(0, 0.06, (nkv * hd, H))
        tensors[p + "self_attn.o_proj.weight"] = r.normal(0, 0.06, (H, nh * hd))
        tensors[p + "mlp.gate_proj.weight"] = r.normal(0, 0.06, (F, H))
        tensors[p + "mlp.up_proj.weight"] = r.normal(0, 0.06, (F, H))
        tensors[p + "mlp.down_proj.weight"] = r.normal(0, 0.04, (H, F))
    bits = {k: oracle.f32_to_bf16_bits(v.astype(np.float32)) for k, v in tensors.items()}
    header, offset, blobs = {}, 0, []
    for name, b in bits.items():
        raw = np.ascontiguousarray(b).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(b.shape), "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(directory / "model.safetensors", "wb") as f:
        f.write(len(text).to_bytes(8, "little"))
        f.write(text)
        for raw in blobs:
            f.write(raw)
    (directory / "config.json").write_text(json.dumps(cfg))
    return {k: oracle.bf16_bits_to_f32(b) for k, b in bits.items()}


def llama3_inv_freq(cfg: dict) -> np.ndarray:
    """Rotary frequencies theta^(-2i/d), then Llama 3's band rule: wavelengths
    above original_context / low_freq_factor are divided by `factor`, those
    below original_context / high_freq_factor are kept, and the band between
    blends the two by (original_context / wavelength - low) / (high - low)."""
    hd = cfg["head_dim"]
    inv = 1.0 / cfg["rope_theta"] ** (np.arange(0, hd, 2, dtype=np.float64) / hd)
    rs = cfg.get("rope_scaling") or {}
    if rs.get("rope_type") != "llama3":
        return inv
    factor, low, high = rs["factor"], rs["low_freq_factor"], rs["high_freq_factor"]
    ctx = rs["original_max_position_embeddings"]
    wavelen = 2 * math.pi / inv
    out = np.where(wavelen > ctx / low, inv / factor, inv)
    smooth = (ctx / wavelen - low) / (high - low)
    medium = (wavelen >= ctx / high) & (wavelen <= ctx / low)
    return np.where(medium, (1 - smooth) * out / factor + smooth * out, out)


class _Float64View(dict):
    """Tensors converted to float64 on first use and dropped from memory by
    `release` (a full-size checkpoint in float64 would be 10 GB)."""

    def __init__(self, source):
        super().__init__()
        self.source = source

    def __missing__(self, name):
        v = self.source[name]
        if v.dtype == np.uint16:
            v = oracle.bf16_bits_to_f32(np.asarray(v))
        out = np.asarray(v, dtype=np.float64)
        self[name] = out
        return out

    def release(self, prefix):
        for k in [k for k in self if k.startswith(prefix)]:
            del self[k]


def forward(cfg: dict, w: dict, tokens, mistake: str | None = None, return_hidden: bool = False,
            last_logits_only: bool = False):
    """Logits of every position of `tokens` (float64 [T, vocab]; only the last
    row's, [1, vocab], with last_logits_only); with return_hidden also the
    residual stream after the embedding and after each layer, and the final
    normed rows. `w` maps tensor names to float values or to bf16 bits
    (uint16, e.g. the memory-mapped arrays of oracle.read_safetensors), and
    is converted to float64 one layer at a time."""
    w = _Float64View(w)
    H = cfg["hidden_size"]
    nh, nkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    G = nh // nkv
    eps = cfg["rms_norm_eps"]
    tokens = np.asarray(tokens)
    T = len(tokens)

    def rms(x, weight):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * weight

    inv = llama3_inv_freq(cfg)
    pos = np.arange(T, dtype=np.float64)
    ang = pos[:, None] * inv[None, :]
    cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]

    def rope(v):  # v: [T, heads, hd]
        if mistake == "rope_interleaved":
            a, b = v[..., 0::2], v[..., 1::2]
            out = np.empty_like(v)
            out[..., 0::2] = a * cos - b * sin
            out[..., 1::2] = b * cos + a * sin
            return out
        lo, hi = v[..., : hd // 2], v[..., hd // 2:]
        return np.concatenate([lo * cos - hi * sin, hi * cos + lo * sin], axis=-1)

    E = w["model.embed_tokens.weight"]
    x = E[tokens].copy()
    hidden = [x.copy()]
    mask = np.triu(np.full((T, T), -np.inf), k=1)
    if mistake == "no_causal_mask":
        mask = np.zeros((T, T))
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        h = rms(x, w[p + "input_layernorm.weight"])
        q = rope((h @ w[p + "self_attn.q_proj.weight"].T).reshape(T, nh, hd))
        k = (h @ w[p + "self_attn.k_proj.weight"].T).reshape(T, nkv, hd)
        if mistake != "rope_on_queries_only":
            k = rope(k)
        v = (h @ w[p + "self_attn.v_proj.weight"].T).reshape(T, nkv, hd)
        o = np.empty((T, nh, hd))
        for head in range(nh):
            g = head % nkv if mistake == "kv_head_modulo" else head // G
            s = q[:, head] @ k[:, g].T / math.sqrt(hd) + mask
            s = np.exp(s - s.max(axis=-1, keepdims=True))
            o[:, head] = (s / s.sum(axis=-1, keepdims=True)) @ v[:, g]
        attn = o.reshape(T, nh * hd) @ w[p + "self_attn.o_proj.weight"].T
        x = attn if mistake == "no_attention_residual" else x + attn
        post = np.ones(H) if mistake == "no_post_norm_weight" else w[p + "post_attention_layernorm.weight"]
        h = rms(x, post)
        g_ = h @ w[p + "mlp.gate_proj.weight"].T
        u_ = h @ w[p + "mlp.up_proj.weight"].T
        if mistake == "swiglu_swapped":
            g_, u_ = u_, g_
        x = x + (g_ / (1 + np.exp(-g_)) * u_) @ w[p + "mlp.down_proj.weight"].T
        hidden.append(x.copy())
        w.release(p)
    final = x if mistake == "no_final_norm" else rms(x, w["model.norm.weight"])
    logits = (final[-1:] if last_logits_only else final) @ E.T
    if return_hidden:
        return logits, hidden, final
    return logits


def drift(got, want) -> dict:
    """The agreement figures of the reference's validator
    (tools/validate_main.cu:95-137) for a [rows, width] tensor (a vector is
    one row): max-abs, RMS of the error over RMS of the reference (rel-RMS),
    and the smallest per-row cosine."""
    a = np.asarray(got, dtype=np.float64)
    b = np.asarray(want, dtype=np.float64)
    assert a.size == b.size, (a.shape, b.shape)
    width = b.shape[-1] if b.ndim > 1 else b.size
    a = a.reshape(-1, width)
    b = b.reshape(-1, width)
    d = a - b
    rms_ref = float(np.sqrt(np.mean(b * b)))
    rms_err = float(np.sqrt(np.mean(d * d)))
    na = np.linalg.norm(a, axis=1)
    nb = np.linalg.norm(b, axis=1)
    live = (na > 0) & (nb > 0)
    cos = np.einsum("ij,ij->i", a[live], b[live]) / (na[live] * nb[live])
    return {
        "max_abs": float(np.abs(d).max()),
        "rms_error": rms_err,
        "rel_rms": rms_err / rms_ref if rms_ref > 0 else 0.0,
        "cosine": float(cos.min()) if cos.size else 1.0,
    }


# How much less accurate than the oracle a prefill may be, layer by layer:
# its rel-RMS distance to float64 within this factor of the oracle's (plus a
# small floor for layers where both are tiny), and every row's cosine to
# float64 at least COSINE_MIN.
ACCURACY_FACTOR = 1.25
ACCURACY_FLOOR = 1e-3
COSINE_MIN = 0.999


def accuracy_report(names, gpu_taps, gpu_logits, oracle_model, tokens, hidden, final, logits64):
    """Per tensor: the GPU's and the oracle's drift from the float64 forward,
    and the GPU's drift from the oracle. `hidden`, `final`, `logits64` come
    from forward(..., return_hidden=True, last_logits_only=True)."""
    rows = []
    for i, name in enumerate(names):
        exact = hidden[i] if i < len(hidden) else final
        orc = oracle_model.tap(i, tokens)
        rows.append((name, drift(gpu_taps[name], exact), drift(orc, exact), drift(gpu_taps[name], orc)))
    return rows


def check_accuracy(rows, logits_row):
    """Asserts the bounds above for every tap row and for the logits row
    (name, gpu-vs-fp64, oracle-vs-fp64, gpu-vs-oracle)."""
    for name, g, o, _ in list(rows) + [logits_row]:
        assert g["rel_rms"] <= ACCURACY_FACTOR * o["rel_rms"] + ACCURACY_FLOOR, (name, g, o)
        assert g["cosine"] >= COSINE_MIN, (name, g)


def format_report(rows) -> str:
    lines = [f"{'tensor':11s} {'rel-RMS gpu':>12s} {'rel-RMS orc':>12s} {'gpu-orc':>9s} {'cos gpu':>9s}"]
    for name, g, o, go in rows:
        lines.append(f"{name:11s} {g['rel_rms']:12.4e} {o['rel_rms']:12.4e} {go['rel_rms']:9.2e} {g['cosine']:9.6f}")
    return "\n".join(lines)
