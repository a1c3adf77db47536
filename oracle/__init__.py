"""ctypes binding of the CPU oracle (oracle/lcr_oracle.{h,cpp}).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, where it is the checker the HIP library is
compared against. The library under test never imports this.
"""

from __future__ import annotations

import ctypes
import json
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "liblcr_oracle.so"

BF16 = 0
FP16 = 1

_lib = None


class KvView(ctypes.Structure):
    _fields_ = [
        ("keys", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("page_size", ctypes.c_int),
        ("page_stride", ctypes.c_int),
        ("head_stride", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
    ]


class Config(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int),
        ("intermediate_size", ctypes.c_int),
        ("num_layers", ctypes.c_int),
        ("num_heads", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("vocab_size", ctypes.c_int),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("rope_llama3", ctypes.c_int),
        ("rope_factor", ctypes.c_float),
        ("rope_low_freq_factor", ctypes.c_float),
        ("rope_high_freq_factor", ctypes.c_float),
        ("rope_original_context", ctypes.c_int),
    ]


_PP = ctypes.POINTER(ctypes.c_void_p)


class Weights(ctypes.Structure):
    _fields_ = [
        ("embed", ctypes.c_void_p),
        ("final_norm", ctypes.c_void_p),
        ("lm_head", ctypes.c_void_p),
        ("input_norm", _PP),
        ("q_proj", _PP),
        ("k_proj", _PP),
        ("v_proj", _PP),
        ("o_proj", _PP),
        ("post_norm", _PP),
        ("gate_proj", _PP),
        ("up_proj", _PP),
        ("down_proj", _PP),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

SIGNATURES = {
    "orc_elem_to_float": (_F, [ctypes.c_uint16, _I]),
    "orc_float_to_elem": (ctypes.c_uint16, [_F, _I]),
    "orc_expf": (_F, [_F]),
    "orc_sincosf": (None, [_F, _P, _P]),
    "orc_rope_inv_freq": (None, [_I, _F, _I, _F, _F, _F, _I, _P]),
    "orc_kv_offset": (ctypes.c_int64, [ctypes.POINTER(KvView), _I, _I, _I]),
    "orc_embedding_lookup": (None, [_P, _P, _P, _I, _I]),
    "orc_rmsnorm": (None, [_I, _P, _P, _P, _I, _I, _F]),
    "orc_add_residual_rmsnorm": (None, [_I, _P, _P, _P, _P, _I, _I, _F]),
    "orc_add_residual": (None, [_I, _P, _P, ctypes.c_int64]),
    "orc_swiglu": (None, [_I, _P, _P, _P, ctypes.c_int64]),
    "orc_swiglu_strided": (None, [_I, _P, _P, _P, _I, _I, _I]),
    "orc_merge_heads": (None, [_P, _P, _I, _I, _I]),
    "orc_rope_q": (None, [_I, _P, _P, _P, _I, _I, _I, _I, _I]),
    "orc_rope_write_kv": (None, [_I, ctypes.POINTER(KvView), _P, _P, _P, _I, _I, _I, _I]),
    "orc_gather_kv": (None, [_P, _P, ctypes.POINTER(KvView), _I]),
    "orc_choose_attention_splits": (_I, [_I, _I, _I]),
    "orc_decode_attention": (None, [_I, _P, _P, ctypes.POINTER(KvView), _I, _I, _I, _F, _I, _I]),
    "orc_causal_softmax": (None, [_I, _P, _P, _I, _I, _I, _I]),
    "orc_prefill_attention": (None, [_I, _P, _P, ctypes.POINTER(KvView), _I, _I, _I, _I, _F, _I]),
    "orc_gemv": (None, [_I, _P, _I, _P, _P, _I, _I]),
    "orc_gemm": (None, [_I, _P, _I, _P, _P, _I, _I, _I]),
    "orc_argmax": (ctypes.c_int32, [_P, _I]),
    "orc_sample": (ctypes.c_int32, [_P, _I, _F, _I, _F, _F]),
    "orc_model_create": (_P, [_I, ctypes.POINTER(Config), ctypes.POINTER(Weights), _I, _I, _I, _I, _I, _I]),
    "orc_model_destroy": (None, [_P]),
    "orc_model_reset": (None, [_P]),
    "orc_model_position": (_I, [_P]),
    "orc_model_decode": (_I, [_P, _I, _P]),
    "orc_model_prefill": (_I, [_P, _P, _I, _I, _P]),
    "orc_model_tap": (ctypes.c_size_t, [_P, _I, _P, ctypes.c_size_t]),
    "orc_model_page_table": (_P, [_P, _I]),
    "orc_model_set_kv": (_I, [_P, _I, _I, _P, _P]),
    "orc_model_set_position": (_I, [_P, _I]),
    "orc_last_error": (ctypes.c_char_p, []),
    "orc_set_threads": (None, [_I]),
    "orc_threads": (_I, []),
}


def build() -> Path:
    """Compiles the oracle with its Makefile (a CPU-only build step)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------------------
# element helpers
# ---------------------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round to nearest even, NaN kept quiet (the reference's __float2bfloat16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def elems_to_f32(bits: np.ndarray, kind: int = BF16) -> np.ndarray:
    if kind == BF16:
        return bf16_bits_to_f32(bits)
    return bits.view(np.float16).astype(np.float32)


def f32_to_elems(x: np.ndarray, kind: int = BF16) -> np.ndarray:
    if kind == BF16:
        return f32_to_bf16_bits(x)
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


# ---------------------------------------------------------------------------
# safetensors (numpy memmap; the checkpoint the GPU path also reads)
# ---------------------------------------------------------------------------

def read_safetensors(path) -> dict:
    path = Path(path)
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    base = 8 + n
    out = {}
    for name, spec in header.items():
        if name == "__metadata__":
            continue
        b, e = spec["data_offsets"]
        dt = {"BF16": np.uint16, "F16": np.uint16, "F32": np.float32}[spec["dtype"]]
        arr = mm[base + b: base + e].view(dt).reshape(spec["shape"])
        out[name] = arr
    return out


def config_struct(cfg: dict) -> Config:
    c = Config()
    c.hidden_size = cfg["hidden_size"]
    c.intermediate_size = cfg["intermediate_size"]
    c.num_layers = cfg["num_hidden_layers"]
    c.num_heads = cfg["num_attention_heads"]
    c.num_kv_heads = cfg.get("num_key_value_heads", cfg["num_attention_heads"])
    c.head_dim = cfg.get("head_dim", cfg["hidden_size"] // cfg["num_attention_heads"])
    c.vocab_size = cfg["vocab_size"]
    c.rms_norm_eps = cfg.get("rms_norm_eps", 1e-5)
    c.rope_theta = cfg.get("rope_theta", 500000.0)
    rs = cfg.get("rope_scaling") or {}
    kind = rs.get("rope_type", rs.get("type", "default"))
    c.rope_llama3 = 1 if kind == "llama3" else 0
    c.rope_factor = rs.get("factor", 32.0)
    c.rope_low_freq_factor = rs.get("low_freq_factor", 1.0)
    c.rope_high_freq_factor = rs.get("high_freq_factor", 4.0)
    c.rope_original_context = rs.get("original_max_position_embeddings", 8192)
    return c


class OracleModel:
    """The whole-model oracle over a checkpoint directory."""

    def __init__(self, model_dir, kind: int = BF16, max_seq: int = 4096, paged: bool = False,
                 page_size: int = 16, prefill_chunk: int = 256, multiprocessors: int = 256,
                 attention_splits: int = 0):
        self.lib = load()
        model_dir = Path(model_dir)
        self.cfg = json.loads((model_dir / "config.json").read_text())
        self.t = read_safetensors(model_dir / "model.safetensors")
        L = self.cfg["num_hidden_layers"]
        self.vocab = self.cfg["vocab_size"]

        def arr(name):
            a = self.t[name]
            return a.ctypes.data

        def per_layer(suffix):
            vals = (ctypes.c_void_p * L)(*[arr(f"model.layers.{i}.{suffix}") for i in range(L)])
            return vals

        self._keep = {}
        w = Weights()
        w.embed = arr("model.embed_tokens.weight")
        w.final_norm = arr("model.norm.weight")
        w.lm_head = arr("lm_head.weight") if "lm_head.weight" in self.t else w.embed
        for field, suffix in [("input_norm", "input_layernorm.weight"), ("q_proj", "self_attn.q_proj.weight"),
                              ("k_proj", "self_attn.k_proj.weight"), ("v_proj", "self_attn.v_proj.weight"),
                              ("o_proj", "self_attn.o_proj.weight"),
                              ("post_norm", "post_attention_layernorm.weight"),
                              ("gate_proj", "mlp.gate_proj.weight"), ("up_proj", "mlp.up_proj.weight"),
                              ("down_proj", "mlp.down_proj.weight")]:
            vals = per_layer(suffix)
            self._keep[field] = vals
            setattr(w, field, ctypes.cast(vals, _PP))
        self._w = w
        self._c = config_struct(self.cfg)
        self.handle = self.lib.orc_model_create(kind, ctypes.byref(self._c), ctypes.byref(self._w), max_seq,
                                                1 if paged else 0, page_size, prefill_chunk,
                                                multiprocessors, attention_splits)
        if not self.handle:
            raise RuntimeError(self.lib.orc_last_error().decode())

    def close(self):
        if getattr(self, "handle", None):
            self.lib.orc_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode(self, token: int) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        rc = self.lib.orc_model_decode(self.handle, int(token), ptr(out))
        if rc != 0:
            raise RuntimeError(self.lib.orc_last_error().decode())
        return out

    def prefill(self, tokens, use_decode_path: bool = False) -> np.ndarray:
        arr_ = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.empty(self.vocab, dtype=np.float32)
        rc = self.lib.orc_model_prefill(self.handle, ptr(arr_), len(arr_), 1 if use_decode_path else 0, ptr(out))
        if rc != 0:
            raise RuntimeError(self.lib.orc_last_error().decode())
        return out

    def reset(self):
        self.lib.orc_model_reset(self.handle)

    @property
    def position(self) -> int:
        return int(self.lib.orc_model_position(self.handle))

    def tap(self, index: int, tokens: int) -> np.ndarray:
        h = self.cfg["hidden_size"]
        out = np.empty(tokens * h, dtype=np.float32)
        n = self.lib.orc_model_tap(self.handle, index, ptr(out), out.size)
        return out[:n].reshape(-1, h)

    def set_kv(self, layer: int, keys: np.ndarray, values: np.ndarray):
        """Writes a layer's cache from logical [kv_head][position][head_dim]
        element arrays (uint16 bits)."""
        k = np.ascontiguousarray(keys, dtype=np.uint16)
        v = np.ascontiguousarray(values, dtype=np.uint16)
        assert k.shape == v.shape and k.ndim == 3
        if self.lib.orc_model_set_kv(self.handle, layer, k.shape[1], ptr(k), ptr(v)) != 0:
            raise RuntimeError(self.lib.orc_last_error().decode())

    def set_position(self, position: int):
        if self.lib.orc_model_set_position(self.handle, position) != 0:
            raise RuntimeError(self.lib.orc_last_error().decode())

    def page_table(self, layer: int, max_pages: int) -> np.ndarray:
        p = self.lib.orc_model_page_table(self.handle, layer)
        if not p:
            return None
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int32)), shape=(max_pages,)).copy()


def argmax(logits: np.ndarray) -> int:
    lib = load()
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib.orc_argmax(ptr(a), a.size))


def sample(logits: np.ndarray, temperature: float, top_k: int, top_p: float, uniform: float) -> int:
    lib = load()
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib.orc_sample(ptr(a), a.size, temperature, top_k, top_p, uniform))
