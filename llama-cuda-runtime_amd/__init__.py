"""Python bindings of the MI355X token-loop library (ctypes over the C-ABI).

The product is the HIP shared library next to this file (liblcr_amd.so for
bf16, liblcr_amd_fp16.so for fp16) and its C headers in include/. This module
only loads it and declares the entry points, so Python code (the tests and
bench.py) drives exactly the code a C or C++ host would. Nothing here computes:
a missing library raises instead of falling back to anything else.

The package directory name contains dashes, so it is loaded by path; use
`load_package()` from tests and scripts:

    import importlib.util, pathlib
    spec = importlib.util.spec_from_file_location(
        "lcr_amd", pathlib.Path("llama-cuda-runtime_amd/__init__.py"))
"""

from __future__ import annotations

import ctypes
import json
import os
from pathlib import Path
from typing import Optional, Sequence

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent

LIB_NAMES = {"bf16": "liblcr_amd.so", "fp16": "liblcr_amd_fp16.so"}

# Llama-3.2-1B geometry, the reference's tests/test_config.cpp:17-44 literal.
LLAMA_3_2_1B_CONFIG = {
    "architectures": ["LlamaForCausalLM"],
    "attention_bias": False,
    "bos_token_id": 128000,
    "eos_token_id": [128001, 128008, 128009],
    "head_dim": 64,
    "hidden_act": "silu",
    "hidden_size": 2048,
    "intermediate_size": 8192,
    "max_position_embeddings": 131072,
    "mlp_bias": False,
    "model_type": "llama",
    "num_attention_heads": 32,
    "num_hidden_layers": 16,
    "num_key_value_heads": 8,
    "rms_norm_eps": 1e-05,
    "rope_scaling": {
        "factor": 32.0,
        "high_freq_factor": 4.0,
        "low_freq_factor": 1.0,
        "original_max_position_embeddings": 8192,
        "rope_type": "llama3",
    },
    "rope_theta": 500000.0,
    "tie_word_embeddings": True,
    "torch_dtype": "bfloat16",
    "vocab_size": 128256,
}

WEIGHT_SEED = 20260904
PROMPT_SEED = 1234
WEIGHT_STD = 0.02


def llama_config(**overrides) -> dict:
    cfg = json.loads(json.dumps(LLAMA_3_2_1B_CONFIG))
    cfg.update(overrides)
    return cfg


class LcrError(RuntimeError):
    pass


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


class ModelOptions(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int),
        ("max_seq", ctypes.c_int),
        ("paged", ctypes.c_int),
        ("page_size", ctypes.c_int),
        ("prefill_chunk", ctypes.c_int),
        ("attention_splits", ctypes.c_int),
        ("fused_decode", ctypes.c_int),
        ("use_graph", ctypes.c_int),
        ("prefill_via_decode", ctypes.c_int),
        ("decode_exchange", ctypes.c_int),
        ("exchange_oproj", ctypes.c_int),
        ("exchange_split", ctypes.c_int),
        ("exchange_spins", ctypes.c_int),
        ("exchange_test_unwritten", ctypes.c_int),
        ("layer_grid", ctypes.c_int),
        ("exchange_head", ctypes.c_int),
    ]


class ModelStats(ctypes.Structure):
    _fields_ = [
        ("weight_bytes_per_token", ctypes.c_uint64),
        ("kv_bytes_per_position", ctypes.c_uint64),
        ("last_prefill_ms", ctypes.c_double),
        ("last_decode_ms", ctypes.c_double),
        ("weight_bytes", ctypes.c_uint64),
        ("arena_peak_bytes", ctypes.c_uint64),
        ("kv_allocated_bytes", ctypes.c_uint64),
        ("multiprocessors", ctypes.c_int),
        ("fused", ctypes.c_int),
        ("vocab_size", ctypes.c_int),
        ("hidden_size", ctypes.c_int),
        ("num_layers", ctypes.c_int),
        ("layer_grid", ctypes.c_int),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t

# name -> (restype, argtypes). Every symbol include/*.h declares.
SIGNATURES = {
    # lcr_kernels.h
    "lcr_last_error_message": (ctypes.c_char_p, []),
    "lcr_elem_name": (ctypes.c_char_p, []),
    "lcr_embedding_lookup": (_I, [_P, _P, _P, _I, _I, _P]),
    "lcr_rmsnorm": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "lcr_add_residual": (_I, [_P, _P, _I64, _P]),
    "lcr_add_residual_rmsnorm": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "lcr_swiglu": (_I, [_P, _P, _P, _I64, _P]),
    "lcr_swiglu_strided": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "lcr_rope_q": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "lcr_rope_write_kv": (_I, [ctypes.POINTER(KvView), _P, _P, _P, _I, _I, _I, _I, _P]),
    "lcr_causal_softmax": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "lcr_merge_heads": (_I, [_P, _P, _I, _I, _I, _P]),
    "lcr_gather_kv": (_I, [_P, _P, ctypes.POINTER(KvView), _I, _P]),
    "lcr_decode_attention": (_I, [_P, _P, ctypes.POINTER(KvView), _I, _I, _I, _F, _I, _I, _P, _P]),
    "lcr_decode_attention_noalloc": (_I, [_P, _P, ctypes.POINTER(KvView), _I, _I, _I, _F, _I, _I, _P]),
    "lcr_decode_attention_scratch_floats": (_SZ, [_I, _I, _I]),
    "lcr_choose_attention_splits": (_I, [_I, _I, _I]),
    "lcr_sample": (_I, [_P, _P, _I, _F, _I, _F, _F, _P, _P]),
    "lcr_sample_scratch_floats": (_SZ, [_I, _I]),
    "lcr_gemv": (_I, [_P, _I, _P, _P, _I, _I, _P]),
    "lcr_gemm": (_I, [_P, _I, _P, _P, _I, _I, _I, _P]),
    "lcr_gemm_ws": (_I, [_P, _I, _P, _P, _I, _I, _I, _P, ctypes.c_size_t, _P]),
    "lcr_gemm_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I]),
    "lcr_gemm_swiglu_ws": (_I, [_P, _P, _P, _I, _I, _I, _P, ctypes.c_size_t, _P]),
    "lcr_gemm_residual_rmsnorm_ws": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, ctypes.c_size_t, _P]),
    "lcr_rope_table": (_I, [_P, _P, _I, _I, _P]),
    "lcr_gemm_qkv_rope_ws": (_I, [_P, ctypes.POINTER(KvView), _P, _P, _P, _I, _I, _I, _I, _I, _P,
                                  ctypes.c_size_t, _P]),
    "lcr_prefill_attention": (_I, [_P, _P, ctypes.POINTER(KvView), _I, _I, _I, _I, _F, _I, _P]),
    # lcr_model.h
    "lcr_model_default_options": (None, [ctypes.POINTER(ModelOptions)]),
    "lcr_model_create": (_I, [ctypes.c_char_p, ctypes.POINTER(ModelOptions), ctypes.POINTER(_P)]),
    "lcr_model_destroy": (None, [_P]),
    "lcr_model_prefill": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "lcr_model_decode": (_I, [_P, ctypes.c_int32, ctypes.POINTER(_P)]),
    "lcr_model_sample": (_I, [_P, _P, _F, _I, _F, _F, ctypes.POINTER(ctypes.c_int32)]),
    "lcr_model_logits_to_host": (_I, [_P, _P, _P]),
    "lcr_model_reset": (_I, [_P]),
    "lcr_model_position": (_I, [_P]),
    "lcr_model_stats_get": (_I, [_P, ctypes.POINTER(ModelStats)]),
    "lcr_model_set_capture_activations": (_I, [_P, _I]),
    "lcr_model_tap_count": (_I, [_P]),
    "lcr_model_tap": (_I, [_P, _I, ctypes.c_char_p, _SZ, ctypes.POINTER(_I), ctypes.POINTER(_I), _P, _SZ]),
    "lcr_model_set_profiling": (_I, [_P, _I]),
    "lcr_model_exchange_status": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "lcr_model_exchange_clear": (_I, [_P]),
    "lcr_model_generate_greedy": (_I, [_P, ctypes.c_int32, _I, _P, ctypes.POINTER(ctypes.c_double)]),
    "lcr_model_generate_sampled": (_I, [_P, ctypes.c_int32, _I, _F, _I, _F, _P, _P,
                                        ctypes.POINTER(ctypes.c_double)]),
    "lcr_model_decode_splits": (_I, [_P, _I]),
    "lcr_model_time_decode_kernel": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_double)]),
    "lcr_model_kv_page_table": (_I, [_P, _I, _P, _I]),
    "lcr_model_kv_geometry": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "lcr_model_set_kv_page_tables": (_I, [_P, _P, _SZ, _I]),
    "lcr_model_fill_kv_normal": (_I, [_P, _U64, _F]),
    "lcr_model_set_position": (_I, [_P, _I]),
    "lcr_model_kv_read": (_I, [_P, _I, _I, _I, _P, _P]),
    "lcr_model_kv_export": (_I, [_P, _I, _I, _P, _P]),
    "lcr_write_synthetic_checkpoint": (_I, [ctypes.c_char_p, ctypes.c_char_p, _U64, _F, _I, _I]),
    "lcr_synthetic_tokens": (_I, [_U64, _I, _I, _P]),
    "lcr_philox_uniforms": (_I, [_U64, _I, _P]),
    "lcr_device_count": (_I, []),
    # lcr_tokenizer.h
    "lcr_tokenizer_create": (_P, [ctypes.c_char_p]),
    "lcr_tokenizer_create_from_json": (_P, [ctypes.c_char_p, _SZ]),
    "lcr_tokenizer_destroy": (None, [_P]),
    "lcr_tokenizer_encode": (_I, [_P, ctypes.c_char_p, _SZ, _I, _I, _P, _SZ, ctypes.POINTER(_SZ)]),
    "lcr_tokenizer_decode": (_I, [_P, _P, _SZ, _I, _P, _SZ, ctypes.POINTER(_SZ)]),
    "lcr_tokenizer_vocab_size": (_I, [_P]),
    "lcr_tokenizer_bos_id": (_I, [_P]),
    "lcr_tokenizer_token_to_id": (_I, [_P, ctypes.c_char_p, _SZ]),
    "lcr_tokenizer_is_special": (_I, [_P, _I]),
    "lcr_split_pretokens": (_I, [ctypes.c_char_p, _SZ, _P, _SZ, ctypes.POINTER(_SZ)]),
    # lcr_runtime.h
    "lcr_device_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "lcr_device_free": (_I, [_P]),
    "lcr_memcpy_htod": (_I, [_P, _P, _SZ]),
    "lcr_memcpy_dtoh": (_I, [_P, _P, _SZ]),
    "lcr_memcpy_dtod": (_I, [_P, _P, _SZ]),
    "lcr_stream_read": (_I, [_P, _SZ, _I, _I, ctypes.POINTER(ctypes.c_float)]),
    "lcr_device_memset": (_I, [_P, _I, _SZ]),
    "lcr_device_synchronize": (_I, []),
}

_LIBS: dict = {}


def library_path(variant: str = "bf16") -> Path:
    return PKG_DIR / LIB_NAMES[variant]


def load_library(variant: str = "bf16"):
    """Loads the HIP library of the given element type, declaring every symbol.

    Raises LcrError when the library has not been built (there is no fallback).
    """
    if variant in _LIBS:
        return _LIBS[variant]
    path = library_path(variant)
    if not path.exists():
        raise LcrError(f"{path} is missing: build it with `python {PKG_DIR / 'build.py'}` "
                       "(or __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIBS[variant] = lib
    return lib


def check(lib, status: int, what: str = "") -> None:
    if status != 0:
        msg = lib.lcr_last_error_message().decode(errors="replace")
        raise LcrError(f"{what}: status {status}: {msg}")


def device_count(variant: str = "bf16") -> int:
    return int(load_library(variant).lcr_device_count())


class Tokenizer:
    """The byte-level BPE tokenizer (include/lcr_tokenizer.h) from a
    tokenizer.json path or its text. No GPU is involved."""

    def __init__(self, path=None, json_text: Optional[str] = None, variant: str = "bf16"):
        self.lib = load_library(variant)
        if json_text is not None:
            raw = json_text.encode()
            self.handle = self.lib.lcr_tokenizer_create_from_json(raw, len(raw))
        else:
            self.handle = self.lib.lcr_tokenizer_create(str(path).encode())
        if not self.handle:
            raise LcrError(self.lib.lcr_last_error_message().decode(errors="replace"))

    def close(self):
        if getattr(self, "handle", None):
            self.lib.lcr_tokenizer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text, add_bos: bool = False, parse_special: bool = True) -> list:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        cap = len(raw) + 8
        while True:
            out = (ctypes.c_int32 * cap)()
            n = ctypes.c_size_t()
            st = self.lib.lcr_tokenizer_encode(self.handle, raw, len(raw), int(add_bos), int(parse_special), out,
                                               cap, ctypes.byref(n))
            if st == 0:
                return list(out[:n.value])
            if n.value <= cap:
                check(self.lib, st, "tokenizer encode")
            cap = n.value

    def decode(self, ids, skip_special: bool = False) -> bytes:
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        cap = 16 * len(ids) + 16
        while True:
            buf = ctypes.create_string_buffer(cap)
            n = ctypes.c_size_t()
            st = self.lib.lcr_tokenizer_decode(self.handle, arr, len(ids), int(skip_special), buf, cap,
                                               ctypes.byref(n))
            if st == 0:
                return buf.raw[:n.value]
            if n.value <= cap:
                check(self.lib, st, "tokenizer decode")
            cap = n.value

    @property
    def vocab_size(self) -> int:
        return int(self.lib.lcr_tokenizer_vocab_size(self.handle))

    @property
    def bos_id(self) -> int:
        return int(self.lib.lcr_tokenizer_bos_id(self.handle))

    def token_to_id(self, token: str) -> int:
        raw = token.encode()
        return int(self.lib.lcr_tokenizer_token_to_id(self.handle, raw, len(raw)))

    def is_special(self, i: int) -> bool:
        return bool(self.lib.lcr_tokenizer_is_special(self.handle, i))


def split_pretokens(text, variant: str = "bf16") -> list:
    """The Llama 3 pretokenizer split (bytes pieces)."""
    lib = load_library(variant)
    raw = text.encode() if isinstance(text, str) else bytes(text)
    cap = len(raw) + 1
    ends = (ctypes.c_size_t * cap)()
    n = ctypes.c_size_t()
    check(lib, lib.lcr_split_pretokens(raw, len(raw), ends, cap, ctypes.byref(n)), "split_pretokens")
    out, start = [], 0
    for i in range(n.value):
        out.append(raw[start:ends[i]])
        start = ends[i]
    return out


def write_synthetic_checkpoint(directory, config: Optional[dict] = None, seed: int = WEIGHT_SEED,
                               stddev: float = WEIGHT_STD, fp16: bool = False,
                               threads: Optional[int] = None, variant: str = "bf16") -> Path:
    """Writes config.json + model.safetensors of a seeded random-init model."""
    lib = load_library(variant)
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    cfg = config or LLAMA_3_2_1B_CONFIG
    if fp16:
        cfg = dict(cfg, torch_dtype="float16")
    threads = threads or min(16, os.cpu_count() or 4)
    check(lib, lib.lcr_write_synthetic_checkpoint(str(directory).encode(), json.dumps(cfg).encode(),
                                                  seed, stddev, 1 if fp16 else 0, threads),
          "write_synthetic_checkpoint")
    return directory


def synthetic_tokens(count: int, vocab: int, seed: int = PROMPT_SEED, variant: str = "bf16"):
    import numpy as np
    lib = load_library(variant)
    out = np.zeros(count, dtype=np.int32)
    check(lib, lib.lcr_synthetic_tokens(seed, count, vocab, out.ctypes.data), "synthetic_tokens")
    return out


# Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
# as 1, 2, 3", SC 2011): the counter-based generator whose draws feed the
# stochastic-sampling comparison, identical floats to the GPU and the oracle.
_PHILOX_M0 = 0xD2511F53
_PHILOX_M1 = 0xCD9E8D57
_PHILOX_W0 = 0x9E3779B9
_PHILOX_W1 = 0xBB67AE85


def philox4x32_10(counter: Sequence[int], key: Sequence[int]) -> list:
    c0, c1, c2, c3 = (int(x) & 0xFFFFFFFF for x in counter)
    k0, k1 = (int(x) & 0xFFFFFFFF for x in key)
    for _ in range(10):
        p0 = _PHILOX_M0 * c0
        p1 = _PHILOX_M1 * c2
        hi0, lo0 = p0 >> 32, p0 & 0xFFFFFFFF
        hi1, lo1 = p1 >> 32, p1 & 0xFFFFFFFF
        c0, c1, c2, c3 = (hi1 ^ c1 ^ k0) & 0xFFFFFFFF, lo1, (hi0 ^ c3 ^ k1) & 0xFFFFFFFF, lo0
        k0 = (k0 + _PHILOX_W0) & 0xFFFFFFFF
        k1 = (k1 + _PHILOX_W1) & 0xFFFFFFFF
    return [c0, c1, c2, c3]


def philox_uniforms(seed: int, count: int) -> list:
    """count floats in [0, 1): draw i is word i%4 of Philox(counter=(i//4,0,0,0),
    key=(seed lo, seed hi)), mapped as (word >> 8) * 2^-24 (exact in float32)."""
    out = []
    key = (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)
    block = None
    for i in range(count):
        if i % 4 == 0:
            block = philox4x32_10((i // 4, 0, 0, 0), key)
        out.append((block[i % 4] >> 8) * (1.0 / 16777216.0))
    return out


class DeviceBuffer:
    """Device memory from include/lcr_runtime.h, with typed host copies."""

    def __init__(self, nbytes: int, dtype=None, count: int = 0, variant: str = "bf16", zero: bool = True):
        self.lib = load_library(variant)
        self.nbytes = int(nbytes)
        self.dtype = dtype
        self.count = count
        ptr = ctypes.c_void_p()
        check(self.lib, self.lib.lcr_device_malloc(ctypes.byref(ptr), max(self.nbytes, 16)), "device_malloc")
        self.ptr = ptr.value
        if zero:
            check(self.lib, self.lib.lcr_device_memset(self.ptr, 0, max(self.nbytes, 16)), "device_memset")

    @classmethod
    def from_array(cls, array, variant: str = "bf16"):
        import numpy as np
        a = np.ascontiguousarray(array)
        buf = cls(a.nbytes, a.dtype, a.size, variant, zero=False)
        check(buf.lib, buf.lib.lcr_memcpy_htod(buf.ptr, a.ctypes.data, a.nbytes), "memcpy_htod")
        return buf

    def to_numpy(self, dtype=None, count=None):
        import numpy as np
        dtype = np.dtype(dtype or self.dtype)
        count = count if count is not None else self.nbytes // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(self.lib, self.lib.lcr_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes), "memcpy_dtoh")
        return out

    def free(self):
        if getattr(self, "ptr", None):
            self.lib.lcr_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(variant: str = "bf16") -> None:
    lib = load_library(variant)
    check(lib, lib.lcr_device_synchronize(), "device_synchronize")


def device_copy(dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
    """Device-to-device copy of nbytes (both buffers must hold them)."""
    if nbytes > min(dst.nbytes, src.nbytes):
        raise LcrError(f"copy of {nbytes} bytes exceeds a buffer ({dst.nbytes}, {src.nbytes})")
    check(dst.lib, dst.lib.lcr_memcpy_dtod(dst.ptr, src.ptr, nbytes), "memcpy_dtod")


def stream_read_gbs(nbytes: int = 1 << 30, blocks: int = 8192, reps: int = 10, variant: str = "bf16") -> float:
    """Read rate (GB/s) of the library's streaming 16-byte loads over a fresh
    device buffer of nbytes (lcr_stream_read: the fastest of `reps` launches)."""
    buf = DeviceBuffer(nbytes, variant=variant)
    try:
        ms = ctypes.c_float()
        check(buf.lib, buf.lib.lcr_stream_read(buf.ptr, nbytes, blocks, reps, ctypes.byref(ms)), "stream_read")
        return nbytes / (ms.value * 1e-3) / 1e9
    finally:
        buf.free()


class Model:
    """lcr::Model through the C-ABI (include/lcr_model.h)."""

    def __init__(self, model_dir, variant: str = "bf16", **options):
        self.lib = load_library(variant)
        opts = ModelOptions()
        self.lib.lcr_model_default_options(ctypes.byref(opts))
        for k, v in options.items():
            if not hasattr(opts, k):
                raise TypeError(f"unknown model option {k}")
            setattr(opts, k, int(v))
        handle = ctypes.c_void_p()
        check(self.lib, self.lib.lcr_model_create(str(model_dir).encode(), ctypes.byref(opts),
                                                  ctypes.byref(handle)), "model_create")
        self.handle = handle
        self.options = opts
        st = self.stats()
        self.vocab = st.vocab_size
        self.hidden = st.hidden_size

    def close(self):
        if getattr(self, "handle", None):
            self.lib.lcr_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def stats(self) -> ModelStats:
        st = ModelStats()
        check(self.lib, self.lib.lcr_model_stats_get(self.handle, ctypes.byref(st)), "stats")
        return st

    def prefill(self, tokens) -> int:
        import numpy as np
        arr = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = ctypes.c_void_p()
        check(self.lib, self.lib.lcr_model_prefill(self.handle, arr.ctypes.data, len(arr), ctypes.byref(out)),
              "prefill")
        return out.value

    def decode(self, token: int) -> int:
        out = ctypes.c_void_p()
        check(self.lib, self.lib.lcr_model_decode(self.handle, int(token), ctypes.byref(out)), "decode")
        return out.value

    def logits(self, device_ptr: int):
        import numpy as np
        host = np.empty(self.vocab, dtype=np.float32)
        check(self.lib, self.lib.lcr_model_logits_to_host(self.handle, device_ptr, host.ctypes.data),
              "logits_to_host")
        return host

    def sample(self, device_ptr: int, temperature=0.0, top_k=0, top_p=1.0, uniform=0.0) -> int:
        out = ctypes.c_int32()
        check(self.lib, self.lib.lcr_model_sample(self.handle, device_ptr, float(temperature), int(top_k),
                                                  float(top_p), float(uniform), ctypes.byref(out)), "sample")
        return int(out.value)

    def reset(self):
        check(self.lib, self.lib.lcr_model_reset(self.handle), "reset")

    @property
    def position(self) -> int:
        return int(self.lib.lcr_model_position(self.handle))

    def generate_greedy(self, first_token: int, steps: int):
        import numpy as np
        out = np.zeros(steps, dtype=np.int32)
        ms = ctypes.c_double()
        check(self.lib, self.lib.lcr_model_generate_greedy(self.handle, int(first_token), int(steps),
                                                           out.ctypes.data, ctypes.byref(ms)),
              "generate_greedy")
        return out, ms.value

    def generate_sampled(self, first_token: int, steps: int, temperature: float, top_k: int, top_p: float,
                         uniforms):
        """The reference's decode + sample loop on the device (uniforms[i] is
        the draw of the i-th sampled id)."""
        import numpy as np
        u = np.ascontiguousarray(np.asarray(uniforms, dtype=np.float32))
        if u.size < steps:
            raise LcrError(f"{steps} steps need {steps} draws, got {u.size}")
        out = np.zeros(steps, dtype=np.int32)
        ms = ctypes.c_double()
        check(self.lib, self.lib.lcr_model_generate_sampled(self.handle, int(first_token), int(steps),
                                                            float(temperature), int(top_k), float(top_p),
                                                            u.ctypes.data, out.ctypes.data, ctypes.byref(ms)),
              "generate_sampled")
        return out, ms.value

    def exchange_status(self):
        """(grid, status): which exchange grid decode steps run (0 none, 1 q/k/v
        and attention, 2 with o_proj too), and whether an exchange wait of a
        past step gave up."""
        enabled, status = ctypes.c_int(), ctypes.c_int()
        check(self.lib, self.lib.lcr_model_exchange_status(self.handle, ctypes.byref(enabled),
                                                           ctypes.byref(status)), "exchange_status")
        return int(enabled.value), int(status.value)

    def exchange_clear(self):
        check(self.lib, self.lib.lcr_model_exchange_clear(self.handle), "exchange_clear")

    def time_decode_kernel(self, kernel: str, launches: int = 64):
        ms, nbytes = ctypes.c_double(), ctypes.c_double()
        check(self.lib, self.lib.lcr_model_time_decode_kernel(self.handle, kernel.encode(), int(launches),
                                                              ctypes.byref(ms), ctypes.byref(nbytes)),
              "time_decode_kernel")
        return ms.value, nbytes.value

    def decode_splits(self, seq_len: int) -> int:
        return int(self.lib.lcr_model_decode_splits(self.handle, int(seq_len)))

    def set_capture_activations(self, enabled: bool):
        check(self.lib, self.lib.lcr_model_set_capture_activations(self.handle, 1 if enabled else 0), "taps")

    def taps(self):
        import numpy as np
        n = self.lib.lcr_model_tap_count(self.handle)
        out = {}
        for i in range(n):
            name = ctypes.create_string_buffer(64)
            tokens, width = ctypes.c_int(), ctypes.c_int()
            check(self.lib, self.lib.lcr_model_tap(self.handle, i, name, 64, ctypes.byref(tokens),
                                                   ctypes.byref(width), None, 0), "tap")
            vals = np.empty(tokens.value * width.value, dtype=np.float32)
            check(self.lib, self.lib.lcr_model_tap(self.handle, i, None, 0, None, None, vals.ctypes.data,
                                                   vals.size), "tap")
            out[name.value.decode()] = vals.reshape(tokens.value, width.value)
        return out

    def kv_geometry(self):
        mp, pp, ps, ln = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(self.lib, self.lib.lcr_model_kv_geometry(self.handle, ctypes.byref(mp), ctypes.byref(pp),
                                                       ctypes.byref(ps), ctypes.byref(ln)), "kv_geometry")
        return {"max_pages": mp.value, "pool_pages": pp.value, "page_size": ps.value, "length": ln.value}

    def kv_page_table(self, layer: int):
        import numpy as np
        g = self.kv_geometry()
        out = np.zeros(g["max_pages"], dtype=np.int32)
        check(self.lib, self.lib.lcr_model_kv_page_table(self.handle, layer, out.ctypes.data, out.size),
              "kv_page_table")
        return out

    def set_kv_page_tables(self, tables, length: int):
        import numpy as np
        arr = np.ascontiguousarray(np.asarray(tables, dtype=np.int32).ravel())
        check(self.lib, self.lib.lcr_model_set_kv_page_tables(self.handle, arr.ctypes.data, arr.size, int(length)),
              "set_kv_page_tables")

    def fill_kv_normal(self, seed: int, stddev: float = 1.0):
        check(self.lib, self.lib.lcr_model_fill_kv_normal(self.handle, seed, stddev), "fill_kv_normal")

    def set_position(self, position: int):
        check(self.lib, self.lib.lcr_model_set_position(self.handle, int(position)), "set_position")

    def kv_read(self, layer: int, head: int, position: int, head_dim: int):
        import numpy as np
        k = np.zeros(head_dim, dtype=np.uint16)
        v = np.zeros(head_dim, dtype=np.uint16)
        check(self.lib, self.lib.lcr_model_kv_read(self.handle, layer, head, position, k.ctypes.data,
                                                   v.ctypes.data), "kv_read")
        return k, v

    def kv_export(self, layer: int, positions: int, num_kv_heads: int, head_dim: int):
        """Keys and values of positions [0, positions) of a layer, as uint16
        element bits in logical [kv_head][position][head_dim] order."""
        import numpy as np
        k = np.zeros((num_kv_heads, positions, head_dim), dtype=np.uint16)
        v = np.zeros((num_kv_heads, positions, head_dim), dtype=np.uint16)
        check(self.lib, self.lib.lcr_model_kv_export(self.handle, layer, positions, k.ctypes.data,
                                                     v.ctypes.data), "kv_export")
        return k, v
